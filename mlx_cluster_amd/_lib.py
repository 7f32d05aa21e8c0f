"""ctypes binding of libmlxc.so, the HIP library declared in include/mlxc.h.

The library is loaded after torch, so it shares torch's HIP runtime (both
resolve the soname libamdhip64.so.7 to the copy torch has already loaded).
There is no fallback: if the library is missing the import fails loudly.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded first: provides the HIP runtime)

# MLXC_LIB selects another build of the same library (for example one
# compiled with different tuning macros); the default is the in-tree build.
IN_TREE_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmlxc.so")
LIB_PATH = os.environ.get("MLXC_LIB") or IN_TREE_LIB

MLXC_OK = 0
MLXC_ERR_INVALID_ARGUMENT = -1
MLXC_ERR_HIP = -2
MLXC_WORK_WORDS = 4
MLXC_STATUS_BAD_NODE = 1
MLXC_STATUS_BAD_ROW = 2
MLXC_RULE_REF_CHAIN = 0
MLXC_RULE_NODE2VEC_EXACT = 1
MLXC_ROWS_UNSORTED = 0
MLXC_ROWS_SORTED = 1
MLXC_ROWS_DETECT = 2
MLXC_ROWS_SYMMETRIC = 4
MLXC_CSR_BAD_ROWPTR = 1
MLXC_CSR_BAD_COL = 2
MLXC_CSR_UNSORTED = 4
MLXC_CSR_ASYMMETRIC = 8
MLXC_OUT_INT64 = 0
MLXC_OUT_INT32 = 1
MLXC_CSR_SYMMETRIZE = 1
MLXC_CSR_DEDUP = 2
MLXC_MAX_TRIALS = 65536
MLXC_NOALLOC_SCRATCH_BYTES = 64 * 1024 * 1024
MLXC_N2V_LAYOUT_DIRECT = 0
MLXC_N2V_LAYOUT_LDS = 1
MLXC_N2V_LAYOUT_CSR = 2
MLXC_N2V_LAYOUT_RECORDS = 3
MLXC_N2V_LAYOUT_RECORDS_HASH = 4
MLXC_N2V_LAYOUT_RECORDS_FULL = 5

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_u64 = ctypes.c_uint64
_dbl = ctypes.c_double
_ptr = ctypes.c_void_p
_size = ctypes.c_size_t

# name -> (restype, argtypes); every function include/mlxc.h declares.
SIGNATURES = {
    "mlxc_version": (ctypes.c_int, []),
    "mlxc_last_error": (ctypes.c_char_p, []),
    "mlxc_random_walk_workspace_bytes": (_size, [_i64, _i64, _i64, _i32]),
    "mlxc_rejection_sampling_workspace_bytes": (_size, [_i64, _i64, _i64, _i32, _dbl, _dbl, _i32]),
    "mlxc_rejection_sampling_layout_bytes": (_size, [_i64, _i64, _i64, _i32, _i32]),
    "mlxc_random_walk": (
        ctypes.c_int,
        [_ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i32, _ptr, _ptr, _i32, _ptr, _size, _ptr],
    ),
    "mlxc_random_walk_noalloc": (
        ctypes.c_int,
        [_ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i32, _ptr, _ptr, _i32, _ptr, _ptr],
    ),
    "mlxc_random_walk_seeded": (
        ctypes.c_int,
        [_ptr, _i64, _ptr, _i64, _ptr, _i64, _i32, _u64, _i64, _ptr, _ptr, _i32, _ptr, _size,
         _ptr],
    ),
    "mlxc_rejection_sampling": (
        ctypes.c_int,
        [_ptr, _i64, _ptr, _i64, _ptr, _i64, _i32, _dbl, _dbl, _u64, _i64, _i32, _i32,
         _ptr, _ptr, _i32, _ptr, _size, _ptr],
    ),
    "mlxc_csr_check": (ctypes.c_int, [_ptr, _i64, _ptr, _i64, _ptr, _size, _ptr, _ptr]),
    "mlxc_philox_uniform": (ctypes.c_int, [_ptr, _i64, _u64, _ptr]),
    "mlxc_csr_build_workspace_bytes": (_size, [_i64, _i64, _i32]),
    "mlxc_csr_build": (
        ctypes.c_int, [_ptr, _ptr, _i64, _i64, _i32, _ptr, _ptr, _ptr, _size, _ptr],
    ),
    "mlxc_csr_build_cpu": (
        ctypes.c_int, [_ptr, _ptr, _i64, _i64, _i32, _ptr, _ptr, _ptr, _ptr],
    ),
    "mlxc_context_windows": (ctypes.c_int, [_ptr, _i64, _i32, _i32, _i32, _ptr, _ptr]),
    "mlxc_negative_windows": (
        ctypes.c_int, [_ptr, _i64, _i32, _i32, _i64, _u64, _i32, _ptr, _ptr],
    ),
    "mlxc_context_windows_cpu": (ctypes.c_int, [_ptr, _i64, _i32, _i32, _i32, _ptr]),
    "mlxc_negative_windows_cpu": (ctypes.c_int, [_ptr, _i64, _i32, _i32, _i64, _u64, _i32, _ptr]),
    "mlxc_random_walk_cpu": (
        ctypes.c_int,
        [_ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i32, _ptr, _ptr, _i32, _i32, _ptr],
    ),
    "mlxc_random_walk_seeded_cpu": (
        ctypes.c_int,
        [_ptr, _i64, _ptr, _i64, _ptr, _i64, _i32, _u64, _i64, _ptr, _ptr, _i32, _i32, _ptr],
    ),
    "mlxc_set_walk_events": (ctypes.c_int, [_ptr, _ptr]),
    "mlxc_publish_status": (ctypes.c_int, [_ptr, _ptr, _ptr]),
    "mlxc_gather_probe": (
        ctypes.c_int, [_ptr, _i64, _i32, _i32, _i32, _i32, _i64, _u64, _ptr, _ptr, _ptr],
    ),
    "mlxc_rejection_sampling_cpu": (
        ctypes.c_int,
        [_ptr, _i64, _ptr, _i64, _ptr, _i64, _i32, _dbl, _dbl, _u64, _i64, _i32, _i32,
         _ptr, _ptr, _i32, _i32, _ptr],
    ),
}

_lib = None


def load() -> ctypes.CDLL:
    """Returns the loaded library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -m mlx_cluster_amd.build_lib` "
            "(this package has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().mlxc_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc == MLXC_OK:
        return
    msg = last_error()
    if rc == MLXC_ERR_INVALID_ARGUMENT:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")
