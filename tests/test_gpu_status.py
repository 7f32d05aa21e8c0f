"""The status bits of malformed input are the same on every kernel path.

Each case of tests/status_cases.py runs through the C ABI with the workspace
that selects each kernel path, and through the host twins; every one must
report the hand-derived bits.  node2vec validates the whole CSR on every
call, so its bits depend neither on the path nor on the seed; the uniform
walk reports what its walks read.
"""
import ctypes
import time

import numpy as np
import pytest
import torch

import mlx_cluster_amd as mc
from mlx_cluster_amd import _lib
from tests import status_cases as sc

pytestmark = pytest.mark.gpu

N2V_MODES = ("lds", "records", "csr", "direct")
ROWS = (_lib.MLXC_ROWS_UNSORTED, _lib.MLXC_ROWS_SORTED, _lib.MLXC_ROWS_DETECT)


def _t(a, cuda):
    return torch.as_tensor(np.asarray(a, dtype=np.int64)).to(cuda)


def _n2v_status(rowptr, col, start, L, seed, rows, mode, cuda):
    lib = _lib.load()
    rowptr, col, start = _t(rowptr, cuda), _t(col, cuda), _t(start, cuda)
    V, E, N = rowptr.numel() - 1, col.numel(), start.numel()
    p, q, rule = 0.5, 2.0, _lib.MLXC_RULE_REF_CHAIN
    query = lambda n_, l_: lib.mlxc_rejection_sampling_workspace_bytes(V, E, n_, l_, p, q, rule)
    layout = {"direct": _lib.MLXC_N2V_LAYOUT_DIRECT, "csr": _lib.MLXC_N2V_LAYOUT_CSR,
              "records": _lib.MLXC_N2V_LAYOUT_RECORDS_FULL, "lds": _lib.MLXC_N2V_LAYOUT_LDS}[mode]
    nbytes = max(lib.mlxc_rejection_sampling_layout_bytes(V, E, N, L, layout), 32)
    if mode == "lds":
        assert query(N, L) == 256  # the query itself selects the LDS walk here
    ws = torch.full(((nbytes + 7) // 8,), -1, dtype=torch.int64, device=cuda)
    n = torch.empty((N, L + 1), dtype=torch.int64, device=cuda)
    e = torch.empty((N, L), dtype=torch.int64, device=cuda)
    rc = lib.mlxc_rejection_sampling(rowptr.data_ptr(), V, col.data_ptr(), E, start.data_ptr(),
                                     N, L, p, q, seed, 0, rule, rows, n.data_ptr(), e.data_ptr(),
                                     _lib.MLXC_OUT_INT64, ws.data_ptr(), nbytes,
                                     torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return int(ws[0].item())


@pytest.mark.parametrize("case", sc.N2V_CASES, ids=[c[0] for c in sc.N2V_CASES])
def test_node2vec_status_same_on_every_path(case, cuda):
    name, rowptr, col, start, want = case
    lib = _lib.load()
    L = 3
    for seed in (0, 1):
        for rows in ROWS:
            got = {mode: _n2v_status(rowptr, col, start, L, seed, rows, mode, cuda)
                   for mode in N2V_MODES}
            got["host"] = sc.host_node2vec_status(lib, rowptr, col, start, L, 0.5, 2.0, seed,
                                                  _lib.MLXC_RULE_REF_CHAIN, rows)
            assert all(v == want for v in got.values()), (name, seed, rows, got)
        if want:
            with pytest.raises(ValueError):
                mc.rejection_sampling(_t(rowptr, cuda), _t(col, cuda), _t(start, cuda), L,
                                      0.5, 2.0, seed=seed)
        else:
            mc.rejection_sampling(_t(rowptr, cuda), _t(col, cuda), _t(start, cuda), L, 0.5, 2.0,
                                  seed=seed)


def _uniform_status(rowptr, col, start, L, mode, seeded, cuda):
    lib = _lib.load()
    rowptr, col, start = _t(rowptr, cuda), _t(col, cuda), _t(start, cuda)
    V, E, N = rowptr.numel() - 1, col.numel(), start.numel()
    nbytes = {"lds": 256, "records": 256 + 16 * (E + N), "csr": 256 + 16 * N, "plain": 32}[mode]
    ws = torch.full(((nbytes + 7) // 8,), -1, dtype=torch.int64, device=cuda)
    n = torch.empty((N, L + 1), dtype=torch.int64, device=cuda)
    e = torch.empty((N, max(L, 1)), dtype=torch.int64, device=cuda)
    stream = torch.cuda.current_stream().cuda_stream
    graph = (rowptr.data_ptr(), V, col.data_ptr(), E, start.data_ptr(), N)
    outs = (n.data_ptr(), e.data_ptr(), _lib.MLXC_OUT_INT64, ws.data_ptr(), nbytes, stream)
    if seeded:
        rc = lib.mlxc_random_walk_seeded(*graph, L, 5, 0, *outs)
    else:
        rand = torch.full((max(N * L, 1),), 0.5, dtype=torch.float32, device=cuda)
        rc = lib.mlxc_random_walk(*graph, rand.data_ptr(), L, *outs)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return int(ws[0].item())


@pytest.mark.parametrize("case", sc.UNI_CASES, ids=[c[0] for c in sc.UNI_CASES])
def test_uniform_status_same_on_every_path(case, cuda):
    """16 walks (the case's starts repeated), so that N * L is a multiple of
    4 and at least 16: the rand tensor then allows the windowed kernels, and
    the record, CSR and LDS workspaces select those walks."""
    name, rowptr, col, start, L, want = case
    lib = _lib.load()
    start = np.resize(np.asarray(start, np.int64), 16)
    for seeded in (False, True):
        got = {mode: _uniform_status(rowptr, col, start, L, mode, seeded, cuda)
               for mode in ("lds", "records", "csr", "plain")}
        got["host"] = sc.host_uniform_status(lib, rowptr, col, start, L,
                                             seed=5 if seeded else None)
        assert all(v == want for v in got.values()), (name, seeded, got)


@pytest.mark.parametrize("case", sc.UNI_CASES, ids=[c[0] for c in sc.UNI_CASES])
def test_published_status_is_the_workspace_word(case, cuda):
    """mlxc_publish_status stores the call's status word into host memory and
    then its flag: the word equals workspace word 0 read back by a copy, and
    the compiled binding's check (which waits on those host words) raises
    exactly when it is non-zero."""
    name, rowptr, col, start, L, want = case
    lib = _lib.load()
    hip = ctypes.CDLL("libamdhip64.so")  # the HIP runtime torch has loaded
    words = ctypes.c_void_p()
    flags = 0x40000000 | 0x2 | 0x1  # hipHostMallocCoherent | Mapped | Portable
    assert hip.hipHostMalloc(ctypes.byref(words), ctypes.c_size_t(16), ctypes.c_uint(flags)) == 0
    try:
        h = (ctypes.c_int64 * 2).from_address(words.value)
        start = np.resize(np.asarray(start, np.int64), 16)
        r, c, s = _t(rowptr, cuda), _t(col, cuda), _t(start, cuda)
        V, E, N = r.numel() - 1, c.numel(), s.numel()
        nbytes = 256 + 16 * (E + N)
        ws = torch.full(((nbytes + 7) // 8,), -1, dtype=torch.int64, device=cuda)
        n = torch.empty((N, L + 1), dtype=torch.int64, device=cuda)
        stream = torch.cuda.current_stream().cuda_stream
        for _ in range(2):  # the second time over the first call's host words
            h[0], h[1] = 0, -1
            rc = lib.mlxc_random_walk_seeded(r.data_ptr(), V, c.data_ptr(), E, s.data_ptr(), N, L,
                                             5, 0, n.data_ptr(), None, _lib.MLXC_OUT_INT64,
                                             ws.data_ptr(), nbytes, stream)
            assert rc == 0, _lib.last_error()
            assert lib.mlxc_publish_status(ws.data_ptr(), words, stream) == 0, _lib.last_error()
            deadline = time.monotonic() + 30
            while h[0] == 0:
                assert time.monotonic() < deadline, "the status was not published"
            assert h[1] == int(ws[0].item()) == want, (name, h[1], want)
    finally:
        torch.cuda.synchronize()
        hip.hipHostFree(words)
    if want:
        with pytest.raises(ValueError):
            mc.random_walk(r, c, s, None, L, seed=5)
    else:
        mc.random_walk(r, c, s, None, L, seed=5)
