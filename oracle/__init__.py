"""numpy wrapper of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared with.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it;
the product (mlx_cluster_amd) never imports it.

Functions follow the reference's CPU evaluation:
  uniform_walk   -> /root/reference/random_walks/RandomWalk.cpp:41-60
  node2vec_walk  -> /root/reference/random_walks/BiasedRandomWalk.cpp:20-28,52-100
  csr_build      -> /root/reference/tests/test_random_walk.py:23-28 (numpy)
  context_windows, negative_windows -> torch_geometric Node2Vec.pos_sample /
                    neg_sample (not in the reference; numpy)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "liboracle.so")

RULE_REF_CHAIN = 0
RULE_NODE2VEC_EXACT = 1
MAX_TRIALS = 65536


class Counts(ctypes.Structure):
    _fields_ = [("moving_steps", ctypes.c_int64), ("sink_walks", ctypes.c_int64),
                ("trials", ctypes.c_int64), ("member_tests", ctypes.c_int64),
                ("member_lines", ctypes.c_int64)]

    def as_dict(self):
        return {k: int(getattr(self, k)) for k, _ in self._fields_}


def build() -> str:
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)
    return LIB_PATH


_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        lib = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i64, i32, u64, u32, dbl = (ctypes.c_int64, ctypes.c_int32, ctypes.c_uint64,
                                   ctypes.c_uint32, ctypes.c_double)
        lib.oracle_philox4x32_10.argtypes = [P, P, P]
        lib.oracle_u32_to_unit_float.argtypes = [u32]
        lib.oracle_u32_to_unit_float.restype = ctypes.c_float
        lib.oracle_philox_uniform_fill.argtypes = [P, i64, u64]
        lib.oracle_philox_uniform_fill_at.argtypes = [P, i64, i64, u64]
        lib.oracle_node2vec_trial0_u0.argtypes = [P, i64, i32, u64]
        lib.oracle_pick_index.argtypes = [ctypes.c_float, i64]
        lib.oracle_pick_index.restype = i64
        lib.oracle_uniform_walk.argtypes = [P, i64, P, i64, P, i64, P, i32, P, P, P]
        lib.oracle_uniform_walk.restype = ctypes.c_int
        lib.oracle_node2vec_probs.argtypes = [dbl, dbl, P]
        lib.oracle_node2vec_walk.argtypes = [P, i64, P, i64, P, i64, i64, i32, dbl, dbl, u64,
                                             i32, i32, P, P, P]
        lib.oracle_node2vec_walk.restype = ctypes.c_int
        lib.oracle_node2vec_walk_libc.argtypes = [P, i64, P, i64, P, i64, i32, dbl, dbl, u32,
                                                  i32, P, P]
        lib.oracle_node2vec_walk_libc.restype = ctypes.c_int
        lib.oracle_csr_flags.argtypes = [P, i64, P, i64]
        lib.oracle_csr_flags.restype = i32
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _i64(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64))


def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    _load().oracle_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def u32_to_unit_float(x: int) -> float:
    return float(np.float32(_load().oracle_u32_to_unit_float(int(x))))


def philox_uniform(n: int, seed: int, first: int = 0) -> np.ndarray:
    """Elements [first, first + n) of the Philox uniform stream of `seed`."""
    out = np.empty(int(n), dtype=np.float32)
    if first == 0:
        _load().oracle_philox_uniform_fill(_p(out), int(n), int(seed) & (2**64 - 1))
    else:
        _load().oracle_philox_uniform_fill_at(_p(out), int(first), int(n), int(seed) & (2**64 - 1))
    return out


def node2vec_trial0_u0(num_walks: int, walk_length: int, seed: int) -> np.ndarray:
    out = np.empty((int(num_walks), int(walk_length)), dtype=np.float32)
    _load().oracle_node2vec_trial0_u0(_p(out), int(num_walks), int(walk_length),
                                      int(seed) & (2**64 - 1))
    return out


def pick_index(r: float, deg: int) -> int:
    return int(_load().oracle_pick_index(float(np.float32(r)), int(deg)))


def uniform_walk(rowptr, col, start, rand, walk_length, *, with_edges=False):
    """Returns (n_out [N, L+1], e_out [N, L] or None, status, counts dict)."""
    rowptr, col, start = _i64(rowptr), _i64(col), _i64(start).reshape(-1)
    rand = np.ascontiguousarray(np.asarray(rand, dtype=np.float32)).reshape(-1)
    N, L = start.size, int(walk_length)
    assert rand.size == N * L
    n_out = np.empty((N, L + 1), dtype=np.int64)
    e_out = np.empty((N, L), dtype=np.int64) if with_edges else None
    counts = Counts()
    st = _load().oracle_uniform_walk(_p(rowptr), rowptr.size - 1, _p(col), col.size, _p(start),
                                     N, _p(rand), L, _p(n_out), _p(e_out),
                                     ctypes.byref(counts))
    return n_out, e_out, st, counts.as_dict()


def node2vec_probs(p: float, q: float) -> np.ndarray:
    out = np.zeros(3, dtype=np.float64)
    _load().oracle_node2vec_probs(float(p), float(q), _p(out))
    return out


def node2vec_walk(rowptr, col, start, walk_length, p, q, seed, *, rule=RULE_REF_CHAIN,
                  rows_sorted=True, with_edges=False, first_walk=0):
    """Returns (n_out, e_out or None, status, counts dict).  Walk n draws from
    the Philox stream of walk index first_walk + n."""
    rowptr, col, start = _i64(rowptr), _i64(col), _i64(start).reshape(-1)
    N, L = start.size, int(walk_length)
    n_out = np.empty((N, L + 1), dtype=np.int64)
    e_out = np.empty((N, L), dtype=np.int64) if with_edges else None
    counts = Counts()
    st = _load().oracle_node2vec_walk(_p(rowptr), rowptr.size - 1, _p(col), col.size, _p(start),
                                      N, int(first_walk), L, float(p), float(q),
                                      int(seed) & (2**64 - 1),
                                      int(rule), 1 if rows_sorted else 0, _p(n_out), _p(e_out),
                                      ctypes.byref(counts))
    return n_out, e_out, st, counts.as_dict()


def node2vec_walk_libc(rowptr, col, start, walk_length, p, q, libc_seed, *,
                       rule=RULE_REF_CHAIN):
    rowptr, col, start = _i64(rowptr), _i64(col), _i64(start).reshape(-1)
    N, L = start.size, int(walk_length)
    n_out = np.empty((N, L + 1), dtype=np.int64)
    st = _load().oracle_node2vec_walk_libc(_p(rowptr), rowptr.size - 1, _p(col), col.size,
                                           _p(start), N, L, float(p), float(q),
                                           int(libc_seed) & 0xFFFFFFFF, int(rule), _p(n_out),
                                           None)
    return n_out, st


def csr_flags(rowptr, col) -> int:
    rowptr, col = _i64(rowptr), _i64(col)
    return int(_load().oracle_csr_flags(_p(rowptr), rowptr.size - 1, _p(col), col.size))


def csr_build(row, col, num_nodes: int, *, symmetrize: bool = False, dedup: bool = False):
    """(rowptr, col) of an edge list, restating the reference tests' pipeline.

    /root/reference/tests/test_random_walk.py:23-28 (and
    test_rejection_sampling.py:22-27) sort the edge index with mlx_graphs
    0.0.7 ``sort_edge_index`` (a dependency absent here; it orders the pairs
    lexicographically by (row, col) and keeps duplicates), then take
    ``rowptr = [0, cumsum(np.unique(row, return_counts=True)[1])]``.  That
    rowptr has no entry for a node without out-edges (and is then not a CSR
    of num_nodes rows); here the counts are ``np.bincount(row,
    minlength=num_nodes)``, which equals the np.unique counts whenever every
    node has an out-edge.  symmetrize appends the reversed pairs first, dedup
    keeps one of each repeated pair.
    """
    row = np.asarray(row, dtype=np.int64).reshape(-1)
    col = np.asarray(col, dtype=np.int64).reshape(-1)
    if symmetrize:
        row, col = np.concatenate([row, col]), np.concatenate([col, row])
    order = np.lexsort((col, row))
    row, col = row[order], col[order]
    if dedup and row.size:
        keep = np.ones(row.size, dtype=bool)
        keep[1:] = (row[1:] != row[:-1]) | (col[1:] != col[:-1])
        row, col = row[keep], col[keep]
    rowptr = np.zeros(num_nodes + 1, dtype=np.int64)
    np.cumsum(np.bincount(row, minlength=num_nodes), out=rowptr[1:])
    return rowptr, col


def philox4x32_10_np(c0, c1, c2, c3, key: int):
    """Philox4x32-10 vectorised over counters (uint64 arrays holding 32-bit
    words), the same rounds as oracle_philox4x32_10 in walk_oracle.c."""
    c0, c1, c2, c3 = (np.asarray(c, dtype=np.uint64) for c in (c0, c1, c2, c3))
    k0, k1 = np.uint64(key & 0xFFFFFFFF), np.uint64((key >> 32) & 0xFFFFFFFF)
    m32 = np.uint64(0xFFFFFFFF)
    for _ in range(10):
        p0 = np.uint64(0xD2511F53) * c0
        p1 = np.uint64(0xCD9E8D57) * c2
        c0, c1, c2, c3 = ((p1 >> np.uint64(32)) ^ c1 ^ k0, p1 & m32,
                          (p0 >> np.uint64(32)) ^ c3 ^ k1, p0 & m32)
        k0 = (k0 + np.uint64(0x9E3779B9)) & m32
        k1 = (k1 + np.uint64(0xBB67AE85)) & m32
    return c0, c1, c2, c3


def context_windows(walks, context_size: int) -> np.ndarray:
    """torch_geometric Node2Vec.pos_sample's windows: for j in range(W), the
    columns j .. j + C - 1 of every walk, concatenated window-major."""
    walks = np.asarray(walks)
    C = int(context_size)
    W = walks.shape[1] - C + 1
    return np.concatenate([walks[:, j:j + C] for j in range(W)], axis=0)


def negative_walks(start, walk_length: int, num_nodes: int, seed: int,
                   walk_ids=None) -> np.ndarray:
    """Node2Vec.neg_sample's walks [start, u_1..u_L] with u_l = (x * V) >> 32,
    x = word 0 of Philox4x32-10(key = seed; counter = (n lo, n hi, l, 0)).
    n is the walk's index, or walk_ids[i] for a sample of walks."""
    start = np.asarray(start, dtype=np.int64).reshape(-1)
    N, L = start.size, int(walk_length)
    ids = np.arange(N) if walk_ids is None else np.asarray(walk_ids).reshape(-1)
    n = np.repeat(ids.astype(np.uint64), L)
    l = np.tile(np.arange(1, L + 1, dtype=np.uint64), N)
    x, _, _, _ = philox4x32_10_np(n & np.uint64(0xFFFFFFFF), n >> np.uint64(32), l,
                                  np.zeros_like(n), int(seed) & (2**64 - 1))
    u = ((x * np.uint64(num_nodes)) >> np.uint64(32)).astype(np.int64).reshape(N, L)
    return np.concatenate([start[:, None], u], axis=1)


def negative_windows(start, walk_length: int, context_size: int, num_nodes: int,
                     seed: int) -> np.ndarray:
    return context_windows(negative_walks(start, walk_length, num_nodes, seed), context_size)
