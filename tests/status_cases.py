"""Malformed graphs and the MLXC_STATUS_* bits every walk path must report.

The contract (include/mlxc.h):
- mlxc_rejection_sampling validates the whole CSR on every call, whatever the
  kernel path and the MLXC_ROWS_* value: BAD_ROW for rowptr[0] != 0,
  rowptr[V] != E or a rowptr entry outside [0, E] / decreasing, BAD_NODE for a
  col value outside [0, V); BAD_NODE also for a start outside [0, V).
- mlxc_random_walk reports what its walks read, the entries the reference's
  loop reads (RandomWalk.cpp:45-54): BAD_NODE for a start or a chosen col value
  outside [0, V), BAD_ROW for the rowptr pair of a node a walk leaves.  The row
  of the node a walk ends at is not read.

The expected bits below are derived by hand from those rules (the walks on
these graphs have out-degree 1 everywhere, so they do not depend on the
uniforms), not from any implementation.
"""
from __future__ import annotations

import ctypes

import numpy as np

BAD_NODE = 1
BAD_ROW = 2

# node2vec: the graph {(0,1), (0,3), (2,1)} on 4 nodes, rowptr [0,2,2,3,3],
# col [1,3,1], and malformed variants.  Seed 0 draws candidate 0 of row(0)
# for walk 0's first step, seed 1 candidate 1 (u0 = 0.399 and 0.890), so one
# seed meets col[1] and the other does not; the bits must not depend on it.
N2V_ROWPTR = [0, 2, 2, 3, 3]
N2V_COL = [1, 3, 1]
N2V_CASES = [
    # (name, rowptr, col, start, expected bits)
    ("well formed", N2V_ROWPTR, N2V_COL, [0, 2, 1, 3], 0),
    ("bad start", N2V_ROWPTR, N2V_COL, [0, 9, 1, 3], BAD_NODE),
    ("negative start", N2V_ROWPTR, N2V_COL, [0, -1], BAD_NODE),
    ("bad col", N2V_ROWPTR, [1, 9, 1], [0, 2, 1, 3], BAD_NODE),
    ("bad col not met", N2V_ROWPTR, [1, 3, -5], [1, 3], BAD_NODE),
    ("decreasing rowptr", [0, 2, 1, 3, 3], N2V_COL, [0, 2, 1, 3], BAD_ROW),
    ("rowptr[V] != E", [0, 1, 1, 2, 2], N2V_COL, [0, 2], BAD_ROW),
    ("rowptr[0] != 0", [1, 2, 2, 3, 3], N2V_COL, [3], BAD_ROW),
    ("rowptr entry > E", [0, 2, 7, 3, 3], N2V_COL, [1], BAD_ROW),
    ("bad col and row", [0, 2, 1, 3, 3], [1, 9, 1], [0], BAD_NODE | BAD_ROW),
    ("all three", [0, 2, 1, 3, 3], [1, 9, 1], [0, 4], BAD_NODE | BAD_ROW),
]

# uniform: the directed 4-cycle 0 -> 1 -> 2 -> 3 -> 0, rowptr [0,1,2,3,4],
# col [1,2,3,0]; every node has out-degree 1, so walks are fixed.
UNI_ROWPTR = [0, 1, 2, 3, 4]
UNI_COL = [1, 2, 3, 0]
UNI_CASES = [
    # (name, rowptr, col, start, walk_length, expected bits)
    ("well formed", UNI_ROWPTR, UNI_COL, [0, 1, 2, 3], 4, 0),
    ("bad start", UNI_ROWPTR, UNI_COL, [0, 9, 1, 3], 3, BAD_NODE),
    ("bad start, L = 0", UNI_ROWPTR, UNI_COL, [0, 9], 0, BAD_NODE),
    # walk from 0 picks col[2] = 7 at its third step
    ("bad col met", UNI_ROWPTR, [1, 2, 7, 0], [0, 3], 3, BAD_NODE),
    # no walk of length 1 from 0 or 1 reaches col[2]
    ("bad col not met", UNI_ROWPTR, [1, 2, 7, 0], [0, 1], 1, 0),
    # the walk leaves node 2, whose row [2, 9) is outside [0, E]
    ("bad row left", [0, 1, 2, 9, 4], UNI_COL, [2, 2], 3, BAD_ROW),
    # row(3) = [3, 9) is malformed: a walk 0 -> 1 -> 2 -> 3 of length 3 ends
    # at 3 without reading it; length 4 leaves 3 and reads it
    ("bad row at the end", [0, 1, 2, 3, 9], UNI_COL, [0, 0, 0, 0], 3, 0),
    ("bad row left at the end", [0, 1, 2, 3, 9], UNI_COL, [0, 0, 0, 0], 4, BAD_ROW),
    ("bad start row, L = 0", [0, 1, 2, 3, 9], UNI_COL, [3, 3], 0, 0),
    ("decreasing row left", [0, 2, 1, 3, 4], UNI_COL, [1], 2, BAD_ROW),
]


def i64(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64))


def host_uniform_status(lib, rowptr, col, start, L, *, seed=None, rand=None):
    """MLXC_STATUS_* bits of mlxc_random_walk_cpu / _seeded_cpu."""
    rowptr, col, start = i64(rowptr), i64(col), i64(start)
    N = start.size
    n_out = np.empty((N, L + 1), np.int64)
    e_out = np.empty((N, max(L, 1)), np.int64)
    status = ctypes.c_int64(-1)
    p = lambda a: a.ctypes.data
    if seed is None:
        rand = np.ascontiguousarray(np.full(max(N * L, 1), 0.5, np.float32) if rand is None
                                    else np.asarray(rand, np.float32))
        rc = lib.mlxc_random_walk_cpu(p(rowptr), rowptr.size - 1, p(col), col.size, p(start), N,
                                      p(rand), L, p(n_out), p(e_out), 0, 2,
                                      ctypes.addressof(status))
    else:
        rc = lib.mlxc_random_walk_seeded_cpu(p(rowptr), rowptr.size - 1, p(col), col.size,
                                             p(start), N, L, seed, 0, p(n_out), p(e_out), 0, 2,
                                             ctypes.addressof(status))
    assert rc == 0
    return int(status.value)


def host_node2vec_status(lib, rowptr, col, start, L, p, q, seed, rule, rows):
    """MLXC_STATUS_* bits of mlxc_rejection_sampling_cpu."""
    rowptr, col, start = i64(rowptr), i64(col), i64(start)
    N = start.size
    n_out = np.empty((N, L + 1), np.int64)
    e_out = np.empty((N, max(L, 1)), np.int64)
    status = ctypes.c_int64(-1)
    ptr = lambda a: a.ctypes.data
    rc = lib.mlxc_rejection_sampling_cpu(ptr(rowptr), rowptr.size - 1, ptr(col), col.size,
                                         ptr(start), N, L, p, q, seed, 0, rule, rows, ptr(n_out),
                                         ptr(e_out), 0, 2, ctypes.addressof(status))
    assert rc == 0
    return int(status.value)
