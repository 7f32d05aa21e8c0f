"""Small hand-built graphs and independent checks shared by the tests."""
from __future__ import annotations

import numpy as np


def csr(num_nodes, edges, *, sort=True):
    """CSR (rowptr, col) of a directed edge list; rows sorted when sort=True
    (otherwise the edge-list order inside each row is kept)."""
    edges = np.asarray(edges, dtype=np.int64).reshape(-1, 2)
    order = np.lexsort((edges[:, 1], edges[:, 0])) if sort else np.argsort(edges[:, 0], kind="stable")
    edges = edges[order]
    rowptr = np.zeros(num_nodes + 1, dtype=np.int64)
    np.cumsum(np.bincount(edges[:, 0], minlength=num_nodes), out=rowptr[1:])
    return rowptr, edges[:, 1].copy()


def undirected(num_nodes, pairs, **kw):
    pairs = np.asarray(pairs, dtype=np.int64).reshape(-1, 2)
    return csr(num_nodes, np.concatenate([pairs, pairs[:, ::-1]]), **kw)


def uniform_transitions_ok(rowptr, col, start, rand, walks):
    """Checks every step of uniform walks with numpy's IEEE float32 arithmetic.

    For each step (u -> v) with uniform r: deg(u) == 0 must give v == u;
    otherwise v == col[rowptr[u] + trunc(f32(r) * f32(deg))] (clamped to the
    row).  Independent of the C oracle: vectorised numpy, not a loop port.
    Returns the number of violating steps.
    """
    rowptr, col = np.asarray(rowptr), np.asarray(col)
    walks = np.asarray(walks)
    N, L1 = walks.shape
    L = L1 - 1
    rand = np.asarray(rand, dtype=np.float32).reshape(N, L)
    bad = int(np.count_nonzero(walks[:, 0] != np.asarray(start).reshape(-1)))
    for l in range(L):
        u, v = walks[:, l], walks[:, l + 1]
        deg = rowptr[u + 1] - rowptr[u]
        prod = rand[:, l] * deg.astype(np.float32)          # float32 * float32 -> float32
        idx = np.minimum(np.trunc(prod).astype(np.int64), np.maximum(deg - 1, 0))
        moving = deg > 0
        expect = np.where(moving, col[np.where(moving, rowptr[u] + idx, 0)], u)
        bad += int(np.count_nonzero(expect != v))
    return bad
