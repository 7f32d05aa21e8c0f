"""CSR construction (mlx_cluster_amd.to_csr), on the CPU."""
import numpy as np
import pytest
import torch

import oracle
from mlx_cluster_amd import to_csr
from tests.graphs import csr


def test_matches_hand_csr_and_keeps_empty_rows():
    edges = np.array([[3, 0], [0, 2], [0, 1], [3, 1], [0, 2]])
    rowptr, col = to_csr(edges.T, 5)
    assert rowptr.tolist() == [0, 3, 3, 3, 5, 5]       # nodes 1, 2, 4 have no out-edges
    assert col.tolist() == [1, 2, 2, 0, 1]             # sorted per row, duplicate kept
    rowptr, col = to_csr(edges.T, 5, dedup=True)
    assert rowptr.tolist() == [0, 2, 2, 2, 4, 4] and col.tolist() == [1, 2, 0, 1]
    ref_rowptr, ref_col = csr(5, np.unique(edges, axis=0))
    assert rowptr.tolist() == ref_rowptr.tolist() and col.tolist() == ref_col.tolist()


def test_reference_pipeline_drops_empty_rows():
    """The reference tests' np.unique rowptr (tests/test_random_walk.py:26-28)
    is shorter than V + 1 when a node has no out-edges; to_csr is not."""
    edges = np.array([[0, 1], [2, 0]])
    _, counts = np.unique(edges[:, 0], return_counts=True)
    assert len(np.concatenate([[0], counts.cumsum()])) == 3   # V + 1 would be 4
    rowptr, _ = to_csr(edges.T, 3)
    assert rowptr.numel() == 4


def test_symmetrize_and_validity():
    rng = np.random.default_rng(0)
    e = rng.integers(0, 50, (2, 400))
    rowptr, col = to_csr(e, 50, symmetrize=True, dedup=True)
    assert oracle.csr_flags(rowptr.numpy(), col.numpy()) == 0
    pairs = set(zip(*e.tolist())) | set(zip(e[1].tolist(), e[0].tolist()))
    got = {(u, int(v)) for u in range(50) for v in col[rowptr[u]:rowptr[u + 1]]}
    assert got == pairs


def test_rejects_bad_input():
    with pytest.raises(ValueError):
        to_csr(np.zeros((3, 2), np.int64))
    with pytest.raises(ValueError):
        to_csr(np.array([[0, 5], [1, 1]]), 3)
    rowptr, col = to_csr(torch.zeros((2, 0), dtype=torch.int64), 4)
    assert rowptr.tolist() == [0, 0, 0, 0, 0] and col.numel() == 0
