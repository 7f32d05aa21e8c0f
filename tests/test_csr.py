"""CSR construction (mlx_cluster_amd.to_csr) on the CPU: the host twin
mlxc_csr_build_cpu against the oracle's restatement of the reference tests'
pipeline (tests/test_random_walk.py:23-28)."""
import numpy as np
import pytest
import torch

import oracle
from mlx_cluster_amd import _lib, to_csr
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


@pytest.mark.parametrize("V,E", [(1, 10), (7, 0), (300, 5000), (70000, 20000), (3_000_001, 9000)])
@pytest.mark.parametrize("symmetrize", [False, True])
@pytest.mark.parametrize("dedup", [False, True])
def test_host_twin_matches_oracle(V, E, symmetrize, dedup):
    rng = np.random.default_rng(V + E)
    row, col = rng.integers(0, V, E), rng.integers(0, V, E)
    row[: E // 3] = row[0] if E else 0       # a heavy row with repeated pairs
    col[: E // 6] = col[0] if E else 0
    rowptr, c = to_csr(np.stack([row, col]), V, symmetrize=symmetrize, dedup=dedup)
    ref_rowptr, ref_col = oracle.csr_build(row, col, V, symmetrize=symmetrize, dedup=dedup)
    np.testing.assert_array_equal(rowptr.numpy(), ref_rowptr)
    np.testing.assert_array_equal(c.numpy(), ref_col)


def test_default_num_nodes_and_int32_input():
    e = torch.tensor([[2, 0, 2], [1, 2, 0]], dtype=torch.int32)
    rowptr, col = to_csr(e)
    assert rowptr.tolist() == [0, 1, 1, 3] and col.tolist() == [2, 0, 1]


def test_rejects_bad_input():
    with pytest.raises(ValueError):
        to_csr(np.zeros((3, 2), np.int64))
    with pytest.raises(ValueError, match="outside"):
        to_csr(np.array([[0, 5], [1, 1]]), 3)
    with pytest.raises(ValueError, match="outside"):
        to_csr(np.array([[0, 1], [-1, 1]]), 3, symmetrize=True)
    with pytest.raises(TypeError):
        to_csr(np.zeros((2, 3), np.float32))
    with pytest.raises(ValueError):
        to_csr(np.zeros((2, 0), np.int64), (1 << 32) + 1)
    rowptr, col = to_csr(torch.zeros((2, 0), dtype=torch.int64), 4)
    assert rowptr.tolist() == [0, 0, 0, 0, 0] and col.numel() == 0
    rowptr, col = to_csr(torch.zeros((2, 0), dtype=torch.int64))
    assert rowptr.tolist() == [0] and col.numel() == 0


def test_abi_argument_checks():
    lib = _lib.load()
    buf = torch.zeros(8, dtype=torch.int64)
    p = buf.data_ptr()
    count = _lib.ctypes.c_int64(0)
    cp = _lib.ctypes.addressof(count)
    assert lib.mlxc_csr_build_cpu(p, p, 2, 4, 4, p, p, cp, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_csr_build_cpu(p, p, 2, -1, 0, p, p, cp, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_csr_build_cpu(None, p, 2, 4, 0, p, p, cp, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_csr_build_cpu(p, p, 2, 4, 0, None, p, cp, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_csr_build_cpu(p, p, 2, 4, 0, p, p, None, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    # the device entry point validates before any HIP call
    assert lib.mlxc_csr_build(p, p, 2, 4, 8, p, p, p, 64, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_csr_build(p, p, 2, 4, 0, p, p, None, 64, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_csr_build(p, p, 2, 4, 0, p, p, p, 1, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    need = lib.mlxc_csr_build_workspace_bytes(4, 2, 0)
    assert lib.mlxc_csr_build(p, p, 2, 4, 0, p, p, p, need - 1, None) == \
        _lib.MLXC_ERR_INVALID_ARGUMENT
    assert "workspace" in _lib.last_error()


def test_workspace_bytes():
    lib = _lib.load()
    # keys of 4 bytes up to 65536 nodes, 5 up to 2^20, 6 up to 2^24, 8 above;
    # two key arrays each, plus a digit byte per entry
    E = 1 << 20
    small = lib.mlxc_csr_build_workspace_bytes(65536, E, 0)
    k5 = lib.mlxc_csr_build_workspace_bytes(65537, E, 0)
    k6 = lib.mlxc_csr_build_workspace_bytes((1 << 20) + 1, E, 0)
    wide = lib.mlxc_csr_build_workspace_bytes((1 << 24) + 1, E, 0)
    assert small >= (2 * 4 + 1) * E and k5 >= (2 * 5 + 1) * E
    assert k6 >= (2 * 6 + 1) * E and wide >= (2 * 8 + 1) * E
    assert k5 - small >= 2 * E and k6 - k5 >= 2 * E and wide - k6 >= 2 * 2 * E
    sym = lib.mlxc_csr_build_workspace_bytes(65537, E, _lib.MLXC_CSR_SYMMETRIZE)
    assert sym >= (2 * 5 + 1) * (2 * E)
    assert lib.mlxc_csr_build_workspace_bytes(-1, 5, 0) == 0
