"""Skip-gram context windows on the CPU: the host twins
(mlxc_context_windows_cpu, mlxc_negative_windows_cpu) against the oracle's
restatement of torch_geometric's Node2Vec.pos_sample / neg_sample."""
import numpy as np
import pytest
import torch

import mlx_cluster_amd as mc
import oracle
from mlx_cluster_amd import _lib


@pytest.mark.parametrize("N,nodes,C", [(0, 5, 3), (1, 1, 1), (5, 6, 6), (100, 21, 10),
                                       (3, 81, 32), (257, 11, 4)])
@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_context_windows_host(N, nodes, C, dtype):
    rng = np.random.default_rng(N + nodes + C)
    walks = torch.from_numpy(rng.integers(0, 2**31 - 1, (N, nodes))).to(dtype)
    got = mc.context_windows(walks, C, stream="cpu")
    assert got.dtype == dtype and got.shape == ((nodes - C + 1) * N, C)
    np.testing.assert_array_equal(got.numpy(), oracle.context_windows(walks.numpy(), C))


@pytest.mark.parametrize("N,L,C,V", [(0, 4, 2, 10), (1, 0, 1, 5), (50, 20, 10, 1 << 20),
                                     (300, 7, 8, 3), (9, 80, 32, (1 << 32))])
def test_negative_windows_host(N, L, C, V):
    start = torch.arange(N, dtype=torch.int64) * 7 % max(V, 1)
    got = mc.negative_windows(start, L, C, V, seed=123, stream="cpu")
    np.testing.assert_array_equal(got.numpy(),
                                  oracle.negative_windows(start.numpy(), L, C, V, 123))
    if V < 2**31:
        g32 = mc.negative_windows(start, L, C, V, seed=123, stream="cpu", out_dtype=torch.int32)
        assert g32.dtype == torch.int32 and torch.equal(g32.long(), got)


def test_seed_default_follows_torch_generator():
    torch.manual_seed(3)
    a = mc.negative_windows(torch.arange(10), 5, 3, 100, stream="cpu")
    torch.manual_seed(3)
    b = mc.negative_windows(torch.arange(10), 5, 3, 100, stream="cpu")
    assert torch.equal(a, b)


def test_argument_checks():
    w = torch.zeros((2, 5), dtype=torch.int64)
    with pytest.raises(ValueError):
        mc.context_windows(w, 6, stream="cpu")
    with pytest.raises(ValueError):
        mc.context_windows(w, 0, stream="cpu")
    with pytest.raises(ValueError):
        mc.context_windows(torch.zeros((2, 40), dtype=torch.int64), 33, stream="cpu")
    with pytest.raises(TypeError):
        mc.context_windows(w.float(), 2, stream="cpu")
    with pytest.raises(ValueError):
        mc.context_windows(torch.zeros(5, dtype=torch.int64), 2, stream="cpu")
    with pytest.raises(ValueError):
        mc.negative_windows(torch.arange(3), 3, 5, 10, seed=1, stream="cpu")
    with pytest.raises(ValueError, match="num_nodes"):
        mc.negative_windows(torch.arange(3), 3, 2, 0, seed=1, stream="cpu")
    with pytest.raises(ValueError, match="num_nodes"):
        mc.negative_windows(torch.arange(3), 3, 2, 2**31, seed=1, stream="cpu",
                            out_dtype=torch.int32)
    with pytest.raises(ValueError, match="nodes per walk"):
        mc.negative_windows(torch.arange(3), 8192, 2, 10, seed=1, stream="cpu")
    with pytest.raises(ValueError, match="nodes per walk"):
        mc.context_windows(torch.zeros((2, 16385), dtype=torch.int32), 2, stream="cpu")
    mc.context_windows(torch.zeros((2, 16384), dtype=torch.int32), 2, stream="cpu")
    lib = _lib.load()
    p = w.data_ptr()
    # device entry points validate before any HIP call
    assert lib.mlxc_context_windows(p, 2, 5, 0, 0, p, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_context_windows(p, 2, 5, 2, 7, p, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_context_windows(None, 2, 5, 2, 0, p, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_negative_windows(p, 2, 4, 2, 0, 1, 0, p, None) == \
        _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_negative_windows(p, 2, -1, 1, 5, 1, 0, p, None) == \
        _lib.MLXC_ERR_INVALID_ARGUMENT
