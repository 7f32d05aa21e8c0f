"""Parity of the HIP context-window kernels (mlxc_context_windows,
mlxc_negative_windows) with the oracle's restatement of torch_geometric's
Node2Vec.pos_sample / neg_sample: bit-exact."""
import numpy as np
import pytest
import torch

import mlx_cluster_amd as mc
import oracle
from mlx_cluster_amd import synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,nodes,C", [(1, 1, 1), (5, 6, 6), (63, 21, 10), (64, 21, 10),
                                       (65, 21, 10), (1000, 81, 32), (4097, 11, 4),
                                       (3, 601, 5)])
@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_context_windows(N, nodes, C, dtype, cuda):
    rng = np.random.default_rng(N * 3 + nodes + C)
    walks = torch.from_numpy(rng.integers(0, 2**31 - 1, (N, nodes))).to(dtype)
    got = mc.context_windows(walks.to(cuda), C)
    assert got.is_cuda and got.dtype == dtype
    np.testing.assert_array_equal(got.cpu().numpy(), oracle.context_windows(walks.numpy(), C))


def test_context_windows_empty(cuda):
    out = mc.context_windows(torch.zeros((0, 9), dtype=torch.int64, device=cuda), 4)
    assert out.shape == (0, 4) and out.is_cuda


@pytest.mark.parametrize("N,L,C,V", [(1, 0, 1, 5), (63, 20, 10, 1 << 20), (129, 7, 8, 3),
                                     (1000, 80, 32, 1 << 32), (5, 4000, 2, 97),
                                     (70, 8191, 3, 11)])
def test_negative_windows(N, L, C, V, cuda):
    start = torch.arange(N, dtype=torch.int64) * 7 % V
    got = mc.negative_windows(start.to(cuda), L, C, V, seed=77)
    ref = oracle.negative_windows(start.numpy(), L, C, V, 77)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    if V < 2**31 and (L + 1) * 4 <= 65536:
        g32 = mc.negative_windows(start.to(cuda), L, C, V, seed=77, out_dtype=torch.int32)
        np.testing.assert_array_equal(g32.cpu().numpy(), ref.astype(np.int32))


def test_host_twins_equal_device(cuda):
    rowptr, col = synth.rmat_csr(12, 40000, seed=2, device=cuda)
    V = rowptr.numel() - 1
    start = torch.arange(3 * V, device=cuda) % V
    walks = mc.random_walk(rowptr, col, start, None, 20, seed=4)
    d = mc.context_windows(walks, 10)
    h = mc.context_windows(walks.cpu(), 10, stream="cpu")
    assert torch.equal(d.cpu(), h)
    dn = mc.negative_windows(start, 20, 10, V, seed=6)
    hn = mc.negative_windows(start.cpu(), 20, 10, V, seed=6, stream="cpu")
    assert torch.equal(dn.cpu(), hn)


def test_c2_walk_windows_full_size(cuda):
    """torch_geometric's defaults (walk_length 20, context 10, 10 walks per
    node) over configuration 2's graph: 10,485,760 walks -> 125,829,120
    windows.  Every window equals its walk slice (checked on the device with
    torch's unfold); negative windows of every 9973rd walk against the oracle."""
    rowptr, col = synth.rmat_csr(20, 1 << 24, seed=0, device=cuda)
    V = rowptr.numel() - 1
    start = torch.arange(10 * V, device=cuda) % V
    walks = mc.random_walk(rowptr, col, start, None, 20, seed=2)
    out = mc.context_windows(walks, 10)
    N, W = walks.shape[0], 21 - 10 + 1
    assert out.shape == (W * N, 10)
    ref = walks.unfold(1, 10, 1).transpose(0, 1).reshape(W * N, 10)
    assert torch.equal(out, ref)
    neg = mc.negative_windows(start, 20, 10, V, seed=9)
    assert neg.shape == (W * N, 10)
    s = torch.arange(0, N, 9973, device=cuda)
    rw = oracle.negative_walks(start[s].cpu().numpy(), 20, V, 9, walk_ids=s.cpu().numpy())
    for j in range(W):
        np.testing.assert_array_equal(neg[j * N + s].cpu().numpy(), rw[:, j:j + 10])
