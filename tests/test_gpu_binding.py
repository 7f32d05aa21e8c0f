"""The compiled fast path of the Python surface (mlx_cluster_amd/_mlxc_torch,
built from csrc/torch_binding.cpp) against the general path and the oracle.

The common call (tensors of the right dtype on the current device, torch's
current stream) goes through the compiled module; every other call through
walks.py's general path.  Both run the same libmlxc.so entry points, so the
walks, edge ids and errors must be the same."""
import numpy as np
import pytest
import torch

import mlx_cluster_amd as mc
import oracle
from mlx_cluster_amd import synth, walks

pytestmark = pytest.mark.gpu


@pytest.fixture
def general_path(monkeypatch):
    monkeypatch.setattr(walks, "_fast", None)


def _graph(cuda):
    rowptr, col = synth.rmat_csr(12, 40_000, seed=3, symmetrize=True)
    return rowptr.to(cuda), col.to(cuda)


def test_binding_is_built_and_loaded():
    assert walks._fast is not None, "the compiled fast path (_mlxc_torch) was not built"


@pytest.mark.parametrize("kw", [dict(), dict(return_edges=True), dict(out_dtype=torch.int32),
                                dict(return_edges=True, out_dtype=torch.int32)])
def test_uniform_same_as_general_path_and_oracle(kw, cuda, monkeypatch):
    rowptr, col = _graph(cuda)
    V, L = rowptr.numel() - 1, 9
    start = torch.arange(3000, device=cuda) % V
    rand = mc.philox_uniform((3000, L), 4, device=cuda)
    fast_r = mc.random_walk(rowptr, col, start, rand, L, **kw)
    fast_s = mc.random_walk(rowptr, col, start, None, L, seed=4, **kw)
    monkeypatch.setattr(walks, "_fast", None)
    slow_r = mc.random_walk(rowptr, col, start, rand, L, **kw)
    slow_s = mc.random_walk(rowptr, col, start, None, L, seed=4, **kw)
    as_tuple = lambda r: r if isinstance(r, tuple) else (r,)
    for a, b in ((fast_r, slow_r), (fast_s, slow_s), (fast_r, fast_s)):
        for x, y in zip(as_tuple(a), as_tuple(b)):
            assert x.dtype == y.dtype and torch.equal(x, y)
    ref, _, st, _ = oracle.uniform_walk(rowptr.cpu().numpy(), col.cpu().numpy(),
                                        start.cpu().numpy(), rand.cpu().numpy(), L)
    assert st == 0
    np.testing.assert_array_equal(as_tuple(fast_r)[0].long().cpu().numpy(), ref)


@pytest.mark.parametrize("rule", ["ref_chain", "node2vec"])
def test_node2vec_same_as_general_path_and_oracle(rule, cuda, monkeypatch):
    rowptr, col = _graph(cuda)
    V, L = rowptr.numel() - 1, 11
    start = torch.arange(2500, device=cuda) % V
    kw = dict(seed=6, rule=rule, return_edges=True)
    fast = mc.rejection_sampling(rowptr, col, start, L, 0.5, 2.0, **kw)
    fast32 = mc.rejection_sampling(rowptr, col, start, L, 0.5, 2.0, out_dtype=torch.int32, **kw)
    monkeypatch.setattr(walks, "_fast", None)
    slow = mc.rejection_sampling(rowptr, col, start, L, 0.5, 2.0, **kw)
    assert torch.equal(fast[0], slow[0]) and torch.equal(fast[1], slow[1])
    assert torch.equal(fast[0], fast32[0].long()) and torch.equal(fast[1], fast32[1].long())
    ref, ref_e, st, _ = oracle.node2vec_walk(rowptr.cpu().numpy(), col.cpu().numpy(),
                                             start.cpu().numpy(), L, 0.5, 2.0, 6,
                                             rule={"ref_chain": 0, "node2vec": 1}[rule],
                                             with_edges=True)
    assert st == 0
    np.testing.assert_array_equal(fast[0].cpu().numpy(), ref)
    np.testing.assert_array_equal(fast[1].cpu().numpy(), ref_e)


def test_errors_as_in_the_general_path(cuda):
    """Malformed starts raise ValueError from the compiled path (check=True);
    with check=False the call returns without synchronising; calls it does
    not take (numpy inputs, 2-D starts, wrong dtypes, a bad rand size) get the
    general path's errors or results."""
    rowptr, col = _graph(cuda)
    V, L = rowptr.numel() - 1, 5
    start = torch.arange(100, device=cuda) % V
    bad = start.clone()
    bad[7] = V + 5
    rand = mc.philox_uniform((100, L), 1, device=cuda)
    with pytest.raises(ValueError, match="outside"):
        mc.random_walk(rowptr, col, bad, rand, L)
    with pytest.raises(ValueError, match="outside"):
        mc.rejection_sampling(rowptr, col, bad, L, 1.0, 1.0, seed=2)
    mc.random_walk(rowptr, col, bad, rand, L, check=False)
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match="num_walks"):
        mc.random_walk(rowptr, col, start, rand[:50], L)
    with pytest.raises(TypeError):
        mc.random_walk(rowptr.int(), col, start, rand, L)
    a = mc.random_walk(rowptr, col, start.reshape(10, 10), rand, L)
    b = mc.random_walk(rowptr.cpu().numpy(), col.cpu().numpy(), start.cpu().numpy(),
                       rand.cpu().numpy(), L)
    assert torch.equal(a, b) and torch.equal(a, mc.random_walk(rowptr, col, start, rand, L))
