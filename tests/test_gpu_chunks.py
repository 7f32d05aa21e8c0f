"""Walk offsets and chunked calls on the GPU.

A call over walks [i0, i1) of a batch with walk_offset=i0 gives rows
i0 .. i1-1 of the whole batch's call, bit for bit: the seeded uniform walk
keys its uniforms by stream position (walk_offset + n) * L + l, the node2vec
walk its Philox counter by walk walk_offset + n, as the reference's loops
index walks globally (RandomWalk.cpp:41, BiasedRandomWalk.cpp:57).  A call
under a memory budget smaller than its outputs runs in such chunks into
pinned host memory and equals the unchunked call; one whose workspace alone
does not fit runs a smaller layout with the same walks.
"""
import numpy as np
import pytest
import torch

import mlx_cluster_amd as mc
import oracle
from mlx_cluster_amd import synth

pytestmark = pytest.mark.gpu


def _cuts(N):
    """Four ragged slices of [0, N)."""
    return [0, N // 4 + 13, N // 2, 3 * N // 4 - 5, N]


def test_c3_four_slices_equal_single_call(cuda):
    """Configuration 3 (node2vec p=0.5 q=2, symmetrized R-MAT 2^20, 4 walks
    per node, L=40) as four slices with walk offsets equals the single call,
    nodes and edges, and 1,000 walks at the head of every slice equal
    oracle.node2vec_walk(first_walk=i0)."""
    rowptr, col = synth.rmat_csr(20, 1 << 24, seed=0, device=cuda, symmetrize=True)
    V = rowptr.numel() - 1
    N, L = 4 * V, 40
    start = torch.arange(N, device=cuda) % V
    kw = dict(seed=3, return_edges=True)
    n, e = mc.rejection_sampling(rowptr, col, start, L, 0.5, 2.0, **kw)
    rp, cl = rowptr.cpu().numpy(), col.cpu().numpy()
    cuts = _cuts(N)
    for i0, i1 in zip(cuts[:-1], cuts[1:]):
        print(f"c3 slice [{i0}, {i1})", flush=True)
        pn, pe = mc.rejection_sampling(rowptr, col, start[i0:i1], L, 0.5, 2.0, walk_offset=i0,
                                       **kw)
        assert torch.equal(pn, n[i0:i1]) and torch.equal(pe, e[i0:i1])
        ref, ref_e, st, _ = oracle.node2vec_walk(rp, cl, start[i0:i0 + 1000].cpu().numpy(), L,
                                                 0.5, 2.0, 3, rule=oracle.RULE_REF_CHAIN,
                                                 with_edges=True, first_walk=i0)
        assert st == 0
        np.testing.assert_array_equal(pn[:1000].cpu().numpy(), ref)
        np.testing.assert_array_equal(pe[:1000].cpu().numpy(), ref_e)


def test_c2_seeded_four_slices_equal_single_call(cuda):
    """Configuration 2 with generated uniforms (R-MAT 2^20, 10 walks per
    node, L=80, seed 2) as four slices with walk offsets equals the single
    call; 2,000 walks at the head of every slice equal the oracle's walk on
    the stream elements [i0 * L, (i0 + 2000) * L)."""
    rowptr, col = synth.rmat_csr(20, 1 << 24, seed=0, device=cuda)
    V = rowptr.numel() - 1
    N, L = 10 * V, 80
    start = torch.arange(N, device=cuda) % V
    n = mc.random_walk(rowptr, col, start, None, L, seed=2)
    rp, cl = rowptr.cpu().numpy(), col.cpu().numpy()
    cuts = _cuts(N)
    for i0, i1 in zip(cuts[:-1], cuts[1:]):
        print(f"c2s slice [{i0}, {i1})", flush=True)
        part = mc.random_walk(rowptr, col, start[i0:i1], None, L, seed=2, walk_offset=i0)
        assert torch.equal(part, n[i0:i1])
        del part
        rand = oracle.philox_uniform(2000 * L, 2, first=i0 * L).reshape(2000, L)
        ref, _, st, _ = oracle.uniform_walk(rp, cl, start[i0:i0 + 2000].cpu().numpy(), rand, L)
        assert st == 0
        np.testing.assert_array_equal(n[i0:i0 + 2000].cpu().numpy(), ref)


def test_c2_seeded_under_a_small_budget(cuda):
    """Configuration 2 with generated uniforms under a 1 GiB budget (its
    output is 6.8 GB): the call runs in chunks into pinned host memory and
    equals the unchunked call."""
    rowptr, col = synth.rmat_csr(20, 1 << 24, seed=0, device=cuda)
    V = rowptr.numel() - 1
    N, L = 10 * V, 80
    start = torch.arange(N, device=cuda) % V
    whole = mc.random_walk(rowptr, col, start, None, L, seed=2).cpu()
    torch.cuda.empty_cache()
    got = mc.random_walk(rowptr, col, start, None, L, seed=2, memory_budget=1 << 30)
    assert got.device.type == "cpu" and got.is_pinned()
    assert torch.equal(got, whole)


def _walk(kind, rowptr, col, start, L, rand, **kw):
    if kind == "uniform":
        return mc.random_walk(rowptr, col, start, rand, L, return_edges=True, **kw)
    if kind == "seeded":
        return mc.random_walk(rowptr, col, start, None, L, seed=9, return_edges=True, **kw)
    rule = "node2vec" if kind == "n2v_exact" else "ref_chain"
    return mc.rejection_sampling(rowptr, col, start, L, 0.5, 2.0, seed=9, rule=rule,
                                 return_edges=True, **kw)


@pytest.mark.parametrize("out_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("kind", ["uniform", "seeded", "n2v_chain", "n2v_exact"])
def test_budgets_equal_the_unchunked_call(kind, out_dtype, cuda):
    """Budgets below the outputs (chunks of 64-walk multiples, a chunk of
    fewer than 64 walks, both through pinned host memory), and budgets that
    hold the outputs but not the fastest workspace (a shrunk workspace: the
    edge records without hub bitmaps, the CSR mode or start records, the
    direct kernels), all equal the unchunked call."""
    rowptr, col = synth.rmat_csr(16, 1 << 20, seed=4, device=cuda, symmetrize=True)
    V = rowptr.numel() - 1
    N, L = 300_001, 20
    start = (torch.arange(N, device=cuda) * 7) % V
    rand = mc.philox_uniform((N, L), 5, device=cuda)
    kw = dict(out_dtype=out_dtype)
    n, e = _walk(kind, rowptr, col, start, L, rand, **kw)
    row_bytes = (2 * L + 1) * n.element_size()
    outs = N * row_bytes
    lib = mc._lib.load()
    if kind in ("uniform", "seeded"):
        ws = lib.mlxc_random_walk_workspace_bytes(V, col.numel(), N, L)
    else:
        ws = lib.mlxc_rejection_sampling_workspace_bytes(V, col.numel(), N, L, 0.5, 2.0,
                                                         int(kind == "n2v_exact"))
    for budget in (outs // 5, outs // 3 + 12345, 2 * 50 * row_bytes + 64,
                   outs + ws - 1, outs + ws // 2, outs + 4096, outs + 64):
        print(f"{kind} {out_dtype} budget {budget} (outputs {outs}, workspace {ws})", flush=True)
        gn, ge = _walk(kind, rowptr, col, start, L, rand, memory_budget=budget, **kw)
        assert gn.device.type == ("cpu" if budget < outs else "cuda")
        assert torch.equal(gn.cpu(), n.cpu()) and torch.equal(ge.cpu(), e.cpu())


def test_chunked_call_reports_a_bad_start_in_a_later_chunk(cuda):
    """The status bits of every chunk reach the caller: a start out of range
    in the last chunk raises ValueError, as in the unchunked call."""
    rowptr, col = synth.rmat_csr(12, 40_000, seed=1, device=cuda)
    V = rowptr.numel() - 1
    N, L = 10_000, 10
    start = torch.arange(N, device=cuda) % V
    start[-1] = V + 3
    for budget in (None, N * (L + 1) * 8 // 4):
        with pytest.raises(ValueError, match="outside"):
            mc.random_walk(rowptr, col, start, None, L, seed=1, memory_budget=budget)
        with pytest.raises(ValueError, match="outside"):
            mc.rejection_sampling(rowptr, col, start, L, 1.0, 2.0, seed=1, memory_budget=budget)


def test_chunked_call_on_a_side_stream(cuda):
    """A chunked call given a torch.cuda.Stream runs its chunks there and
    still equals the unchunked call on torch's current stream."""
    rowptr, col = synth.rmat_csr(14, 200_000, seed=2, device=cuda, symmetrize=True)
    V = rowptr.numel() - 1
    N, L = 50_000, 15
    start = torch.arange(N, device=cuda) % V
    want = mc.rejection_sampling(rowptr, col, start, L, 2.0, 0.5, seed=4, rule="node2vec")
    side = torch.cuda.Stream(cuda)
    got = mc.rejection_sampling(rowptr, col, start, L, 2.0, 0.5, seed=4, rule="node2vec",
                                stream=side, memory_budget=N * (L + 1) * 8 // 6)
    assert torch.equal(got, want.cpu())
