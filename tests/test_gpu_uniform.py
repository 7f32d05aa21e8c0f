"""Parity of the HIP uniform walk (libmlxc.so) with the CPU oracle.

Bit-exact: node sequences and edge ids must equal the oracle's restatement of
RandomWalk.cpp:41-60 for the same rand tensor.
"""
import numpy as np
import pytest
import torch

import mlx_cluster_amd as mc
import oracle
from mlx_cluster_amd import synth
from tests.graphs import csr, undirected, uniform_transitions_ok

pytestmark = pytest.mark.gpu


def run_both(rowptr, col, start, rand, L, cuda):
    rowptr, col, start = (np.asarray(a, dtype=np.int64) for a in (rowptr, col, start))
    rand = np.asarray(rand, dtype=np.float32).reshape(start.size, L)
    n_ref, e_ref, st, _ = oracle.uniform_walk(rowptr, col, start, rand, L, with_edges=True)
    assert st == 0
    n, e = mc.random_walk(torch.from_numpy(rowptr).to(cuda), torch.from_numpy(col).to(cuda),
                          torch.from_numpy(start).to(cuda), torch.from_numpy(rand).to(cuda), L,
                          return_edges=True)
    return n.cpu().numpy(), e.cpu().numpy(), n_ref, e_ref


def assert_parity(rowptr, col, start, rand, L, cuda):
    n, e, n_ref, e_ref = run_both(rowptr, col, start, rand, L, cuda)
    np.testing.assert_array_equal(n, n_ref)
    np.testing.assert_array_equal(e, e_ref)
    return n


def test_fixture_c1(c1, cuda):
    rowptr, col, start, rand = (torch.from_numpy(c1[k]).to(cuda)
                                for k in ("rowptr", "col", "start", "rand"))
    L = int(c1["walk_length"])
    n, e = mc.random_walk(rowptr, col, start, rand, L, return_edges=True)
    np.testing.assert_array_equal(n.cpu().numpy(), c1["uniform_nodes"])
    np.testing.assert_array_equal(e.cpu().numpy(), c1["uniform_edges"])
    # default call returns the node sequences only, as the reference op does
    n2 = mc.random_walk(rowptr, col, start, rand, L)
    assert n2.shape == (2000, L + 1) and n2.dtype == torch.int64
    assert torch.equal(n2, n)


def test_hand_graphs(cuda):
    rowptr, col = csr(3, [(0, 1), (1, 2), (2, 0)])
    n = assert_parity(rowptr, col, [0, 2], np.full((2, 4), 0.7), 4, cuda)
    assert n.tolist() == [[0, 1, 2, 0, 1], [2, 0, 1, 2, 0]]
    rowptr, col = csr(4, [(0, 1), (1, 3)])  # sink 3, isolated 2
    n = assert_parity(rowptr, col, [0, 2], np.full((2, 5), 0.5), 5, cuda)
    assert n.tolist() == [[0, 1, 3, 3, 3, 3], [2, 2, 2, 2, 2, 2]]
    rowptr, col = csr(2, [(0, 0), (0, 1), (1, 0)])  # self-loop
    n = assert_parity(rowptr, col, [0, 0], [[0.1, 0.1], [0.75, 0.1]], 2, cuda)
    assert n.tolist() == [[0, 0, 0], [0, 1, 0]]
    rowptr, col = undirected(5, [(0, 1), (0, 2), (0, 3), (0, 4)])
    r = np.array([[k / 4 + 0.01, 0.3] for k in range(4)], np.float32)
    n = assert_parity(rowptr, col, [0, 0, 0, 0], r, 2, cuda)
    assert n[:, 1].tolist() == [1, 2, 3, 4]


def test_out_of_range_rand_is_clamped_like_oracle(cuda):
    rowptr, col = csr(4, [(0, 1), (0, 2), (0, 3), (1, 0), (2, 0), (3, 0)])
    r = np.array([[1.0, 0.5], [2.5, 0.5], [-0.5, 0.5], [np.nan, 0.5], [np.inf, 0.5],
                  [1 - 2 ** -24, 0.5]], np.float32)
    n = assert_parity(rowptr, col, [0] * 6, r, 2, cuda)
    assert n[:, 1].tolist() == [3, 3, 1, 1, 3, 3]


@pytest.mark.parametrize("N,L", [(0, 5), (1, 1), (7, 0), (255, 3), (257, 17), (5000, 40),
                                 (70_001, 9)])
def test_ragged_sizes(N, L, cuda):
    rowptr, col = synth.rmat_csr(10, 6000, seed=N + L)
    V = rowptr.numel() - 1
    start = (np.arange(N) * 7919) % V
    rand = oracle.philox_uniform(N * L, seed=N * 31 + L)
    assert_parity(rowptr.numpy(), col.numpy(), start, rand, L, cuda)


def test_rmat_scale16_with_sinks(cuda):
    rowptr, col = synth.rmat_csr(16, 1 << 20, seed=3)
    rowptr, col = rowptr.numpy(), col.numpy()
    assert (np.diff(rowptr) == 0).sum() > 1000  # many absorbing nodes
    V = rowptr.size - 1
    start = np.arange(4 * V) % V
    L = 30
    rand = oracle.philox_uniform(start.size * L, seed=77)
    n = assert_parity(rowptr, col, start, rand, L, cuda)
    assert uniform_transitions_ok(rowptr, col, start, rand, n) == 0


def test_philox_uniform_matches_oracle(cuda):
    for n, seed in [(1, 0), (3, 5), (4, 5), (1001, 2**63 + 12345), (1 << 18, 9)]:
        got = mc.philox_uniform(n, seed, device=cuda).cpu().numpy()
        np.testing.assert_array_equal(got, oracle.philox_uniform(n, seed))


def test_repeatable_and_side_stream(cuda):
    rowptr, col = synth.rmat_csr(12, 40_000, seed=5, device=cuda)
    V = rowptr.numel() - 1
    start = torch.arange(3 * V, device=cuda) % V
    rand = mc.philox_uniform((start.numel(), 25), 4, device=cuda)
    a = mc.random_walk(rowptr, col, start, rand, 25)
    s = torch.cuda.Stream(device=cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    b = mc.random_walk(rowptr, col, start, rand, 25, stream=s)
    torch.cuda.current_stream(cuda).wait_stream(s)
    assert torch.equal(a, b)


def test_side_stream_call_is_ordered_and_keeps_its_memory(cuda):
    """A call on a side stream with check=False: its kernels run after the
    work queued on torch's current stream (here an input written there
    behind a spin kernel of bounded length), and the allocator hands out
    none of the call's memory (workspace, input copies) while they run: a
    zero-fill of the workspace's size queued on the current stream right
    after the call must not reach the walk's edge records.  Nodes, edges and
    node2vec walks equal the oracle's."""
    rowptr, col = synth.rmat_csr(12, 40_000, seed=5)
    rowptr, col = rowptr.numpy(), col.numpy()
    V, L = rowptr.size - 1, 30
    start = (np.arange(20 * V) % V).astype(np.int64)   # many steps per edge: records
    rand = oracle.philox_uniform(start.size * L, 6).reshape(start.size, L)
    n_ref, e_ref, _, _ = oracle.uniform_walk(rowptr, col, start, rand, L, with_edges=True)
    n2v_ref, _, _, _ = oracle.node2vec_walk(rowptr, col, start, L, 0.5, 2.0, 9)
    cur = torch.cuda.current_stream(cuda)
    s = torch.cuda.Stream(device=cuda)
    rand_dev = torch.full(rand.shape, 0.5, dtype=torch.float32, device=cuda)
    lib = mc._lib.load()
    ws_words = lib.mlxc_random_walk_workspace_bytes(V, col.size, start.size, L) // 8 + 1
    torch.cuda._sleep(20_000_000)          # bounded spin on the current stream
    rand_dev.copy_(torch.from_numpy(rand).to(cuda, non_blocking=False))
    n, e = mc.random_walk(rowptr, col, start, rand_dev, L, stream=s, check=False,
                          return_edges=True)
    junk = torch.zeros(ws_words, dtype=torch.int64, device=cuda)
    torch.cuda._sleep(20_000_000)
    junk.fill_(0)
    w = mc.rejection_sampling(rowptr, col, start, L, 0.5, 2.0, seed=9, stream=s, check=False)
    junk2 = torch.zeros(ws_words * 2, dtype=torch.int64, device=cuda)
    s.synchronize()
    cur.synchronize()
    np.testing.assert_array_equal(n.cpu().numpy(), n_ref)
    np.testing.assert_array_equal(e.cpu().numpy(), e_ref)
    np.testing.assert_array_equal(w.cpu().numpy(), n2v_ref)
    del junk, junk2


def test_numpy_inputs_are_copied(c1, cuda):
    n = mc.random_walk(c1["rowptr"], c1["col"], c1["start"], c1["rand"], int(c1["walk_length"]))
    assert n.is_cuda
    np.testing.assert_array_equal(n.cpu().numpy(), c1["uniform_nodes"])


def test_bad_graph_raises(cuda):
    rowptr, col = csr(3, [(0, 1), (1, 2)])
    rand = np.zeros((1, 3), np.float32)
    with pytest.raises(ValueError, match="outside"):
        mc.random_walk(rowptr, col, np.array([5]), rand, 3)
    with pytest.raises(ValueError, match="outside"):
        mc.random_walk(rowptr, np.array([7, 2]), np.array([0]), rand, 3)
    with pytest.raises(ValueError, match="rowptr"):
        mc.random_walk(np.array([0, 2, 1, 2]), col, np.array([0]), rand, 3)
    with pytest.raises(ValueError, match="rowptr"):
        mc.random_walk(np.array([0, 1, 9, 2]), col, np.array([0]), rand, 3)


def test_c2_full_size_properties(cuda):
    """Configuration 2 at full size (R-MAT 2^20, 10 walks per node, L=80):
    every one of the 838,860,800 steps is checked against numpy-free torch
    float32 arithmetic on the device, and a sample of walks bit-exactly
    against the oracle; the unwindowed kernel gives the same walks in full."""
    rowptr, col = synth.rmat_csr(20, 1 << 24, seed=0, device=cuda)
    V = rowptr.numel() - 1
    N, L = 10 * V, 80
    start = torch.arange(N, device=cuda) % V
    rand = mc.philox_uniform((N, L), 2, device=cuda)
    n = mc.random_walk(rowptr, col, start, rand, L)
    assert torch.equal(n[:, 0], start)
    bad = 0
    for l in range(L):
        u, v = n[:, l], n[:, l + 1]
        rs = rowptr[u]
        deg = rowptr[u + 1] - rs
        prod = rand[:, l] * deg.to(torch.float32)
        idx = torch.minimum(prod.to(torch.int64), (deg - 1).clamp_min(0))
        moving = deg > 0
        expect = torch.where(moving, col[torch.where(moving, rs + idx, 0)], u)
        bad += int((expect != v).sum())
    assert bad == 0
    g = torch.Generator().manual_seed(0)
    sample = torch.randint(0, N, (4000,), generator=g).to(cuda)
    rp, cl = rowptr.cpu().numpy(), col.cpu().numpy()
    n_ref, _, st, _ = oracle.uniform_walk(rp, cl, start[sample].cpu().numpy(),
                                          rand[sample].cpu().numpy(), L)
    assert st == 0
    np.testing.assert_array_equal(n[sample].cpu().numpy(), n_ref)
    # the unwindowed kernel (the path of graphs beyond int32 ids, forced by a
    # minimal workspace) gives the same walks in full
    n2 = torch.empty_like(n)
    _abi_walk(rowptr, col, start, rand.data_ptr(), L, n2.data_ptr(), ws_bytes=32)
    assert torch.equal(n2, n)


def test_c4_full_size_properties(cuda):
    """Configuration 4 at full size (R-MAT 2^24 with 2^28 samples, one walk
    per node, L=20), which the workspace query sends to the CSR walk (fewer
    than 4 steps per edge): every one of the 335,544,320 steps and its edge id
    is checked against torch float32 arithmetic on the device, and 4,000
    sampled walks bit-exactly against the oracle, nodes and edges; the
    unwindowed kernel gives the same walks and edges in full."""
    rowptr, col = synth.rmat_csr(24, 1 << 28, seed=0, device=cuda)
    V, E = rowptr.numel() - 1, col.numel()
    N, L = V, 20
    assert N * L < 4 * E  # the CSR walk, not edge records
    from mlx_cluster_amd import _lib
    assert _lib.load().mlxc_random_walk_workspace_bytes(V, E, N, L) == 256 + 16 * N
    start = torch.arange(N, device=cuda)
    rand = mc.philox_uniform((N, L), 4, device=cuda)
    n, e = mc.random_walk(rowptr, col, start, rand, L, return_edges=True)
    assert torch.equal(n[:, 0], start)
    bad = 0
    for l in range(L):
        u, v = n[:, l], n[:, l + 1]
        rs = rowptr[u]
        deg = rowptr[u + 1] - rs
        prod = rand[:, l] * deg.to(torch.float32)
        idx = torch.minimum(prod.to(torch.int64), (deg - 1).clamp_min(0))
        moving = deg > 0
        edge = torch.where(moving, rs + idx, -1)
        expect = torch.where(moving, col[edge.clamp_min(0)], u)
        bad += int((expect != v).sum()) + int((edge != e[:, l]).sum())
        del u, v, rs, deg, prod, idx, moving, edge, expect
    assert bad == 0
    g = torch.Generator().manual_seed(4)
    sample = torch.randint(0, N, (4000,), generator=g).to(cuda)
    rp, cl = rowptr.cpu().numpy(), col.cpu().numpy()
    n_ref, e_ref, st, _ = oracle.uniform_walk(rp, cl, start[sample].cpu().numpy(),
                                              rand[sample].cpu().numpy(), L, with_edges=True)
    assert st == 0
    np.testing.assert_array_equal(n[sample].cpu().numpy(), n_ref)
    np.testing.assert_array_equal(e[sample].cpu().numpy(), e_ref)
    # the unwindowed kernel (the path of graphs beyond int32 ids, forced by a
    # minimal workspace) gives the same walks and edges in full
    n2, e2 = torch.empty_like(n), torch.empty_like(e)
    _abi_walk(rowptr, col, start, rand.data_ptr(), L, n2.data_ptr(), e_out=e2, ws_bytes=32)
    assert torch.equal(n2, n) and torch.equal(e2, e)


def _abi_walk(rowptr, col, start, rand_t, L, n_out_t, *, e_out=None, ws_bytes=None,
              out_type=0):
    """Calls mlxc_random_walk directly so each kernel path can be selected:
    edge records (full workspace, many steps per edge), CSR reads with start
    records (workspace for start records only), and the unwindowed kernel
    (minimal workspace, edge output or unaligned buffers)."""
    from mlx_cluster_amd import _lib
    lib = _lib.load()
    V, E = rowptr.numel() - 1, col.numel()
    if ws_bytes is None:
        ws_bytes = 256 + 16 * (E + start.numel())  # room for edge + start records
    ws = torch.empty((ws_bytes + 7) // 8, dtype=torch.int64, device=rowptr.device)
    rc = lib.mlxc_random_walk(rowptr.data_ptr(), V, col.data_ptr(), E, start.data_ptr(),
                              start.numel(), rand_t, L, n_out_t,
                              None if e_out is None else e_out.data_ptr(), out_type,
                              ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    assert int(ws[0].item()) == 0


@pytest.mark.parametrize("N,L", [(1, 1), (33, 5), (257, 4), (1000, 16), (4096, 23),
                                 (20_000, 80)])
def test_all_kernel_paths_agree(N, L, cuda):
    # small graph (E <= 300) so that most shapes take >= 4 * E steps: the
    # full workspace then selects the edge-record walk; N * L not a multiple
    # of 4 selects the unwindowed kernel whatever the workspace
    rowptr, col = synth.rmat_csr(7, 300, seed=N, device=cuda)
    V = rowptr.numel() - 1
    start = (torch.arange(N, device=cuda) * 131) % V
    rand = mc.philox_uniform(N * L + 1, 17, device=cuda)
    ref, ref_e, st, _ = oracle.uniform_walk(rowptr.cpu().numpy(), col.cpu().numpy(),
                                            start.cpu().numpy(), rand[:N * L].cpu().numpy(), L,
                                            with_edges=True)
    assert st == 0
    E = col.numel()
    workspaces = {"records": 256 + 16 * (E + N), "csr": 256 + 16 * N, "plain": 32}
    for name, ws in workspaces.items():
        for edges in (False, True):
            out = torch.full((N, L + 1), -7, dtype=torch.int64, device=cuda)
            e = torch.full((N, L), -7, dtype=torch.int64, device=cuda) if edges else None
            _abi_walk(rowptr, col, start, rand.data_ptr(), L, out.data_ptr(), e_out=e,
                      ws_bytes=ws)
            np.testing.assert_array_equal(out.cpu().numpy(), ref, err_msg=f"{name} {edges}")
            if edges:
                np.testing.assert_array_equal(e.cpu().numpy(), ref_e, err_msg=f"{name} edges")
    # unaligned rand (4-byte offset), n_out and e_out (8-byte offsets): unwindowed kernel
    rand_u = mc.philox_uniform(N * L + 1, 0, device=cuda)
    rand_u[1:] = rand[:N * L]
    big = torch.full((N * (L + 1) + 1,), -7, dtype=torch.int64, device=cuda)
    big_e = torch.full((N * L + 1,), -7, dtype=torch.int64, device=cuda)
    e_view = big_e[1:]
    _abi_walk(rowptr, col, start, rand_u.data_ptr() + 4, L, big.data_ptr() + 8, e_out=e_view)
    np.testing.assert_array_equal(big[1:].view(N, L + 1).cpu().numpy(), ref, err_msg="unaligned")
    np.testing.assert_array_equal(e_view.view(N, L).cpu().numpy(), ref_e, err_msg="unaligned e")


def _hub_graph(V, hub_degrees, core_entries, seed):
    """V nodes, most of them isolated: 1000 core nodes spread over the id
    range with core_entries entries between them (a fifth of them to the
    hubs), and hubs at the top ids whose rows of the given lengths point back
    into the core, so that walks keep entering and leaving the hubs."""
    rng = np.random.default_rng(seed)
    core = np.arange(1000, dtype=np.int64) * (V // 1000)
    hubs = V - 1 - np.arange(len(hub_degrees), dtype=np.int64)
    to_hub = rng.random(core_entries) < 0.2
    pick = lambda ids, n: ids[rng.integers(0, ids.size, n)]  # noqa: E731
    row = np.concatenate([np.repeat(hubs, hub_degrees), pick(core, core_entries)])
    col = np.concatenate([pick(core, int(sum(hub_degrees))),
                          np.where(to_hub, pick(hubs, core_entries), pick(core, core_entries))])
    order = np.lexsort((col, row))
    rowptr = np.zeros(V + 1, np.int64)
    np.cumsum(np.bincount(row, minlength=V), out=rowptr[1:])
    return rowptr, col[order], core, hubs


@pytest.mark.parametrize("packed", [True, False])
def test_record_formats_and_long_rows(packed, cuda):
    """Edge records of 8 bytes (26 bits of node id, 22 of row begin and a
    16-bit degree field) and of 16 bytes (one more bit of row begin leaves
    15), on a graph of 2^26 nodes whose hub rows hold 65,532 entries (the
    longest the 8-byte degree field holds), 65,533 (the shortest it does not)
    and 100,000: a walk leaving a longer row reads the row's end from rowptr
    first.  Sampled walks and edge ids against the oracle; generated
    uniforms and the int32 output give the same walks."""
    from mlx_cluster_amd import _lib
    V, L = 1 << 26, 40
    rowptr, col, core, hubs = _hub_graph(V, [65_532, 65_533, 100_000],
                                         2_500_000 if packed else 4_300_000, seed=26)
    E = col.size
    assert (E < 1 << 22) == packed
    N = 4 * E // L + 1001                  # >= 4 steps per edge: the record walk
    start = np.where(np.arange(N) % 4 == 0, hubs[np.arange(N) % 3], core[np.arange(N) % 1000])
    assert _lib.load().mlxc_random_walk_workspace_bytes(V, E, N, L) == \
        256 + (8 if packed else 16) * (E + N)
    rp, cl, st = (torch.from_numpy(a).to(cuda) for a in (rowptr, col, start))
    rand = mc.philox_uniform((N, L), 31, device=cuda)
    n, e = mc.random_walk(rp, cl, st, rand, L, return_edges=True)
    sample = np.random.default_rng(1).choice(N, 3000, replace=False)
    n_ref, e_ref, status, _ = oracle.uniform_walk(rowptr, col, start[sample],
                                                  rand.cpu().numpy()[sample], L, with_edges=True)
    assert status == 0
    np.testing.assert_array_equal(n.cpu().numpy()[sample], n_ref)
    np.testing.assert_array_equal(e.cpu().numpy()[sample], e_ref)
    assert np.isin(n_ref[:, :-1], hubs[1:]).sum() > 1000   # steps leaving the long rows
    assert torch.equal(mc.random_walk(rp, cl, st, None, L, seed=31), n)
    n32 = mc.random_walk(rp, cl, st, None, L, seed=31, out_dtype=torch.int32)
    assert torch.equal(n32.long(), n)


def test_packed_degree_field_cap(cuda):
    """The widest degree code (24 bits: 14 bits of node id and 26 of row
    begin leave more): a row of 2^24 - 4 entries, the longest the code
    holds, and one of 2^24 - 3, read through the long-row phase.  Sampled
    walks and edge ids against the oracle."""
    from mlx_cluster_amd import _lib
    V, L = 1 << 14, 40
    rowptr, col, core, hubs = _hub_graph(V, [(1 << 24) - 4, (1 << 24) - 3], 200_000, seed=24)
    E = col.size
    assert (1 << 25) < E < (1 << 26)
    N = 4 * E // L + 1001
    start = np.where(np.arange(N) % 2 == 0, hubs[np.arange(N) % 2], core[np.arange(N) % 1000])
    assert _lib.load().mlxc_random_walk_workspace_bytes(V, E, N, L) == 256 + 8 * (E + N)
    rp, cl, st = (torch.from_numpy(a).to(cuda) for a in (rowptr, col, start))
    rand = mc.philox_uniform((N, L), 5, device=cuda)
    n, e = mc.random_walk(rp, cl, st, rand, L, return_edges=True)
    sample = np.random.default_rng(2).choice(N, 2000, replace=False)
    n_ref, e_ref, status, _ = oracle.uniform_walk(rowptr, col, start[sample],
                                                  rand.cpu().numpy()[sample], L, with_edges=True)
    assert status == 0
    np.testing.assert_array_equal(n.cpu().numpy()[sample], n_ref)
    np.testing.assert_array_equal(e.cpu().numpy()[sample], e_ref)
    assert np.isin(n_ref[:, :-1], hubs).sum() > 1000


@pytest.mark.parametrize("N,L", [(1, 1), (37, 5), (1000, 16), (4096, 23), (30_000, 80)])
def test_seeded_uniforms_match_rand_tensor(N, L, cuda):
    """rand=None, seed=s generates in the kernel exactly the stream
    philox_uniform((N, L), s) holds: every kernel path (edge records, CSR
    reads, edge output) gives the walks of the explicit tensor, and the oracle's."""
    rowptr, col = synth.rmat_csr(9, 3000, seed=N, device=cuda)
    V = rowptr.numel() - 1
    start = (torch.arange(N, device=cuda) * 17) % V
    seed = 0xABCDEF0123 + N
    rand = mc.philox_uniform((N, L), seed, device=cuda)
    want = mc.random_walk(rowptr, col, start, rand, L)
    got = mc.random_walk(rowptr, col, start, None, L, seed=seed)
    assert torch.equal(got, want)
    got_n, got_e = mc.random_walk(rowptr, col, start, None, L, seed=seed, return_edges=True)
    want_n, want_e = mc.random_walk(rowptr, col, start, rand, L, return_edges=True)
    assert torch.equal(got_n, want) and torch.equal(got_e, want_e)
    ref, _, st, _ = oracle.uniform_walk(rowptr.cpu().numpy(), col.cpu().numpy(),
                                        start.cpu().numpy(), oracle.philox_uniform(N * L, seed), L)
    assert st == 0
    np.testing.assert_array_equal(got.cpu().numpy(), ref)


def test_cpu_twin_equals_gpu(cuda):
    """stream='cpu' (host twin) and the GPU kernels give the same walks and
    edges, with a rand tensor and with generated uniforms."""
    rowptr, col = synth.rmat_csr(16, 600_000, seed=6)
    V = rowptr.numel() - 1
    start = torch.arange(4 * V) % V
    L = 21
    rand = mc.philox_uniform((start.numel(), L), 5, device=cuda)
    g = mc.random_walk(rowptr.to(cuda), col.to(cuda), start.to(cuda), rand, L, return_edges=True)
    c = mc.random_walk(rowptr, col, start, rand.cpu(), L, return_edges=True, stream="cpu")
    assert torch.equal(g[0].cpu(), c[0]) and torch.equal(g[1].cpu(), c[1])
    g = mc.random_walk(rowptr.to(cuda), col.to(cuda), start.to(cuda), None, L, seed=5)
    c = mc.random_walk(rowptr, col, start, None, L, seed=5, stream="cpu")
    assert torch.equal(g.cpu(), c)


@pytest.mark.parametrize("L", [7, 8, 9, 600])
def test_long_and_block_sized_walks_with_sinks(L, cuda):
    """Walk lengths around one 64-byte output block and far beyond it, on a
    graph with many out-degree-0 nodes: completed blocks of many lanes at once
    and sink tails of hundreds of blocks, all stored cooperatively by the
    wavefront.  Nodes and edges bit-exact against the oracle for the record
    walk (full workspace) and the CSR walk (start records only), and nodes
    for generated uniforms."""
    rowptr, col = synth.rmat_csr(10, 4000, seed=44, device=cuda)
    V, E = rowptr.numel() - 1, col.numel()
    N = 3000  # N * L >= 4 * E and a multiple of 4: both windowed walks apply
    assert N * L >= 4 * E and (N * L) % 4 == 0
    start = (torch.arange(N, device=cuda) * 7) % V
    rand = mc.philox_uniform((N, L), 8, device=cuda)
    n_ref, e_ref, st, counts = oracle.uniform_walk(rowptr.cpu().numpy(), col.cpu().numpy(),
                                                   start.cpu().numpy(), rand.cpu().numpy(), L,
                                                   with_edges=True)
    assert st == 0 and counts["sink_walks"] > N // 4
    for ws_bytes in (256 + 16 * (E + N), 256 + 16 * N):
        n = torch.empty((N, L + 1), dtype=torch.int64, device=cuda)
        e = torch.empty((N, L), dtype=torch.int64, device=cuda)
        _abi_walk(rowptr, col, start, rand.data_ptr(), L, n.data_ptr(), e_out=e, ws_bytes=ws_bytes)
        np.testing.assert_array_equal(n.cpu().numpy(), n_ref)
        np.testing.assert_array_equal(e.cpu().numpy(), e_ref)
    g = mc.random_walk(rowptr, col, start, None, L, seed=8)
    np.testing.assert_array_equal(g.cpu().numpy(), n_ref)


@pytest.mark.parametrize("L", [7, 9, 80, 600])
def test_int32_output_all_kernel_paths(L, cuda):
    """out_type MLXC_OUT_INT32 (8-entry blocks of 32 bytes, two lanes per
    block in the wavefront stores): nodes and edges equal the int64 output
    for the record walk, the CSR walk and the unwindowed kernel, and the
    oracle."""
    rowptr, col = synth.rmat_csr(10, 4000, seed=46, device=cuda)
    V, E = rowptr.numel() - 1, col.numel()
    N = 3000
    start = (torch.arange(N, device=cuda) * 5) % V
    rand = mc.philox_uniform((N, L), 9, device=cuda)
    n_ref, e_ref, st, _ = oracle.uniform_walk(rowptr.cpu().numpy(), col.cpu().numpy(),
                                              start.cpu().numpy(), rand.cpu().numpy(), L,
                                              with_edges=True)
    assert st == 0
    for ws_bytes in (256 + 16 * (E + N), 256 + 16 * N, 32):
        n = torch.empty((N, L + 1), dtype=torch.int32, device=cuda)
        e = torch.empty((N, L), dtype=torch.int32, device=cuda)
        _abi_walk(rowptr, col, start, rand.data_ptr(), L, n.data_ptr(), e_out=e,
                  ws_bytes=ws_bytes, out_type=1)
        np.testing.assert_array_equal(n.cpu().numpy(), n_ref)
        np.testing.assert_array_equal(e.cpu().numpy(), e_ref)
    g = mc.random_walk(rowptr, col, start, None, L, seed=9, out_dtype=torch.int32)
    assert g.dtype == torch.int32
    np.testing.assert_array_equal(g.cpu().numpy(), n_ref)


@pytest.mark.parametrize("V,E_target", [(50, 300), (2708, 10556), (3000, 14336 - 3001)])
def test_lds_walk(V, E_target, cuda):
    """Graphs whose rowptr and col fit in LDS (V + 1 + E <= 14,336 entries) on
    calls of 1 to 2^20 steps take the LDS walk (the workspace query asks for
    the 256-byte header only).  Nodes and edges bit-exact against the oracle
    with a rand tensor and generated uniforms, int64 and int32 output, sinks
    included; a graph one entry over the limit takes the record walk with
    the same results."""
    from mlx_cluster_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(V)
    pairs = rng.integers(0, V, (E_target, 2))
    pairs[: V // 5, 0] = np.arange(V // 5) * 5 % V  # a spread of rows
    rowptr, col = csr(V, pairs)
    keep = np.ones(V, bool)
    keep[rng.integers(0, V, V // 10)] = False  # some sinks: drop their rows' entries
    row_of = np.repeat(np.arange(V), np.diff(rowptr))
    rowptr, col = csr(V, np.stack([row_of[keep[row_of]], col[keep[row_of]]], 1))
    E = col.size
    assert V + 1 + E <= 14336
    for N, L in ((1, 1), (300, 7), (2000, 5), (4000, 80)):
        assert lib.mlxc_random_walk_workspace_bytes(V, E, N, L) == 256
        start = (np.arange(N) * 7) % V
        rand = mc.philox_uniform((N, L), N + L, device=cuda)
        n_ref, e_ref, st, counts = oracle.uniform_walk(rowptr, col, start, rand.cpu().numpy(), L,
                                                       with_edges=True)
        assert st == 0
        t = lambda a: torch.as_tensor(a).to(cuda)
        n, e = mc.random_walk(t(rowptr), t(col), t(start), rand, L, return_edges=True)
        np.testing.assert_array_equal(n.cpu().numpy(), n_ref)
        np.testing.assert_array_equal(e.cpu().numpy(), e_ref)
        n32 = mc.random_walk(t(rowptr), t(col), t(start), rand, L, out_dtype=torch.int32)
        np.testing.assert_array_equal(n32.cpu().numpy(), n_ref)
        g = mc.random_walk(t(rowptr), t(col), t(start), None, L, seed=N + L)
        np.testing.assert_array_equal(g.cpu().numpy(), n_ref)
    # exactly at the limit (the LDS walk) and one entry over it (the record walk)
    base = np.stack([np.repeat(np.arange(V), np.diff(rowptr)), col], 1)
    for total, lds in ((14336, True), (14337, False)):
        rp2, cl2 = csr(V, np.concatenate([base, np.tile([[0, 1]], (total - (V + 1 + E), 1))]))
        assert V + 1 + cl2.size == total
        N, L = 2000, 5
        assert (lib.mlxc_random_walk_workspace_bytes(V, cl2.size, N, L) == 256) == lds
        start = (np.arange(N) * 3) % V
        rand = mc.philox_uniform((N, L), 77, device=cuda)
        n_ref, _, st, _ = oracle.uniform_walk(rp2, cl2, start, rand.cpu().numpy(), L)
        assert st == 0
        n = mc.random_walk(torch.as_tensor(rp2).to(cuda), torch.as_tensor(cl2).to(cuda),
                           torch.as_tensor(start).to(cuda), rand, L)
        np.testing.assert_array_equal(n.cpu().numpy(), n_ref)


def test_lds_walk_flags_bad_input(cuda):
    """Out-of-range starts, col entries and rowptr entries met by an LDS walk
    raise ValueError, as on the other paths."""
    rowptr, col = csr(4, [(0, 1), (1, 2), (2, 3), (3, 0)])
    t = lambda a: torch.as_tensor(np.asarray(a, dtype=np.int64)).to(cuda)
    rand = torch.full((2, 3), 0.5, device=cuda)
    with pytest.raises(ValueError):
        mc.random_walk(t(rowptr), t(col), t([0, 9]), rand, 3)
    with pytest.raises(ValueError):
        mc.random_walk(t(rowptr), t([1, 2, 7, 0]), t([0, 1]), rand, 3)
    with pytest.raises(ValueError):
        mc.random_walk(t([0, 1, 2, 9, 4]), t(col), t([2, 2]), rand, 3)
    # the same graph, well formed: no error
    n = mc.random_walk(t(rowptr), t(col), t([0, 1]), rand, 3)
    np.testing.assert_array_equal(n.cpu().numpy(), [[0, 1, 2, 3], [1, 2, 3, 0]])


def _check_steps(rowptr, col, rand, n, e, L):
    """Mismatches between the walks and their steps re-derived with torch
    float32 arithmetic on the device (RandomWalk.cpp:45-58: the degree
    rounded to float32, multiplied by r, truncated)."""
    bad = 0
    for l in range(L):
        u, v = n[:, l], n[:, l + 1]
        rs = rowptr[u]
        deg = rowptr[u + 1] - rs
        idx = torch.minimum((rand[:, l] * deg.to(torch.float32)).to(torch.int64),
                            (deg - 1).clamp_min(0))
        moving = deg > 0
        edge = torch.where(moving, rs + idx, -1)
        expect = torch.where(moving, col[edge.clamp_min(0)], u)
        bad += int((expect != v).sum()) + int((edge != e[:, l]).sum())
    return bad


def test_graph_beyond_int32_edge_ids(cuda):
    """A graph of 2^31 + 2^20 CSR entries (2^20 nodes of degree 2049, 17.2 GB
    of col): the workspace query asks for 16-byte start records, and the
    wide CSR walk runs with int64 edge ids.  Every step and edge id is
    re-derived on the device, the unwindowed kernel gives the same walks and
    edges, and 2,000 walks are bit-exact against the oracle; 4,096 node2vec
    walks (the direct kernel, linear scans of the unsorted rows) are too; a
    bad col entry and a bad rowptr entry met by a walk raise.  Then a row of 2^31 + 5
    entries: its start record marks it long, the walk reads its bounds from
    rowptr and picks with the float32 rule's rounded degree."""
    from mlx_cluster_amd import _lib
    q = _lib.load().mlxc_random_walk_workspace_bytes
    V, deg, L = 1 << 20, 2049, 20
    E = V * deg
    assert E > 2**31 - 1
    rowptr = torch.arange(V + 1, device=cuda, dtype=torch.int64) * deg
    g = torch.Generator(device=cuda).manual_seed(11)
    col = torch.randint(0, V, (E,), device=cuda, generator=g, dtype=torch.int64)
    N = V
    start = torch.arange(N, device=cuda, dtype=torch.int64)
    rand = mc.philox_uniform((N, L), 7, device=cuda)
    assert q(V, E, N, L) == 256 + 16 * N
    n, e = mc.random_walk(rowptr, col, start, rand, L, return_edges=True)
    assert torch.equal(n[:, 0], start)
    assert _check_steps(rowptr, col, rand, n, e, L) == 0
    assert int(e.max()) > 2**31  # edge ids beyond int32
    n2, e2 = torch.empty_like(n), torch.empty_like(e)
    _abi_walk(rowptr, col, start, rand.data_ptr(), L, n2.data_ptr(), e_out=e2, ws_bytes=32)
    assert torch.equal(n2, n) and torch.equal(e2, e)
    del n2, e2
    sample = torch.randint(0, N, (2000,), generator=torch.Generator().manual_seed(3)).to(cuda)
    rp, cl = rowptr.cpu().numpy(), col.cpu().numpy()
    n_ref, e_ref, st, _ = oracle.uniform_walk(rp, cl, start[sample].cpu().numpy(),
                                              rand[sample].cpu().numpy(), L, with_edges=True)
    assert st == 0
    np.testing.assert_array_equal(n[sample].cpu().numpy(), n_ref)
    np.testing.assert_array_equal(e[sample].cpu().numpy(), e_ref)
    # node2vec on the same graph takes its direct kernel (int64 positions);
    # the rows are unsorted, so the device check picks linear scans
    w = mc.rejection_sampling(rowptr, col, start[:4096], 5, 0.5, 2.0, seed=13, return_edges=True)
    w_ref, we_ref, st, _ = oracle.node2vec_walk(rp, cl, start[:4096].cpu().numpy(), 5, 0.5, 2.0,
                                                13, rule=oracle.RULE_REF_CHAIN, rows_sorted=False,
                                                with_edges=True)
    assert st == 0
    np.testing.assert_array_equal(w[0].cpu().numpy(), w_ref)
    np.testing.assert_array_equal(w[1].cpu().numpy(), we_ref)
    del cl, rp, w
    # malformed input met by a walk: walk 0's first edge, then its start's row
    first = int(e[0, 0])
    col[first] = V
    with pytest.raises(ValueError, match="outside"):
        mc.random_walk(rowptr, col, start[:64], rand[:64], L)
    col[first] = 0
    rowptr[1] = E + 1
    with pytest.raises(ValueError, match="rowptr"):
        mc.random_walk(rowptr, col, start[:64], rand[:64], L)
    del col, n, e, rowptr
    torch.cuda.empty_cache()

    # one row of 2^31 + 5 entries (node 0) and one of 3 (node 1)
    E2 = 2**31 + 8
    rowptr = torch.tensor([0, E2 - 3, E2], device=cuda, dtype=torch.int64)
    col = torch.randint(0, 2, (E2,), device=cuda, generator=g, dtype=torch.int64)
    N, L = 4096, 6
    start = torch.arange(N, device=cuda, dtype=torch.int64) % 2
    rand = mc.philox_uniform((N, L), 8, device=cuda)
    assert q(2, E2, N, L) == 256 + 16 * N
    n, e = mc.random_walk(rowptr, col, start, rand, L, return_edges=True)
    assert _check_steps(rowptr, col, rand, n, e, L) == 0
    assert int(e[start == 0, 0].max()) > 2**30  # first steps spread over the long row
    n2, e2 = torch.empty_like(n), torch.empty_like(e)
    _abi_walk(rowptr, col, start, rand.data_ptr(), L, n2.data_ptr(), e_out=e2, ws_bytes=32)
    assert torch.equal(n2, n) and torch.equal(e2, e)
    del col, n, e, n2, e2
    torch.cuda.empty_cache()
