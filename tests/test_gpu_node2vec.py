"""Parity of the HIP node2vec walk (libmlxc.so) with the CPU oracle.

Bit-exact on the shared Philox stream for both acceptance rules, plus
distribution checks against the closed-form transition weights.
"""
import numpy as np
import pytest
import torch
from scipy import stats

import mlx_cluster_amd as mc
import oracle
from mlx_cluster_amd import synth
from tests.graphs import csr, undirected
from tests.test_oracle import class_counts, three_class_graph

pytestmark = pytest.mark.gpu

RULE_NAME = {oracle.RULE_REF_CHAIN: "ref_chain", oracle.RULE_NODE2VEC_EXACT: "node2vec"}


def _abi_walk(rowptr, col, start, L, p, q, seed, rule, rows, mode, out_dtype=torch.int64,
              expect_status=0):
    """mlxc_rejection_sampling through the C ABI, with edge output, in the
    layout the workspace selects (mlxc_rejection_sampling_layout_bytes):
    "direct" (the direct CSR kernel), "lds" (the LDS walk, for graphs and
    calls small enough), "csr" (the record kernel in CSR mode), "records_plain"
    (edge records, index-level searches), "records_nohub" (edge records and
    the row hash tables) or "records" (the tables and the hub bitmaps; the
    tables and bitmaps serve calls that search rows).  Asserts the call's
    status word equals expect_status."""
    from mlx_cluster_amd import _lib
    lib = _lib.load()
    N = start.numel()
    V, E = rowptr.numel() - 1, col.numel()
    n = torch.empty((N, L + 1), dtype=out_dtype, device=start.device)
    e = torch.empty((N, L), dtype=out_dtype, device=start.device)
    out_type = _lib.MLXC_OUT_INT32 if out_dtype == torch.int32 else _lib.MLXC_OUT_INT64
    layout = {"direct": _lib.MLXC_N2V_LAYOUT_DIRECT, "lds": _lib.MLXC_N2V_LAYOUT_LDS,
              "csr": _lib.MLXC_N2V_LAYOUT_CSR, "records_plain": _lib.MLXC_N2V_LAYOUT_RECORDS,
              "records_nohub": _lib.MLXC_N2V_LAYOUT_RECORDS_HASH,
              "records": _lib.MLXC_N2V_LAYOUT_RECORDS_FULL}[mode]
    nbytes = lib.mlxc_rejection_sampling_layout_bytes(V, E, N, L, layout)
    assert nbytes > 0, mode
    ws = torch.zeros((nbytes + 7) // 8, dtype=torch.int64, device=start.device)
    ptr = lambda t: t.data_ptr() if t.numel() else None
    rc = lib.mlxc_rejection_sampling(ptr(rowptr), V, ptr(col), E,
                                     ptr(start), N, L, p, q, seed, 0, rule, rows, ptr(n), ptr(e),
                                     out_type, ws.data_ptr(), nbytes,
                                     torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    assert int(ws[0].item()) == expect_status, f"{mode}: status {int(ws[0].item())}"
    return n, e


def gpu_walk(rowptr, col, start, L, p, q, seed, rule, cuda, **kw):
    """Runs the walk without and with edge output (the mode the workspace
    query picks) and through the C ABI in each of the three modes (edge
    records, CSR mode, the direct kernel); all node outputs must agree, and all
    edge outputs.  Returns (nodes, edges)."""
    t = lambda a: torch.as_tensor(np.asarray(a, dtype=np.int64)).to(cuda)
    args = (t(rowptr), t(col), t(start), L, p, q)
    n_rec = mc.rejection_sampling(*args, seed=seed, rule=RULE_NAME[rule], **kw)
    n, e = mc.rejection_sampling(*args, seed=seed, rule=RULE_NAME[rule], return_edges=True, **kw)
    np.testing.assert_array_equal(n_rec.cpu().numpy(), n.cpu().numpy(),
                                  err_msg="record walk: nodes differ with edge output")
    rows = {None: 2, True: 1, False: 0}[kw.get("rows_sorted")]
    if kw.get("symmetric"):
        rows |= 4  # MLXC_ROWS_SYMMETRIC
    for mode in ("direct", "csr", "records_plain", "records_nohub", "records"):
        nm, em = _abi_walk(*args[:3], L, p, q, seed, rule, rows, mode)
        np.testing.assert_array_equal(nm.cpu().numpy(), n.cpu().numpy(),
                                      err_msg=f"{mode} walk nodes differ")
        np.testing.assert_array_equal(em.cpu().numpy(), e.cpu().numpy(),
                                      err_msg=f"{mode} walk edges differ")
    return n.cpu().numpy(), e.cpu().numpy()


def assert_parity(rowptr, col, start, L, p, q, seed, rule, cuda, sorted_rows=True, **kw):
    n_ref, e_ref, st, counts = oracle.node2vec_walk(rowptr, col, start, L, p, q, seed, rule=rule,
                                                    rows_sorted=sorted_rows, with_edges=True)
    assert st == 0
    n, e = gpu_walk(rowptr, col, start, L, p, q, seed, rule, cuda, **kw)
    np.testing.assert_array_equal(n, n_ref)
    np.testing.assert_array_equal(e, e_ref)
    return n, counts


def test_fixture_c1(c1, cuda):
    names = sorted({k[4:-6] for k in c1 if k.startswith("n2v_") and k.endswith("_nodes")})
    assert len(names) == 5
    for name in names:
        p, q, rule, seed = c1[f"n2v_{name}_params"]
        n, e = gpu_walk(c1["rowptr"], c1["col"], c1["start"], int(c1["walk_length"]), p, q,
                        int(seed), int(rule), cuda)
        np.testing.assert_array_equal(n, c1[f"n2v_{name}_nodes"])
        np.testing.assert_array_equal(e, c1[f"n2v_{name}_edges"])


@pytest.mark.parametrize("p,q", [(0.5, 2.0), (4.0, 0.25), (1.0, 3.0), (2.0, 0.5)])
@pytest.mark.parametrize("rule", [oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT])
def test_rmat_symmetrized(p, q, rule, cuda):
    rowptr, col = synth.rmat_csr(12, 40_000, seed=11, symmetrize=True)
    rowptr, col = rowptr.numpy(), col.numpy()
    V = rowptr.size - 1
    start = np.arange(2 * V) % V
    assert_parity(rowptr, col, start, 20, p, q, 1234, rule, cuda)


@pytest.mark.parametrize("rule", [oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT])
def test_unsorted_rows_use_linear_scan(rule, cuda):
    rng = np.random.default_rng(2)
    rowptr, col = undirected(500, rng.integers(0, 500, (4000, 2)), sort=False)
    assert oracle.csr_flags(rowptr, col) & 4  # rows really are unsorted
    assert mc.csr_check(rowptr, col) == oracle.csr_flags(rowptr, col)
    start = np.arange(1000) % 500
    assert_parity(rowptr, col, start, 15, 0.5, 2.0, 5, rule, cuda, sorted_rows=False)
    # the same graph declared sorted by the caller on sorted rows
    srp, scol = undirected(500, rng.integers(0, 500, (4000, 2)))
    assert_parity(srp, scol, start, 15, 0.5, 2.0, 5, rule, cuda, rows_sorted=True)


def test_trial_cap_matches_oracle(cuda):
    """p = q = 1e6 makes prob_2 = 1e-6: most steps hit the 65,536-trial cap
    and keep their last candidate, identically in oracle and kernels."""
    rowptr, col = undirected(40, [(i, (i * 7 + 3) % 40) for i in range(40)] +
                             [(i, (i * 11 + 5) % 40) for i in range(40)])
    start = np.arange(64) % 40
    assert_parity(rowptr, col, start, 3, 1e6, 1e6, 8, oracle.RULE_NODE2VEC_EXACT, cuda)


def test_p1_q1_equals_uniform_walk(cuda):
    rowptr, col = synth.rmat_csr(12, 40_000, seed=12)
    V = rowptr.numel() - 1
    start = torch.arange(V) % V
    L = 16
    n, _ = gpu_walk(rowptr.numpy(), col.numpy(), start.numpy(), L, 1.0, 1.0, 99,
                    oracle.RULE_REF_CHAIN, cuda)
    rand = torch.from_numpy(oracle.node2vec_trial0_u0(V, L, 99))
    u = mc.random_walk(rowptr.to(cuda), col.to(cuda), start.to(cuda), rand.to(cuda), L)
    np.testing.assert_array_equal(n, u.cpu().numpy())


@pytest.mark.parametrize("N,L", [(0, 4), (1, 1), (3, 0), (300, 2), (1025, 7)])
def test_ragged_sizes(N, L, cuda):
    rowptr, col = undirected(64, np.random.default_rng(N).integers(0, 64, (200, 2)))
    start = np.arange(N) % 64
    assert_parity(rowptr, col, start, L, 0.7, 1.5, N + L, oracle.RULE_NODE2VEC_EXACT, cuda)


@pytest.mark.parametrize("p,q,rule", [(0.5, 2.0, oracle.RULE_NODE2VEC_EXACT),
                                      (4.0, 0.25, oracle.RULE_NODE2VEC_EXACT),
                                      (4.0, 0.25, oracle.RULE_REF_CHAIN)])
def test_transition_chi_square(p, q, rule, cuda):
    K, M = 3, 4
    (rowptr, col), a, b = three_class_graph(K, M)
    N = 1_000_000
    n, _ = gpu_walk(rowptr, col, np.zeros(N, np.int64), 2, p, q, 2024, rule, cuda)
    p0, p1, p2 = oracle.node2vec_probs(p, q)
    w = (p0, p1, p2) if rule == oracle.RULE_NODE2VEC_EXACT else (max(p0, p2), max(p1, p2), p2)
    expect = np.array([w[0], K * w[1], M * w[2]])
    expect = expect / expect.sum() * N
    assert stats.chisquare(class_counts(n, a, b), expect).pvalue > 0.01


def test_hub_graph_parity(cuda):
    """Small version of configuration 5: BA-style graph with hubs (long rows,
    many membership tests), p=4, q=0.25, both rules."""
    rowptr, col = synth.ba_hub_csr(20_000, 5, 4, 5_000, seed=3)
    rowptr, col = rowptr.numpy(), col.numpy()
    start = np.arange(20_000)
    for rule in (oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT):
        _, counts = assert_parity(rowptr, col, start, 12, 4.0, 0.25, 55, rule, cuda)
        if rule == oracle.RULE_NODE2VEC_EXACT:
            assert counts["member_tests"] > 0


@pytest.mark.parametrize("rule,p,q", [(oracle.RULE_REF_CHAIN, 0.5, 2.0),
                                      (oracle.RULE_NODE2VEC_EXACT, 4.0, 0.25)])
def test_hub_bitmaps_parity(rule, p, q, cuda):
    """Hub rows answered by their bitmaps: 600,000 nodes (bitmaps of three
    LDS chunks), 8 hubs of 20,000 entries (the chunks' block-wide bound
    search) and tens of rows of some hundreds, with (p, q) for which a
    quarter (chain) or three quarters (analytic rule) of the draws can need a
    neighbour test.  Every mode (edge records with and without bitmaps, CSR
    mode, direct kernel) against the oracle, for sorted rows, rows shuffled
    inside (each chunk scans its row) and the symmetric hint."""
    rowptr, col = synth.ba_hub_csr(600_000, 3, 8, 20_000, seed=5)
    rowptr, col = rowptr.numpy(), col.numpy()
    deg = np.diff(rowptr)
    assert deg.max() >= 20_000 and (deg >= 512).sum() >= 20
    start = (np.arange(200_000) * 3) % 600_000
    _, counts = assert_parity(rowptr, col, start, 10, p, q, 77, rule, cuda)
    assert counts["member_tests"] > 50_000
    assert_parity(rowptr, col, start, 10, p, q, 78, rule, cuda, symmetric=True)
    rng = np.random.default_rng(6)
    shuffled = col.copy()
    for u in np.flatnonzero(deg >= 512):
        shuffled[rowptr[u]:rowptr[u + 1]] = rng.permutation(shuffled[rowptr[u]:rowptr[u + 1]])
    assert_parity(rowptr, shuffled, start, 10, p, q, 79, rule, cuda, sorted_rows=False)


@pytest.mark.parametrize("rule", [oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT])
def test_return_dominated_walks(rule, cuda):
    """Small p: a trial with r >= prob1 and r >= prob2 is accepted only as a
    return to t.  On a directed graph without back edges no return exists, so
    with p = 1e-6 nearly every step runs to the trial cap and keeps its last
    candidate; on an undirected graph returns are frequent."""
    edges = [(i, (i + 1) % 64) for i in range(64)] + [(i, (i + 2) % 64) for i in range(64)]
    rowptr, col = csr(64, edges)
    start = np.arange(16)
    _, counts = assert_parity(rowptr, col, start, 4, 1e-6, 1.0, 21, rule, cuda)
    assert counts["trials"] > 16 * 2 * 60_000
    rowptr, col = synth.rmat_csr(11, 20_000, seed=5, symmetrize=True)
    rowptr, col = rowptr.numpy(), col.numpy()
    start = np.arange(rowptr.size - 1)
    for p, q in ((1e-3, 1.0), (0.5, 2.0), (0.25, 0.5)):
        assert_parity(rowptr, col, start, 15, p, q, 8, rule, cuda)


@pytest.mark.parametrize("rule", [oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT])
def test_return_biased_graph_shapes(rule, cuda):
    """p < 1, where most trials can only accept a return to t: a directed
    graph (many edges without a reverse), a symmetric graph with self-loops,
    and a multigraph whose rows hold some nodes twice must all match the
    oracle, in every mode."""
    rowptr, col = synth.rmat_csr(11, 20_000, seed=6)
    rowptr, col = rowptr.numpy(), col.numpy()
    V = rowptr.size - 1
    start = np.arange(2 * V) % V
    _, counts = assert_parity(rowptr, col, start, 12, 0.25, 4.0, 31, rule, cuda)
    assert counts["trials"] > 2 * counts["moving_steps"]
    rng = np.random.default_rng(12)
    pairs = np.unique(np.sort(rng.integers(0, 300, (2500, 2)), axis=1), axis=0)
    loops = np.stack([np.arange(0, 300, 7)] * 2, axis=1)
    pairs = pairs[pairs[:, 0] != pairs[:, 1]]
    rowptr, col = csr(300, np.concatenate([pairs, pairs[:, ::-1], loops]))
    assert np.all((np.diff(col) != 0) | (np.diff(np.repeat(np.arange(300), np.diff(rowptr)))) != 0)
    start = np.arange(900) % 300
    for p, q in ((0.3, 1.0), (0.05, 2.0)):
        assert_parity(rowptr, col, start, 16, p, q, 4, rule, cuda)
    rowptr, col = csr(300, np.concatenate([pairs, pairs[:, ::-1], pairs[:5]]))  # 5 duplicates
    assert_parity(rowptr, col, start, 16, 0.3, 1.0, 4, rule, cuda)


@pytest.mark.parametrize("p,q", [(0.5, 2.0), (2.0, 0.5), (1.0, 3.0), (4.0, 0.25)])
@pytest.mark.parametrize("rule", [oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT])
def test_symmetric_hint(p, q, rule, cuda):
    """symmetric=True (MLXC_ROWS_SYMMETRIC) on symmetric graphs: the shorter
    of row(x) and row(t) is searched, with the oracle's results (which search
    row(x)), in every mode; sorted and unsorted rows."""
    rowptr, col = synth.rmat_csr(12, 40_000, seed=17, symmetrize=True)
    rowptr, col = rowptr.numpy(), col.numpy()
    V = rowptr.size - 1
    start = np.arange(2 * V) % V
    _, counts = assert_parity(rowptr, col, start, 20, p, q, 99, rule, cuda, symmetric=True)
    if (p, q) == (0.5, 2.0):
        assert counts["member_tests"] > 1000
    rng = np.random.default_rng(8)
    rowptr, col = undirected(300, rng.integers(0, 300, (2500, 2)), sort=False)
    start = np.arange(600) % 300
    assert_parity(rowptr, col, start, 8, p, q, 5, rule, cuda, sorted_rows=False,
                  rows_sorted=False, symmetric=True)
    rowptr, col = synth.ba_hub_csr(20_000, 5, 4, 5_000, seed=3)
    rowptr, col = rowptr.numpy(), col.numpy()
    assert_parity(rowptr, col, np.arange(20_000), 12, p, q, 55, rule, cuda, symmetric=True)


def test_csr_check_matches_oracle(cuda):
    """csr_check equals the oracle's flags, and a malformed graph raises on
    every call whether or not a walk meets the bad entry: seed 0 takes
    candidate 0 of row(0) at walk 0's first step and never reads col[1] = 9,
    seed 1 takes candidate 1 (both checked on the oracle's stream here)."""
    rowptr, col = csr(4, [(0, 1), (0, 3), (2, 1)])
    cases = [(rowptr, col), (rowptr, np.array([3, 1, 1])), (rowptr, np.array([1, 9, 1])),
             (np.array([0, 2, 1, 3, 3]), col), (np.array([0, 2, 2, 3, 4]), col)]
    for rp, cl in cases:
        assert mc.csr_check(rp, cl) == oracle.csr_flags(rp, cl)
    u0 = {s: float(oracle.node2vec_trial0_u0(1, 1, s)[0, 0]) for s in (0, 1)}
    assert mc.csr_check(rowptr, col) == 8  # directed
    assert oracle.pick_index(u0[0], 2) == 0 and oracle.pick_index(u0[1], 2) == 1
    for seed in (0, 1):
        for stream in (None, "cpu"):
            with pytest.raises(ValueError, match="outside"):
                mc.rejection_sampling(rowptr, np.array([1, 9, 1]), np.array([0]), 3, 1.0, 1.0,
                                      seed=seed, stream=stream)
            with pytest.raises(ValueError, match="rowptr"):
                mc.rejection_sampling(np.array([0, 2, 1, 3, 3]), col, np.array([0]), 3, 1.0, 1.0,
                                      seed=seed, stream=stream)
            with pytest.raises(ValueError, match="rowptr"):  # rowptr[V] != E, every row valid
                mc.rejection_sampling(np.array([0, 1, 1, 2, 2]), col, np.array([0]), 3, 1.0, 1.0,
                                      seed=seed, stream=stream)


def test_csr_check_asymmetry(cuda):
    """MLXC_CSR_ASYMMETRIC tells a caller whether the promise behind
    symmetric=True holds: set on directed graphs, clear on symmetrized ones
    (with duplicates and self-loops), equal to the oracle's brute force; left
    clear on unsorted or malformed graphs."""
    for seed, sym in ((1, False), (2, True), (3, False), (4, True)):
        rowptr, col = synth.rmat_csr(11, 20_000, seed=seed, symmetrize=sym)
        rowptr, col = rowptr.numpy(), col.numpy()
        want = oracle.csr_flags(rowptr, col)
        assert want == (0 if sym else 8)
        assert mc.csr_check(rowptr, col) == want
    rp, cl = undirected(300, np.random.default_rng(5).integers(0, 300, (3000, 2)))
    assert mc.csr_check(rp, cl) == oracle.csr_flags(rp, cl) == 0
    cl2 = cl.copy()
    cl2[17] = (cl2[17] + 1) % 300  # one entry changed: its reverse is missing
    assert mc.csr_check(rp, cl2) == oracle.csr_flags(rp, cl2)
    # symmetric=True on a directed graph: caught by the check before the walk
    rowptr, col = synth.rmat_csr(11, 20_000, seed=1)
    assert mc.csr_check(rowptr, col) & 8
    # unsorted rows: bit 2 only
    rp3, cl3 = undirected(300, np.random.default_rng(6).integers(0, 300, (3000, 2)), sort=False)
    assert mc.csr_check(rp3, cl3) == oracle.csr_flags(rp3, cl3) == 4


def test_seed_none_follows_torch_manual_seed(c1, cuda):
    torch.manual_seed(3)
    a = mc.rejection_sampling(c1["rowptr"], c1["col"], c1["start"], 5, 1.0, 3.0)
    torch.manual_seed(3)
    b = mc.rejection_sampling(c1["rowptr"], c1["col"], c1["start"], 5, 1.0, 3.0)
    assert torch.equal(a, b)


@pytest.mark.parametrize("rule", ["ref_chain", "node2vec"])
def test_cpu_twin_equals_gpu(rule, cuda):
    """stream='cpu' (host twin) and the GPU kernels give the same node2vec
    walks and edges on a hub graph, for sorted and unsorted row handling."""
    rowptr, col = synth.ba_hub_csr(50_000, 5, 4, 8_000, seed=9)
    start = torch.arange(100_000) % 50_000
    for rows_sorted in (None, False):
        kw = dict(seed=17, rule=rule, rows_sorted=rows_sorted, return_edges=True)
        g = mc.rejection_sampling(rowptr.to(cuda), col.to(cuda), start.to(cuda), 15, 4.0, 0.25, **kw)
        c = mc.rejection_sampling(rowptr, col, start, 15, 4.0, 0.25, stream="cpu", **kw)
        assert torch.equal(g[0].cpu(), c[0]) and torch.equal(g[1].cpu(), c[1])


@pytest.mark.parametrize("L", [8, 300])
def test_long_walks_with_sinks(L, cuda):
    """Directed R-MAT graph (many nodes of out-degree 0): sink tails of up to
    hundreds of 64-byte blocks and walks ending on a block boundary, stored
    cooperatively by the wavefront; both rules, bit-exact."""
    rowptr, col = synth.rmat_csr(10, 4000, seed=45)
    rowptr, col = rowptr.numpy(), col.numpy()
    start = (np.arange(2000) * 7) % (rowptr.size - 1)
    for rule in (oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT):
        _, counts = assert_parity(rowptr, col, start, L, 0.5, 2.0, 71, rule, cuda)
        assert counts["sink_walks"] > 500


@pytest.mark.parametrize("rule", ["ref_chain", "node2vec"])
def test_int32_output(rule, cuda):
    """out_dtype=torch.int32: the walk with and without edges, and through
    the C ABI in each mode (edge records, CSR mode, the direct kernel), gives
    the int64 results, narrowed."""
    rowptr, col = synth.rmat_csr(12, 40_000, seed=13, symmetrize=True)
    rowptr, col = rowptr.to(cuda), col.to(cuda)
    start = torch.arange(9000, device=cuda) % (rowptr.numel() - 1)
    kw = dict(seed=5, rule=rule, return_edges=True)
    a = mc.rejection_sampling(rowptr, col, start, 21, 0.5, 2.0, **kw)
    b = mc.rejection_sampling(rowptr, col, start, 21, 0.5, 2.0, out_dtype=torch.int32, **kw)
    assert b[0].dtype == torch.int32
    assert torch.equal(a[0], b[0].long()) and torch.equal(a[1], b[1].long())
    c = mc.rejection_sampling(rowptr, col, start, 21, 0.5, 2.0, out_dtype=torch.int32, seed=5,
                              rule=rule)
    assert torch.equal(a[0], c.long())
    for mode in ("direct", "csr", "records"):
        rule_id = {name: k for k, name in RULE_NAME.items()}[rule]
        n, e = _abi_walk(rowptr, col, start, 21, 0.5, 2.0, 5, rule_id, 2, mode,
                         out_dtype=torch.int32)
        assert n.dtype == torch.int32
        assert torch.equal(a[0], n.long()) and torch.equal(a[1], e.long()), mode


def test_c3_full_size_properties(cuda):
    """Configuration 3 at full size (node2vec p=0.5, q=2 on the symmetrized
    R-MAT 2^20 graph, 4 walks per node, L=40).  Every one of the 167,772,160
    steps follows its recorded edge (inside the row of the current node, and
    col[e] is the next node) or stays, with edge id -1, at a node of
    out-degree 0; and three blocks of 2,000 walks (start, middle and end of
    the walk-id range, hence of the Philox counters) are bit-exact against the
    oracle, nodes and edges.  The direct kernel (the path of graphs beyond
    int32 ids, forced by a minimal workspace) gives the same walks in full."""
    rowptr, col = synth.rmat_csr(20, 1 << 24, seed=0, device=cuda, symmetrize=True)
    V, E = rowptr.numel() - 1, col.numel()
    N, L = 4 * V, 40
    start = torch.arange(N, device=cuda) % V
    n, e = mc.rejection_sampling(rowptr, col, start, L, 0.5, 2.0, seed=3, return_edges=True)
    assert torch.equal(n[:, 0], start)
    dn, de = _abi_walk(rowptr, col, start, L, 0.5, 2.0, 3, oracle.RULE_REF_CHAIN,
                       mc._lib.MLXC_ROWS_DETECT, "direct")
    assert torch.equal(dn, n) and torch.equal(de, e)
    del dn, de
    bad = 0
    for l in range(L):
        u, v, el = n[:, l], n[:, l + 1], e[:, l]
        rs, re = rowptr[u], rowptr[u + 1]
        stay = (el == -1) & (re == rs) & (v == u)
        move = (el >= rs) & (el < re) & (col[el.clamp(0, E - 1)] == v)
        bad += int((~(stay | move)).sum())
    assert bad == 0
    rp, cl = rowptr.cpu().numpy(), col.cpu().numpy()
    for s0 in (0, N // 2, N - 2000):
        ref, ref_e, st, _ = oracle.node2vec_walk(rp, cl, start[s0:s0 + 2000].cpu().numpy(), L,
                                                 0.5, 2.0, 3, rule=oracle.RULE_REF_CHAIN,
                                                 rows_sorted=True, with_edges=True, first_walk=s0)
        assert st == 0
        np.testing.assert_array_equal(n[s0:s0 + 2000].cpu().numpy(), ref)
        np.testing.assert_array_equal(e[s0:s0 + 2000].cpu().numpy(), ref_e)


@pytest.mark.parametrize("rule", ["ref_chain", "node2vec"])
def test_c5_full_size_properties(rule, cuda):
    """Configuration 5 at full size (BA graph of 4,000,000 nodes, m = 20, plus
    64 hubs of 500,000 neighbours; p = 4, q = 0.25, 2 walks per node, L = 30),
    with the reference chain (CSR mode: every draw accepts) and the analytic
    rule (edge records, frequent searches of hub rows, which the hub bitmaps
    answer).  Every step follows its recorded edge or stays at a node of
    out-degree 0.  52,128 walks are bit-exact against the oracle, nodes and
    edges: 25 blocks of 1,000 spread over the walk-id range, both walks of
    each of the 64 hubs, and the first walks of 27,000 nodes drawn from the
    hubs' neighbours (their walks step onto hubs, whose rows the acceptance
    test searches).  The direct kernel (the path of graphs beyond int32 ids,
    forced by a minimal workspace) gives the same walks in full."""
    rowptr, col = synth.ba_hub_csr(4_000_000, 20, 64, 500_000, seed=0, device=cuda)
    V, E = rowptr.numel() - 1, col.numel()
    N, L = 2 * V, 30
    start = torch.arange(N, device=cuda) % V
    n, e = mc.rejection_sampling(rowptr, col, start, L, 4.0, 0.25, seed=5, rule=rule,
                                 return_edges=True)
    assert torch.equal(n[:, 0], start)
    rule_id = {name: k for k, name in RULE_NAME.items()}[rule]
    dn, de = _abi_walk(rowptr, col, start, L, 4.0, 0.25, 5, rule_id, mc._lib.MLXC_ROWS_DETECT,
                       "direct")
    assert torch.equal(dn, n) and torch.equal(de, e)
    del dn, de
    bad = 0
    for l in range(L):
        u, v, el = n[:, l], n[:, l + 1], e[:, l]
        rs, re = rowptr[u], rowptr[u + 1]
        stay = (el == -1) & (re == rs) & (v == u)
        move = (el >= rs) & (el < re) & (col[el.clamp(0, E - 1)] == v)
        bad += int((~(stay | move)).sum())
    assert bad == 0
    rp, cl = rowptr.cpu().numpy(), col.cpu().numpy()
    n_h, e_h = n.cpu().numpy(), e.cpu().numpy()
    checked = 0
    for s0 in np.linspace(0, N - 1000, 25).astype(np.int64):
        ref, ref_e, st, _ = oracle.node2vec_walk(rp, cl, start[s0:s0 + 1000].cpu().numpy(), L,
                                                 4.0, 0.25, 5, rule=rule_id, rows_sorted=True,
                                                 with_edges=True, first_walk=int(s0))
        assert st == 0
        np.testing.assert_array_equal(n_h[s0:s0 + 1000], ref)
        np.testing.assert_array_equal(e_h[s0:s0 + 1000], ref_e)
        checked += 1000
    # walk n starts at node n % V: the hubs' walks, and the first walks of hub
    # neighbours (each checked with the oracle told its walk id)
    deg = np.diff(rp)
    hubs = np.flatnonzero(deg >= 500_000)
    assert hubs.size == 64
    nbrs = np.unique(np.concatenate([cl[rp[h]:rp[h + 1]] for h in hubs]))
    picks = np.random.default_rng(5).choice(nbrs, 27_000, replace=False)
    ids = np.concatenate([hubs, hubs + V, picks])
    for w in ids:
        ref, ref_e, st, _ = oracle.node2vec_walk(rp, cl, np.array([w % V]), L, 4.0, 0.25, 5,
                                                 rule=rule_id, rows_sorted=True, with_edges=True,
                                                 first_walk=int(w))
        assert st == 0
        np.testing.assert_array_equal(n_h[w], ref[0])
        np.testing.assert_array_equal(e_h[w], ref_e[0])
        checked += 1
    assert checked >= 50_000
    print(f"c5 {rule}: {checked} walks bit-exact against the oracle", flush=True)


@pytest.mark.parametrize("rule", [oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT])
def test_lds_walk(rule, cuda):
    """Graphs whose rowptr and col fit in LDS (V + 1 + E <= 14,336 entries) on
    calls of 1 to 2^20 steps take the LDS walk: the workspace query asks for
    the 256-byte header.  Bit-exact nodes and edges against the oracle for
    sorted, detected and unsorted rows, p < 1 and p > 1, int32 output, at the
    size limit; one entry over it, the record walk gives the same walks;
    malformed input raises ValueError."""
    from mlx_cluster_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(rule + 3)
    V = 1500
    pairs = rng.integers(0, V, (5000, 2))
    rowptr, col = undirected(V, pairs)
    urowptr, ucol = undirected(V, pairs, sort=False)  # the same rows, unsorted
    assert np.array_equal(urowptr, rowptr) and oracle.csr_flags(urowptr, ucol) & 4
    t = lambda a: torch.as_tensor(np.asarray(a, dtype=np.int64)).to(cuda)
    for N, L, p, q in ((1, 1, 0.5, 2.0), (700, 9, 0.25, 4.0), (3000, 30, 2.0, 0.5)):
        assert lib.mlxc_rejection_sampling_workspace_bytes(V, col.size, N, L, p, q, rule) == 256
        start = (np.arange(N) * 11) % V
        for rp, cl, rows_sorted in ((rowptr, col, None), (rowptr, col, True)):
            n_ref, e_ref, st, _ = oracle.node2vec_walk(rp, cl, start, L, p, q, 9, rule=rule,
                                                       rows_sorted=True, with_edges=True)
            assert st == 0
            n, e = mc.rejection_sampling(t(rp), t(cl), t(start), L, p, q, seed=9,
                                         rule=RULE_NAME[rule], rows_sorted=rows_sorted,
                                         return_edges=True)
            np.testing.assert_array_equal(n.cpu().numpy(), n_ref)
            np.testing.assert_array_equal(e.cpu().numpy(), e_ref)
            n32 = mc.rejection_sampling(t(rp), t(cl), t(start), L, p, q, seed=9,
                                        rule=RULE_NAME[rule], out_dtype=torch.int32)
            np.testing.assert_array_equal(n32.cpu().numpy(), n_ref)
        # unsorted rows: detected, and stated
        n_ref, _, st, _ = oracle.node2vec_walk(urowptr, ucol, start, L, p, q, 9, rule=rule,
                                               rows_sorted=False, with_edges=True)
        assert st == 0
        for rows_sorted in (None, False):
            n = mc.rejection_sampling(t(urowptr), t(ucol), t(start), L, p, q, seed=9,
                                      rule=RULE_NAME[rule], rows_sorted=rows_sorted)
            np.testing.assert_array_equal(n.cpu().numpy(), n_ref)
    # at the limit and one entry over it
    base = np.stack([np.repeat(np.arange(V), np.diff(rowptr)), col], 1)
    for total, lds in ((14336, True), (14337, False)):
        rp2, cl2 = csr(V, np.concatenate([base, np.tile([[0, 1]], (total - (V + 1 + col.size), 1))]))
        N, L = 2000, 6
        assert (lib.mlxc_rejection_sampling_workspace_bytes(V, cl2.size, N, L, 0.5, 2.0, rule)
                == 256) == lds
        start = (np.arange(N) * 3) % V
        n_ref, _, st, _ = oracle.node2vec_walk(rp2, cl2, start, L, 0.5, 2.0, 4, rule=rule,
                                               rows_sorted=True, with_edges=True)
        n = mc.rejection_sampling(t(rp2), t(cl2), t(start), L, 0.5, 2.0, seed=4,
                                  rule=RULE_NAME[rule])
        np.testing.assert_array_equal(n.cpu().numpy(), n_ref)
    # malformed input
    rp3, cl3 = csr(4, [(0, 1), (1, 2), (1, 3), (2, 3), (3, 0), (3, 1)])
    with pytest.raises(ValueError):
        mc.rejection_sampling(t(rp3), t(cl3), t([0, 9]), 3, 0.5, 2.0, seed=1, rule=RULE_NAME[rule])
    with pytest.raises(ValueError):
        mc.rejection_sampling(t(rp3), t([1, 2, 3, 7, 0, 1]), t([0, 1, 2, 3]), 4, 0.5, 2.0,
                              seed=1, rule=RULE_NAME[rule])


@pytest.mark.parametrize("rule", [oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT])
def test_lds_walk_many_walks(rule, cuda):
    """The LDS walk spreads its walks over at most one block per compute unit,
    256 to 1,024 walking threads a block: 50,000 walks take about 200 blocks
    of 256 walkers, 300,000 take a block per compute unit of 1,024 walkers
    that each run two walks or more.  Bit-exact against the oracle, nodes
    and edges."""
    from mlx_cluster_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(11 + rule)
    V = 900
    rowptr, col = undirected(V, rng.integers(0, V, (3000, 2)))
    t = lambda a: torch.as_tensor(np.asarray(a, dtype=np.int64)).to(cuda)
    for N, L in ((50_000, 4), (300_000, 3)):
        assert lib.mlxc_rejection_sampling_workspace_bytes(V, col.size, N, L, 0.5, 2.0, rule) == 256
        start = (np.arange(N) * 7) % V
        n_ref, e_ref, st, _ = oracle.node2vec_walk(rowptr, col, start, L, 0.5, 2.0, 21, rule=rule,
                                                   rows_sorted=True, with_edges=True)
        assert st == 0
        n, e = mc.rejection_sampling(t(rowptr), t(col), t(start), L, 0.5, 2.0, seed=21,
                                     rule=RULE_NAME[rule], return_edges=True)
        np.testing.assert_array_equal(n.cpu().numpy(), n_ref)
        np.testing.assert_array_equal(e.cpu().numpy(), e_ref)


@pytest.mark.parametrize("N", [3000, 6000, 12000, 24000, 40000])
def test_lds_walk_lane_groups(N, cuda):
    """The LDS walk runs each walk on a group of lanes that try consecutive
    trials of its step at once: on 256 compute units, 16 lanes up to 4,096
    walks, then 8, 4 and 2 up to 8,192, 16,384 and 32,768, and one lane
    beyond.  One call per group size, both rules, and with q = 30 too, where
    most candidates away from t are rejected and steps take many rounds:
    bit-exact against the oracle, nodes and edges."""
    rng = np.random.default_rng(N)
    V = 700
    rowptr, col = undirected(V, rng.integers(0, V, (2500, 2)))
    t = lambda a: torch.as_tensor(np.asarray(a, dtype=np.int64)).to(cuda)
    start = (np.arange(N) * 13) % V
    L = 6
    for rule in (oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT):
        for p, q in ((0.5, 2.0), (1.0, 30.0)):
            n_ref, e_ref, st, _ = oracle.node2vec_walk(rowptr, col, start, L, p, q, 5, rule=rule,
                                                       rows_sorted=True, with_edges=True)
            assert st == 0
            n, e = mc.rejection_sampling(t(rowptr), t(col), t(start), L, p, q, seed=5,
                                         rule=RULE_NAME[rule], return_edges=True)
            np.testing.assert_array_equal(n.cpu().numpy(), n_ref, err_msg=f"{rule} {p} {q}")
            np.testing.assert_array_equal(e.cpu().numpy(), e_ref, err_msg=f"{rule} {p} {q}")


def test_lds_walks_random_sweep(cuda):
    """Random small graphs (directed and undirected, duplicates and
    self-loops kept) under the LDS limit, random walk counts and lengths:
    the uniform and node2vec LDS walks (the Python API's default for these
    sizes) are bit-exact against the oracle for both rules and several
    (p, q)."""
    from mlx_cluster_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(2024)
    t = lambda a: torch.as_tensor(np.asarray(a, dtype=np.int64)).to(cuda)
    for case in range(12):
        V = int(rng.integers(2, 2000))
        E_pairs = int(rng.integers(1, 6000))
        pairs = rng.integers(0, V, (E_pairs, 2))
        rowptr, col = (undirected(V, pairs) if case % 2 else csr(V, pairs))
        if V + 1 + col.size > 14336:
            continue
        N = int(rng.integers(1, 3000))
        L = int(rng.integers(1, 50))
        start = rng.integers(0, V, N)
        # the Python API takes the LDS walks here, whatever N * L is
        assert lib.mlxc_random_walk_workspace_bytes(V, col.size, N, L) == 256
        assert lib.mlxc_rejection_sampling_workspace_bytes(V, col.size, N, L, 1.0, 1.0, 0) == 256
        rand = mc.philox_uniform((N, L), case, device=cuda)
        n_ref, e_ref, st, _ = oracle.uniform_walk(rowptr, col, start, rand.cpu().numpy(), L,
                                                  with_edges=True)
        assert st == 0
        n, e = mc.random_walk(t(rowptr), t(col), t(start), rand, L, return_edges=True)
        np.testing.assert_array_equal(n.cpu().numpy(), n_ref, err_msg=f"uniform case {case}")
        np.testing.assert_array_equal(e.cpu().numpy(), e_ref, err_msg=f"uniform edges {case}")
        for p, q in ((1.0, 1.0), (0.3, 3.0), (4.0, 0.25)):
            for rule in (oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT):
                n_ref, e_ref, st, _ = oracle.node2vec_walk(rowptr, col, start, L, p, q, case,
                                                           rule=rule, rows_sorted=True,
                                                           with_edges=True)
                assert st == 0
                n, e = mc.rejection_sampling(t(rowptr), t(col), t(start), L, p, q, seed=case,
                                             rule=RULE_NAME[rule], return_edges=True)
                np.testing.assert_array_equal(n.cpu().numpy(), n_ref,
                                              err_msg=f"node2vec case {case} {p} {q} {rule}")
                np.testing.assert_array_equal(e.cpu().numpy(), e_ref)


@pytest.mark.parametrize("rule", [oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT])
def test_row_hash_tables_overflow_and_size_limit(rule, cuda):
    """Row hash tables at their edges.  Node 0's row holds 20 ids that all
    fall in bucket 0 of its 3-bucket table: 16 fill that bucket and 4 move on
    to bucket 1, and a lookup of an absent id whose bucket is the full one
    reads bucket 1 too.  Node 1's row has 1,023 entries (the longest row with
    a table) and node 2's 1,024 (none: index levels).  The 20 ids are joined
    in a chain and the hub rows are linked, so walks step from one of the ids
    to node 0 and test the previous node against row 0.  Walks starting at
    the 20 ids and at random nodes are bit-exact against the oracle in every
    layout, sorted and unsorted rows."""
    B = 3

    def bucket(t):
        return (((t * 0x9E3779B1) & 0xFFFFFFFF) * B) >> 32

    V = 3000
    ids = [t for t in range(3, V) if bucket(t) == 0][:20]
    rng = np.random.default_rng(rule + 17)
    others = [t for t in range(3, V) if t not in set(ids)]
    pairs = [(0, c) for c in ids] + list(zip(ids[:-1], ids[1:]))
    pairs += [(1, c) for c in rng.choice(others, 1023 - 1, replace=False)] + [(1, 2)]
    pairs += [(2, c) for c in rng.choice(others, 1024 - 1, replace=False)]
    pairs += [(int(a), int(b)) for a, b in rng.integers(3, V, (4000, 2)) if a != b]
    rowptr, col = undirected(V, pairs)
    deg = np.diff(rowptr)
    assert (deg[0], deg[1], deg[2]) == (20, 1023, 1024)
    start = np.concatenate([np.repeat(ids, 200), rng.integers(0, V, 6000)])
    for sorted_rows in (True, False):
        r, c = rowptr, col
        if not sorted_rows:  # the same rows, each reversed
            c = np.concatenate([col[rowptr[v]:rowptr[v + 1]][::-1] for v in range(V)])
        assert_parity(r, c, start, 12, 0.5, 2.0, 99, rule, cuda, sorted_rows=sorted_rows,
                      rows_sorted=sorted_rows)
