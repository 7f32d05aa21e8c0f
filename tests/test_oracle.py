"""Pins the CPU oracle (oracle/) before it is trusted as the GPU's checker.

The reference's own tests hold no golden vectors (they print, and load Cora
over the network: /root/reference/tests/test_random_walk.py:18,38), so the
oracle is pinned by published known answers (Philox), an independent library
(rocRAND), hand-derived walks on tiny graphs, numpy's IEEE float32, closed
forms of the node2vec transition probabilities (chi-square), and identities
between the functions (p = q = 1 is the uniform walk).
"""
import os

import numpy as np
import pytest
from scipy import stats

import oracle
from tests.graphs import csr, undirected, uniform_transitions_ok

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# ------------------------------------------------------------------ Philox


@pytest.mark.parametrize("ctr,key,expect", [
    # Random123 known-answer vectors for philox4x32-10 (kat_vectors).
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
])
def test_philox_known_answers(ctr, key, expect):
    assert list(oracle.philox4x32_10(ctr, key)) == expect


def test_philox_matches_rocrand():
    """64 vectors written by rocRAND's philox4x32_10_engine::ten_rounds
    (tests/golden/philox_rocrand_vectors.cpp)."""
    n = 0
    with open(os.path.join(GOLDEN, "philox_rocrand.txt")) as f:
        for line in f:
            if line.startswith("#"):
                continue
            w = [int(x, 16) for x in line.split()]
            assert list(oracle.philox4x32_10(w[0:4], w[4:6])) == w[6:10]
            n += 1
    assert n == 64


def test_unit_float_endpoints():
    assert oracle.u32_to_unit_float(0) == 0.0
    assert oracle.u32_to_unit_float(0xFF) == 0.0
    assert oracle.u32_to_unit_float(0x100) == 2.0 ** -24
    assert oracle.u32_to_unit_float(0xFFFFFFFF) == 1.0 - 2.0 ** -24


def test_uniform_fill_layout():
    """Element i is word i % 4 of block i // 4 (counter (i//4, 0, 0, 0))."""
    seed = 0x1234_5678_9ABC_DEF0
    u = oracle.philox_uniform(11, seed)
    key = [seed & 0xFFFFFFFF, seed >> 32]
    for i in range(11):
        w = oracle.philox4x32_10([i // 4, 0, 0, 0], key)[i % 4]
        assert u[i] == np.float32((int(w) >> 8) * 2.0 ** -24)
    assert u.min() >= 0.0 and u.max() < 1.0


@pytest.mark.parametrize("first", [1, 6, 4096 * 80 + 3, (1 << 34) + 5])
def test_uniform_fill_at_offset(first):
    """Elements [first, first + n) of the stream: each rebuilt from one
    Philox block (counter (pos//4 lo, pos//4 hi, 0, 0)), the high counter
    word included past 2^34; and equal to the slice of the fill from 0."""
    seed = 0x0BAD_5EED_0000_0042
    n = 13
    u = oracle.philox_uniform(n, seed, first=first)
    key = [seed & 0xFFFFFFFF, seed >> 32]
    for i in range(n):
        pos = first + i
        w = oracle.philox4x32_10([(pos >> 2) & 0xFFFFFFFF, pos >> 34, 0, 0], key)[pos % 4]
        assert u[i] == np.float32((int(w) >> 8) * 2.0 ** -24)
    if first < 1 << 20:
        assert np.array_equal(oracle.philox_uniform(first + n, seed)[first:], u)


def test_uniform_fill_is_uniform():
    u = oracle.philox_uniform(200_000, 7)
    assert stats.kstest(u, "uniform").pvalue > 0.01


# --------------------------------------------------------- index selection


@pytest.mark.parametrize("r,deg,expect", [
    (0.0, 1, 0), (0.0, 5, 0), (0.5, 2, 1), (0.25, 4, 1), (0.999, 4, 3),
    (1.0 - 2.0 ** -24, 3, 2), (1.0 - 2.0 ** -24, 1 << 24, (1 << 24) - 1),
    (0.5, (1 << 24) + 1, 1 << 23),
    # outside [0, 1): clamped into the row instead of reading past it
    (1.0, 7, 6), (2.5, 7, 6), (-0.5, 7, 0), (float("nan"), 7, 0), (float("inf"), 7, 6),
])
def test_pick_index_known(r, deg, expect):
    assert oracle.pick_index(r, deg) == expect


def test_pick_index_is_float32_not_float64():
    """RandomWalk.cpp:51-53 multiplies in float32.  Find products whose
    float32 rounding crosses an integer (so float64 truncation differs) and
    check the oracle follows numpy's IEEE float32 multiply on them."""
    rng = np.random.default_rng(0)
    r = rng.random(400_000, dtype=np.float32)
    deg = rng.integers(1 << 20, 1 << 24, 400_000)
    f32 = np.trunc(r * deg.astype(np.float32)).astype(np.int64)
    f64 = np.trunc(r.astype(np.float64) * deg.astype(np.float64)).astype(np.int64)
    diff = np.nonzero(f32 != f64)[0]
    assert diff.size > 10  # such cases exist and are exercised
    for i in diff[:200]:
        assert oracle.pick_index(float(r[i]), int(deg[i])) == min(f32[i], deg[i] - 1)


def test_pick_index_never_leaves_row_below_2p24():
    # Brute force over the top of [0,1): r = 1 - k * 2^-24, all deg up to 4096.
    for deg in range(1, 4097):
        for k in (1, 2, 3):
            assert oracle.pick_index(1.0 - k * 2.0 ** -24, deg) <= deg - 1


# ------------------------------------------------------------ uniform walk


def walk(rowptr, col, start, rand, L, **kw):
    n, e, st, counts = oracle.uniform_walk(rowptr, col, start, rand, L, with_edges=True, **kw)
    return n, e, st, counts


def test_uniform_directed_cycle():
    rowptr, col = csr(3, [(0, 1), (1, 2), (2, 0)])
    n, e, st, c = walk(rowptr, col, [0, 2], np.full((2, 4), 0.7, np.float32), 4)
    assert st == 0
    assert n.tolist() == [[0, 1, 2, 0, 1], [2, 0, 1, 2, 0]]
    assert e.tolist() == [[0, 1, 2, 0], [2, 0, 1, 2]]
    assert c["moving_steps"] == 8 and c["sink_walks"] == 0


def test_uniform_star_index_choice():
    # centre 0 <-> leaves 1..4; row(0) = [1, 2, 3, 4]
    rowptr, col = undirected(5, [(0, 1), (0, 2), (0, 3), (0, 4)])
    r = np.array([[k / 4 + 0.01, 0.3] for k in range(4)], np.float32)
    n, e, st, _ = walk(rowptr, col, [0, 0, 0, 0], r, 2)
    assert n.tolist() == [[0, 1, 0], [0, 2, 0], [0, 3, 0], [0, 4, 0]]
    assert e[:, 0].tolist() == [0, 1, 2, 3]


def test_uniform_extremes_pick_first_and_last():
    rowptr, col = csr(4, [(0, 3), (0, 1), (0, 2)])  # row(0) sorted: [1, 2, 3]
    n, _, _, _ = walk(rowptr, col, [0, 0], np.array([[0.0], [1 - 2 ** -24]], np.float32), 1)
    assert n[:, 1].tolist() == [1, 3]


def test_uniform_sink_absorbs():
    # 0 -> 1 -> 3, node 3 has out-degree 0, node 2 isolated
    rowptr, col = csr(4, [(0, 1), (1, 3)])
    n, e, st, c = walk(rowptr, col, [0, 2], np.full((2, 5), 0.5, np.float32), 5)
    assert n.tolist() == [[0, 1, 3, 3, 3, 3], [2, 2, 2, 2, 2, 2]]
    assert e.tolist() == [[0, 1, -1, -1, -1], [-1, -1, -1, -1, -1]]
    assert c["moving_steps"] == 2 and c["sink_walks"] == 2


def test_uniform_self_loop():
    rowptr, col = csr(2, [(0, 0), (0, 1), (1, 0)])
    n, _, _, _ = walk(rowptr, col, [0, 0], np.array([[0.1, 0.1], [0.75, 0.1]], np.float32), 2)
    assert n.tolist() == [[0, 0, 0], [0, 1, 0]]


def test_uniform_zero_length_and_empty():
    rowptr, col = csr(3, [(0, 1)])
    n, e, st, _ = walk(rowptr, col, [2, 0, 1], np.zeros((3, 0), np.float32), 0)
    assert n.tolist() == [[2], [0], [1]] and e.shape == (3, 0) and st == 0
    n, e, st, _ = walk(rowptr, col, np.zeros(0, np.int64), np.zeros(0, np.float32), 4)
    assert n.shape == (0, 5) and st == 0


def test_uniform_bad_indices_flagged():
    rowptr, col = csr(3, [(0, 1), (1, 2)])
    _, _, st, _ = walk(rowptr, col, [3], np.zeros((1, 2), np.float32), 2)
    assert st == -1
    _, _, st, _ = walk(rowptr, np.array([7, 2]), [0], np.zeros((1, 2), np.float32), 2)
    assert st == -1
    _, _, st, _ = walk(np.array([0, 2, 1, 2]), col, [0], np.zeros((1, 2), np.float32), 2)
    assert st == -1


def random_graph(num_nodes, num_edges, seed, sink_frac=0.2):
    rng = np.random.default_rng(seed)
    src = rng.integers(0, num_nodes, num_edges)
    keep = rng.random(num_nodes) >= sink_frac
    src = src[keep[src]]
    dst = rng.integers(0, num_nodes, src.size)
    return csr(num_nodes, np.stack([src, dst], 1))


def test_uniform_transitions_random_graph():
    rowptr, col = random_graph(500, 3000, 1)
    start = np.arange(500).repeat(3)
    L = 12
    rand = oracle.philox_uniform(start.size * L, 2)
    n, _, st, _ = walk(rowptr, col, start, rand, L)
    assert st == 0
    assert uniform_transitions_ok(rowptr, col, start, rand, n) == 0
    # a planted wrong answer is caught by the same check
    n[7, 3] = (n[7, 3] + 1) % 500
    assert uniform_transitions_ok(rowptr, col, start, rand, n) > 0


def test_uniform_distribution_chi_square():
    rowptr, col = csr(8, [(0, k) for k in range(1, 8)])  # 7 out-neighbours
    N = 70_000
    rand = oracle.philox_uniform(N, 11)
    n, _, _, _ = walk(rowptr, col, np.zeros(N, np.int64), rand, 1)
    counts = np.bincount(n[:, 1], minlength=8)[1:]
    assert stats.chisquare(counts).pvalue > 0.01


def test_uniform_fixture_c1(c1):
    n, e, st, _ = walk(c1["rowptr"], c1["col"], c1["start"], c1["rand"], int(c1["walk_length"]))
    assert st == 0
    np.testing.assert_array_equal(n, c1["uniform_nodes"])
    np.testing.assert_array_equal(e, c1["uniform_edges"])
    assert uniform_transitions_ok(c1["rowptr"], c1["col"], c1["start"], c1["rand"], n) == 0


# ---------------------------------------------------------- node2vec walk


@pytest.mark.parametrize("p,q,expect", [
    (1.0, 3.0, (1.0, 1.0, 1 / 3)),
    (0.5, 2.0, (1.0, 0.5, 0.25)),
    (4.0, 0.25, (0.0625, 0.25, 1.0)),
    (1.0, 1.0, (1.0, 1.0, 1.0)),
])
def test_node2vec_probs_closed_form(p, q, expect):
    np.testing.assert_allclose(oracle.node2vec_probs(p, q), expect, rtol=0, atol=1e-15)


def n2v(rowptr, col, start, L, p, q, seed, rule=oracle.RULE_REF_CHAIN, sorted_rows=True):
    n, e, st, c = oracle.node2vec_walk(rowptr, col, start, L, p, q, seed, rule=rule,
                                       rows_sorted=sorted_rows, with_edges=True)
    assert st == 0
    return n, e, c


@pytest.mark.parametrize("rule", [oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT])
def test_node2vec_p1_q1_is_uniform_walk(rule):
    """With p = q = 1 every candidate is accepted at trial 0, so the walk is
    the uniform walk driven by the trial-0 candidate uniforms."""
    rowptr, col = random_graph(400, 2500, 3)
    start = np.arange(400).repeat(2)
    L = 9
    n, e, c = n2v(rowptr, col, start, L, 1.0, 1.0, 42, rule)
    rand = oracle.node2vec_trial0_u0(start.size, L, 42)
    nu, eu, _, _ = walk(rowptr, col, start, rand, L)
    np.testing.assert_array_equal(n, nu)
    np.testing.assert_array_equal(e, eu)


def test_node2vec_ref_chain_degenerates_when_q_small():
    """F1: with p=4, q=0.25 the reference chain accepts every candidate
    (prob_2 = 1), so it equals the uniform walk on the trial-0 stream; the
    analytic rule does not."""
    rowptr, col = undirected(300, np.random.default_rng(4).integers(0, 300, (1500, 2)))
    start = np.arange(300)
    n, _, c = n2v(rowptr, col, start, 8, 4.0, 0.25, 9, oracle.RULE_REF_CHAIN)
    nu, _, _, _ = walk(rowptr, col, start, oracle.node2vec_trial0_u0(300, 8, 9), 8)
    np.testing.assert_array_equal(n, nu)
    assert c["member_tests"] == 0
    ne, _, ce = n2v(rowptr, col, start, 8, 4.0, 0.25, 9, oracle.RULE_NODE2VEC_EXACT)
    assert not np.array_equal(ne, nu) and ce["trials"] > c["trials"]


def test_node2vec_rules_agree_when_q_large():
    """When q >= max(p, 1) the chain's effective weights equal the analytic
    ones draw for draw, so both rules give identical walks."""
    rowptr, col = undirected(300, np.random.default_rng(5).integers(0, 300, (1500, 2)))
    start = np.arange(300).repeat(2)
    a, ea, _ = n2v(rowptr, col, start, 10, 0.5, 2.0, 17, oracle.RULE_REF_CHAIN)
    b, eb, _ = n2v(rowptr, col, start, 10, 0.5, 2.0, 17, oracle.RULE_NODE2VEC_EXACT)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(ea, eb)


def test_node2vec_forced_and_sink_steps():
    # path 0 - 1 - 2 plus isolated 3: every interior step is forced or a
    # back-and-forth choice; degree-1 rows take no draw.
    rowptr, col = undirected(4, [(0, 1), (1, 2)])
    n, e, _ = n2v(rowptr, col, [0, 3], 4, 1.0, 1.0, 1)
    assert n[1].tolist() == [3] * 5 and e[1].tolist() == [-1] * 4
    assert n[0, 1] == 1 and e[0, 0] == 0          # row(0) = [1], forced
    assert all(n[0, k] in (0, 2) for k in (2, 4))  # from 1: 0 or 2
    assert all(n[0, k] == 1 for k in (1, 3))       # from 0 or 2: back to 1


def test_node2vec_binary_search_equals_linear_scan():
    rowptr, col = undirected(200, np.random.default_rng(6).integers(0, 200, (1200, 2)))
    start = np.arange(200).repeat(3)
    for rule in (oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT):
        a, _, ca = n2v(rowptr, col, start, 12, 0.7, 3.0, 8, rule, sorted_rows=True)
        b, _, cb = n2v(rowptr, col, start, 12, 0.7, 3.0, 8, rule, sorted_rows=False)
        np.testing.assert_array_equal(a, b)
        assert ca["member_tests"] == cb["member_tests"] > 0


def three_class_graph(K, M):
    """t0 -> v; row(v) = {t0, a1..aK, b1..bM}; every a_i links to t0, no b_j
    does.  Walks of length 2 from t0 choose out[:, 2] with class weights
    (w0, K w1, M w2)."""
    t0, v = 0, 1
    a = list(range(2, 2 + K))
    b = list(range(2 + K, 2 + K + M))
    edges = [(t0, v)] + [(v, x) for x in [t0] + a + b] + [(x, t0) for x in a] + [(x, v) for x in b]
    return csr(2 + K + M, edges), a, b


def class_counts(out, a, b):
    x = out[:, 2]
    return np.array([np.sum(x == 0), np.sum(np.isin(x, a)), np.sum(np.isin(x, b))])


@pytest.mark.parametrize("p,q,rule", [
    (0.5, 2.0, oracle.RULE_NODE2VEC_EXACT), (4.0, 0.25, oracle.RULE_NODE2VEC_EXACT),
    (2.0, 0.5, oracle.RULE_NODE2VEC_EXACT), (0.5, 2.0, oracle.RULE_REF_CHAIN),
    (4.0, 0.25, oracle.RULE_REF_CHAIN), (2.0, 0.5, oracle.RULE_REF_CHAIN),
])
def test_node2vec_transition_chi_square(p, q, rule):
    """Transition frequencies match the closed-form weights: analytic
    (1/p, 1, 1/q) for the exact rule; (max(p0,p2), max(p1,p2), p2) for the
    reference chain (BiasedRandomWalk.cpp:86-91)."""
    K, M = 3, 4
    (rowptr, col), a, b = three_class_graph(K, M)
    N = 60_000
    n, _, _ = n2v(rowptr, col, np.zeros(N, np.int64), 2, p, q, 1234, rule)
    p0, p1, p2 = oracle.node2vec_probs(p, q)
    w = (p0, p1, p2) if rule == oracle.RULE_NODE2VEC_EXACT else (max(p0, p2), max(p1, p2), p2)
    expect = np.array([w[0], K * w[1], M * w[2]])
    expect = expect / expect.sum() * N
    assert stats.chisquare(class_counts(n, a, b), expect).pvalue > 0.01


@pytest.mark.parametrize("p,q,rule", [
    (0.5, 2.0, oracle.RULE_NODE2VEC_EXACT), (4.0, 0.25, oracle.RULE_NODE2VEC_EXACT),
    (1.0, 3.0, oracle.RULE_NODE2VEC_EXACT), (4.0, 0.25, oracle.RULE_REF_CHAIN),
    (0.5, 2.0, oracle.RULE_REF_CHAIN),
])
def test_node2vec_return_probability_on_trees(p, q, rule):
    """On a tree no neighbour of v other than t is adjacent to t, so from v
    (reached from t) the walk returns to t with probability
    w0 / (w0 + (deg(v) - 1) * w2): (1/p) / ((1/p) + (deg(v) - 1)/q) for the
    analytic rule, max(p0, p2) and p2 for the reference chain.  Checked on a
    random tree over every step that has a previous node and deg(v) >= 2:
    the count of returns against the sum of the per-step probabilities."""
    rng = np.random.default_rng(int(p * 100 + q * 10 + rule))
    V = 400
    parent = [int(rng.integers(0, i)) for i in range(1, V)]
    rowptr, col = undirected(V, [(i + 1, parent[i]) for i in range(V - 1)])
    deg = np.diff(rowptr)
    N, L = 20_000, 12
    n, _, _ = n2v(rowptr, col, rng.integers(0, V, N), L, p, q, 77, rule)
    p0, p1, p2 = oracle.node2vec_probs(p, q)
    w0 = p0 if rule == oracle.RULE_NODE2VEC_EXACT else max(p0, p2)
    prev, cur, nxt = n[:, :-2].ravel(), n[:, 1:-1].ravel(), n[:, 2:].ravel()
    k = deg[cur]
    use = k >= 2
    prob = w0 / (w0 + (k[use] - 1) * p2)
    returns = np.count_nonzero(nxt[use] == prev[use])
    z = (returns - prob.sum()) / np.sqrt((prob * (1 - prob)).sum())
    assert abs(z) < 4.5, (returns, prob.sum())
    # deg(v) == 1 is forced back to t (BiasedRandomWalk.cpp:76-78)
    assert np.all(nxt[k == 1] == prev[k == 1])


def test_node2vec_libc_stream_chi_square():
    """The libc-rand() restatement (the reference's own draw pattern) gives
    the same transition law as the Philox-driven one."""
    K, M = 3, 4
    (rowptr, col), a, b = three_class_graph(K, M)
    N = 60_000
    n, st = oracle.node2vec_walk_libc(rowptr, col, np.zeros(N, np.int64), 2, 0.5, 2.0, 1)
    assert st == 0
    p0, p1, p2 = oracle.node2vec_probs(0.5, 2.0)
    expect = np.array([p0, K * p1, M * p2])
    expect = expect / expect.sum() * N
    assert stats.chisquare(class_counts(n, a, b), expect).pvalue > 0.01


def test_node2vec_fixture_c1(c1):
    names = sorted({k[4:-6] for k in c1 if k.startswith("n2v_") and k.endswith("_nodes")})
    assert len(names) == 5
    for name in names:
        p, q, rule, seed = c1[f"n2v_{name}_params"]
        n, e, _ = n2v(c1["rowptr"], c1["col"], c1["start"], int(c1["walk_length"]), p, q,
                      int(seed), int(rule))
        np.testing.assert_array_equal(n, c1[f"n2v_{name}_nodes"])
        np.testing.assert_array_equal(e, c1[f"n2v_{name}_edges"])


def test_node2vec_walks_follow_edges(c1):
    rowptr, col = c1["rowptr"], c1["col"]
    n = c1["n2v_p05_q2_ref_nodes"]
    for l in range(n.shape[1] - 1):
        u, v = n[:, l], n[:, l + 1]
        ok = [(rowptr[x + 1] == rowptr[x] and y == x) or y in col[rowptr[x]:rowptr[x + 1]]
              for x, y in zip(u, v)]
        assert all(ok)


# -------------------------------------------------------------- CSR flags


def test_csr_flags():
    rowptr, col = csr(4, [(0, 1), (0, 3), (2, 1)])
    assert oracle.csr_flags(rowptr, col) == 8                         # directed: no (1, 0)
    srp, scol = undirected(4, [(0, 1), (0, 3), (2, 1)])
    assert oracle.csr_flags(srp, scol) == 0
    assert oracle.csr_flags(rowptr, np.array([3, 1, 1])) == 4         # row 0 unsorted
    assert oracle.csr_flags(rowptr, np.array([1, 9, 1])) == 2         # col out of range
    assert oracle.csr_flags(np.array([0, 2, 1, 3, 3]), col) & 1      # decreasing rowptr
    assert oracle.csr_flags(np.array([0, 2, 2, 3, 4]), col) & 1      # rowptr[V] != E


def test_csr_asymmetry_flag_brute_force():
    """Bit 3 against a set of pairs: random graphs with duplicates and
    self-loops, symmetrized (clear) and with one reverse entry removed or one
    directed entry added (set)."""
    rng = np.random.default_rng(31)
    for case in range(40):
        V = int(rng.integers(1, 60))
        pairs = rng.integers(0, V, (int(rng.integers(0, 200)), 2))
        rowptr, col = undirected(V, pairs)
        pairs_set = set()
        for u in range(V):
            pairs_set.update((u, int(v)) for v in col[rowptr[u]:rowptr[u + 1]])
        assert all((v, u) in pairs_set for u, v in pairs_set)
        assert oracle.csr_flags(rowptr, col) == 0
        if len(pairs) == 0:
            continue
        # drop every copy of one entry (u, v) with u != v: (v, u) loses its reverse
        u, v = (int(x) for x in pairs[int(rng.integers(0, len(pairs)))])
        edges = [(a, int(b)) for a in range(V) for b in col[rowptr[a]:rowptr[a + 1]]]
        kept = [e for e in edges if e != (u, v)]
        rp2, cl2 = csr(V, kept) if kept else (np.zeros(V + 1, np.int64), np.zeros(0, np.int64))
        want = any((b, a) not in set(kept) for a, b in kept)
        assert bool(oracle.csr_flags(rp2, cl2) & 8) == want, case
        assert want == (u != v)
        # one extra directed entry
        a, b = (int(x) for x in rng.integers(0, V, 2))
        rp3, cl3 = csr(V, edges + [(a, b)])
        assert bool(oracle.csr_flags(rp3, cl3) & 8) == ((b, a) not in set(edges) and a != b), case


# ---------------------------------------------------------------- CSR build

def _brute_csr(row, col, V, symmetrize, dedup):
    """Pure-Python CSR: sorted() of the (row, col) tuples, per-node loops."""
    pairs = list(zip(row.tolist(), col.tolist()))
    if symmetrize:
        pairs += [(c, r) for r, c in pairs]
    pairs = sorted(set(pairs)) if dedup else sorted(pairs)
    rowptr = [0]
    for v in range(V):
        rowptr.append(rowptr[-1] + sum(1 for r, _ in pairs if r == v))
    return rowptr, [c for _, c in pairs]


@pytest.mark.parametrize("seed", range(6))
def test_csr_build_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    V = int(rng.integers(1, 20))
    E = int(rng.integers(0, 60))
    row, col = rng.integers(0, V, E), rng.integers(0, V, E)
    for symmetrize in (False, True):
        for dedup in (False, True):
            rowptr, c = oracle.csr_build(row, col, V, symmetrize=symmetrize, dedup=dedup)
            ref_rowptr, ref_col = _brute_csr(row, col, V, symmetrize, dedup)
            assert rowptr.tolist() == ref_rowptr and c.tolist() == ref_col


def test_csr_build_equals_reference_pipeline_without_empty_rows():
    """tests/test_random_walk.py:26-28 takes rowptr from np.unique counts; on a
    graph where every node has an out-edge that is exactly this rowptr."""
    rng = np.random.default_rng(3)
    V = 50
    row = np.concatenate([np.arange(V), rng.integers(0, V, 300)])
    col = rng.integers(0, V, row.size)
    rowptr, c = oracle.csr_build(row, col, V)
    order = np.lexsort((col, row))
    _, counts = np.unique(row[order], return_counts=True)
    assert rowptr.tolist() == np.concatenate([[0], counts.cumsum()]).tolist()
    assert c.tolist() == col[order].tolist()


def test_csr_build_hand_case():
    row, col = np.array([3, 0, 0, 3, 0]), np.array([0, 2, 1, 1, 2])
    rowptr, c = oracle.csr_build(row, col, 5)
    assert rowptr.tolist() == [0, 3, 3, 3, 5, 5] and c.tolist() == [1, 2, 2, 0, 1]
    rowptr, c = oracle.csr_build(row, col, 5, dedup=True)
    assert rowptr.tolist() == [0, 2, 2, 2, 4, 4] and c.tolist() == [1, 2, 0, 1]
    rowptr, c = oracle.csr_build(np.array([0]), np.array([1]), 2, symmetrize=True)
    assert rowptr.tolist() == [0, 1, 2] and c.tolist() == [1, 0]


# ---------------------------------------------------------------- context windows

def test_philox_np_matches_c_oracle():
    rng = np.random.default_rng(9)
    for _ in range(64):
        c = rng.integers(0, 2**32, 4)
        k = int(rng.integers(0, 2**63)) * 2 + int(rng.integers(0, 2))
        ref = oracle.philox4x32_10(c, [k & 0xFFFFFFFF, k >> 32])
        got = oracle.philox4x32_10_np(*[np.array([x], dtype=np.uint64) for x in c], k)
        assert [int(g[0]) for g in got] == [int(x) for x in ref]


def test_context_windows_brute_force_and_unfold():
    """Pure-Python loops, and torch's unfold (an independent library routine)."""
    import torch
    rng = np.random.default_rng(4)
    for N, nodes, C in ((1, 1, 1), (3, 5, 2), (7, 9, 9), (5, 21, 10)):
        walks = rng.integers(0, 1000, (N, nodes))
        got = oracle.context_windows(walks, C)
        W = nodes - C + 1
        brute = [[int(walks[n][j + k]) for k in range(C)] for j in range(W) for n in range(N)]
        assert got.tolist() == brute
        unf = torch.from_numpy(walks).unfold(1, C, 1).transpose(0, 1).reshape(W * N, C)
        assert got.tolist() == unf.tolist()


def test_negative_walks_closed_form():
    start = np.array([7, 3, 2**40])
    rw = oracle.negative_walks(start, 4, 1000, seed=5)
    assert rw.shape == (3, 5) and rw[:, 0].tolist() == start.tolist()
    for n in range(3):
        for l in range(1, 5):
            x = int(oracle.philox4x32_10([n, 0, l, 0], [5, 0])[0])
            assert rw[n, l] == (x * 1000) >> 32
    u = oracle.negative_walks(np.zeros(20000, np.int64), 8, 37, seed=11)[:, 1:].reshape(-1)
    counts = np.bincount(u, minlength=37)
    assert u.min() >= 0 and u.max() < 37
    assert stats.chisquare(counts).pvalue > 1e-4
