"""The host twins behind stream='cpu' (mlxc_*_cpu in libmlxc.so).

Bit-exact against the oracle and the committed C1 fixture, independent of
the thread count, and with the device path's argument and status handling.
No GPU needed: these entry points take host pointers.
"""
import numpy as np
import pytest
import torch

import mlx_cluster_amd as mc
import oracle
from mlx_cluster_amd import synth
from tests import status_cases
from tests.graphs import csr, undirected, uniform_transitions_ok

RULE_NAME = {oracle.RULE_REF_CHAIN: "ref_chain", oracle.RULE_NODE2VEC_EXACT: "node2vec"}


def n2v_cpu(rowptr, col, start, L, p, q, seed, rule, **kw):
    n, e = mc.rejection_sampling(rowptr, col, start, L, p, q, seed=seed, rule=RULE_NAME[rule],
                                 return_edges=True, stream="cpu", **kw)
    return n.numpy(), e.numpy()


def test_c1_fixture(c1):
    L = int(c1["walk_length"])
    n, e = mc.random_walk(c1["rowptr"], c1["col"], c1["start"], c1["rand"], L, stream="cpu",
                          return_edges=True)
    assert n.device.type == "cpu" and n.dtype == torch.int64
    np.testing.assert_array_equal(n.numpy(), c1["uniform_nodes"])
    np.testing.assert_array_equal(e.numpy(), c1["uniform_edges"])
    names = sorted({k[4:-6] for k in c1 if k.startswith("n2v_") and k.endswith("_nodes")})
    assert len(names) == 5
    for name in names:
        p, q, rule, seed = c1[f"n2v_{name}_params"]
        n, e = n2v_cpu(c1["rowptr"], c1["col"], c1["start"], L, p, q, int(seed), int(rule))
        np.testing.assert_array_equal(n, c1[f"n2v_{name}_nodes"])
        np.testing.assert_array_equal(e, c1[f"n2v_{name}_edges"])


@pytest.mark.parametrize("N,L", [(0, 5), (1, 0), (7, 1), (1000, 13), (4097, 3)])
def test_uniform_ragged_matches_oracle(N, L):
    rowptr, col = synth.rmat_csr(10, 6000, seed=N + L)
    rowptr, col = rowptr.numpy(), col.numpy()
    V = rowptr.size - 1
    start = np.arange(N, dtype=np.int64) % V
    rand = oracle.philox_uniform(N * L, 77).reshape(N, L)
    n_ref, e_ref, st, _ = oracle.uniform_walk(rowptr, col, start, rand, L, with_edges=True)
    assert st == 0
    n, e = mc.random_walk(rowptr, col, start, rand, L, stream="cpu", return_edges=True)
    np.testing.assert_array_equal(n.numpy(), n_ref)
    np.testing.assert_array_equal(e.numpy(), e_ref)
    assert uniform_transitions_ok(rowptr, col, start, rand, n.numpy()) == 0


def test_uniform_seeded_equals_rand_tensor():
    rowptr, col = synth.rmat_csr(11, 20000, seed=4)
    V = rowptr.numel() - 1
    start = torch.arange(3 * V) % V
    L = 9  # N * L not a multiple of 4: blocks straddle walks
    rand = torch.from_numpy(oracle.philox_uniform(start.numel() * L, 123456789).reshape(-1, L))
    a = mc.random_walk(rowptr, col, start, rand, L, stream="cpu")
    b = mc.random_walk(rowptr, col, start, None, L, seed=123456789, stream="cpu")
    assert torch.equal(a, b)


@pytest.mark.parametrize("threads", [1, 2, 7])
def test_thread_count_does_not_change_results(threads):
    rowptr, col = synth.rmat_csr(11, 20000, seed=5, symmetrize=True)
    V = rowptr.numel() - 1
    start = torch.arange(5000) % V
    ref = mc.rejection_sampling(rowptr, col, start, 12, 0.5, 2.0, seed=9, stream="cpu")
    got = mc.rejection_sampling(rowptr, col, start, 12, 0.5, 2.0, seed=9, stream="cpu",
                                threads=threads)
    assert torch.equal(ref, got)
    ref = mc.random_walk(rowptr, col, start, None, 12, seed=3, stream="cpu")
    got = mc.random_walk(rowptr, col, start, None, 12, seed=3, stream="cpu", threads=threads)
    assert torch.equal(ref, got)


@pytest.mark.parametrize("p,q", [(0.5, 2.0), (4.0, 0.25), (1.0, 1.0)])
@pytest.mark.parametrize("rule", [oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT])
def test_node2vec_matches_oracle(p, q, rule):
    rowptr, col = synth.rmat_csr(10, 12000, seed=21, symmetrize=True)
    rowptr, col = rowptr.numpy(), col.numpy()
    V = rowptr.size - 1
    start = np.arange(2 * V) % V
    n_ref, e_ref, st, _ = oracle.node2vec_walk(rowptr, col, start, 10, p, q, 31, rule=rule,
                                               with_edges=True)
    assert st == 0
    for rows_sorted in (None, True, False):
        n, e = n2v_cpu(rowptr, col, start, 10, p, q, 31, rule, rows_sorted=rows_sorted)
        np.testing.assert_array_equal(n, n_ref)
        np.testing.assert_array_equal(e, e_ref)


def test_node2vec_unsorted_rows_detected():
    rng = np.random.default_rng(8)
    rowptr, col = undirected(300, rng.integers(0, 300, (2500, 2)), sort=False)
    assert oracle.csr_flags(rowptr, col) & 4
    start = np.arange(600) % 300
    for rule in RULE_NAME:
        n_ref, e_ref, st, _ = oracle.node2vec_walk(rowptr, col, start, 8, 0.25, 4.0, 5,
                                                   rule=rule, rows_sorted=False, with_edges=True)
        assert st == 0
        for rows_sorted in (None, False):
            n, e = n2v_cpu(rowptr, col, start, 8, 0.25, 4.0, 5, rule, rows_sorted=rows_sorted)
            np.testing.assert_array_equal(n, n_ref)
            np.testing.assert_array_equal(e, e_ref)


def test_symmetric_flag_is_accepted_and_checked():
    """MLXC_ROWS_SYMMETRIC combines with the row orders; the host twin gives
    the same walks (it always searches row(x)); other bits are rejected."""
    rowptr, col = synth.rmat_csr(10, 12000, seed=21, symmetrize=True)
    start = torch.arange(2000) % (rowptr.numel() - 1)
    a = mc.rejection_sampling(rowptr, col, start, 10, 0.5, 2.0, seed=4, stream="cpu")
    b = mc.rejection_sampling(rowptr, col, start, 10, 0.5, 2.0, seed=4, stream="cpu",
                              symmetric=True)
    assert torch.equal(a, b)
    from mlx_cluster_amd import _lib
    lib = _lib.load()
    out = torch.empty((1, 3), dtype=torch.int64)
    ptr = lambda t: t.data_ptr()
    for rows in (3, 7, 8, -1):
        rc = lib.mlxc_rejection_sampling_cpu(ptr(rowptr), rowptr.numel() - 1, ptr(col), col.numel(),
                                             ptr(start), 1, 2, 1.0, 1.0, 1, 0, 0, rows, ptr(out), None,
                                             _lib.MLXC_OUT_INT64, 1, None)
        assert rc == _lib.MLXC_ERR_INVALID_ARGUMENT, rows
    for rows in (4, 5, 6):
        rc = lib.mlxc_rejection_sampling_cpu(ptr(rowptr), rowptr.numel() - 1, ptr(col), col.numel(),
                                             ptr(start), 1, 2, 1.0, 1.0, 1, 0, 0, rows, ptr(out), None,
                                             _lib.MLXC_OUT_INT64, 1, None)
        assert rc == _lib.MLXC_OK, rows


def test_trial_cap_matches_oracle():
    rowptr, col = undirected(40, [(i, (i * 7 + 3) % 40) for i in range(40)] +
                             [(i, (i * 11 + 5) % 40) for i in range(40)])
    start = np.arange(64) % 40
    n_ref, e_ref, st, _ = oracle.node2vec_walk(rowptr, col, start, 3, 1e6, 1e6, 8,
                                               rule=oracle.RULE_NODE2VEC_EXACT, with_edges=True)
    n, e = n2v_cpu(rowptr, col, start, 3, 1e6, 1e6, 8, oracle.RULE_NODE2VEC_EXACT)
    np.testing.assert_array_equal(n, n_ref)
    np.testing.assert_array_equal(e, e_ref)


def test_sinks_and_empty_rows():
    # node 3 has out-degree 0 and node 4 none at all; walks stay put there
    rowptr, col = csr(5, [(0, 1), (1, 2), (2, 3), (2, 0)])
    start = np.array([0, 3, 4, 2], dtype=np.int64)
    rand = np.full((4, 6), 0.75, dtype=np.float32)
    n, e = mc.random_walk(rowptr, col, start, rand, 6, stream="cpu", return_edges=True)
    n_ref, e_ref, _, _ = oracle.uniform_walk(rowptr, col, start, rand, 6, with_edges=True)
    np.testing.assert_array_equal(n.numpy(), n_ref)
    np.testing.assert_array_equal(e.numpy(), e_ref)
    assert (n.numpy()[1] == 3).all() and (e.numpy()[1] == -1).all()


def test_malformed_graphs_raise():
    rowptr, col = csr(4, [(0, 1), (0, 3), (2, 1)])
    with pytest.raises(ValueError, match="outside"):
        mc.random_walk(rowptr, np.array([1, 9, 1]), np.array([0, 0, 0, 0]),
                       np.full((4, 3), 0.9, np.float32), 3, stream="cpu")
    with pytest.raises(ValueError, match="outside"):
        mc.random_walk(rowptr, col, np.array([5]), np.zeros((1, 3), np.float32), 3, stream="cpu")
    with pytest.raises(ValueError, match="rowptr"):
        mc.random_walk(np.array([0, 2, 1, 3, 3]), col, np.array([1]),
                       np.zeros((1, 3), np.float32), 3, stream="cpu")
    # the DETECT pass validates the whole graph, as the device preparation pass does
    with pytest.raises(ValueError, match="outside"):
        mc.rejection_sampling(rowptr, np.array([1, 9, 1]), np.array([2]), 3, 1.0, 1.0,
                              stream="cpu")
    with pytest.raises(ValueError, match="rowptr"):
        mc.rejection_sampling(np.array([0, 2, 1, 3, 3]), col, np.array([0]), 3, 1.0, 1.0,
                              stream="cpu")
    # check=False returns whatever the stopped walks hold, without raising
    out = mc.random_walk(rowptr, col, np.array([5]), np.zeros((1, 3), np.float32), 3,
                         stream="cpu", check=False)
    assert out.shape == (1, 4) and int(out[0, 0]) == 5


@pytest.mark.parametrize("stream", ["cpu", torch.device("cpu")])
def test_both_spellings_of_the_cpu_stream(stream):
    rowptr, col = csr(3, [(0, 1), (1, 2), (2, 0)])
    out = mc.random_walk(rowptr, col, np.array([0, 1]), None, 4, seed=1, stream=stream)
    assert out.tolist() == [[0, 1, 2, 0, 1], [1, 2, 0, 1, 2]]


def test_threads_argument_validation():
    rowptr, col = csr(3, [(0, 1), (1, 2), (2, 0)])
    for bad in (0, -1, 2.5, True):
        with pytest.raises(ValueError, match="threads"):
            mc.random_walk(rowptr, col, np.array([0]), None, 2, seed=1, stream="cpu", threads=bad)


def test_gpu_only_helpers_refuse_the_cpu_stream():
    rowptr, col = csr(3, [(0, 1), (1, 2), (2, 0)])
    with pytest.raises(ValueError, match="GPU only"):
        mc.csr_check(rowptr, col, stream="cpu")
    with pytest.raises(ValueError, match="GPU only"):
        mc.philox_uniform(8, 1, stream="cpu")


def test_int32_output_equals_int64():
    rowptr, col = synth.rmat_csr(11, 20000, seed=6)
    V = rowptr.numel() - 1
    start = torch.arange(3 * V) % V
    for seed_kw in (dict(seed=4), None):
        rand = None if seed_kw else torch.from_numpy(oracle.philox_uniform(start.numel() * 9, 4)
                                                      .reshape(-1, 9))
        kw = seed_kw or {}
        a = mc.random_walk(rowptr, col, start, rand, 9, stream="cpu", return_edges=True, **kw)
        b = mc.random_walk(rowptr, col, start, rand, 9, stream="cpu", return_edges=True,
                           out_dtype=torch.int32, **kw)
        assert b[0].dtype == torch.int32 and b[1].dtype == torch.int32
        assert torch.equal(a[0], b[0].long()) and torch.equal(a[1], b[1].long())
    a = mc.rejection_sampling(rowptr, col, start, 7, 0.5, 2.0, seed=3, stream="cpu",
                              return_edges=True)
    b = mc.rejection_sampling(rowptr, col, start, 7, 0.5, 2.0, seed=3, stream="cpu",
                              return_edges=True, out_dtype=torch.int32)
    assert torch.equal(a[0], b[0].long()) and torch.equal(a[1], b[1].long())


def test_out_dtype_validation():
    rowptr, col = csr(3, [(0, 1), (1, 2), (2, 0)])
    with pytest.raises(TypeError, match="out_dtype"):
        mc.random_walk(rowptr, col, np.array([0]), None, 2, seed=1, stream="cpu",
                       out_dtype=torch.int16)
    with pytest.raises(TypeError, match="out_dtype"):
        mc.rejection_sampling(rowptr, col, np.array([0]), 2, 1.0, 1.0, stream="cpu",
                              out_dtype=torch.float32)


@pytest.mark.parametrize("case", status_cases.N2V_CASES, ids=[c[0] for c in status_cases.N2V_CASES])
def test_node2vec_status_bits(case):
    """The host twin validates the whole CSR on every call: the hand-derived
    bits for every row mode and both seeds (one of which never meets the bad
    col entry of the 'bad col' case)."""
    from mlx_cluster_amd import _lib
    name, rowptr, col, start, want = case
    for seed in (0, 1):
        for rows in (0, 1, 2):
            got = status_cases.host_node2vec_status(_lib.load(), rowptr, col, start, 3, 0.5, 2.0,
                                                    seed, 0, rows)
            assert got == want, (name, seed, rows, got)


@pytest.mark.parametrize("case", status_cases.UNI_CASES, ids=[c[0] for c in status_cases.UNI_CASES])
def test_uniform_status_bits(case):
    """The host twin reports what the walks read (a start, the row of a node
    a walk leaves, a chosen col entry): the hand-derived bits."""
    from mlx_cluster_amd import _lib
    name, rowptr, col, start, L, want = case
    for seed in (None, 5):
        got = status_cases.host_uniform_status(_lib.load(), rowptr, col, start, L, seed=seed)
        assert got == want, (name, seed, got)


# ------------------------------------------------------------ walk offsets


@pytest.mark.parametrize("cuts", [(0, 1000), (0, 1, 64, 999, 1000), (0, 333, 334, 1000)])
def test_seeded_uniform_slices_equal_whole_call(cuts):
    """walk_offset: the call on start[i0:i1] with walk_offset=i0 gives rows
    i0 .. i1-1 of the whole call, and those rows are the oracle's walk on the
    stream elements [i0 * L, i1 * L)."""
    rowptr, col = synth.rmat_csr(11, 20000, seed=8)
    rowptr_h, col_h = rowptr.numpy(), col.numpy()
    V, L, seed = rowptr.numel() - 1, 11, 31
    start = torch.arange(1000) * 7 % V
    whole_n, whole_e = mc.random_walk(rowptr, col, start, None, L, seed=seed, stream="cpu",
                                      return_edges=True)
    for i0, i1 in zip(cuts[:-1], cuts[1:]):
        n, e = mc.random_walk(rowptr, col, start[i0:i1], None, L, seed=seed, walk_offset=i0,
                              stream="cpu", return_edges=True)
        assert torch.equal(n, whole_n[i0:i1]) and torch.equal(e, whole_e[i0:i1])
        rand = oracle.philox_uniform((i1 - i0) * L, seed, first=i0 * L).reshape(-1, L)
        n_ref, e_ref, st, _ = oracle.uniform_walk(rowptr_h, col_h, start[i0:i1].numpy(), rand, L,
                                                  with_edges=True)
        assert st == 0
        np.testing.assert_array_equal(n.numpy(), n_ref)
        np.testing.assert_array_equal(e.numpy(), e_ref)


@pytest.mark.parametrize("rule", [oracle.RULE_REF_CHAIN, oracle.RULE_NODE2VEC_EXACT])
def test_node2vec_slices_equal_whole_call(rule):
    """walk_offset on the node2vec walk: slices equal the whole call and the
    oracle's walk with first_walk = i0 (Philox counter = global walk index)."""
    rowptr, col = synth.rmat_csr(11, 20000, seed=9, symmetrize=True)
    rowptr_h, col_h = rowptr.numpy(), col.numpy()
    V, L, seed, p, q = rowptr.numel() - 1, 9, 12, 0.5, 2.0
    start = torch.arange(900) * 5 % V
    whole_n, whole_e = n2v_cpu(rowptr, col, start, L, p, q, seed, rule)
    for i0, i1 in ((0, 300), (300, 301), (301, 900)):
        n, e = n2v_cpu(rowptr, col, start[i0:i1], L, p, q, seed, rule, walk_offset=i0)
        np.testing.assert_array_equal(n, whole_n[i0:i1])
        np.testing.assert_array_equal(e, whole_e[i0:i1])
        n_ref, e_ref, st, _ = oracle.node2vec_walk(rowptr_h, col_h, start[i0:i1].numpy(), L, p,
                                                   q, seed, rule=rule, with_edges=True,
                                                   first_walk=i0)
        assert st == 0
        np.testing.assert_array_equal(n, n_ref)
        np.testing.assert_array_equal(e, e_ref)


def test_walk_offset_far_into_the_stream():
    """An offset past 2^32 walks reaches the counter's high word: the host
    twin equals the oracle there."""
    rowptr, col = synth.rmat_csr(9, 4000, seed=2, symmetrize=True)
    rowptr_h, col_h = rowptr.numpy(), col.numpy()
    start = torch.arange(50) % (rowptr.numel() - 1)
    first, L = (1 << 33) + 17, 6
    n = mc.random_walk(rowptr, col, start, None, L, seed=5, walk_offset=first, stream="cpu")
    rand = oracle.philox_uniform(50 * L, 5, first=first * L).reshape(50, L)
    np.testing.assert_array_equal(n.numpy(),
                                  oracle.uniform_walk(rowptr_h, col_h, start.numpy(), rand, L)[0])
    n, _ = n2v_cpu(rowptr, col, start, L, 2.0, 0.5, 3, oracle.RULE_NODE2VEC_EXACT,
                   walk_offset=first)
    np.testing.assert_array_equal(n, oracle.node2vec_walk(
        rowptr_h, col_h, start.numpy(), L, 2.0, 0.5, 3, rule=oracle.RULE_NODE2VEC_EXACT,
        first_walk=first)[0])


def test_first_walk_checked_by_the_abi():
    from mlx_cluster_amd import _lib
    lib = _lib.load()
    rowptr, col = csr(3, [(0, 1), (1, 2), (2, 0)])
    start = np.array([0, 1], dtype=np.int64)
    out = np.empty((2, 5), np.int64)
    p = lambda a: a.ctypes.data
    for first in (-1, 2**63 // 4):  # negative; (first + N) * L past int64
        rc = lib.mlxc_random_walk_seeded_cpu(p(rowptr), 3, p(col), 3, p(start), 2, 4, 1, first,
                                             p(out), None, 0, 1, None)
        assert rc == _lib.MLXC_ERR_INVALID_ARGUMENT and "first_walk" in _lib.last_error()
        rc = lib.mlxc_rejection_sampling_cpu(p(rowptr), 3, p(col), 3, p(start), 2, 4, 1.0, 1.0,
                                             1, first, 0, 1, p(out), None, 0, 1, None)
        assert rc == _lib.MLXC_ERR_INVALID_ARGUMENT and "first_walk" in _lib.last_error()
