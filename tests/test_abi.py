"""The C-ABI library loads and exports what include/mlxc.h declares.

CPU-only: argument errors are rejected on the host before any HIP call, so
they can be exercised without a GPU.
"""
import ctypes
import os
import re

import numpy as np
import pytest

from mlx_cluster_amd import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "mlxc.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mlxc_\w+)\s*\(", text)))


def test_header_declares_the_path():
    names = declared_functions()
    assert {"mlxc_random_walk", "mlxc_rejection_sampling", "mlxc_version",
            "mlxc_last_error"} <= set(names)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_header_constants_match_binding():
    text = open(HEADER).read()
    for name in ["MLXC_OK", "MLXC_ERR_INVALID_ARGUMENT", "MLXC_ERR_HIP", "MLXC_WORK_WORDS",
                 "MLXC_STATUS_BAD_NODE", "MLXC_STATUS_BAD_ROW", "MLXC_RULE_REF_CHAIN",
                 "MLXC_RULE_NODE2VEC_EXACT", "MLXC_ROWS_UNSORTED", "MLXC_ROWS_SORTED",
                 "MLXC_ROWS_DETECT", "MLXC_CSR_BAD_ROWPTR", "MLXC_CSR_BAD_COL",
                 "MLXC_CSR_UNSORTED", "MLXC_MAX_TRIALS"]:
        m = re.search(rf"#define {name} \(?(-?\d+)\)?", text)
        assert m, name
        assert int(m.group(1)) == getattr(_lib, name), name


def test_version():
    assert _lib.load().mlxc_version() == 301


FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first


WS = 64  # workspace bytes passed with FAKE


@pytest.mark.parametrize("args,msg", [
    ((FAKE, -1, FAKE, 0, FAKE, 1, FAKE, 1, FAKE, None, FAKE, WS, None), "num_nodes"),
    ((FAKE, 1, FAKE, -1, FAKE, 1, FAKE, 1, FAKE, None, FAKE, WS, None), "num_edges"),
    ((FAKE, 1, FAKE, 0, FAKE, -1, FAKE, 1, FAKE, None, FAKE, WS, None), "num_walks"),
    ((FAKE, 1, FAKE, 0, FAKE, 1, FAKE, -2, FAKE, None, FAKE, WS, None), "walk_length"),
    ((FAKE, 1, FAKE, 0, FAKE, 1, FAKE, 2**31 - 1, FAKE, None, FAKE, WS, None), "2^31 - 1"),
    ((FAKE, 1, FAKE, 0, FAKE, 1, FAKE, 1, FAKE, None, None, WS, None), "workspace"),
    ((FAKE, 1, FAKE, 0, FAKE, 1, FAKE, 1, FAKE, None, FAKE, 16, None), "MLXC_WORK_WORDS"),
    ((FAKE, 1, FAKE, 0, FAKE, 1, FAKE, 1, FAKE, None, ctypes.c_void_p(0x1008), WS, None),
     "aligned"),
    ((None, 1, FAKE, 0, FAKE, 1, FAKE, 1, FAKE, None, FAKE, WS, None), "NULL"),
    ((FAKE, 1, FAKE, 0, FAKE, 1, None, 3, FAKE, None, FAKE, WS, None), "rand"),
    ((FAKE, 1, FAKE, 0, FAKE, 2**62, FAKE, 8, FAKE, None, FAKE, WS, None), "overflows"),
])
def test_random_walk_rejects_bad_arguments(args, msg):
    lib = _lib.load()
    args = args[:10] + (_lib.MLXC_OUT_INT64,) + args[10:]  # out_type after d_e_out
    assert lib.mlxc_random_walk(*args) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert msg in _lib.last_error()


@pytest.mark.parametrize("num_nodes,num_edges,e_out,out_type,msg", [
    (1, 0, None, 5, "out_type"),
    (2**31, 0, None, 1, "MLXC_OUT_INT32"),
    (1, 2**31, FAKE, 1, "MLXC_OUT_INT32"),
])
def test_out_type_is_checked(num_nodes, num_edges, e_out, out_type, msg):
    lib = _lib.load()
    for fn in (lib.mlxc_random_walk, lambda *a: lib.mlxc_random_walk_cpu(*a[:11], 1, None)):
        rc = fn(FAKE, num_nodes, FAKE, num_edges, FAKE, 1, FAKE, 1, FAKE, e_out, out_type, FAKE,
                WS, None)
        assert rc == _lib.MLXC_ERR_INVALID_ARGUMENT and msg in _lib.last_error()


@pytest.mark.parametrize("p,q,rule,msg", [
    (0.0, 1.0, 0, "p and q"), (1.0, -1.0, 0, "p and q"), (float("inf"), 1.0, 0, "p and q"),
    (1.0, float("nan"), 0, "p and q"), (1.0, 1.0, 7, "rule"),
])
def test_rejection_sampling_rejects_bad_arguments(p, q, rule, msg):
    lib = _lib.load()
    rc = lib.mlxc_rejection_sampling(FAKE, 1, FAKE, 0, FAKE, 0, 3, p, q, 1, 0, rule, 1, FAKE, None,
                                     0, FAKE, WS, None)
    assert rc == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert msg in _lib.last_error()


def test_rejection_sampling_rejects_bad_row_mode():
    lib = _lib.load()
    rc = lib.mlxc_rejection_sampling(FAKE, 1, FAKE, 0, FAKE, 0, 3, 1.0, 1.0, 1, 0, 0, 3, FAKE, None,
                                     0, FAKE, WS, None)
    assert rc == _lib.MLXC_ERR_INVALID_ARGUMENT and "rows" in _lib.last_error()


def test_other_entry_points_reject_bad_arguments():
    lib = _lib.load()
    assert lib.mlxc_philox_uniform(FAKE, -1, 0, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_philox_uniform(None, 0, 0, None) == _lib.MLXC_OK  # empty is a no-op
    flags = ctypes.c_int32(0)
    assert lib.mlxc_csr_check(FAKE, -1, FAKE, 0, FAKE, WS, ctypes.addressof(flags), None) \
        == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_csr_check(FAKE, 1, FAKE, 0, FAKE, WS, None, None) \
        == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_csr_check(FAKE, 1, FAKE, 0, FAKE, 8, ctypes.addressof(flags), None) \
        == _lib.MLXC_ERR_INVALID_ARGUMENT


def test_publish_status_checks_its_pointers():
    lib = _lib.load()
    assert lib.mlxc_publish_status(None, FAKE, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert "workspace" in _lib.last_error()
    assert lib.mlxc_publish_status(FAKE, None, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_publish_status(FAKE, ctypes.c_void_p(0x1004), None) \
        == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert "h_status" in _lib.last_error()


def test_walk_events_are_set_in_pairs():
    lib = _lib.load()
    assert lib.mlxc_set_walk_events(FAKE, None) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert "both events" in _lib.last_error()
    assert lib.mlxc_set_walk_events(None, FAKE) == _lib.MLXC_ERR_INVALID_ARGUMENT
    assert lib.mlxc_set_walk_events(None, None) == _lib.MLXC_OK


def test_window_launches_beyond_the_grid_limit_are_rejected():
    """A window launch runs one 256-thread block per tile of walks (64 walks
    of up to 128 int64 nodes, one walk of 8192): more tiles than a grid
    dimension holds (2^32 - 1 work-items) fail with a message before any
    device call; the largest call that fits passes the check."""
    lib = _lib.load()
    max_tiles = (2**32 - 1) // 256
    for nodes, per_tile in ((2, 64), (8192, 1)):
        too_many = max_tiles * per_tile + 1
        rc = lib.mlxc_context_windows(FAKE, too_many, nodes, 2, _lib.MLXC_OUT_INT64, FAKE, None)
        assert rc == _lib.MLXC_ERR_INVALID_ARGUMENT and "split the call" in _lib.last_error()
        rc = lib.mlxc_negative_windows(FAKE, too_many, nodes - 1, 2, 10, 1, _lib.MLXC_OUT_INT64,
                                       FAKE, None)
        assert rc == _lib.MLXC_ERR_INVALID_ARGUMENT and "split the call" in _lib.last_error()


def test_workspace_size_query():
    """Edge and start records take 8 bytes each when node ids, row begins and
    at least 16 bits of degree pack into 64 bits, else 16; start records
    alone (the CSR walk, and the wide CSR walk of graphs with 2^31 or more
    entries) always take 16."""
    q = _lib.load().mlxc_random_walk_workspace_bytes
    E = 10**6                                     # above the small-graph size 32768 * 4
    assert q(10, E, E, 4) == 256 + 8 * 2 * E      # 4E steps >= 4 * E edges: records
    assert q(10, E, E - 1, 4) == 256 + 16 * (E - 1)  # fewer steps: start records only
    assert q(10, 32768 * 4, 1, 4) == 256 + 8 * (32768 * 4 + 1)   # small graph: records
    assert q(10, 32768 * 4 + 1, 1, 4) == 256 + 16 * 1
    # graphs whose rowptr and col fit in LDS (V + 1 + E <= 14336 entries), on
    # calls of 1 to 2^20 steps: the LDS walk, selected by a 256-byte workspace
    assert q(10, 100, 1, 4) == 256
    assert q(10, 14336 - 11, 2000, 5) == 256
    assert q(10, 14336 - 10, 2000, 5) == 256 + 8 * (14336 - 10 + 2000)   # one entry more
    assert q(10, 100, 2**18, 4) == 256
    assert q(10, 100, 2**18 + 1, 4) == 256 + 8 * (100 + 2**18 + 1)      # > 2^20 steps
    assert q(10, 100, 5, 0) == 256 + 16 * 5              # no step: start records only
    assert q(10, 0, 0, 0) == 256 + 16 * 0
    # 24 bits of node id + 24 of row begin leave 16 for the degree; 25 do not
    assert q(1 << 24, (1 << 24) - 1, 1 << 24, 4) == 256 + 8 * ((1 << 24) - 1 + (1 << 24))
    assert q(1 << 24, 1 << 24, 1 << 24, 4) == 256 + 16 * 2 * (1 << 24)
    assert q((1 << 24) + 1, (1 << 24) - 1, 1 << 24, 4) == 256 + 16 * ((1 << 24) - 1 + (1 << 24))
    assert q(2**31 - 1, E, E, 4) == 256 + 16 * 2 * E
    assert q(2**31, 5, 1, 1) == 32                 # node ids beyond int32: the plain walk
    assert q(5, 2**31, 3, 1) == 256 + 16 * 3       # 2^31 entries: the wide CSR walk's starts
    assert q(2**31, 2**31, 3, 1) == 32
    assert q(-1, 5, 1, 1) == 32
    assert q(5, 5, -1, 1) == 32
    assert q(5, 5, 1, -1) == 32


def test_python_check_maps_codes():
    with pytest.raises(ValueError):
        _lib.load().mlxc_philox_uniform(FAKE, -1, 0, None)
        _lib.check(_lib.MLXC_ERR_INVALID_ARGUMENT, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.MLXC_ERR_HIP, "x")


def test_noalloc_checks_its_arguments():
    """mlxc_random_walk_noalloc checks its arguments before any HIP call; its
    scratch size is the header's."""
    lib = _lib.load()
    text = open(HEADER).read()
    assert "#define MLXC_NOALLOC_SCRATCH_BYTES (64 * 1024 * 1024)" in text
    assert _lib.MLXC_NOALLOC_SCRATCH_BYTES == 64 * 1024 * 1024
    rc = lib.mlxc_random_walk_noalloc(FAKE, 4, FAKE, 3, FAKE, 2, None, 5, FAKE, None, 0, None,
                                      None)
    assert rc == _lib.MLXC_ERR_INVALID_ARGUMENT and "rand" in _lib.last_error()
    rc = lib.mlxc_random_walk_noalloc(FAKE, 4, FAKE, 3, FAKE, 2, FAKE, 5, FAKE, None, 7, None,
                                      None)
    assert rc == _lib.MLXC_ERR_INVALID_ARGUMENT and "out_type" in _lib.last_error()


def test_row_hash_table_regions_are_disjoint():
    """The node2vec walk's row hash tables: row x of begin b and degree d has
    d // 8 + 1 buckets starting at bucket b // 8 + x.  Over random degree
    sequences (empty rows, rows inside one 16-entry block, rows up to past the
    1,024-entry limit) the tables of consecutive rows never overlap and all of
    them end by bucket E // 8 + V + 1; the layout query reserves that many
    64-byte buckets between the record layout and the hash layout."""
    lib = _lib.load()
    rng = np.random.default_rng(7)
    for trial in range(20):
        V = int(rng.integers(1, 3000))
        deg = rng.choice([0, 1, 2, 15, 16, 17, 100, 1023, 1024, 1500], V) * (trial % 2) + \
            rng.integers(0, 40, V)
        rowptr = np.concatenate([[0], np.cumsum(deg)])
        E = int(rowptr[-1])
        b, d, x = rowptr[:-1], deg, np.arange(V)
        start, count = b // 8 + x, d // 8 + 1
        hashed = (d > 1) & (d < 1024) & (((b ^ (b + d - 1)) >> 4) != 0)
        s, c = start[hashed], count[hashed]
        assert np.all(s[1:] >= s[:-1] + c[:-1])
        if hashed.any():
            assert (s + c).max() <= E // 8 + V + 1
        base = lib.mlxc_rejection_sampling_layout_bytes(V, E, 100, 10, _lib.MLXC_N2V_LAYOUT_RECORDS)
        with_tables = lib.mlxc_rejection_sampling_layout_bytes(
            V, E, 100, 10, _lib.MLXC_N2V_LAYOUT_RECORDS_HASH)
        assert with_tables - base >= 64 * (E // 8 + V + 2)


def test_layout_query_orders_the_layouts():
    """Each layout of mlxc_rejection_sampling holds the one before it; the
    LDS walk is offered only within its limits, the CSR-mode and record
    layouts only for ids below 2^31."""
    lib = _lib.load()
    q = lambda V, E, N, L, k: lib.mlxc_rejection_sampling_layout_bytes(V, E, N, L, k)
    sizes = [q(2**20, 31_000_000, 4 * 2**20, 40, k) for k in range(6)]
    assert sizes[0] == 32 and sizes[1] == 0
    assert sizes[2] < sizes[3] < sizes[4] <= sizes[5]
    assert q(2708, 10556, 2000, 5, _lib.MLXC_N2V_LAYOUT_LDS) == 256
    assert q(2**31, 10, 10, 5, _lib.MLXC_N2V_LAYOUT_RECORDS) == 0
    assert q(10, 2**31, 10, 5, _lib.MLXC_N2V_LAYOUT_CSR) == 0
    assert q(10, 10, 10, 5, 6) == 0 and q(-1, 10, 10, 5, 3) == 0
    # the fastest layout the workspace query returns is one of these
    full = lib.mlxc_rejection_sampling_workspace_bytes(2**20, 31_000_000, 4 * 2**20, 40, 0.5,
                                                       2.0, 0)
    assert full == sizes[5]
    # a call that never searches a row (p = q = 1: every draw accepts) gets
    # the records without tables or bitmaps
    assert lib.mlxc_rejection_sampling_workspace_bytes(2**20, 31_000_000, 4 * 2**20, 40, 1.0,
                                                       1.0, 0) == sizes[3]
