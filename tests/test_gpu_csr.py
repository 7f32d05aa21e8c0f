"""Parity of the HIP CSR build (mlxc_csr_build, via to_csr on a GPU) with the
oracle's restatement of the reference tests' pipeline
(tests/test_random_walk.py:23-28): bit-exact rowptr and col."""
import math

import numpy as np
import pytest
import torch

import mlx_cluster_amd as mc
import oracle
from mlx_cluster_amd import _lib, synth

pytestmark = pytest.mark.gpu


def assert_parity(row, col, V, cuda, symmetrize=False, dedup=False):
    row, col = np.asarray(row, np.int64), np.asarray(col, np.int64)
    ei = torch.from_numpy(np.stack([row, col])).to(cuda)
    rowptr, c = mc.to_csr(ei, V, symmetrize=symmetrize, dedup=dedup)
    assert rowptr.is_cuda and c.is_cuda
    ref_rowptr, ref_col = oracle.csr_build(row, col, V, symmetrize=symmetrize, dedup=dedup)
    np.testing.assert_array_equal(rowptr.cpu().numpy(), ref_rowptr)
    np.testing.assert_array_equal(c.cpu().numpy(), ref_col)


def test_hand_case(cuda):
    row, col = [3, 0, 0, 3, 0], [0, 2, 1, 1, 2]
    for sym in (False, True):
        for dedup in (False, True):
            assert_parity(row, col, 5, cuda, sym, dedup)


def test_empty_and_single_node(cuda):
    for V in (0, 1, 5):
        rowptr, c = mc.to_csr(torch.zeros((2, 0), dtype=torch.int64, device=cuda), V)
        assert rowptr.tolist() == [0] * (V + 1) and c.numel() == 0
    # one node: every key is 0 (no key bits at all)
    assert_parity([0] * 9000, [0] * 9000, 1, cuda)
    assert_parity([0] * 9000, [0] * 9000, 1, cuda, symmetrize=True, dedup=True)


@pytest.mark.parametrize("E", [1, 63, 4095, 4096, 4097, 3 * 4096 + 5, 100_003])
@pytest.mark.parametrize("V", [2, 255, 257, 65536, 65537, 3_000_001])
def test_random_lists(E, V, cuda):
    """Tile-ragged sizes; 32-bit keys (V <= 65536) and 64-bit keys."""
    rng = np.random.default_rng(E * 7 + V)
    row, col = rng.integers(0, V, E), rng.integers(0, V, E)
    assert_parity(row, col, V, cuda)
    assert_parity(row, col, V, cuda, symmetrize=True, dedup=True)


def test_64_bit_keys(cuda):
    """More than 2^24 nodes: keys wider than 48 bits, stored whole (smaller
    graphs split theirs into 32 + 16 bits).  Ids near both ends of the range,
    a hub row and repeated pairs."""
    rng = np.random.default_rng(64)
    V, E = (1 << 25) + 7, 150_003
    row, col = rng.integers(0, V, E), rng.integers(0, V, E)
    row[:20_000] = V - 1
    col[20_000:24_000] = rng.integers(0, 3, 4000)
    col[24_000:26_000] = V - 2
    row[30_000:32_000] = row[40_000:42_000]
    col[30_000:32_000] = col[40_000:42_000]
    for sym, dedup in ((False, False), (True, True)):
        assert_parity(row, col, V, cuda, sym, dedup)


@pytest.mark.parametrize("sym,dedup", [(False, False), (False, True), (True, False),
                                       (True, True)])
def test_skewed_with_duplicates(sym, dedup, cuda):
    """A hub row holding most entries, long runs of one digit and repeated
    pairs crossing tile boundaries."""
    rng = np.random.default_rng(11)
    V, E = 40_000, 70_000
    row, col = rng.integers(0, V, E), rng.integers(0, V, E)
    row[:50_000] = 17
    col[10_000:30_000] = 3
    col[30_000:34_000] = rng.integers(0, 4, 4000)
    assert_parity(row, col, V, cuda, sym, dedup)


def _rows_of_lengths(lengths, V, rng, col_range=None):
    """An edge list, shuffled, whose rows 0, k, 2k, ... hold the given numbers
    of entries (k spreads the rows over the node ids)."""
    k = max(1, V // len(lengths))
    row = np.repeat(np.arange(len(lengths), dtype=np.int64) * k, lengths)
    col = rng.integers(0, col_range or V, row.size)
    perm = rng.permutation(row.size)
    return row[perm], col[perm]


@pytest.mark.parametrize("V", [300, 65536, 3_000_001])
def test_row_lengths_around_tiles(V, cuda):
    """Rows of lengths around the radix passes' 8192-key tiles and their
    4096-entry finish chunks (one entry to several tiles), shuffled, with
    repeated pairs and a long last row: digit runs that cross tile and
    chunk boundaries.  V = 300 and 65536 give 32-bit keys, 3_000_001 64-bit
    keys."""
    rng = np.random.default_rng(V)
    base = [1, 2, 63, 64, 4095, 4096, 4097, 6000, 8191, 8192, 8193, 12_000, 20_000]
    lengths = list(rng.permutation(base * 3)) + [3, 4100, 9000]
    row, col = _rows_of_lengths(lengths, min(V, 300), rng, col_range=V)
    for sym, dedup in ((False, False), (False, True), (True, True)):
        assert_parity(row, col, V, cuda, sym, dedup)


def test_many_long_rows(cuda):
    """1500 rows of 8500 to 12000 entries over 5000 columns: every tile holds
    one or two rows, whose columns repeat many times."""
    rng = np.random.default_rng(3)
    V = 1 << 20
    lengths = rng.integers(8_500, 12_000, 1500)
    row, col = _rows_of_lengths(lengths, V, rng, col_range=5000)
    assert_parity(row, col, V, cuda)
    assert_parity(row, col, V, cuda, dedup=True)


def test_rmat_2_20(cuda):
    """The generator of configurations 2 and 3: R-MAT 2^20, 2^24 samples."""
    row, col = synth.rmat_edges(20, 1 << 24, seed=0, device=cuda)
    r, c = row.cpu().numpy(), col.cpu().numpy()
    for sym, dedup in ((False, True), (True, True), (False, False)):
        rowptr, cc = mc.to_csr(torch.stack([row, col]), 1 << 20, symmetrize=sym, dedup=dedup)
        ref_rowptr, ref_col = oracle.csr_build(r, c, 1 << 20, symmetrize=sym, dedup=dedup)
        np.testing.assert_array_equal(rowptr.cpu().numpy(), ref_rowptr)
        np.testing.assert_array_equal(cc.cpu().numpy(), ref_col)


def test_ids_out_of_range_raise(cuda):
    for row, col in (([0, 5], [1, 1]), ([0, 1], [-1, 1]), ([0, 2**40], [1, 1])):
        ei = torch.tensor([row, col], dtype=torch.int64, device=cuda)
        with pytest.raises(ValueError, match="outside"):
            mc.to_csr(ei, 3)
        with pytest.raises(ValueError, match="outside"):
            mc.to_csr(ei, 3, symmetrize=True, dedup=True)
    # the device stays usable afterwards
    assert_parity([2, 0, 1], [0, 2, 2], 3, cuda)


def test_side_stream_and_host_twin(cuda):
    rng = np.random.default_rng(5)
    V, E = 100_000, 250_000
    ei = torch.from_numpy(rng.integers(0, V, (2, E))).to(cuda)
    s = torch.cuda.Stream(device=cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(s):
        rowptr, col = mc.to_csr(ei, V, symmetrize=True, dedup=True, stream=s)
    s.synchronize()
    hrowptr, hcol = mc.to_csr(ei.cpu(), V, symmetrize=True, dedup=True)
    assert torch.equal(rowptr.cpu(), hrowptr) and torch.equal(col.cpu(), hcol)


def test_abi_status_words(cuda):
    """Workspace word 0 = status bits, word 1 = entries written."""
    lib = _lib.load()
    row = torch.tensor([1, 1, 0, 1], dtype=torch.int64, device=cuda)
    col = torch.tensor([0, 0, 1, 0], dtype=torch.int64, device=cuda)
    rowptr = torch.empty(3, dtype=torch.int64, device=cuda)
    out = torch.empty(4, dtype=torch.int64, device=cuda)
    nbytes = lib.mlxc_csr_build_workspace_bytes(2, 4, _lib.MLXC_CSR_DEDUP)
    work = torch.full(((nbytes + 7) // 8,), -1, dtype=torch.int64, device=cuda)
    rc = lib.mlxc_csr_build(row.data_ptr(), col.data_ptr(), 4, 2, _lib.MLXC_CSR_DEDUP,
                            rowptr.data_ptr(), out.data_ptr(), work.data_ptr(), nbytes,
                            torch.cuda.current_stream(cuda).cuda_stream)
    assert rc == 0
    assert work[:2].tolist() == [0, 2]
    assert rowptr.tolist() == [0, 1, 2] and out[:2].tolist() == [1, 0]


def test_c4_full_size_properties(cuda):
    """Configuration 4's edge list (R-MAT 2^24, 2^28 samples, 64-bit keys,
    six radix passes) at full size, against an independent device result
    instead of the oracle: the sorted unique keys row * V + col of the input
    (torch.unique).  rowptr must equal their cumulative row counts (torch
    bincount) and the (row, col) sequence must equal them entry for entry,
    hence sorted and free of repeats."""
    V = 1 << 24
    row, col = synth.rmat_edges(24, 1 << 28, seed=0, device=cuda)
    rowptr, c = mc.to_csr(torch.stack([row, col]), V, dedup=True)
    del row, col
    row, col = synth.rmat_edges(24, 1 << 28, seed=0, device=cuda)
    key = torch.unique(row * V + col)
    del row, col
    assert rowptr[-1].item() == c.numel() == key.numel()
    urow = key // V
    expect = torch.zeros(V + 1, dtype=torch.int64, device=cuda)
    torch.cumsum(torch.bincount(urow, minlength=V), 0, out=expect[1:])
    assert torch.equal(rowptr, expect)
    out_row = torch.repeat_interleave(torch.arange(V, device=cuda), rowptr.diff())
    out_key = out_row * V + c
    assert bool((out_key[1:] > out_key[:-1]).all())
    assert torch.equal(out_key, key)


def test_build_beyond_int32_entries(cuda):
    """A build whose input and output both pass int32 positions, against an
    answer known in closed form (torch's unique and boolean indexing are not
    usable at this size): the n = 2^31 + 2^20 distinct keys
    k_j = j * 2^16 + 12345 (row k >> 24 of 2^24 nodes, 256 entries a row),
    laid out in the order pi(i) = (a * i + b) mod n with a coprime to n, then
    2^20 of them repeated: 2^31 + 2^21 pairs, two 17 GB arrays.  Sorting and
    deduplicating must give col = k_j mod 2^24 for every j and
    rowptr = min(256 * r, n)."""
    from mlx_cluster_amd import _lib
    lib = _lib.load()
    V = 1 << 24
    n, dup = (1 << 31) + (1 << 20), 1 << 20
    E = n + dup
    a, b = 1_000_000_007, 77_777
    assert math.gcd(a, n) == 1
    pos = torch.arange(E, device=cuda, dtype=torch.int64)
    j = torch.where(pos < n, (pos * a + b) % n, pos - n)  # a * i < 2^63
    del pos
    key = j * (1 << 16) + 12345
    del j
    row, col = key >> 24, key & (V - 1)
    del key
    flags = _lib.MLXC_CSR_DEDUP
    nbytes = lib.mlxc_csr_build_workspace_bytes(V, E, flags)
    work = torch.empty((nbytes + 7) // 8, dtype=torch.int64, device=cuda)
    rowptr = torch.empty(V + 1, dtype=torch.int64, device=cuda)
    out = torch.empty(E, dtype=torch.int64, device=cuda)
    rc = lib.mlxc_csr_build(row.data_ptr(), col.data_ptr(), E, V, flags, rowptr.data_ptr(),
                            out.data_ptr(), work.data_ptr(), nbytes,
                            torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    bits, count = (int(x) for x in work[:2].tolist())
    del work, row, col
    torch.cuda.empty_cache()
    assert bits == 0 and count == n
    expect_rowptr = torch.clamp(torch.arange(V + 1, device=cuda, dtype=torch.int64) * 256, max=n)
    assert torch.equal(rowptr, expect_rowptr)
    del expect_rowptr
    expect_col = (torch.arange(n, device=cuda, dtype=torch.int64) * (1 << 16) + 12345) & (V - 1)
    assert torch.equal(out[:n], expect_col)
    del expect_col, out, rowptr
    torch.cuda.empty_cache()


def test_rowptr_of_2_28_nodes(cuda):
    """num_nodes = 2^28 + 3 (a rowptr of 2 GB): the rowptr scans take the
    levelled form (65,537 chunks, whose sums are scanned first).  A few
    thousand pairs, clustered at both ends of the id range, equal the oracle;
    rowptr equals bincount + cumsum of the rows, and the call's time is
    printed."""
    import time
    V = (1 << 28) + 3
    rng = np.random.default_rng(28)
    row = np.concatenate([rng.integers(0, 5000, 3000), rng.integers(V - 5000, V, 3000),
                          rng.integers(0, V, 2000)])
    col = rng.integers(0, V, row.size)
    ei = torch.from_numpy(np.stack([row, col])).to(cuda)
    for dedup in (False, True):
        mc.to_csr(ei, V, dedup=dedup)  # warm
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        rowptr, c = mc.to_csr(ei, V, dedup=dedup)
        torch.cuda.synchronize()
        print(f"to_csr, {row.size} pairs over {V} nodes (dedup={dedup}): "
              f"{(time.perf_counter() - t0) * 1e3:.2f} ms", flush=True)
        ref = torch.zeros(V + 1, dtype=torch.int64, device=cuda)
        torch.cumsum(torch.bincount(ei[0], minlength=V), 0, out=ref[1:])
        assert torch.equal(rowptr, ref)
        order = np.lexsort((col, row))
        np.testing.assert_array_equal(c.cpu().numpy(), col[order])
        del rowptr, c, ref
