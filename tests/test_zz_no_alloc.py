"""mlxc_random_walk_noalloc: the walk with its workspace in the library's
per-GPU scratch array instead of a caller's buffer.

Through the C ABI, its outputs and status must equal mlxc_random_walk's with
a workspace of the queried size, on consecutive calls that reuse the array
(the second smaller than the first, and after a call that left error bits).
"""
import ctypes

import numpy as np
import pytest
import torch

import mlx_cluster_amd as mc
import oracle
from mlx_cluster_amd import _lib, synth

pytestmark = pytest.mark.gpu


def _walk(rowptr, col, start, rand, L, *, noalloc, edges=True, out_type=0):
    """One call of either entry point; returns (nodes, edges, status)."""
    lib = _lib.load()
    V, E, N = rowptr.numel() - 1, col.numel(), start.numel()
    dtype = torch.int32 if out_type == _lib.MLXC_OUT_INT32 else torch.int64
    n = torch.full((N, L + 1), -7, dtype=dtype, device=rowptr.device)
    e = torch.full((N, L), -7, dtype=dtype, device=rowptr.device) if edges else None
    stream = torch.cuda.current_stream().cuda_stream
    args = (rowptr.data_ptr(), V, col.data_ptr(), E, start.data_ptr(), N, rand.data_ptr(), L,
            n.data_ptr(), None if e is None else e.data_ptr(), out_type)
    if noalloc:
        status = torch.full((1,), -1, dtype=torch.int64, device=rowptr.device)
        rc = lib.mlxc_random_walk_noalloc(*args, status.data_ptr(), stream)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        st = int(status.item())
    else:
        nbytes = lib.mlxc_random_walk_workspace_bytes(V, E, N, L)
        ws = torch.full(((nbytes + 7) // 8,), -1, dtype=torch.int64, device=rowptr.device)
        rc = lib.mlxc_random_walk(*args, ws.data_ptr(), nbytes, stream)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        st = int(ws[0].item())
    return n, e, st


def _same(rowptr, col, start, rand, L, **kw):
    a = _walk(rowptr, col, start, rand, L, noalloc=False, **kw)
    b = _walk(rowptr, col, start, rand, L, noalloc=True, **kw)
    assert torch.equal(a[0], b[0])
    if a[1] is not None:
        assert torch.equal(a[1], b[1])
    assert a[2] == b[2]
    return b


def test_noalloc_equals_workspace_entry_point(cuda):
    """Two calls in a row on the records layout (many steps per edge), the
    second smaller; then the CSR-walk layout and the LDS walk; every result
    equal to mlxc_random_walk's, and the first also to the oracle's."""
    rowptr, col = synth.rmat_csr(14, 120_000, seed=21, device=cuda)
    V = rowptr.numel() - 1
    # call 1: 200,000 walks x 16 steps (records: N*L >= 4E; 8 bytes each), 2.5 MB of workspace
    N, L = 200_000, 16
    start = (torch.arange(N, device=cuda) * 7) % V
    rand = mc.philox_uniform((N, L), 3, device=cuda)
    lib = _lib.load()
    E = col.numel()
    assert lib.mlxc_random_walk_workspace_bytes(V, E, N, L) == 256 + 8 * (E + N)
    n, e, st = _same(rowptr, col, start, rand, L)
    assert st == 0
    ref, ref_e, rst, _ = oracle.uniform_walk(rowptr.cpu().numpy(), col.cpu().numpy(),
                                             start.cpu().numpy(), rand.cpu().numpy(), L,
                                             with_edges=True)
    assert rst == 0
    np.testing.assert_array_equal(n.cpu().numpy(), ref)
    np.testing.assert_array_equal(e.cpu().numpy(), ref_e)
    # call 2: smaller, reusing the array the first call filled
    N2, L2 = 3_001, 5
    start2 = (torch.arange(N2, device=cuda) * 13) % V
    rand2 = mc.philox_uniform((N2, L2), 4, device=cuda)
    _same(rowptr, col, start2, rand2, L2)
    _same(rowptr, col, start2, rand2, L2, edges=False, out_type=_lib.MLXC_OUT_INT32)
    # CSR-walk layout (fewer than 4 steps per edge): start records only
    N3, L3 = 20_000, 2
    assert lib.mlxc_random_walk_workspace_bytes(V, E, N3, L3) == 256 + 16 * N3
    start3 = torch.arange(N3, device=cuda) % V
    rand3 = mc.philox_uniform((N3, L3), 5, device=cuda)
    _same(rowptr, col, start3, rand3, L3)
    # the LDS walk (graph within the LDS limit)
    rp4, cl4 = synth.rmat_csr(9, 3_000, seed=2, device=cuda)
    N4, L4 = 1_000, 7
    assert lib.mlxc_random_walk_workspace_bytes(rp4.numel() - 1, cl4.numel(), N4, L4) == 256
    start4 = torch.arange(N4, device=cuda) % (rp4.numel() - 1)
    rand4 = mc.philox_uniform((N4, L4), 6, device=cuda)
    _same(rp4, cl4, start4, rand4, L4)


def test_noalloc_status_is_per_call(cuda):
    """A call that sets error bits, then a well-formed smaller call: each
    reports its own status, as the workspace entry point does."""
    rowptr, col = synth.rmat_csr(12, 40_000, seed=5, device=cuda)
    V = rowptr.numel() - 1
    N, L = 10_000, 12
    start = torch.arange(N, device=cuda) % V
    start[17] = V + 3  # out of range: MLXC_STATUS_BAD_NODE
    rand = mc.philox_uniform((N, L), 9, device=cuda)
    n, _, st = _walk(rowptr, col, start, rand, L, noalloc=True)
    assert st == _lib.MLXC_STATUS_BAD_NODE
    ok = start[:5_000] % V
    n_a, e_a, st_a = _walk(rowptr, col, ok, rand[:5_000], L, noalloc=False)
    n_b, e_b, st_b = _walk(rowptr, col, ok, rand[:5_000], L, noalloc=True)
    assert st_a == 0 and st_b == 0
    assert torch.equal(n_a, n_b) and torch.equal(e_a, e_b)
    # d_status may be NULL
    lib = _lib.load()
    out = torch.empty((5_000, L + 1), dtype=torch.int64, device=cuda)
    rc = lib.mlxc_random_walk_noalloc(rowptr.data_ptr(), V, col.data_ptr(), col.numel(),
                                      ok.data_ptr(), 5_000, rand.data_ptr(), L, out.data_ptr(),
                                      None, 0, None, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(out, n_a)


def test_noalloc_beyond_the_scratch_runs_a_smaller_layout(cuda):
    """Calls whose fastest layout exceeds MLXC_NOALLOC_SCRATCH_BYTES run the
    largest layout the scratch holds: configuration 2's graph with 2^20 walks
    of 80 steps (packed records of 137 MB; the start records of 16 MB fit),
    then 2^23 walks of 6 steps (start records of 134 MB: the direct kernel),
    each equal to mlxc_random_walk with the full workspace, nodes, edges and
    status."""
    lib = _lib.load()
    rowptr, col = synth.rmat_csr(20, 1 << 24, seed=0, device=cuda)
    V, E = rowptr.numel() - 1, col.numel()
    for N, L in ((1 << 20, 80), (1 << 23, 6)):
        assert lib.mlxc_random_walk_workspace_bytes(V, E, N, L) > _lib.MLXC_NOALLOC_SCRATCH_BYTES
        start = torch.arange(N, device=cuda) % V
        rand = mc.philox_uniform((N, L), 11, device=cuda)
        _same(rowptr, col, start, rand, L)
