"""mlxc_set_walk_events: the HIP events a walk call records around its walk
kernel, which bench.py uses to time that kernel alone.

Each case runs a call between two outer events with the hook set and checks
that the library recorded the pair inside the call, in order, that the walks
are the same as without the hook, and that after mlxc_set_walk_events(NULL,
NULL) a call leaves the events alone."""
import numpy as np
import pytest
import torch

import mlx_cluster_amd as mc
from mlx_cluster_amd import _lib, synth

pytestmark = pytest.mark.gpu


def _events(n):
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for e in ev:  # torch creates an event's HIP handle at its first record
        e.record()
    torch.cuda.synchronize()
    return ev


def _graphs(cuda):
    big = synth.rmat_csr(14, 200_000, seed=5, symmetrize=True)
    small = synth.cora_like(seed=0)
    t = lambda a: torch.as_tensor(a).to(cuda)
    return {"rmat": tuple(t(a) for a in big), "cora": tuple(t(a) for a in small)}


@pytest.mark.parametrize("graph", ["rmat", "cora"])
@pytest.mark.parametrize("kind", ["uniform", "seeded", "node2vec"])
def test_events_bracket_the_walk_kernel(graph, kind, cuda):
    rowptr, col = _graphs(cuda)[graph]
    V, L, N = rowptr.numel() - 1, 6, 4000
    start = torch.arange(N, device=cuda) % V
    rand = mc.philox_uniform((N, L), 9, device=cuda)
    if kind == "uniform":
        call = lambda: mc.random_walk(rowptr, col, start, rand, L)
    elif kind == "seeded":
        call = lambda: mc.random_walk(rowptr, col, start, None, L, seed=9)
    else:
        call = lambda: mc.rejection_sampling(rowptr, col, start, L, 0.5, 2.0, seed=9)
    plain = call()
    lib = _lib.load()
    o0, o1, w0, w1 = _events(4)
    o0.record()
    _lib.check(lib.mlxc_set_walk_events(w0.cuda_event, w1.cuda_event), "set")
    try:
        hooked = call()
    finally:
        _lib.check(lib.mlxc_set_walk_events(None, None), "clear")
    o1.record()
    torch.cuda.synchronize()
    assert torch.equal(plain, hooked)
    call_ms, walk_ms = o0.elapsed_time(o1), w0.elapsed_time(w1)
    assert o0.elapsed_time(w0) >= 0 and w1.elapsed_time(o1) >= 0, "recorded inside the call"
    assert 0 < walk_ms <= call_ms
    t0, t1 = o0.elapsed_time(w0), o0.elapsed_time(w1)
    again = call()
    torch.cuda.synchronize()
    assert torch.equal(plain, again)
    assert (o0.elapsed_time(w0), o0.elapsed_time(w1)) == (t0, t1), \
        "a call after the hook was cleared re-recorded an event"


def test_empty_call_records_nothing(cuda):
    rowptr, col = _graphs(cuda)["cora"]
    start = torch.empty(0, dtype=torch.int64, device=cuda)
    lib = _lib.load()
    o0, w0, w1 = _events(3)
    before = (o0.elapsed_time(w0), o0.elapsed_time(w1))
    _lib.check(lib.mlxc_set_walk_events(w0.cuda_event, w1.cuda_event), "set")
    try:
        out = mc.random_walk(rowptr, col, start, None, 5, seed=1)
    finally:
        _lib.check(lib.mlxc_set_walk_events(None, None), "clear")
    torch.cuda.synchronize()
    assert out.shape == (0, 6)
    assert (o0.elapsed_time(w0), o0.elapsed_time(w1)) == before
    np.testing.assert_array_equal(out.cpu().numpy(), np.zeros((0, 6), np.int64))
