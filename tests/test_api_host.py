"""Host-side argument handling of the Python API (no GPU needed: every case
here is rejected before the device is touched)."""
import numpy as np
import pytest
import torch

import mlx_cluster_amd as mc
from tests.graphs import csr

ROWPTR, COL = csr(3, [(0, 1), (1, 2), (2, 0)])
START = np.array([0, 1], dtype=np.int64)
RAND = np.zeros((2, 4), dtype=np.float32)


def test_reference_signature_order():
    import inspect
    sig = inspect.signature(mc.random_walk)
    assert list(sig.parameters)[:5] == ["rowptr", "col", "start", "rand", "walk_length"]
    assert sig.parameters["stream"].kind is inspect.Parameter.KEYWORD_ONLY
    sig = inspect.signature(mc.rejection_sampling)
    assert list(sig.parameters)[:6] == ["rowptr", "col", "start", "walk_length", "p", "q"]
    assert sig.parameters["stream"].kind is inspect.Parameter.KEYWORD_ONLY


@pytest.mark.parametrize("kw,exc", [
    (dict(rowptr=ROWPTR.astype(np.int32)), TypeError),
    (dict(col=COL.astype(np.float64)), TypeError),
    (dict(start=START.astype(np.int32)), TypeError),
    (dict(rand=RAND.astype(np.float64)), TypeError),
    (dict(rand=np.zeros((2, 3), np.float32)), ValueError),
    (dict(walk_length=-1), ValueError),
    (dict(walk_length=2.0), TypeError),
    (dict(rowptr=np.zeros(0, np.int64)), ValueError),
    (dict(col=COL.reshape(1, -1)), ValueError),
    (dict(rowptr=[0, 1, 2, 3]), TypeError),
])
def test_random_walk_validation(kw, exc):
    args = dict(rowptr=ROWPTR, col=COL, start=START, rand=RAND, walk_length=4)
    args.update(kw)
    with pytest.raises(exc):
        mc.random_walk(args["rowptr"], args["col"], args["start"], args["rand"],
                       args["walk_length"])


def test_seed_and_rand_are_exclusive():
    with pytest.raises(ValueError, match="seed"):
        mc.random_walk(ROWPTR, COL, START, None, 4)
    with pytest.raises(ValueError, match="either"):
        mc.random_walk(ROWPTR, COL, START, RAND, 4, seed=3)


def test_bad_stream_type():
    with pytest.raises(TypeError):
        mc.random_walk(ROWPTR, COL, START, RAND, 4, stream=3.5)


@pytest.mark.parametrize("p,q,rule,exc", [
    (0.0, 1.0, "ref_chain", ValueError), (1.0, -2.0, "ref_chain", ValueError),
    (float("nan"), 1.0, "ref_chain", ValueError), (1.0, float("inf"), "ref_chain", ValueError),
    (1.0, 1.0, "bogus", ValueError),
])
def test_rejection_sampling_validation(p, q, rule, exc):
    with pytest.raises(exc):
        mc.rejection_sampling(ROWPTR, COL, START, 4, p, q, rule=rule)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
def test_no_gpu_fails_loudly():
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mc.random_walk(ROWPTR, COL, START, RAND, 4)
