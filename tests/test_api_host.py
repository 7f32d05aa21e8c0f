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


def test_device_named_as_stream_is_where_the_call_runs():
    from mlx_cluster_amd.walks import _resolve_device
    host_tensor = torch.zeros(1)
    assert _resolve_device("cuda:1", (host_tensor,)) == torch.device("cuda", 1)
    assert _resolve_device(torch.device("cuda", 3), ()) == torch.device("cuda", 3)
    with pytest.raises(ValueError, match="expected a GPU"):
        _resolve_device("meta", ())


def test_to_csr_stream_must_be_a_stream():
    with pytest.raises(TypeError, match="torch.cuda.Stream"):
        mc.to_csr(np.array([[0, 1], [1, 0]]), 2, stream="cuda:0")


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


def test_walk_offset_validation():
    with pytest.raises(ValueError, match="walk_offset"):
        mc.random_walk(ROWPTR, COL, START, RAND, 4, walk_offset=3, stream="cpu")
    with pytest.raises(ValueError, match="walk_offset"):
        mc.random_walk(ROWPTR, COL, START, None, 4, seed=1, walk_offset=-1, stream="cpu")
    with pytest.raises(TypeError, match="walk_offset"):
        mc.rejection_sampling(ROWPTR, COL, START, 4, 1.0, 1.0, walk_offset=1.5, stream="cpu")
    with pytest.raises(ValueError, match="memory_budget"):
        mc.random_walk(ROWPTR, COL, START, None, 4, seed=1, memory_budget=0, stream="cpu")


# -------------------------------------------------- chunk planning (host logic)

def _records_query(E):
    """A workspace query shaped like the uniform walk's: records (8 bytes per
    edge and walk) when the call takes at least 4 steps per edge, else 16
    bytes per walk."""
    return lambda n: 256 + (8 * (E + n) if n * 20 >= 4 * E else 16 * n)


def test_plan_one_call_when_everything_fits():
    from mlx_cluster_amd.walks import _plan
    q = _records_query(1000)
    assert _plan(10_000, 168, q, 10_000 * 168 + q(10_000)) == ("device", None, q(10_000))


def test_plan_shrinks_the_workspace_before_chunking():
    from mlx_cluster_amd.walks import _MIN_WORKSPACE, _plan
    q = _records_query(10**6)
    N, row = 10_000, 168
    budget = N * row + 5000
    mode, chunk, ws = _plan(N, row, q, budget)
    assert (mode, chunk) == ("device", None) and _MIN_WORKSPACE <= ws <= 5000 and ws % 16 == 0


@pytest.mark.parametrize("N,row,E,budget", [
    (100_000, 168, 1000, 4_000_000), (100_000, 168, 10**6, 4_000_000),
    (1_000_000, 656, 16 * 10**6, 300 * 2**20), (777, 48, 10, 20_000), (50, 8, 10, 300)])
def test_plan_chunks_fit_the_budget(N, row, E, budget):
    """Outputs larger than the budget: chunks whose two staging buffers and
    workspace fit it, whole multiples of 64 walks when a chunk holds that
    many, as large as the budget allows."""
    from mlx_cluster_amd.walks import _CHUNK_ALIGN, _MIN_WORKSPACE, _plan
    q = _records_query(E)
    mode, chunk, ws = _plan(N, row, q, budget)
    assert mode == "host" and 1 <= chunk <= N
    assert 2 * chunk * row + ws <= budget and ws >= _MIN_WORKSPACE
    if chunk >= _CHUNK_ALIGN:
        assert chunk % _CHUNK_ALIGN == 0
        bigger = chunk + _CHUNK_ALIGN
        assert bigger > N or 2 * bigger * row + min(q(bigger), _MIN_WORKSPACE) > budget or \
            2 * bigger * row + q(bigger) > budget


def test_plan_rejects_a_budget_below_one_walk():
    from mlx_cluster_amd.walks import _plan
    with pytest.raises(ValueError, match="memory_budget"):
        _plan(10, 1000, lambda n: 256 + 16 * n, 1000)


def test_binding_declines_cpu_tensors():
    """The compiled fast path takes only device tensors: given CPU tensors it
    returns None, and the general path then reports the missing GPU (or, for
    stream='cpu', runs the host twins)."""
    from mlx_cluster_amd import walks
    if walks._fast is None:
        pytest.skip("the compiled fast path is not built")
    r = torch.from_numpy(ROWPTR)
    c = torch.from_numpy(COL)
    s = torch.from_numpy(START)
    assert walks._fast.random_walk(r, c, s, torch.from_numpy(RAND), 4, None, True, False,
                                   False) is None
    assert walks._fast.rejection_sampling(r, c, s, 4, 1.0, 1.0, 1, 0, 2, True, False,
                                          False) is None
    n = mc.random_walk(r, c, s, torch.from_numpy(RAND), 4, stream="cpu")
    assert n.shape == (2, 5)


def test_fast_path_only_with_the_in_tree_library(tmp_path):
    """The compiled fast path is linked to the in-tree libmlxc.so: another
    build selected by MLXC_LIB must not be bypassed through it."""
    import os
    import subprocess
    import sys
    code = "import mlx_cluster_amd.walks as w; print(w._fast is None)"
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, MLXC_LIB=str(tmp_path / "libmlxc.so"))
    out = subprocess.run([sys.executable, "-c", code], cwd=repo, env=env, capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "True"
