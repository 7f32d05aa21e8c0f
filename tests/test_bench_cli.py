"""bench.py's contract checks that need no GPU: more than one GPU is refused
with a message, and every configuration it accepts is described."""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args):
    return subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120)


@pytest.mark.parametrize("n", ["2", "8"])
def test_more_than_one_gpu_is_refused(n):
    res = run_bench("--gpus", n)
    assert res.returncode == 2
    assert "one GPU" in res.stderr or "single MI355X" in res.stderr
    assert res.stdout == ""


def test_configurations_are_listed():
    sys.path.insert(0, REPO)
    import bench
    names = set(bench.CONFIGS) | set(bench.CSR_CONFIGS) | set(bench.WIN_CONFIGS)
    assert {"c2", "c3", "c4", "c5", "csr4", "win2"} <= names
    assert not (set(bench.CONFIGS) & set(bench.CSR_CONFIGS))
    res = run_bench("--help")
    assert res.returncode == 0
    for name in ("c2", "csr4", "win2"):
        assert name in res.stdout
