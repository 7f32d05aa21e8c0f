"""include/mlxc.h and libmlxc.so used from plain C99: tests/c_abi_example.c
is compiled with gcc (-std=c99 -Wall -Werror) against the in-tree library
and run.  Host twins only, so no GPU is needed."""
import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(REPO, "mlx_cluster_amd")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_c_abi_example(tmp_path):
    exe = tmp_path / "c_abi_example"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-I",
                    os.path.join(REPO, "include"), os.path.join(REPO, "tests", "c_abi_example.c"),
                    "-L", LIBDIR, "-lmlxc", f"-Wl,-rpath,{LIBDIR}", "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stderr
    assert "c abi example ok" in res.stdout
