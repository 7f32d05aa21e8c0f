"""Builds libmlxc.so (HIP kernels + C ABI) in-tree for gfx950.

Usage: python -m mlx_cluster_amd.build_lib   (or build() from __graft_entry__)
"""
from __future__ import annotations

import hashlib
import os
import re
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
SOURCES = [os.path.join(CSRC, f) for f in
           ("mlxc_api.hip", "prep_kernels.hip", "uniform_walk.hip", "node2vec_walk.hip",
            "csr_build.hip", "windows.hip", "gather_probe.hip", "host_walk.cpp", "host_csr.cpp")]
OUT = os.path.join(PKG_DIR, "libmlxc.so")
INCLUDE = os.path.join(REPO_DIR, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("MLXC_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off: the walk's index is an IEEE float32 product that must
# round exactly as the reference's scalar code; no fused or reassociated math.
# -packed-fp32-ops off: keep the compiler from emitting packed FP32 forms.
FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


BUILD_DIR = os.path.join(REPO_DIR, "_build")


def _run(cmd: list[str], verbose: bool, what: str) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed building {what}")


def build(verbose: bool = False, extra_flags: list[str] | None = None, out: str = OUT) -> str:
    """Compiles every source to an object (in parallel; each translation unit
    carries its own gfx950 code object, no cross-unit device calls) and links
    them into `out`."""
    from concurrent.futures import ThreadPoolExecutor

    tag = hashlib.sha256(" ".join(extra_flags or []).encode()).hexdigest()[:8]
    obj_dir = os.path.join(BUILD_DIR, f"{os.path.basename(out)}-{tag}")
    os.makedirs(obj_dir, exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    objs = [os.path.join(obj_dir, os.path.basename(src) + ".o") for src in SOURCES]
    jobs = max(1, min(len(SOURCES), os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(lambda so: _run([HIPCC, *compile_flags, *(extra_flags or []), "-I", INCLUDE,
                                       "-I", CSRC, "-c", so[0], "-o", so[1]], verbose, so[0]),
                      zip(SOURCES, objs)))
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", out + ".tmp"],
         verbose, out)
    os.replace(out + ".tmp", out)
    return out


BINDING_SRC = os.path.join(CSRC, "torch_binding.cpp")


def binding_path() -> str:
    import sysconfig
    return os.path.join(PKG_DIR, "_mlxc_torch" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_binding(verbose: bool = False, lib: str = OUT) -> str:
    """Compiles the compiled fast path (torch_binding.cpp, host code only)
    against torch's headers and libraries and the in-tree libmlxc.so, with
    hipcc and no source translation step."""
    import sysconfig

    import torch
    import torch.utils.cpp_extension as ce
    out = binding_path()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_EXTENSION_NAME=_mlxc_torch", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-I", INCLUDE, "-I", sysconfig.get_paths()["include"]]
    for d in ce.include_paths(device_type="cuda"):
        cmd += ["-isystem", d]
    cmd += [BINDING_SRC, "-o", out + ".tmp"]
    for d in ce.library_paths(device_type="cuda"):
        cmd += ["-L", d, f"-Wl,-rpath,{d}"]
    cmd += ["-L", os.path.dirname(lib), "-Wl,-rpath,$ORIGIN", "-lmlxc",
            "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
            "-lamdhip64"]
    _run(cmd, verbose, out)
    os.replace(out + ".tmp", out)
    return out


def source_files() -> list[str]:
    """Every file the library is built from (kernels, headers, C ABI)."""
    return sorted([os.path.join(CSRC, f) for f in os.listdir(CSRC)] +
                  [os.path.join(INCLUDE, "mlxc.h")])


def _code_only(text: str) -> str:
    """C/C++ source without comments, trailing blanks and empty lines."""
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return "\n".join(line.rstrip() for line in text.splitlines() if line.strip())


# The device code each profiled kernel family is built from (its kernels and
# launchers, the preparation kernels the walks run first, the shared device
# helpers): a profile stays matched to a build as long as these files' code
# is unchanged.
# walk_host.h is in every family: its constants (records_fit,
# kSmallGraphEdgesPerStep) choose which kernels a call runs.
KERNEL_SOURCES = {
    "uniform_walk": ["walk_device.h", "walk_host.h", "prep_kernels.hip", "uniform_walk.hip"],
    "node2vec_walk": ["walk_device.h", "walk_host.h", "prep_kernels.hip", "node2vec_walk.hip"],
    "csr_build": ["walk_device.h", "walk_host.h", "csr_build.hip"],
    "context_windows": ["walk_device.h", "walk_host.h", "windows.hip"],
    # the probe's kernel uses nothing from the walk headers (its launcher only
    # their host helpers)
    "gather_probe": ["gather_probe.hip"],
}


def source_hash(kind: str | None = None) -> str:
    """sha256[:16] over the code of the source files of one kernel family
    (KERNEL_SOURCES; every source file when kind is None) and the C ABI
    header, comments excluded, so that a profile taken of a build stays
    matched to it across comment edits and changes to unrelated kernels."""
    files = source_files()
    if kind is not None:
        wanted = set(KERNEL_SOURCES[kind]) | {"mlxc.h"}
        files = [f for f in files if os.path.basename(f) in wanted]
    h = hashlib.sha256()
    for path in files:
        h.update(os.path.basename(path).encode())
        h.update(_code_only(open(path, encoding="utf-8").read()).encode())
    return h.hexdigest()[:16]


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_binding(verbose=True))
