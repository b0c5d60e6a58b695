"""Build libtda_hip.so in-tree: hipcc for the gfx950 kernels, g++ for the host-only C ABI.

    python -m tda_amd.build          # or tda_amd.build.build()

The library lands next to this file (tda_amd/libtda_hip.so), so it travels with the source
tree; objects go to tda_amd/_build/.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(HERE, "libtda_hip.so")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", os.path.join(ROCM, "bin", "hipcc"))
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"

# Packed fp32 VALU ops are switched off for all device code.
HIP_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]

HIP_SOURCES = ["tda_fwd.hip", "tda_fwd_sparse.hip", "tda_fwd_decode.hip", "tda_bwd.hip", "tda_bwd_fast.hip",
               "tda_wide.hip", "tda_noalloc.hip"]
HOST_SOURCES = ["tda_host.cpp"]
# host-only code that calls the HIP runtime API (no device code): g++ against the ROCm headers
HIP_HOST_SOURCES = ["tda_timing.cpp"]
HIP_HOST_FLAGS = [f"-I{ROCM}/include", "-D__HIP_PLATFORM_AMD__"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless noise
    err = "\n".join(ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every source and link LIB_PATH.  Always rebuilds.  Returns the library path."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD_DIR, exist_ok=True)
    cmds, objs = [], []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD_DIR, src + ".o")
        cmds.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD_DIR, src + ".o")
        cmds.append([CXX, *HOST_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in HIP_HOST_SOURCES:
        obj = os.path.join(BUILD_DIR, src + ".o")
        cmds.append([CXX, *HOST_FLAGS, *HIP_HOST_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    jobs = jobs or min(len(cmds), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    shutil.move(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
