"""Build the cortexsdr_amd HIP library in-tree for gfx950.

    python -m cortexsdr_amd.build        # -> cortexsdr_amd/libcortexsdr_amd.so

One hipcc invocation per source into objects under cortexsdr_amd/_build/, then one link.
Cross-compiles without a GPU. The packed-fp32 target feature is switched off for all
device code (hipcc still emits scalar and vector fp32 math).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcortexsdr_amd.so")
BIN = os.path.join(HERE, "bin")
TOOLS = os.path.join(CSRC, "tools")
ROOT = os.path.dirname(HERE)

ARCH = os.environ.get("CSDR_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return p


def common_flags() -> list[str]:
    return [
        "-std=c++17", "-O3", "-fPIC", "-Wall", "-Wno-unused-result",
        "-I" + os.path.join(ROOT, "include"),
    ]


def device_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-fno-gpu-flush-denormals-to-zero",
        "-munsafe-fp-atomics",
    ]


def compile_one(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if src.endswith(".hip"):
        cmd = [hipcc(), "-x", "hip", *common_flags(), *device_flags(), "-c", src, "-o", obj]
    else:
        cmd = [hipcc(), *common_flags(), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    # (tools/ holds executables, built after the library)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    # host tools linked against the library (rpath to the package directory)
    os.makedirs(BIN, exist_ok=True)
    for src in sorted(glob.glob(os.path.join(TOOLS, "*.cpp"))):
        exe = os.path.join(BIN, "cortexsdr_" + os.path.splitext(os.path.basename(src))[0])
        cmd = [hipcc(), *common_flags(), src, "-L" + HERE, "-lcortexsdr_amd",
               "-Wl,-rpath,$ORIGIN/..", "-o", exe + ".tmp"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"tool build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
        os.replace(exe + ".tmp", exe)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
