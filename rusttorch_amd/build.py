"""Build librtgpu.so (HIP kernels + C++ runtime) for gfx950, in-tree.

Usage: python -m rusttorch_amd.build  (or rusttorch_amd.build.build()).
Objects go to rusttorch_amd/_build/, the library to rusttorch_amd/lib/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "librtgpu.so")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function", f"-I{os.path.join(PKG, '..', 'include')}"]

SOURCES = ["kernels.hip", "decode_persistent.hip", "decode_persistent_inst_mini.hip",
           "decode_persistent_inst_small.hip", "decode_persistent_inst_medium.hip",
           "decode_persistent_inst_large.hip", "rtg_runtime.cpp", "safetensors_reader.cpp",
           "tokenizer.cpp", "sampling.hip", "bgemv.hip", "scratch.hip", "decode_tile.hip", "rows.hip"]


def _compile(src: str) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJ, src + ".o")
    if src.endswith(".hip"):
        cmd = [HIPCC, f"--offload-arch={ARCH}", *DEVICE_FLAGS, *COMMON, "-c", path, "-o", obj]
    else:
        cmd = [HIPCC, *COMMON, "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every source (always, no staleness check) and link the library."""
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    # seeded weight generator (host-only helper for synthetic inputs)
    so = os.path.join(LIBDIR, "libsynth.so")
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-o", so + ".tmp", os.path.join(CSRC, "synth.c"), "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"synth build failed: {' '.join(cmd)}\n{r.stderr}")
    os.replace(so + ".tmp", so)
    if verbose:
        print("built", LIB)
    return LIB


def clean() -> None:
    shutil.rmtree(OBJ, ignore_errors=True)


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
