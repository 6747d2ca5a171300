"""Builds atlas_amd/libatlas_kernels.so with hipcc for gfx950.

The reference compiles kernels/matmul.cu with nvcc from build.rs
(crates/atlas-tensor/build.rs:19-107); this is the hipcc equivalent: one
shared library with the extern "C" ABI of include/atlas_kernels.h and
include/atlas_engine.h, linked against the HIP runtime and hipBLASLt (the
bf16 and int8 prompt GEMMs of 17..1024 rows, used only when ATLAS_PROMPT_BLAS=1
at model creation; every other kernel, and by default those GEMMs too, is
hand-written HIP).

Usage: python -m atlas_amd.build   (or atlas_amd.build.build())
Environment: ATLAS_HIP_ARCH overrides the target (default gfx950).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libatlas_kernels.so")

SOURCES = ["gemv.hip", "skinny.hip", "attention.hip", "fused.hip", "errors.cpp", "runtime.cpp",
           "capi.cpp", "engine.cpp", "st_format.cpp", "loader.cpp", "blas.cpp"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build atlas_amd")


def flags() -> list[str]:
    arch = os.environ.get("ATLAS_HIP_ARCH", "gfx950")
    return [f"--offload-arch={arch}", "-O3", "-std=c++17", "-fPIC", "-Wall",
            "-Wno-unused-function", "-fvisibility=hidden",
            # packed FP32 VALU ops are kept out of every kernel
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", os.path.join(HERE, "..", "include")]


def _compile(src: str) -> str:
    obj = os.path.join(OUT_DIR, src + ".o")
    path = os.path.join(CSRC, src)
    cmd = [hipcc()] + flags() + ["-c", path, "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={os.environ.get('ATLAS_HIP_ARCH', 'gfx950')}", "-shared",
           "-fPIC", "-o", tmp] + objs + ["-lhipblaslt", "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
