"""Build recipe for the native library (hipcc, gfx950 only).

`build()` compiles every time it is called:
  brovisionml_amd/lib/libbvml_dsine.so  -- HIP kernels, the C ABI
                                          (include/bvml_dsine.h) and the C++
                                          drop-in layer (include/brovisionml/)
Run as `python -m brovisionml_amd.build`.
"""
from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "brovisionml_amd")
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libbvml_dsine.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed fp32 instructions are disabled for all device code: only the scalar
# fp32 forms are generated.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # leading scalar kernel arguments (up to 14 dwords) arrive preloaded in
    # SGPRs; the code object keeps a prologue that loads them on firmware
    # without the feature
    "-mllvm", "-amdgpu-kernarg-preload-count=10",
    "-Wall",
]

SOURCES = [
    os.path.join(CSRC, "dsine_ops.hip"),   # kernels + C ABI
    os.path.join(CSRC, "upsample.hip"),    # convex upsample + normalise
    os.path.join(CSRC, "dsine_ops.cpp"),   # C++ drop-in (brovisionml::dsine)
    os.path.join(CSRC, "tensor.cpp"),      # brotensor::Tensor subset
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError("build failed: " + " ".join(cmd))


def build_library() -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *HIP_FLAGS, "-I", os.path.join(ROOT, "include"), "-shared",
           "-o", tmp, *SOURCES]
    _run(cmd)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build_library())
