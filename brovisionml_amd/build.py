"""Build recipe for the native libraries (hipcc for gfx950, g++ for plain C++).

`build_library()` compiles every time it is called, into brovisionml_amd/lib/:
  libbvml_dsine.so        HIP kernels and the CPU branch behind one C ABI
                          (include/bvml_dsine.h); extern "C" symbols only
  libbvml_dsine_cxx.so    the C++ drop-in of the ops, brovisionml::dsine::*
                          (dsine_ops.cpp, include/brovisionml/dsine_ops.h),
                          plain C++ over the C ABI; brotensor::Tensor left
                          undefined, to be resolved by brotensor or by the
                          subset below
  libbvml_dsine_refine.so the native NRN refiner (refiner.cpp,
                          refiner_cpu.cpp, include/bvml_dsine_refine.h): C++
                          over the C ABI; extern "C" symbols only
  libbvml_dsine_refine_cxx.so  the C++ drop-in brovisionml::dsine::Refiner
                          (dsine_refine.cpp, include/brovisionml/dsine_refine.h)
                          over the refiner's C ABI; brotensor::Tensor left
                          undefined, like libbvml_dsine_cxx.so
  libbrotensor_subset.so  the brotensor::Tensor subset of
                          include/brotensor/tensor.h, for standalone use and
                          the C++ tests; a brovisionml build links brotensor
Run as `python -m brovisionml_amd.build`.
"""
from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "brovisionml_amd")
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libbvml_dsine.so")
LIB_CXX = os.path.join(LIBDIR, "libbvml_dsine_cxx.so")
LIB_TENSOR = os.path.join(LIBDIR, "libbrotensor_subset.so")
LIB_REFINE = os.path.join(LIBDIR, "libbvml_dsine_refine.so")
LIB_REFINE_CXX = os.path.join(LIBDIR, "libbvml_dsine_refine_cxx.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

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

# Host C++ (the CPU branch, the C++ layer).  Contraction off keeps the CPU
# branch's double arithmetic in the reference's operation order.
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-Wall",
             "-Wextra", "-pthread"]

SOURCES = [
    os.path.join(CSRC, "dsine_ops.hip"),      # AngMF / RayReLU kernels + C ABI
    os.path.join(CSRC, "upsample.hip"),       # convex upsample + normalise
    os.path.join(CSRC, "gru.hip"),            # the refiner's fused elementwise steps
    os.path.join(CSRC, "heads.hip"),          # the refiner's heads after their 3x3 layer
    os.path.join(CSRC, "conv.hip"),           # the refiner's 3x3 / 5x5 convolutions
]
HOST_SOURCES = [
    os.path.join(CSRC, "dsine_ops_cpu.cpp"),  # CPU branch (C ABI *_cpu_f32)
    os.path.join(CSRC, "status.cpp"),         # error state, bvml_dsine_last_error
    os.path.join(CSRC, "pack.cpp"),           # weight packing for the matrix-core kernels
]
CXX_SOURCES = [os.path.join(CSRC, "dsine_ops.cpp")]     # the ops' public dispatch
REFINE_CXX_SOURCES = [os.path.join(CSRC, "dsine_refine.cpp")]  # the Refiner class
TENSOR_SOURCES = [os.path.join(CSRC, "tensor.cpp")]
REFINE_SOURCES = [os.path.join(CSRC, "refiner.cpp"),      # device path, weights, C ABI
                  os.path.join(CSRC, "refiner_cpu.cpp")]  # host path
# the allocation-free forward and its device scratch array (hipcc)
REFINE_HIP_SOURCE = os.path.join(CSRC, "refiner_noalloc.hip")
# host C++ against the HIP runtime headers
HIP_HOST_FLAGS = ["-D__HIP_PLATFORM_AMD__", "-isystem", os.path.join(ROCM, "include")]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError("build failed: " + " ".join(cmd))


def _install(tmp: str, dst: str) -> None:
    os.replace(tmp, dst)


def build_library() -> str:
    """Builds the five libraries; returns the C ABI library's path."""
    os.makedirs(LIBDIR, exist_ok=True)
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    host_objs = []
    for src in HOST_SOURCES:
        obj = os.path.join(objdir, os.path.basename(src) + ".o")
        _run([CXX, *CXX_FLAGS, "-I", INCLUDE, "-c", src, "-o", obj])
        host_objs.append(obj)
    # objects first: hipcc reads every file after a .hip source as HIP
    _run([HIPCC, *HIP_FLAGS, "-I", INCLUDE, "-shared", "-o", LIB + ".tmp", *host_objs, *SOURCES,
          "-Wl,--version-script=" + os.path.join(CSRC, "libbvml_dsine.map")])
    _install(LIB + ".tmp", LIB)
    noalloc_obj = os.path.join(objdir, "refiner_noalloc.hip.o")
    _run([HIPCC, *HIP_FLAGS, "-I", INCLUDE, "-c", REFINE_HIP_SOURCE, "-o", noalloc_obj])
    _run([CXX, *CXX_FLAGS, *HIP_HOST_FLAGS, "-I", INCLUDE, "-shared", "-o", LIB_REFINE + ".tmp",
          *REFINE_SOURCES, noalloc_obj, "-L", LIBDIR, "-lbvml_dsine", "-L", os.path.join(ROCM, "lib"),
          "-lamdhip64", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + os.path.join(ROCM, "lib"),
          "-Wl,--version-script=" + os.path.join(CSRC, "libbvml_dsine_refine.map")])
    _install(LIB_REFINE + ".tmp", LIB_REFINE)
    _run([CXX, *CXX_FLAGS, "-I", INCLUDE, "-shared", "-o", LIB_REFINE_CXX + ".tmp",
          *REFINE_CXX_SOURCES, "-L", LIBDIR, "-lbvml_dsine_refine", "-Wl,-rpath,$ORIGIN",
          "-Wl,--version-script=" + os.path.join(CSRC, "libbvml_dsine_refine_cxx.map")])
    _install(LIB_REFINE_CXX + ".tmp", LIB_REFINE_CXX)
    _run([CXX, *CXX_FLAGS, "-I", INCLUDE, "-shared", "-o", LIB_CXX + ".tmp", *CXX_SOURCES,
          "-L", LIBDIR, "-lbvml_dsine", "-Wl,-rpath,$ORIGIN",
          "-Wl,--version-script=" + os.path.join(CSRC, "libbvml_dsine_cxx.map")])
    _install(LIB_CXX + ".tmp", LIB_CXX)
    _run([HIPCC, "-O2", "-std=c++17", "-fPIC", "-I", INCLUDE, "-shared", "-o", LIB_TENSOR + ".tmp",
          *TENSOR_SOURCES])
    _install(LIB_TENSOR + ".tmp", LIB_TENSOR)
    return LIB


# The language standards the drop-in C++ is checked against: brovisionml
# builds as C++20 (its CMakeLists.txt sets CMAKE_CXX_STANDARD 20); the
# library's own build uses C++17, so the sources take both.
CXX_STANDARDS = ("c++17", "c++20")


def check_brotensor_api() -> None:
    """Compiles the C++ layer and the launchers header against a header that
    declares only what brovisionml's sources use of brotensor::Tensor
    (tests/cpp/brotensor_api/brotensor/tensor.h), warnings as errors, under
    each of CXX_STANDARDS."""
    api = os.path.join(ROOT, "tests", "cpp", "brotensor_api")
    for std in CXX_STANDARDS:
        for src in (*CXX_SOURCES, *REFINE_CXX_SOURCES, os.path.join(api, "launchers_check.cpp")):
            _run([CXX, "-std=" + std, "-fsyntax-only", "-Wall", "-Wextra", "-Werror", "-I", api,
                  "-I", INCLUDE, src])


if __name__ == "__main__":
    print(build_library())
    check_brotensor_api()
