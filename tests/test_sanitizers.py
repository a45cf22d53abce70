"""The host code under AddressSanitizer and UBSan: the C++ layer's dispatch
and error paths, the CPU branch, the error state and the C oracle, built
with g++/gcc -fsanitize=address,undefined into one executable
(tests/cpp/test_dsine_ops.cpp in cpu mode, the device entry points replaced
by stubs that abort: tests/cpp/no_device.cpp) and run here.  A sanitizer
report fails the run (-fno-sanitize-recover, halt_on_error)."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from brovisionml_amd.build import CSRC, INCLUDE, ROOT

OUT = os.path.join(ROOT, "tests", "cpp", "_build", "sanitize")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
       "-g", "-O1"]
HIP_HOST = ["-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include"]


def _run(cmd, **kw):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, **kw)
    assert proc.returncode == 0, " ".join(cmd) + "\n" + proc.stdout[-4000:]
    return proc.stdout


@pytest.fixture(scope="module")
def sanitized_exe():
    if shutil.which("g++") is None or shutil.which("gcc") is None:
        pytest.skip("needs g++ and gcc")
    os.makedirs(OUT, exist_ok=True)
    objs = []
    oracle_o = os.path.join(OUT, "oracle.o")
    _run(["gcc", "-std=c11", "-fPIC", "-ffp-contract=off", "-fopenmp", *SAN, "-c",
          os.path.join(ROOT, "oracle", "dsine_ops_oracle.c"), "-o", oracle_o])
    objs.append(oracle_o)
    for src in (os.path.join(ROOT, "tests", "cpp", "test_dsine_ops.cpp"),
                os.path.join(ROOT, "tests", "cpp", "no_device.cpp"),
                os.path.join(CSRC, "dsine_ops.cpp"), os.path.join(CSRC, "dsine_ops_cpu.cpp"),
                os.path.join(CSRC, "status.cpp"), os.path.join(CSRC, "tensor.cpp")):
        obj = os.path.join(OUT, os.path.basename(src) + ".o")
        _run(["g++", "-std=c++17", "-ffp-contract=off", "-pthread", *SAN, *HIP_HOST,
              "-I", INCLUDE, "-c", src, "-o", obj])
        objs.append(obj)
    exe = os.path.join(OUT, "test_dsine_ops_san")
    _run(["g++", *SAN, "-pthread", "-fopenmp", *objs, "-L", "/opt/rocm/lib", "-lamdhip64",
          "-Wl,-rpath,/opt/rocm/lib", "-o", exe])
    return exe


def test_host_code_under_asan_and_ubsan(sanitized_exe):
    env = dict(os.environ, ASAN_OPTIONS="halt_on_error=1:detect_leaks=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    out = _run([sanitized_exe, "cpu"], env=env, timeout=600)
    assert "OK" in out and "ERROR" not in out and "runtime error" not in out, out
