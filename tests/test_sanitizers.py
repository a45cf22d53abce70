"""The host code under AddressSanitizer and UBSan: the C++ layer's dispatch
and error paths, the CPU branch, the error state and the C oracle, built
with g++/gcc -fsanitize=address,undefined into one executable
(tests/cpp/test_dsine_ops.cpp in cpu mode, the device entry points replaced
by stubs that abort: tests/cpp/no_device.cpp) and run here; and the Refiner
class with the native refiner's checkpoint reader and host path
(tests/cpp/test_dsine_refine.cpp: its error paths, a CPU forward and a set
of malformed checkpoints) the same way.  A sanitizer report fails the run
(-fno-sanitize-recover, halt_on_error)."""
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


@pytest.fixture(scope="module")
def sanitized_refine_exe(sanitized_exe):
    objs = []
    for src in (os.path.join(ROOT, "tests", "cpp", "test_dsine_refine.cpp"),
                os.path.join(ROOT, "tests", "cpp", "no_device.cpp"),
                os.path.join(CSRC, "dsine_refine.cpp"), os.path.join(CSRC, "refiner.cpp"),
                os.path.join(CSRC, "refiner_cpu.cpp"), os.path.join(CSRC, "dsine_ops_cpu.cpp"),
                os.path.join(CSRC, "pack.cpp"), os.path.join(CSRC, "status.cpp"),
                os.path.join(CSRC, "tensor.cpp")):
        obj = os.path.join(OUT, os.path.basename(src) + ".o")
        _run(["g++", "-std=c++17", "-ffp-contract=off", "-pthread", *SAN, *HIP_HOST,
              "-I", INCLUDE, "-c", src, "-o", obj])
        objs.append(obj)
    exe = os.path.join(OUT, "test_dsine_refine_san")
    _run(["g++", *SAN, "-pthread", *objs, "-L", "/opt/rocm/lib", "-lamdhip64",
          "-Wl,-rpath,/opt/rocm/lib", "-o", exe])
    return exe


def test_host_code_under_asan_and_ubsan(sanitized_exe):
    env = dict(os.environ, ASAN_OPTIONS="halt_on_error=1:detect_leaks=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    out = _run([sanitized_exe, "cpu"], env=env, timeout=600)
    assert "OK" in out and "ERROR" not in out and "runtime error" not in out, out


def _malformed_checkpoints(tmp_path):
    """Checkpoints the reader must refuse cleanly: truncated, lying headers,
    bad JSON, deep nesting, out-of-range numbers and offsets."""
    import json
    import struct
    from tests.test_refiner_native_host import write_safetensors
    from brovisionml_amd import refiner as rf
    files = []

    def raw(name, data):
        p = str(tmp_path / name)
        with open(p, "wb") as f:
            f.write(data)
        files.append(p)

    raw("empty", b"")
    raw("short", b"\x01\x02")
    raw("len_only", struct.pack("<Q", 16))
    raw("len_huge", struct.pack("<Q", (1 << 64) - 1) + b"{}")
    raw("not_json", struct.pack("<Q", 8) + b"abcdefgh")
    raw("deep", struct.pack("<Q", 400) + b"[" * 200 + b"]" * 200)
    raw("bad_escape", struct.pack("<Q", 8) + b'{"\\q":1}')
    raw("lone_surrogate", struct.pack("<Q", 12) + b'{"\\ud800":1}')
    raw("num_tail", struct.pack("<Q", 10) + b'{"a":1e}  ')
    raw("ctrl_char", struct.pack("<Q", 8) + b'{"a\x01":1}')
    w = rf.random_weights(2)
    for name, patch in (
            ("offset_float", lambda h: h["gru.convz.bias"].update(data_offsets=[0.5, 256])),
            ("offset_huge", lambda h: h["gru.convz.bias"].update(data_offsets=[0, 1 << 62])),
            ("shape_huge", lambda h: h["gru.convz.bias"].update(shape=[1 << 41, 1 << 41])),
            ("shape_string", lambda h: h["gru.convz.bias"].update(shape=["64"])),
            ("entry_list", lambda h: h.update({"gru.convz.bias": [1, 2]})),
            ("dtype_number", lambda h: h["gru.convz.bias"].update(dtype=4))):
        p = str(tmp_path / name)
        write_safetensors(p, w, header_patch=patch)
        files.append(p)
    p = str(tmp_path / "truncated")
    write_safetensors(p, w, truncate=1000)
    files.append(p)
    p = str(tmp_path / "good")
    write_safetensors(p, w, metadata={"k": "v \u00e9"})
    files.append(p)
    assert json  # the writer's JSON is json.dumps
    return files


def test_refiner_host_code_under_asan_and_ubsan(sanitized_refine_exe, tmp_path):
    from tests.test_refiner_native_host import cpp_case
    env = dict(os.environ, ASAN_OPTIONS="halt_on_error=1:detect_leaks=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    out = _run([sanitized_refine_exe, "errors"], env=env, timeout=600)
    assert "OK" in out and "ERROR" not in out and "runtime error" not in out, out
    wpath, cpath, *_ = cpp_case(tmp_path, H=6, W=5)
    out = _run([sanitized_refine_exe, "run", "cpu", wpath, cpath, str(tmp_path / "o.bin")],
               env=env, timeout=600)
    assert "OK" in out and "ERROR" not in out and "runtime error" not in out, out
    files = _malformed_checkpoints(tmp_path)
    out = _run([sanitized_refine_exe, "parse", *files], env=env, timeout=600)
    assert "ERROR" not in out and "runtime error" not in out, out
    lines = out.strip().splitlines()
    assert lines[-2].endswith("good: ok"), out
    assert all(": dsine::Refiner: " in line for line in lines[:-2]), out
