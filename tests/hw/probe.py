"""ctypes binding of tests/hw/_build/libbvml_probe.so (built by
__graft_entry__.build() from tests/hw/probe.hip): hardware-function error
sweeps and a streaming-read kernel.  Test and measurement infrastructure."""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libbvml_probe.so")
OPS = {"sin": 0, "cos": 1, "rsq": 2, "rcp": 3, "exp2": 4, "sqrt": 5}

_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} missing: run __graft_entry__.build()")
        lib = ctypes.CDLL(LIB)
        d, f, i, vp, sz = ctypes.c_double, ctypes.c_float, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
        lib.bvml_probe_hw_error.argtypes = [i, f, f, i, ctypes.POINTER(d), ctypes.POINTER(d),
                                            ctypes.POINTER(f)]
        lib.bvml_probe_hw_error.restype = i
        lib.bvml_probe_stream_read.argtypes = [vp, sz, i, vp, sz, vp]
        lib.bvml_probe_stream_read.restype = i
        lib.bvml_probe_read_partials.argtypes = [sz, i]
        lib.bvml_probe_read_partials.restype = sz
        lib.bvml_probe_angmf_loop.argtypes = [vp, ctypes.POINTER(ctypes.c_ulonglong), i, d, d, d, d,
                                              i, i, i, i, ctypes.c_uint, d, vp,
                                              ctypes.POINTER(f)]
        lib.bvml_probe_angmf_loop.restype = i
        _lib = lib
    return _lib


def hw_error(op: str, lo: float, hi: float, negative: bool = False):
    """(max abs error, max relative error, argument of the latter) of the
    hardware function over every float of magnitude in [lo, hi]."""
    a, r, g = ctypes.c_double(), ctypes.c_double(), ctypes.c_float()
    st = load().bvml_probe_hw_error(OPS[op], lo, hi, int(negative), ctypes.byref(a),
                                    ctypes.byref(r), ctypes.byref(g))
    if st != 0:
        raise RuntimeError(f"bvml_probe_hw_error failed: {st}")
    return a.value, r.value, g.value


def stream_read(ptr: int, n: int, unroll: int, out_ptr: int, out_len: int,
                stream: int = 0) -> None:
    """One streaming read of n floats at ptr (unroll float4 loads per lane);
    per-wave partial sums into out (out_len floats)."""
    st = load().bvml_probe_stream_read(ptr, n, unroll, out_ptr, out_len, stream)
    if st != 0:
        raise RuntimeError(f"bvml_probe_stream_read failed: {st}")


def read_partials(n: int, unroll: int) -> int:
    return load().bvml_probe_read_partials(n, unroll)


def angmf_loop(fn_ptr: int, ptrs, intr, B: int, H: int, W: int, k: int, flags: int,
               spin_us: float, stream: int = 0) -> float:
    """Seconds for len(ptrs) calls of the angmf_propagate_f32 entry point at
    fn_ptr enqueued back to back from C++ (call i on the six pointers
    ptrs[i]: pred_norm, prob, xy, angle, ray, out), timed by events after a
    spin of spin_us microseconds that holds the stream while they are
    enqueued."""
    flat = (ctypes.c_ulonglong * (6 * len(ptrs)))(*[int(p) for row in ptrs for p in row])
    ms = ctypes.c_float()
    fu, cu, fv, cv = intr
    st = load().bvml_probe_angmf_loop(fn_ptr, flat, len(ptrs), fu, cu, fv, cv, B, H, W, k, flags,
                                      spin_us, stream, ctypes.byref(ms))
    if st != 0:
        raise RuntimeError(f"bvml_probe_angmf_loop failed: {st}")
    return ms.value * 1e-3
