"""ctypes binding of the C ABI declared in include/bvml_dsine.h.

The library is the in-tree build product brovisionml_amd/lib/libbvml_dsine.so.
There is no fallback: if it is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

from .build import LIB, LIB_REFINE

# Status codes (include/bvml_dsine.h)
OK = 0
ENULL = -1
ESHAPE = -2
EK = -3
ESIZE = -4
EALIAS = -5
EFLAGS = -6
EPARAM = -7
EUNSUP = -8

DEFAULT = 0
FP64 = 1
RAY_FROM_INTRINSICS = 2
LOGITS = 4

# Every symbol include/bvml_dsine.h declares.
EXPORTS = (
    "bvml_dsine_ray_relu_f32",
    "bvml_dsine_angmf_propagate_f32",
    "bvml_dsine_build_ray8_f32",
    "bvml_dsine_build_uv8_f32",
    "bvml_dsine_convex_upsample_f32",
    "bvml_dsine_convex_upsample_bias_f32",
    "bvml_dsine_angmf_recompute_ratio",
    "bvml_dsine_angmf_plan",
    "bvml_dsine_ray_relu_cpu_f32",
    "bvml_dsine_angmf_propagate_cpu_f32",
    "bvml_dsine_gru_gates_f32",
    "bvml_dsine_gru_update_f32",
    "bvml_dsine_bias_act_f32",
    "bvml_dsine_heads_mlp_f32",
    "bvml_dsine_heads_pack_f32",
    "bvml_dsine_heads_packed_size",
    "bvml_dsine_conv_packed_size",
    "bvml_dsine_conv_pack_f32",
    "bvml_dsine_conv_f32",
    "bvml_dsine_conv_gru_gates_f32",
    "bvml_dsine_conv_gru_update_f32",
    "bvml_dsine_conv_gru_gates_sum_f32",
    "bvml_dsine_conv_gru_update_sum_f32",
    "bvml_dsine_conv_heads_f32",
    "bvml_dsine_last_error",
    "bvml_dsine_version",
)

# Every symbol include/bvml_dsine_refine.h declares.
REFINE_EXPORTS = (
    "bvml_dsine_refiner_create",
    "bvml_dsine_refiner_destroy",
    "bvml_dsine_refiner_load_file",
    "bvml_dsine_refiner_set_tensor",
    "bvml_dsine_refiner_tensor_numel",
    "bvml_dsine_refiner_get_tensor",
    "bvml_dsine_refiner_forward",
    "bvml_dsine_refiner_forward_cpu",
    "bvml_dsine_refiner_forward_noalloc",
    "bvml_dsine_refiner_last_error",
)
EWEIGHTS = -9
EFILE = -10
ELIB = -11

_lib = None
_refine = None


def load(path: str = LIB) -> ctypes.CDLL:
    """Load (once) and type the native library; raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"brovisionml_amd: native library {path} is missing; run "
            "`python -m brovisionml_amd.build` (hipcc, gfx950) first")
    lib = ctypes.CDLL(path)
    vp, i, ll, d, u = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_double, ctypes.c_uint
    lib.bvml_dsine_ray_relu_f32.argtypes = [vp, vp, i, i, i, ll, vp]
    lib.bvml_dsine_ray_relu_f32.restype = i
    lib.bvml_dsine_angmf_propagate_f32.argtypes = [
        vp, vp, vp, vp, vp, d, d, d, d, i, i, i, i, ll, vp, u, vp]
    lib.bvml_dsine_angmf_propagate_f32.restype = i
    lib.bvml_dsine_build_ray8_f32.argtypes = [vp, d, d, d, d, i, i, vp]
    lib.bvml_dsine_build_ray8_f32.restype = i
    lib.bvml_dsine_build_uv8_f32.argtypes = [vp, d, d, d, d, i, i, vp]
    lib.bvml_dsine_build_uv8_f32.restype = i
    lib.bvml_dsine_convex_upsample_f32.argtypes = [vp, vp, i, i, i, i, i, i, ctypes.c_float, vp,
                                                   u, vp]
    lib.bvml_dsine_convex_upsample_f32.restype = i
    lib.bvml_dsine_convex_upsample_bias_f32.argtypes = [vp, vp, vp, i, i, i, i, i, i,
                                                        ctypes.c_float, vp, u, vp]
    lib.bvml_dsine_convex_upsample_bias_f32.restype = i
    ip = ctypes.POINTER(ctypes.c_int)
    lib.bvml_dsine_angmf_plan.argtypes = [i, i, i, i, d, d, d, d, u, ip, ip, ip, ip]
    lib.bvml_dsine_angmf_plan.restype = i
    lib.bvml_dsine_angmf_recompute_ratio.argtypes = [i, u]
    lib.bvml_dsine_angmf_recompute_ratio.restype = d
    lib.bvml_dsine_ray_relu_cpu_f32.argtypes = [vp, vp, i, i, i, ll, i]
    lib.bvml_dsine_ray_relu_cpu_f32.restype = i
    lib.bvml_dsine_angmf_propagate_cpu_f32.argtypes = [
        vp, vp, vp, vp, vp, d, d, d, d, i, i, i, i, ll, vp, u, i]
    lib.bvml_dsine_angmf_propagate_cpu_f32.restype = i
    lib.bvml_dsine_gru_gates_f32.argtypes = [vp, vp, vp, vp, i, ll, vp, vp, vp]
    lib.bvml_dsine_gru_gates_f32.restype = i
    lib.bvml_dsine_gru_update_f32.argtypes = [vp, vp, vp, vp, i, ll, vp, vp, vp]
    lib.bvml_dsine_gru_update_f32.restype = i
    lib.bvml_dsine_bias_act_f32.argtypes = [vp, vp, i, ll, i, vp]
    lib.bvml_dsine_bias_act_f32.restype = i
    pp = ctypes.POINTER(vp)
    lib.bvml_dsine_heads_mlp_f32.argtypes = [vp, vp, vp, vp, pp, pp, ip, i, i, i, pp, vp]
    lib.bvml_dsine_heads_mlp_f32.restype = i
    lib.bvml_dsine_heads_pack_f32.argtypes = [vp, pp, ip, i, vp, pp]
    lib.bvml_dsine_heads_pack_f32.restype = i
    lib.bvml_dsine_heads_packed_size.argtypes = [i]
    lib.bvml_dsine_heads_packed_size.restype = ll
    lib.bvml_dsine_conv_packed_size.argtypes = [i, i, i]
    lib.bvml_dsine_conv_packed_size.restype = ll
    lib.bvml_dsine_conv_pack_f32.argtypes = [vp, i, i, i, i, vp]
    lib.bvml_dsine_conv_pack_f32.restype = i
    lib.bvml_dsine_conv_f32.argtypes = [vp, i, i, i, vp, i, i, vp, vp]
    lib.bvml_dsine_conv_f32.restype = i
    lib.bvml_dsine_conv_gru_gates_f32.argtypes = [vp, i, i, i, vp, i, vp, vp, vp, vp, vp, vp]
    lib.bvml_dsine_conv_gru_gates_f32.restype = i
    lib.bvml_dsine_conv_gru_update_f32.argtypes = [vp, i, i, i, vp, i, vp, vp, vp, vp, vp, vp]
    lib.bvml_dsine_conv_gru_update_f32.restype = i
    lib.bvml_dsine_conv_gru_gates_sum_f32.argtypes = [vp, i, i, i, vp, i, vp, vp, vp, vp, vp, vp,
                                                      vp]
    lib.bvml_dsine_conv_gru_gates_sum_f32.restype = i
    lib.bvml_dsine_conv_gru_update_sum_f32.argtypes = [vp, i, i, i, vp, i, vp, vp, vp, vp, vp, vp,
                                                       vp]
    lib.bvml_dsine_conv_gru_update_sum_f32.restype = i
    lib.bvml_dsine_conv_heads_f32.argtypes = [vp, i, i, i, vp, i, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.bvml_dsine_conv_heads_f32.restype = i
    lib.bvml_dsine_last_error.argtypes = []
    lib.bvml_dsine_last_error.restype = ctypes.c_char_p
    lib.bvml_dsine_version.argtypes = []
    lib.bvml_dsine_version.restype = ctypes.c_char_p
    _lib = lib
    return lib


def load_refine(path: str = LIB_REFINE) -> ctypes.CDLL:
    """Load (once) and type the native refiner library (include/bvml_dsine_refine.h);
    raises if it was not built."""
    global _refine
    if _refine is not None:
        return _refine
    load()
    if not os.path.exists(path):
        raise RuntimeError(
            f"brovisionml_amd: native library {path} is missing; run "
            "`python -m brovisionml_amd.build` first")
    lib = ctypes.CDLL(path)
    vp, i, ll, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float
    lib.bvml_dsine_refiner_create.argtypes = [ctypes.POINTER(vp)]
    lib.bvml_dsine_refiner_create.restype = i
    lib.bvml_dsine_refiner_destroy.argtypes = [vp]
    lib.bvml_dsine_refiner_destroy.restype = None
    lib.bvml_dsine_refiner_load_file.argtypes = [vp, ctypes.c_char_p]
    lib.bvml_dsine_refiner_load_file.restype = i
    lib.bvml_dsine_refiner_set_tensor.argtypes = [vp, ctypes.c_char_p, vp, ll]
    lib.bvml_dsine_refiner_set_tensor.restype = i
    lib.bvml_dsine_refiner_tensor_numel.argtypes = [ctypes.c_char_p]
    lib.bvml_dsine_refiner_tensor_numel.restype = ll
    lib.bvml_dsine_refiner_get_tensor.argtypes = [vp, ctypes.c_char_p, vp, ll]
    lib.bvml_dsine_refiner_get_tensor.restype = i
    lib.bvml_dsine_refiner_forward.argtypes = [vp, vp, vp, vp, i, i, f, f, f, f, i, i, i, i, i, i,
                                               vp, vp, vp]
    lib.bvml_dsine_refiner_forward.restype = i
    lib.bvml_dsine_refiner_forward_cpu.argtypes = [vp, vp, vp, vp, i, i, f, f, f, f, i, i, i, i,
                                                   i, i, vp, vp, i]
    lib.bvml_dsine_refiner_forward_cpu.restype = i
    lib.bvml_dsine_refiner_forward_noalloc.argtypes = lib.bvml_dsine_refiner_forward.argtypes
    lib.bvml_dsine_refiner_forward_noalloc.restype = i
    lib.bvml_dsine_refiner_last_error.argtypes = []
    lib.bvml_dsine_refiner_last_error.restype = ctypes.c_char_p
    _refine = lib
    return lib


def refine_last_error() -> str:
    return load_refine().bvml_dsine_refiner_last_error().decode()


def last_error() -> str:
    return load().bvml_dsine_last_error().decode()


def ray_relu_f32(normal: int, ray: int, B: int, H: int, W: int,
                 ray_bstride: int, stream: int = 0) -> int:
    """Raw call; pointers are integer device addresses. Returns the status."""
    return load().bvml_dsine_ray_relu_f32(normal, ray, B, H, W, ray_bstride, stream)


def angmf_propagate_f32(pred_norm: int, prob: int, xy: int, angle: int, ray: int,
                        fu: float, cu: float, fv: float, cv: float,
                        B: int, H: int, W: int, k: int, ray_bstride: int,
                        out: int, flags: int = DEFAULT, stream: int = 0) -> int:
    """Raw call; pointers are integer device addresses. Returns the status."""
    return load().bvml_dsine_angmf_propagate_f32(
        pred_norm, prob, xy, angle, ray, fu, cu, fv, cv, B, H, W, k,
        ray_bstride, out, flags, stream)


def build_ray8_f32(ray: int, fu: float, cu: float, fv: float, cv: float, H: int, W: int,
                   stream: int = 0) -> int:
    """Raw call; `ray` is an integer device address of 3*H*W floats."""
    return load().bvml_dsine_build_ray8_f32(ray, fu, cu, fv, cv, H, W, stream)


def build_uv8_f32(uv: int, fu: float, cu: float, fv: float, cv: float, H: int, W: int,
                  stream: int = 0) -> int:
    """Raw call; `uv` is an integer device address of 2*H*W floats."""
    return load().bvml_dsine_build_uv8_f32(uv, fu, cu, fv, cv, H, W, stream)


def convex_upsample_f32(x: int, mask: int, B: int, C: int, H: int, W: int, scale: int,
                        normalize: bool, eps: float, out: int, flags: int = DEFAULT,
                        stream: int = 0) -> int:
    """Raw call; pointers are integer device addresses. Returns the status."""
    return load().bvml_dsine_convex_upsample_f32(x, mask, B, C, H, W, scale, int(bool(normalize)),
                                                 eps, out, flags, stream)


def convex_upsample_bias_f32(x: int, mask: int, mask_bias: int, B: int, C: int, H: int, W: int,
                             scale: int, normalize: bool, eps: float, out: int,
                             flags: int = DEFAULT, stream: int = 0) -> int:
    """Raw call with a per-channel mask bias (0 for none); pointers are
    integer device addresses. Returns the status."""
    return load().bvml_dsine_convex_upsample_bias_f32(x, mask, mask_bias, B, C, H, W, scale,
                                                      int(bool(normalize)), eps, out, flags,
                                                      stream)


def angmf_recompute_ratio(k: int, flags: int = DEFAULT) -> float:
    """The fast path's cancellation threshold at window size k: pixels with
    |acc|^2 below this times sum (prob/|p|)^2 are recomputed in double (0
    with FP64, -1 for an unsupported k)."""
    return load().bvml_dsine_angmf_recompute_ratio(k, flags)


def ray_relu_cpu_f32(normal: int, ray: int, B: int, H: int, W: int, ray_bstride: int,
                     nthreads: int = 0) -> int:
    """Raw call of the CPU branch; pointers are host addresses."""
    return load().bvml_dsine_ray_relu_cpu_f32(normal, ray, B, H, W, ray_bstride, nthreads)


def angmf_propagate_cpu_f32(pred_norm: int, prob: int, xy: int, angle: int, ray: int,
                            fu: float, cu: float, fv: float, cv: float,
                            B: int, H: int, W: int, k: int, ray_bstride: int,
                            out: int, flags: int = DEFAULT, nthreads: int = 0) -> int:
    """Raw call of the CPU branch; pointers are host addresses."""
    return load().bvml_dsine_angmf_propagate_cpu_f32(
        pred_norm, prob, xy, angle, ray, fu, cu, fv, cv, B, H, W, k, ray_bstride, out, flags,
        nthreads)


def angmf_plan_full(B: int, H: int, W: int, k: int, fu: float, cu: float, fv: float,
                    cv: float, flags: int = DEFAULT):
    """(fp32 kernel?, waves per 64-pixel group, tile width, tile height,
    non-temporal plane loads?) of the launch bvml_dsine_angmf_propagate_f32
    makes for these arguments; raises on a rejected argument."""
    g, tw, th, nt = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    st = load().bvml_dsine_angmf_plan(B, H, W, k, fu, cu, fv, cv, flags, ctypes.byref(g),
                                      ctypes.byref(tw), ctypes.byref(th), ctypes.byref(nt))
    if st < 0:
        raise RuntimeError(f"angmf_plan: {last_error()} (status {st})")
    return bool(st), g.value, tw.value, th.value, bool(nt.value)


def angmf_plan(B: int, H: int, W: int, k: int, fu: float, cu: float, fv: float, cv: float,
               flags: int = DEFAULT):
    """(fp32 kernel?, waves per 64-pixel group, tile width, tile height) of the
    launch bvml_dsine_angmf_propagate_f32 makes for these arguments; raises
    on a rejected argument."""
    return angmf_plan_full(B, H, W, k, fu, cu, fv, cv, flags)[:4]


def gru_gates_f32(zr: int, bias_z: int, bias_r: int, h: int, C: int, HW: int, z: int, rh: int,
                  stream: int = 0) -> int:
    """Raw call; pointers are integer device addresses. Returns the status."""
    return load().bvml_dsine_gru_gates_f32(zr, bias_z, bias_r, h, C, HW, z, rh, stream)


def gru_update_f32(q_pre: int, bias_q: int, z: int, h: int, C: int, HW: int, h_new: int,
                   h_copy: int = 0, stream: int = 0) -> int:
    """Raw call; pointers are integer device addresses. Returns the status."""
    return load().bvml_dsine_gru_update_f32(q_pre, bias_q, z, h, C, HW, h_new, h_copy, stream)


def heads_pack_f32(w2, w4s):
    """Host packing of the heads' 1x1 weights for bvml_dsine_heads_mlp_f32:
    w2 (nheads, 64, 64[, 1, 1]) float32, w4s a list of (outs[h], 64[, 1, 1]);
    returns (w2p, [w4p_h]) as float32 numpy arrays."""
    import numpy as np
    lib = load()
    w2 = np.ascontiguousarray(np.asarray(w2, np.float32).reshape(-1, 64, 64))
    nh = w2.shape[0]
    w4s = [np.ascontiguousarray(np.asarray(w, np.float32).reshape(-1, 64)) for w in w4s]
    outs = (ctypes.c_int * nh)(*[w.shape[0] for w in w4s])
    w2p = np.empty(nh * 4096, np.float32)
    w4p = [np.empty(lib.bvml_dsine_heads_packed_size(w.shape[0]), np.float32) for w in w4s]
    vp = ctypes.c_void_p
    st = lib.bvml_dsine_heads_pack_f32(w2.ctypes.data, (vp * nh)(*[w.ctypes.data for w in w4s]),
                                       outs, nh, w2p.ctypes.data,
                                       (vp * nh)(*[w.ctypes.data for w in w4p]))
    if st != OK:
        raise RuntimeError(f"heads_pack: {last_error()} (status {st})")
    return w2p, w4p


def heads_mlp_f32(t0: int, b0: int, w2p: int, b2: int, w4p, b4, outs, H: int, W: int, out,
                  stream: int = 0) -> int:
    """Raw call; pointers are integer device addresses, w4p / b4 / out lists
    of them (0 in b4 for no bias), outs the output counts. Returns the status."""
    vp = ctypes.c_void_p
    nh = len(outs)
    return load().bvml_dsine_heads_mlp_f32(
        t0, b0, w2p, b2, (vp * nh)(*w4p), (vp * nh)(*[b or None for b in b4]),
        (ctypes.c_int * nh)(*outs), nh, H, W, (vp * nh)(*out), stream)


def heads_w2q_f32(w2):
    """Each head's middle-layer weights (nheads, 64, 64[, 1, 1]) in the
    last-layer layout bvml_dsine_conv_heads_f32 reads (W2 packed as a
    64-output last layer), back to back; a float32 numpy array."""
    import numpy as np
    w2 = np.asarray(w2, np.float32).reshape(-1, 64, 64)
    return np.concatenate(heads_pack_f32(w2, list(w2))[1])


def conv_heads_f32(x: int, cin: int, H: int, W: int, wp: int, b0: int, w2q: int, b2: int, w4p,
                   b4, outs, out, stream: int = 0) -> int:
    """Raw call of bvml_dsine_conv_heads_f32; pointers are integer device
    addresses, w4p / b4 / out lists of them (0 in b4 for no bias), outs the
    output counts. Returns the status."""
    vp = ctypes.c_void_p
    nh = len(outs)
    return load().bvml_dsine_conv_heads_f32(
        x, cin, H, W, wp, nh, b0, w2q, b2, (vp * nh)(*w4p), (vp * nh)(*[b or None for b in b4]),
        (ctypes.c_int * nh)(*outs), (vp * nh)(*out), stream)


def conv_pack_f32(w, interleave: bool = False):
    """Host packing of OIHW conv weights (cout, cin, k, k) for the
    bvml_dsine_conv_* kernels; returns a float32 numpy array."""
    import numpy as np
    w = np.ascontiguousarray(np.asarray(w, np.float32))
    cout, cin, k, _ = w.shape
    lib = load()
    n = lib.bvml_dsine_conv_packed_size(cout, cin, k)
    if n < 0:
        raise RuntimeError("conv_pack: unsupported shape")
    wp = np.empty(n, np.float32)
    st = lib.bvml_dsine_conv_pack_f32(w.ctypes.data, cout, cin, k, int(bool(interleave)),
                                      wp.ctypes.data)
    if st != OK:
        raise RuntimeError(f"conv_pack: {last_error()} (status {st})")
    return wp


def bias_act_f32(x: int, bias: int, C: int, HW: int, relu: bool, stream: int = 0) -> int:
    """Raw call; pointers are integer device addresses. Returns the status."""
    return load().bvml_dsine_bias_act_f32(x, bias, C, HW, int(bool(relu)), stream)
