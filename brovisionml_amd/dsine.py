"""Python mirror of brovisionml's DSINE op interface on HIP device tensors.

Same names, argument meaning and error behaviour as the C++ entry points in
include/brovisionml/dsine_ops.h (the reference's
include/brovisionml/dsine_ops.h:19-54):

  ray_relu(normal, ray, H, W)                    in place
  angmf_propagate(pred_norm, prob, xy, angle, ray, fu, cu, fv, cv, H, W, out)

and the refiner's post-propagate step (src/dsine_refine.cpp:276-282), whose
reference is brotensor's convex_upsample_forward + l2_normalize_nchw_forward:

  convex_upsample(x, mask, N, C, H, W, scale, out)
  convex_upsample_normalize(x, mask, N, C, H, W, scale, eps, out)   fused

Tensors are torch tensors (torch is only the allocator and stream provider
here), fp32, contiguous, in the reference's NCHW layout:
(1, C*H*W), (C, H, W), or batched (B, C, H, W) / (B, C*H*W).  A batch of B
samples is inferred from pred_norm / normal; the window size k from prob.
`ray` may hold one map (3*H*W, shared) or one per sample.

ray_relu and angmf_propagate dispatch on the tensors' device as the
reference's public dispatch does (src/dsine_ops.cpp:178-215): CPU tensors run
the library's CPU branch (double precision in the reference's operation
order, equal to the reference CPU twin bit for bit), tensors on the GPU the
gfx950 kernels.  The convex upsample replaces brotensor's GPU kernels only:
CPU tensors raise.

Errors raise RuntimeError with the reference's "dsine ops: " prefix
(src/dsine_ops.cpp:18-22).
"""
from __future__ import annotations

import math

from . import _lib

_WHO = "dsine ops: "


def _fail(msg: str):
    raise RuntimeError(_WHO + msg)


def _check_tensors(op: str, tensors, cpu_ok: bool = False) -> None:
    dev = tensors[0].device
    for t in tensors[1:]:
        if t.device != dev:
            if op == "ray_relu":
                _fail("ray_relu: normal and ray must share a device")
            if op.startswith("convex_upsample"):
                _fail(f"{op}: x and mask must share a device")
            _fail(f"{op}: all inputs must share a device")
    if dev.type == "cpu" and not cpu_ok:
        _fail(f"{op}: tensors are on the CPU; this op replaces brotensor's GPU kernels only")
    if dev.type not in ("cpu", "cuda"):
        _fail(f"{op}: tensors on a device this library does not run (CPU and the HIP GPU only)")
    import torch
    for t in tensors:
        if t.dtype != torch.float32:
            _fail(f"{op}: tensors must be float32")
        if not t.is_contiguous():
            _fail(f"{op}: tensors must be contiguous")


def _stream_of(t) -> int:
    import torch
    return torch.cuda.current_stream(t.device).cuda_stream


def _ray_stride(op: str, ray, B: int, HW: int) -> int:
    if ray.numel() == 3 * HW:
        return 0
    if ray.numel() == 3 * HW * B:
        return 3 * HW
    _fail(f"{op}: ray must hold 3*H*W or B*3*H*W elements")


def _raise_status(op: str, status: int) -> None:
    if status != _lib.OK:
        _fail(f"{op}: {_lib.last_error()} (status {status})")


def ray_relu(normal, ray, H: int, W: int) -> None:
    """RayReLU (eps 1e-2) in place on `normal` (src/dsine_ops.cpp:55-76)."""
    _check_tensors("ray_relu", [normal, ray], cpu_ok=True)
    HW = H * W
    if HW == 0:
        return
    if normal.numel() % (3 * HW):
        _fail("ray_relu: normal must hold B*3*H*W elements")
    B = normal.numel() // (3 * HW)
    bstride = _ray_stride("ray_relu", ray, B, HW)
    if normal.device.type == "cpu":
        _raise_status("ray_relu", _lib.ray_relu_cpu_f32(normal.data_ptr(), ray.data_ptr(), B, H,
                                                        W, bstride))
        return
    with _device(normal):
        st = _lib.ray_relu_f32(normal.data_ptr(), ray.data_ptr(), B, H, W, bstride,
                               _stream_of(normal))
    _raise_status("ray_relu", st)


def angmf_propagate(pred_norm, prob, xy, angle, ray, fu: float, cu: float,
                    fv: float, cv: float, H: int, W: int, out=None, *,
                    precise: bool = False, logits: bool = False):
    """Fused AngMF propagate (src/dsine_ops.cpp:78-172).  Returns `out`
    (allocated like pred_norm when None; must not alias any input).
    precise=True runs the double-precision kernel.  ray=None forms each
    pixel's ray from fu, cu, fv, cv in the kernel, bit-identical to
    build_ray8 (src/dsine_decoder.cpp:242-293).  logits=True takes prob and
    angle as the heads' raw logits and applies the refiner's activations
    (src/dsine_refine.cpp:262-267: sigmoid, and sigmoid * pi) in the kernel.
    CPU tensors run the CPU branch, which is double precision in the
    reference's order whatever `precise` says."""
    _check_tensors("angmf_propagate", [pred_norm, prob, xy, angle] + ([] if ray is None else [ray]),
                   cpu_ok=True)
    import torch
    HW = H * W
    if out is None:
        out = torch.empty_like(pred_norm)
    elif out.device != pred_norm.device or out.dtype != pred_norm.dtype \
            or not out.is_contiguous() or out.numel() != pred_norm.numel():
        _fail("angmf_propagate: out must match pred_norm's device, dtype and size")
    if HW == 0:
        return out
    if pred_norm.numel() % (3 * HW):
        _fail("angmf_propagate: pred_norm must hold B*3*H*W elements")
    B = pred_norm.numel() // (3 * HW)
    if B == 0:
        return out
    if prob.numel() % (B * HW):
        _fail("angmf_propagate: prob must hold B*k*k*H*W elements")
    K2 = prob.numel() // (B * HW)
    k = math.isqrt(K2)
    if k * k != K2:
        _fail("angmf_propagate: prob channel count is not a square")
    if xy.numel() != 2 * K2 * B * HW or angle.numel() != K2 * B * HW:
        _fail("angmf_propagate: xy must hold 2*k*k and angle k*k planes per sample")
    bstride = 0 if ray is None else _ray_stride("angmf_propagate", ray, B, HW)
    flags = _lib.FP64 if precise else _lib.DEFAULT
    if ray is None:
        flags |= _lib.RAY_FROM_INTRINSICS
    if logits:
        flags |= _lib.LOGITS
    if pred_norm.device.type == "cpu":
        st = _lib.angmf_propagate_cpu_f32(
            pred_norm.data_ptr(), prob.data_ptr(), xy.data_ptr(), angle.data_ptr(),
            0 if ray is None else ray.data_ptr(), float(fu), float(cu), float(fv), float(cv),
            B, H, W, k, bstride, out.data_ptr(), flags)
        _raise_status("angmf_propagate", st)
        return out
    with _device(pred_norm):
        st = _lib.angmf_propagate_f32(
            pred_norm.data_ptr(), prob.data_ptr(), xy.data_ptr(), angle.data_ptr(),
            0 if ray is None else ray.data_ptr(), float(fu), float(cu), float(fv), float(cv),
            B, H, W, k, bstride, out.data_ptr(), flags, _stream_of(pred_norm))
    _raise_status("angmf_propagate", st)
    return out


def _upsample(op: str, x, mask, N: int, C: int, H: int, W: int, scale: int, out,
              normalize: bool, eps: float, precise: bool, mask_bias=None):
    _check_tensors(op, [x, mask] + ([] if mask_bias is None else [mask_bias]))
    import torch
    if min(N, C, H, W) < 0 or scale < 1:
        _fail(f"{op}: N, C, H and W must be >= 0 and scale >= 1")
    HW = H * W
    if x.numel() != N * C * HW:
        _fail(f"{op}: x holds {x.numel()} elements, expected N*C*H*W = {N * C * HW}")
    if mask.numel() != N * 9 * scale * scale * HW:
        _fail(f"{op}: mask holds {mask.numel()} elements, expected N*9*scale^2*H*W")
    if mask_bias is not None and mask_bias.numel() != 9 * scale * scale:
        _fail(f"{op}: mask_bias holds {mask_bias.numel()} elements, expected 9*scale^2")
    n_out = N * C * scale * scale * HW
    if out is None:
        out = torch.empty((N, C, scale * H, scale * W), dtype=torch.float32, device=x.device)
    elif out.device != x.device or out.dtype != torch.float32 or not out.is_contiguous() \
            or out.numel() != n_out:
        _fail(f"{op}: out must be a contiguous float32 tensor of N*C*(scale*H)*(scale*W) "
              "elements on x's device")
    if n_out == 0:
        return out
    flags = _lib.FP64 if precise else _lib.DEFAULT
    with _device(x):
        st = _lib.convex_upsample_bias_f32(x.data_ptr(), mask.data_ptr(),
                                           0 if mask_bias is None else mask_bias.data_ptr(),
                                           N, C, H, W, scale, normalize, float(eps),
                                           out.data_ptr(), flags, _stream_of(x))
    _raise_status(op, st)
    return out


def convex_upsample(x, mask, N: int, C: int, H: int, W: int, scale: int = 8, out=None, *,
                    precise: bool = False, mask_bias=None):
    """Convex upsample by `scale` with a 9-tap softmax mask: brotensor's
    convex_upsample_forward as the refiner calls it (src/dsine_refine.cpp:278,
    arithmetic of include/brovisionml/dsine_refine.h:91-97).  x (N, C, H, W),
    mask (N, 9*scale^2, H, W), mask_bias an optional (9*scale^2,) per-channel
    bias added to the mask; returns out (N, C, scale*H, scale*W)."""
    return _upsample("convex_upsample", x, mask, N, C, H, W, scale, out, False, 0.0, precise,
                     mask_bias)


def convex_upsample_normalize(x, mask, N: int, C: int, H: int, W: int, scale: int = 8,
                              eps: float = 1e-12, out=None, *, precise: bool = False,
                              mask_bias=None):
    """convex_upsample followed by the channel L2-normalise with eps, fused:
    the pair the refiner runs after each propagate (src/dsine_refine.cpp:276-282,
    l2_normalize_nchw_forward with eps 1e-12f)."""
    return _upsample("convex_upsample_normalize", x, mask, N, C, H, W, scale, out, True, eps,
                     precise, mask_bias)


def build_ray8(fu: float, cu: float, fv: float, cv: float, H: int, W: int, device=None):
    """The (3, H, W) fp32 ray map of build_ray8 (src/dsine_decoder.cpp:242-293)
    from the grid-scaled intrinsics, formed on the device."""
    import torch
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    ray = torch.empty((3, H, W), dtype=torch.float32, device=dev)
    if H * W == 0:
        return ray
    with _device(ray):
        st = _lib.build_ray8_f32(ray.data_ptr(), float(fu), float(cu), float(fv), float(cv), H, W,
                                 _stream_of(ray))
    _raise_status("build_ray8", st)
    return ray


def _maps(op: str, C: int, HW: int, **tensors) -> None:
    """Every tensor a contiguous float32 map of C*HW floats (or C for a
    bias) on one HIP device."""
    import torch
    dev = None
    for name, t in tensors.items():
        want = C if name.startswith("bias") else C * HW
        if t.device.type != "cuda":
            _fail(f"{op}: {name} is not on a HIP device")
        if dev is not None and t.device != dev:
            _fail(f"{op}: all tensors must share a device")
        dev = t.device
        if t.dtype != torch.float32 or not t.is_contiguous():
            _fail(f"{op}: {name} must be a contiguous float32 tensor")
        if t.numel() != want:
            _fail(f"{op}: {name} holds {t.numel()} elements, expected {want}")


def gru_gates(zr, bias_z, bias_r, h, C: int, HW: int, z, rh) -> None:
    """The ConvGRU's gates (src/dsine_refine.cpp:149-151) after one
    convolution of convz and convr stacked, without bias: zr holds 2*C planes
    (convz's, then convr's); writes z = sigmoid(zr[:C] + bias_z) and
    rh = sigmoid(zr[C:] + bias_r) * h.  Tensors may be channel slices of
    larger maps as long as each is contiguous."""
    _maps("gru_gates", C, HW, h=h, z=z, rh=rh, bias_z=bias_z, bias_r=bias_r)
    _maps("gru_gates", 2 * C, HW, zr=zr)
    with _device(zr):
        st = _lib.gru_gates_f32(zr.data_ptr(), bias_z.data_ptr(), bias_r.data_ptr(), h.data_ptr(),
                                C, HW, z.data_ptr(), rh.data_ptr(), _stream_of(zr))
    _raise_status("gru_gates", st)


def gru_update(q_pre, bias_q, z, h, C: int, HW: int, h_new, h_copy=None) -> None:
    """h_new = (1 - z) h + z tanh(q_pre + bias_q) (src/dsine_refine.cpp:
    152-157), also into h_copy when given; h_new may be h."""
    extra = {} if h_copy is None else {"h_copy": h_copy}
    _maps("gru_update", C, HW, q_pre=q_pre, z=z, h=h, h_new=h_new, bias_q=bias_q, **extra)
    with _device(q_pre):
        st = _lib.gru_update_f32(q_pre.data_ptr(), bias_q.data_ptr(), z.data_ptr(), h.data_ptr(),
                                 C, HW, h_new.data_ptr(),
                                 0 if h_copy is None else h_copy.data_ptr(), _stream_of(q_pre))
    _raise_status("gru_update", st)


def bias_act(x, bias, C: int, HW: int, relu: bool) -> None:
    """x = x + bias (per channel), then ReLU if relu, in place: a
    convolution's bias and the head's relu_forward (src/dsine_refine.cpp:
    119-127) in one pass."""
    _maps("bias_act", C, HW, x=x, bias=bias)
    with _device(x):
        st = _lib.bias_act_f32(x.data_ptr(), bias.data_ptr(), C, HW, relu, _stream_of(x))
    _raise_status("bias_act", st)


class _device:
    """Make the tensor's device current for the launch."""

    def __init__(self, t):
        self.t = t

    def __enter__(self):
        import torch
        self.ctx = torch.cuda.device(self.t.device)
        self.ctx.__enter__()

    def __exit__(self, *exc):
        self.ctx.__exit__(*exc)
