"""DSINE NRN refiner on the HIP device: the 5-iteration loop of brovisionml's
Refiner::forward (src/dsine_refine.cpp:212-294; the spec comment at
include/brovisionml/dsine_refine.h:1-111), driving this package's kernels.

Per iteration (src/dsine_refine.cpp:255-287):
  h_new     = ConvGRU(h, feat_map)                 convz/convr/convq 5x5, 130 -> 64
  hin       = cat(h_new, uv_8)                      66 channels
  prob, xy, angle = the three heads on hin          (25, 50, 25 channels)
  pred_norm = angmf_propagate(pred_norm, sigmoid(prob), xy, sigmoid(angle)*pi, ray_8)
  up        = normalize(convex_upsample(pred_norm, up_prob_head(hin)))
  h         = h_new
after pred_norm = RayReLU(decoder.normal, ray_8) and feat_map = cat(decoder.feature,
uv_8).  The result is the last iteration's up-sampled normals, cropped to the
unpadded image.

What runs where:
  * RayReLU, the propagate and the convex upsample + normalise are the
    package's gfx950 kernels (C ABI in include/bvml_dsine.h); the propagate
    takes the heads' raw logits and applies the activations itself
    (BVML_DSINE_LOGITS), so the two activation passes of :262-267 are gone;
    the upsample fuses convex_upsample_forward and l2_normalize_nchw_forward
    (:278-282); the ray map comes from bvml_dsine_build_ray8_f32 on the device.
  * The ConvGRU and the heads' convolutions (the reference's brotensor
    conv2d_forward, :94-101) are torch's F.conv2d in fp32 and without bias,
    with MIOpen switched off, so torch runs them as im2col + an fp32 GEMM: a
    fixed algorithm per shape, the same rounding in every process (MIOpen
    picks its algorithm by estimated or measured time, which changes with
    the process's history, and its Winograd kernels round differently from a
    direct sum); their biases, activations and the GRU's
    gate arithmetic run in the package's fused elementwise kernels
    (bvml_dsine_gru_gates_f32, bvml_dsine_gru_update_f32,
    bvml_dsine_bias_act_f32), the up-mask head's last bias in the upsample
    (bvml_dsine_convex_upsample_bias_f32).

Weights are the checkpoint's top-level tensors gru.conv{z,r,q}.{weight,bias}
and {prob,xy,angle,up_prob}_head.{0,2,4}.{weight,bias} (:161-180), loaded
from a safetensors file or drawn at random for synthetic runs (no checkpoint
ships in this environment).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from . import dsine, workloads

K_UP = 8            # downsample_ratio (src/dsine_refine.cpp:24)
N_ITER = 5          # num_iter_test (:25)
PS = 5              # the propagate's window (:24 of src/dsine_ops.cpp)
K_PI = float(np.float32(3.14159265358979323846))  # the float kPi (:26)
HEAD_OUT = {"prob_head": PS * PS, "xy_head": 2 * PS * PS, "angle_head": PS * PS,
            "up_prob_head": 9 * K_UP * K_UP}


@dataclass
class DecoderOutput:
    """The decoder's /8-grid maps (include/brovisionml/dsine_decoder.h:96-102):
    normal (1, 3, h8, w8) unit normals, feature (1, 64, h8, w8), hidden
    (1, 64, h8, w8); fp32 tensors on the device."""
    normal: object
    feature: object
    hidden: object


@dataclass(frozen=True)
class Crop:
    """The part of DsineTransform the refiner uses
    (include/brovisionml/dsine_preprocess.h:48-57): the unpadded size and the
    top/left padding."""
    orig_h: int
    orig_w: int
    pad_t: int = 0
    pad_l: int = 0


def weight_shapes(hidden: int = 64, feature: int = 64) -> dict:
    """Checkpoint tensor name -> shape (OIHW weights, (C_out,) biases)."""
    inp = feature + 2          # feat_map = cat(feature, uv_8)
    shapes = {}
    for g in ("convz", "convr", "convq"):
        shapes[f"gru.{g}.weight"] = (hidden, hidden + inp, 5, 5)
        shapes[f"gru.{g}.bias"] = (hidden,)
    for head, out in HEAD_OUT.items():
        for idx, (ci, co, k) in zip((0, 2, 4), ((hidden + 2, 64, 3), (64, 64, 1), (64, out, 1))):
            shapes[f"{head}.{idx}.weight"] = (co, ci, k, k)
            shapes[f"{head}.{idx}.bias"] = (co,)
    return shapes


def random_weights(seed: int, hidden: int = 64, feature: int = 64) -> dict:
    """Synthetic weights: uniform(-1/sqrt(fan_in), 1/sqrt(fan_in)) for each
    convolution's weight and bias (torch's default initialisation bound), as
    float32 numpy arrays."""
    rng = np.random.default_rng(seed)
    shapes = weight_shapes(hidden, feature)
    out = {}
    for name, shape in shapes.items():
        conv = name.rsplit(".", 1)[0]
        bound = 1.0 / math.sqrt(math.prod(shapes[conv + ".weight"][1:]))
        out[name] = rng.uniform(-bound, bound, shape).astype(np.float32)
    return out


def load_safetensors(path: str) -> dict:
    """The checkpoint's refiner tensors as float32 numpy arrays, weights
    reshaped to OIHW (the reference stores (C_out, C_in*k*k) as well)."""
    from safetensors.numpy import load_file
    raw = load_file(path)
    shapes = weight_shapes()
    out = {}
    for name, shape in shapes.items():
        if name not in raw:
            raise RuntimeError(f"dsine::Refiner: missing tensor '{name}'")
        out[name] = np.asarray(raw[name], np.float32).reshape(shape)
    return out


def uv_map(intr: workloads.Intrinsics, H: int, W: int, orig_h: int, orig_w: int):
    """build_uv (src/dsine_decoder.cpp:242-274): ray_x, ray_y on the (H, W)
    grid, double arithmetic rounded to float; (2, H, W) float32 numpy."""
    fu, cu, fv, cv = workloads.scaled_intrinsics(intr, H, W, orig_h, orig_w)
    x = np.arange(W, dtype=np.float64)
    y = np.arange(H, dtype=np.float64)
    rx = (((x + 0.5) - cu) / fu).astype(np.float32)
    ry = (((y + 0.5) - cv) / fv).astype(np.float32)
    return np.stack([np.broadcast_to(rx, (H, W)), np.broadcast_to(ry[:, None], (H, W))])


class Refiner:
    """Refiner::forward on the device.  `weights` as weight_shapes() names
    them (numpy or torch); hidden / feature are the checkpoint's widths.

    The convolutions run without their bias as torch's F.conv2d with MIOpen
    off (im2col + an fp32 GEMM, the same algorithm in every process): convz
    and convr as one 2*hidden-channel convolution, the four
    heads' first 3x3 convolutions as one, their 1x1 middle convolutions as one
    grouped convolution.  Biases, activations and the gate arithmetic run in
    this package's fused kernels (bvml_dsine_gru_gates_f32,
    bvml_dsine_gru_update_f32, bvml_dsine_bias_act_f32), which write into the
    channel slices of persistent [h | feature | uv], [r*h | feature | uv] and
    [h_new | uv] maps, so no concatenation is materialised per iteration."""

    def __init__(self, weights: dict, device, hidden: int = 64, feature: int = 64):
        import torch
        self.device = torch.device(device)
        self.hidden, self.feature = hidden, feature
        shapes = weight_shapes(hidden, feature)
        self.w = {}
        for name, shape in shapes.items():
            t = torch.as_tensor(np.asarray(weights[name], np.float32)).reshape(shape)
            self.w[name] = t.to(self.device).contiguous()
        w = self.w
        heads = list(HEAD_OUT)
        self.w_zr = torch.cat([w["gru.convz.weight"], w["gru.convr.weight"]]).contiguous()
        self.b_z, self.b_r = w["gru.convz.bias"], w["gru.convr.bias"]
        self.w_q, self.b_q = w["gru.convq.weight"], w["gru.convq.bias"]
        self.w_h0 = torch.cat([w[f"{h}.0.weight"] for h in heads]).contiguous()
        self.b_h0 = torch.cat([w[f"{h}.0.bias"] for h in heads]).contiguous()
        self.w_h2 = torch.cat([w[f"{h}.2.weight"] for h in heads]).contiguous()
        self.b_h2 = torch.cat([w[f"{h}.2.bias"] for h in heads]).contiguous()
        self.heads = heads

    def conditioning(self, intr: workloads.Intrinsics, H: int, W: int, orig_h: int, orig_w: int):
        """(ray_8, uv_8, (fu, cu, fv, cv)) on the device for an (H, W) grid: the
        ray map from bvml_dsine_build_ray8_f32, the uv map from build_uv."""
        import torch
        fuv = workloads.scaled_intrinsics(intr, H, W, orig_h, orig_w)
        ray8 = dsine.build_ray8(*fuv, H, W, device=self.device)
        uv8 = torch.from_numpy(np.ascontiguousarray(uv_map(intr, H, W, orig_h, orig_w)))
        return ray8, uv8.to(self.device)[None], fuv

    def _heads(self, hin, H: int, W: int):
        """The four get_prediction_head stacks (src/dsine_refine.cpp:119-127)
        on hin: (prob, xy, angle, up_mask) logits, up_mask without its last
        layer's bias (the upsample adds it)."""
        import torch.nn.functional as F
        nh = len(self.heads)
        t = F.conv2d(hin, self.w_h0, None, padding=1)
        dsine.bias_act(t, self.b_h0, nh * 64, H * W, relu=True)
        t = F.conv2d(t, self.w_h2, None, groups=nh)
        dsine.bias_act(t, self.b_h2, nh * 64, H * W, relu=True)
        # the up-mask head's last layer runs without its bias: the upsample
        # adds it to the mask as it loads it (one fp32 add per value, as the
        # bias pass would round it), so the 576 planes are not read and
        # written once more
        return [F.conv2d(t[:, 64 * i:64 * (i + 1)], self.w[f"{h}.4.weight"],
                         None if h == "up_prob_head" else self.w[f"{h}.4.bias"]).contiguous()
                for i, h in enumerate(self.heads)]

    def forward(self, dec: DecoderOutput, intr: workloads.Intrinsics, orig_h: int, orig_w: int,
                crop: Crop | None = None, trace: list | None = None, cond=None,
                hidden_trace: list | None = None, heads_trace: list | None = None):
        """The refined normals (1, 3, h, w) at the unpadded resolution
        (crop.orig_h x crop.orig_w; the whole 8*h8 x 8*w8 map without crop).
        trace, when given, receives each iteration's (pred_norm, up) pair,
        hidden_trace a copy of each iteration's h_new (1, C, h8, w8),
        heads_trace each iteration's propagate inputs (pred_norm before the
        iteration, and the prob, xy and angle heads' raw logits);
        cond, when given, is conditioning()'s result for these intrinsics (so
        the call does no host-to-device copy and can be captured in a graph)."""
        import torch
        with torch.backends.cudnn.flags(enabled=False):
            return self._forward(dec, intr, orig_h, orig_w, crop, trace, cond, hidden_trace,
                                 heads_trace)

    def _forward(self, dec, intr, orig_h, orig_w, crop, trace, cond, hidden_trace, heads_trace):
        import torch
        import torch.nn.functional as F
        _, _, H, W = dec.normal.shape
        C, HW = self.hidden, H * W
        ray8, uv8, (fu, cu, fv, cv) = (cond if cond is not None
                                       else self.conditioning(intr, H, W, orig_h, orig_w))
        pred_norm = dec.normal.contiguous().clone()
        dsine.ray_relu(pred_norm, ray8, H, W)
        # hx = [h | feature | uv], rhx = [r*h | feature | uv], hin = [h_new | uv]
        # (submodules.ConvGRU's cat([h, x]) and cat([r*h, x]) with
        # x = feat_map = cat(feature, uv_8), and the heads' cat(h_new, uv_8))
        cx = self.feature + 2
        hx = torch.empty((1, C + cx, H, W), dtype=torch.float32, device=self.device)
        hx[:, :C] = dec.hidden
        hx[:, C:C + self.feature] = dec.feature
        hx[:, C + self.feature:] = uv8
        rhx = torch.empty_like(hx)
        rhx[:, C:] = hx[:, C:]
        hin = torch.empty((1, C + 2, H, W), dtype=torch.float32, device=self.device)
        hin[:, C:] = uv8
        z = torch.empty((1, C, H, W), dtype=torch.float32, device=self.device)
        h = hx[:, :C]
        up = None
        for _ in range(N_ITER):
            # ConvGRU (src/dsine_refine.cpp:138-159): h_new overwrites h in hx
            zr = F.conv2d(hx, self.w_zr, None, padding=2)
            dsine.gru_gates(zr, self.b_z, self.b_r, h, C, HW, z, rhx[:, :C])
            qp = F.conv2d(rhx, self.w_q, None, padding=2)
            dsine.gru_update(qp, self.b_q, z, h, C, HW, h, hin[:, :C])
            prob, xy, angle, up_mask = self._heads(hin, H, W)
            if heads_trace is not None:
                heads_trace.append((pred_norm, prob, xy, angle))
            pred_norm = dsine.angmf_propagate(pred_norm, prob, xy, angle, ray8, fu, cu, fv, cv,
                                              H, W, logits=True)
            up = dsine.convex_upsample_normalize(pred_norm, up_mask, 1, 3, H, W, K_UP,
                                                 float(np.float32(1e-12)),
                                                 mask_bias=self.w["up_prob_head.4.bias"])
            if trace is not None:
                trace.append((pred_norm, up))
            if hidden_trace is not None:
                hidden_trace.append(h.clone())
        if crop is None:
            return up
        return up[:, :, crop.pad_t:crop.pad_t + crop.orig_h,
                  crop.pad_l:crop.pad_l + crop.orig_w].contiguous()


class NativeRefiner:
    """Refiner::forward in C++ (libbvml_dsine_refine.so, the C ABI of
    include/bvml_dsine_refine.h): the same loop as Refiner above, with no
    Python or torch in it: the 5x5 ConvGRU convolutions on this package's
    fp32 matrix-core kernels with the gates and update fused, the heads'
    3x3 layer on the same kernels, the rest of the heads in one fused pass,
    the rest this package's kernels, the up-mask head and the upsample in
    the last iteration only: the same bits in every process.  Weights from a safetensors file (`path`, read by
    the library) or a dict as weight_shapes() names them."""

    def __init__(self, weights: dict | None = None, path: str | None = None):
        import ctypes
        from . import _lib
        self._lib = _lib.load_refine()
        h = ctypes.c_void_p()
        self._check("create", self._lib.bvml_dsine_refiner_create(ctypes.byref(h)))
        self._h = h
        if path is not None:
            self.load_file(path)
        if weights is not None:
            for name in weight_shapes():
                self.set_tensor(name, weights[name])

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.bvml_dsine_refiner_destroy(h)
            self._h = None

    def _check(self, op: str, status: int) -> None:
        if status != 0:
            from . import _lib
            raise RuntimeError(f"dsine::Refiner: {_lib.refine_last_error()} (status {status})")

    def load_file(self, path: str) -> None:
        self._check("load_file", self._lib.bvml_dsine_refiner_load_file(self._h, path.encode()))

    def set_tensor(self, name: str, value) -> None:
        a = np.ascontiguousarray(np.asarray(value, np.float32)).reshape(-1)
        self._check("set_tensor", self._lib.bvml_dsine_refiner_set_tensor(
            self._h, name.encode(), a.ctypes.data, a.size))

    def get_tensor(self, name: str) -> np.ndarray:
        n = self._lib.bvml_dsine_refiner_tensor_numel(name.encode())
        if n < 0:
            raise RuntimeError(f"dsine::Refiner: unknown tensor '{name}'")
        a = np.empty(n, np.float32)
        self._check("get_tensor", self._lib.bvml_dsine_refiner_get_tensor(
            self._h, name.encode(), a.ctypes.data, n))
        return a

    def forward(self, dec: DecoderOutput, intr: workloads.Intrinsics, orig_h: int, orig_w: int,
                crop: Crop | None = None, coarse: bool = False, out=None, nthreads: int = 0):
        """The refined normals (1, 3, h, w) at the unpadded resolution (the
        whole 8*h8 x 8*w8 map without crop); with coarse=True also each
        iteration's propagated /8-grid normal, (N_ITER, 3, h8, w8).  The
        decoder maps are contiguous fp32 torch tensors, all on the GPU (the
        device path, asynchronous on the current stream) or all on the CPU
        (the host path, on nthreads threads, 0 = all); the results live
        there too.  `out`, when given, is the result tensor to fill."""
        import torch
        _, _, H, W = dec.normal.shape
        dev = dec.normal.device
        for t in (dec.normal, dec.feature, dec.hidden):
            if t.device != dev or t.dtype != torch.float32 or not t.is_contiguous():
                raise RuntimeError("dsine::Refiner: decoder maps must be contiguous fp32 tensors "
                                   "on one device")
        c = crop if crop is not None else Crop(8 * H, 8 * W)
        if out is None:
            out = torch.empty((1, 3, c.orig_h, c.orig_w), dtype=torch.float32, device=dev)
        cz = (torch.empty((N_ITER, 3, H, W), dtype=torch.float32, device=dev) if coarse
              else None)
        args = (self._h, dec.normal.data_ptr(), dec.feature.data_ptr(), dec.hidden.data_ptr(),
                H, W, intr.fx, intr.fy, intr.cx, intr.cy, orig_h, orig_w, c.pad_t, c.pad_l,
                c.orig_h, c.orig_w, out.data_ptr(), cz.data_ptr() if cz is not None else None)
        if dev.type == "cpu":
            st = self._lib.bvml_dsine_refiner_forward_cpu(*args, nthreads)
        else:
            with torch.cuda.device(dev):
                st = self._lib.bvml_dsine_refiner_forward(
                    *args, torch.cuda.current_stream(dev).cuda_stream)
        self._check("forward", st)
        return (out, cz) if coarse else out
