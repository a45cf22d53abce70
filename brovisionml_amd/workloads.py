"""Synthetic workloads and the camera closed forms that feed the two ops.

The ops take a per-pixel unit ray map and grid-scaled intrinsics that the
reference builds on the host before the refinement loop:
  intrins_from_fov   src/dsine_preprocess.cpp:35-46 (float-rounded fx, fy, cx, cy)
  scaled_intrinsics  src/dsine_refine.cpp:232-237  (fu, cu, fv, cv with +0.5)
  build_ray8         src/dsine_decoder.cpp:242-259,276-293 (get_ray_core + L2)
They are restated here in double with the same float roundings, vectorised
with numpy.

The five workloads are the op's benchmark/parity shapes:
  0  B=1,  60x80,   k=5  plumbing (a 480x640 image)
  1  B=1,  128x128, k=5  4 chained calls (out feeds the next pred_norm)
  2  B=1,  256x256, k=5  headline shape; angles U[0, pi/4]
  3  B=32, 60x80,   k=5  many small frames, per-sample seeds
  4  B=4,  512x512, k=7  bandwidth stress; +z-biased normals
Inputs: unit normals from N(0,1)^3 (config 4: z ~ U(0.5,1), xy ~ N(0,1),
renormalised), angle planes from the stated distribution, raw xy planes
N(0,1), prob = sigmoid(L) with L ~ N(0,1), computed once on the host.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Intrinsics:
    fx: float
    fy: float
    cx: float
    cy: float


def _f32(v: float) -> float:
    return float(np.float32(v))


def intrins_from_fov(orig_h: int, orig_w: int, fov_deg: float = 60.0) -> Intrinsics:
    """src/dsine_preprocess.cpp:35-46: f = (max(H,W)/2)/tan(fov/2), principal
    point at the image centre - 0.5; every field rounded to float."""
    k_pi = 3.14159265358979323846
    half_fov_rad = (float(np.float32(fov_deg)) / 2.0) * k_pi / 180.0
    f = (max(orig_h, orig_w) / 2.0) / math.tan(half_fov_rad)
    return Intrinsics(fx=_f32(f), fy=_f32(f), cx=_f32(orig_w / 2.0 - 0.5),
                      cy=_f32(orig_h / 2.0 - 0.5))


def scaled_intrinsics(intr: Intrinsics, H: int, W: int, orig_h: int, orig_w: int):
    """src/dsine_refine.cpp:232-237: (fu, cu, fv, cv) on the (H, W) grid, with
    the +0.5 on the principal point."""
    sw = W / orig_w
    sh = H / orig_h
    return (intr.fx * sw, (intr.cx + 0.5) * sw, intr.fy * sh, (intr.cy + 0.5) * sh)


def build_ray8(intr: Intrinsics, H: int, W: int, orig_h: int, orig_w: int) -> np.ndarray:
    """src/dsine_decoder.cpp:242-259 (get_ray_core) and :276-293 (build_ray8):
    ray_x/ray_y in double rounded to float, then L2-normalise [x, y, 1] in
    double and round each channel to float.  Returns (3, H, W) float32."""
    fu, cu, fv, cv = scaled_intrinsics(intr, H, W, orig_h, orig_w)
    xs = np.arange(W, dtype=np.float64)
    ys = np.arange(H, dtype=np.float64)
    rx = (((xs + 0.5) - cu) / fu).astype(np.float32).astype(np.float64)
    ry = (((ys + 0.5) - cv) / fv).astype(np.float32).astype(np.float64)
    X = np.broadcast_to(rx[None, :], (H, W))
    Y = np.broadcast_to(ry[:, None], (H, W))
    inv = 1.0 / np.maximum(np.sqrt(X * X + Y * Y + 1.0), 1e-12)
    out = np.empty((3, H, W), dtype=np.float32)
    out[0] = X * inv
    out[1] = Y * inv
    out[2] = 1.0 * inv
    return out


@dataclass(frozen=True)
class Workload:
    index: int
    name: str
    B: int
    H: int
    W: int
    k: int
    calls: int          # chained calls per step (out feeds the next pred_norm)
    angle: str          # "normal:<sigma>" or "uniform:<lo>:<hi>"
    normals: str        # "sphere" or "zbias"
    seed: int

    @property
    def HW(self) -> int:
        return self.H * self.W

    @property
    def K2(self) -> int:
        return self.k * self.k

    def intrinsics(self):
        intr = intrins_from_fov(8 * self.H, 8 * self.W, 60.0)
        return intr, scaled_intrinsics(intr, self.H, self.W, 8 * self.H, 8 * self.W)

    def algorithmic_bytes(self, shared_ray: bool = True) -> int:
        """Bytes one step must move at least once: every input plane read once
        (halo re-reads not counted), out written once, per call."""
        R = 1 if shared_ray else self.B
        per_call = (self.B * self.HW * 4 * (3 + self.K2 + 2 * self.K2 + self.K2)
                    + R * self.HW * 4 * 3 + self.B * self.HW * 4 * 3)
        return self.calls * per_call


WORKLOADS = [
    Workload(0, "dsine-angmf-60x80-k5", 1, 60, 80, 5, 1, "normal:0.1", "sphere", 1000),
    Workload(1, "dsine-angmf-128x128-k5-chain4", 1, 128, 128, 5, 4, "normal:0.1", "sphere", 1001),
    Workload(2, "dsine-angmf-256x256-k5", 1, 256, 256, 5, 1, "uniform:0:0.7853981633974483",
             "sphere", 1002),
    Workload(3, "dsine-angmf-b32-60x80-k5", 32, 60, 80, 5, 1, "normal:0.1", "sphere", 1003),
    Workload(4, "dsine-angmf-b4-512x512-k7", 4, 512, 512, 7, 1, "normal:0.2", "zbias", 1004),
]


def _unit_normals(rng: np.random.Generator, HW: int, kind: str) -> np.ndarray:
    if kind == "sphere":
        v = rng.standard_normal((3, HW))
    elif kind == "zbias":
        v = np.empty((3, HW))
        v[0:2] = rng.standard_normal((2, HW))
        v[2] = rng.uniform(0.5, 1.0, HW)
    else:
        raise ValueError(kind)
    v /= np.sqrt((v * v).sum(axis=0, keepdims=True))
    return v.astype(np.float32)


def _angles(rng: np.random.Generator, shape, spec: str) -> np.ndarray:
    kind, *par = spec.split(":")
    if kind == "normal":
        return (rng.standard_normal(shape) * float(par[0])).astype(np.float32)
    if kind == "uniform":
        return rng.uniform(float(par[0]), float(par[1]), shape).astype(np.float32)
    raise ValueError(spec)


# Seed offset between independent draws of a workload (draw 0 is the stated
# seed; sample b of draw d uses seed + d * DRAW_STRIDE + b).
DRAW_STRIDE = 100003


def make_sample(wl: Workload, b: int = 0, draw: int = 0):
    """Inputs of sample b of draw `draw` (0: the workload's stated seed):
    dict of float32 arrays shaped (C, H*W)."""
    rng = np.random.default_rng(wl.seed + draw * DRAW_STRIDE + b)
    HW, K2 = wl.HW, wl.K2
    pred = _unit_normals(rng, HW, wl.normals)
    angle = _angles(rng, (K2, HW), wl.angle)
    xy = rng.standard_normal((2 * K2, HW), dtype=np.float32)
    logits = rng.standard_normal((K2, HW), dtype=np.float32)
    prob = (1.0 / (1.0 + np.exp(-logits.astype(np.float64)))).astype(np.float32)
    return {"pred_norm": pred, "prob": prob, "xy": xy, "angle": angle}


def make_inputs(wl: Workload, draw: int = 0):
    """All B samples of draw `draw` stacked: pred_norm (B,3,HW), prob
    (B,K2,HW), xy (B,2K2,HW), angle (B,K2,HW); ray (3,HW) shared;
    (fu,cu,fv,cv)."""
    samples = [make_sample(wl, b, draw) for b in range(wl.B)]
    out = {key: np.ascontiguousarray(np.stack([s[key] for s in samples]))
           for key in samples[0]}
    intr, (fu, cu, fv, cv) = wl.intrinsics()
    out["ray"] = build_ray8(intr, wl.H, wl.W, 8 * wl.H, 8 * wl.W).reshape(3, wl.HW)
    out["intrinsics"] = (fu, cu, fv, cv)
    return out


@dataclass(frozen=True)
class UpsampleWorkload:
    """The refiner's post-propagate step (src/dsine_refine.cpp:276-282): the
    C-channel normal map on the /8 grid upsampled by s with a 9*s*s-channel
    softmax mask, then L2-normalised."""
    name: str
    B: int
    C: int
    H: int
    W: int
    s: int
    mask_sigma: float   # mask logits ~ N(0, sigma^2)
    seed: int

    @property
    def HW(self) -> int:
        return self.H * self.W

    def algorithmic_bytes(self) -> int:
        """x and the mask read once, out written once."""
        return self.B * self.HW * 4 * (self.C + 9 * self.s * self.s + self.C * self.s * self.s)


# the refiner's shape at the 2048x2048 headline image (the 256x256 grid of
# the propagate workload), and at 480x640
UPSAMPLE_WORKLOADS = [
    UpsampleWorkload("dsine-upsample-256x256-s8", 1, 3, 256, 256, 8, 1.0, 2000),
    UpsampleWorkload("dsine-upsample-60x80-s8", 1, 3, 60, 80, 8, 1.0, 2001),
]


def make_upsample_inputs(wl: UpsampleWorkload, draw: int = 0):
    """x (B, C, H, W) unit normals drawn independently per pixel (the case
    with the most cancellation between neighbours), mask (B, 9*s*s, H, W);
    draw d > 0 is an independent draw (seed + d * DRAW_STRIDE)."""
    rng = np.random.default_rng(wl.seed + draw * DRAW_STRIDE)
    x = np.stack([_unit_normals(rng, wl.HW, "sphere").reshape(wl.C, wl.H, wl.W)
                  for _ in range(wl.B)])
    mask = (wl.mask_sigma * rng.standard_normal((wl.B, 9 * wl.s * wl.s, wl.H, wl.W),
                                                dtype=np.float32)).astype(np.float32)
    return np.ascontiguousarray(x), mask
