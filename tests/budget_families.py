"""Input families for the fast kernel's tier-1 error budget.

Each family stresses one mechanism of the fp32 arithmetic (test
infrastructure; tests/test_tier1_budget.py runs them through the CPU model,
tests/test_gpu_budget.py through the kernel):
  random         the benchmark's distribution: isotropic unit normals,
                 angles U[0, pi/4], xy N(0, 1), prob sigmoid(N(0, 1))
  wideangle      angles U[-3.2, 3.2], the fast path's whole domain
  widefov        a 140 degree field of view (source rays up to |P0| ~ 2.9)
  antipode       normals facing away from the camera and small rotations:
                 most terms land near -ray, where RayReLU's clamp leaves
                 |p| near eps and amplifies the rotation's rounding by 1/|p|
  antipode_mix   half the pixels facing the camera, half away
  checker        a checkerboard of nearly opposite normals with uniform
                 weights: sums that nearly cancel
  checker_clamp  the same with directions perpendicular to the ray, so
                 about half the terms are clamped
  qcancel        xy pairs perpendicular to the pixel's own normal: q cancels
  grazing        normals perpendicular to the viewing ray (g = P0.m ~ 0)
  grazing_qcancel  both: g and q cancel, the axis's worst conditioning
  logits         raw logits N(0, 30^2) for prob (saturated activations) and
                 N(0, 9) for angle, activated in the kernel (BVML_DSINE_LOGITS)
  logits_mild    logits N(0, 1) for both
"""
from __future__ import annotations

import numpy as np

from brovisionml_amd import workloads as wl

FAMILIES = ("random", "wideangle", "widefov", "antipode", "antipode_mix", "checker",
            "checker_clamp", "qcancel", "grazing", "grazing_qcancel", "logits", "logits_mild")


def _unit(v) -> np.ndarray:
    return (v / np.linalg.norm(v, axis=0, keepdims=True)).astype(np.float32)


def family(name: str, rng: np.random.Generator, H: int = 64, W: int = 64, k: int = 5) -> dict:
    """One draw of a family: pred_norm (3, HW), prob (K2, HW) (raw logits when
    `logits`), xy (2 K2, HW), angle (K2, HW) (raw logits when `logits`), ray
    (3, HW), intr (fu, cu, fv, cv), and H, W, k, logits."""
    HW, K2 = H * W, k * k
    fov = 140.0 if name == "widefov" else 60.0
    intr = wl.intrins_from_fov(8 * H, 8 * W, fov)
    fuv = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    ray = wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, HW)
    n = _unit(rng.standard_normal((3, HW)))
    th = rng.uniform(0, np.pi / 4, (K2, HW)).astype(np.float32)
    xy = rng.standard_normal((2 * K2, HW)).astype(np.float32)
    prob = (1 / (1 + np.exp(-rng.standard_normal((K2, HW))))).astype(np.float32)
    logits = False
    yy, xx = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
    checker = np.where(((yy + xx) % 2).ravel() == 0, 1.0, -1.0)
    if name == "wideangle":
        th = rng.uniform(-3.2, 3.2, (K2, HW)).astype(np.float32)
    elif name == "antipode":
        n = _unit(-ray + 0.05 * rng.standard_normal((3, HW)))
        th = (0.05 * rng.standard_normal((K2, HW))).astype(np.float32)
    elif name == "antipode_mix":
        away = rng.uniform(size=HW) < 0.5
        n = _unit(np.where(away, -ray, ray) + 0.08 * rng.standard_normal((3, HW)))
        th = (0.1 * rng.standard_normal((K2, HW))).astype(np.float32)
    elif name == "checker":
        d = _unit(rng.standard_normal((3, 1)) + 0 * ray)
        n = _unit(d * checker + 0.02 * rng.standard_normal((3, HW)))
        th = (0.02 * rng.standard_normal((K2, HW))).astype(np.float32)
        prob = rng.uniform(0.0, 1.0, (K2, HW)).astype(np.float32)
    elif name == "checker_clamp":
        d = _unit(np.cross(ray, rng.standard_normal((3, 1)) + 0 * ray, axis=0))
        n = _unit(d * checker + 0.05 * rng.standard_normal((3, HW)))
        th = (0.05 * rng.standard_normal((K2, HW))).astype(np.float32)
        prob = rng.uniform(0.0, 1.0, (K2, HW)).astype(np.float32)
    elif name == "qcancel":
        s = rng.standard_normal((K2, HW))
        xy = np.concatenate([-n[1][None] * s, n[0][None] * s]).astype(np.float32)
        xy += (1e-3 * rng.standard_normal(xy.shape)).astype(np.float32)
    elif name == "grazing":
        n = _unit(np.cross(ray, rng.standard_normal((3, HW)), axis=0)
                  + 0.01 * rng.standard_normal((3, HW)))
    elif name == "grazing_qcancel":
        n = _unit(np.cross(ray, rng.standard_normal((3, HW)), axis=0)
                  + 0.01 * rng.standard_normal((3, HW)))
        s = rng.standard_normal((K2, HW))
        xy = np.concatenate([-n[1][None] * s, n[0][None] * s]).astype(np.float32)
        xy += (1e-3 * rng.standard_normal(xy.shape)).astype(np.float32)
    elif name == "logits":
        logits = True
        prob = (30.0 * rng.standard_normal((K2, HW))).astype(np.float32)
        th = (3.0 * rng.standard_normal((K2, HW))).astype(np.float32)
    elif name == "logits_mild":
        logits = True
        prob = rng.standard_normal((K2, HW)).astype(np.float32)
        th = rng.standard_normal((K2, HW)).astype(np.float32)
    elif name not in ("random", "widefov"):
        raise ValueError(name)
    return dict(pred_norm=n, prob=prob, xy=xy, angle=th, ray=ray, intr=fuv, H=H, W=W, k=k,
                logits=logits)


def activated(d: dict):
    """(prob, angle) as the op takes them: the refiner's activations of the
    logits, correctly rounded (sigmoid in double rounded to float; the angle
    the float product with the float pi), or the planes themselves."""
    if not d["logits"]:
        return d["prob"], d["angle"]
    def sig(x):
        return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)
    return sig(d["prob"]), sig(d["angle"]) * np.float32(np.pi)


def exact_terms(oracle, d: dict):
    """The oracle's output (3, HW) and the cancellation ratio
    |acc|^2 / sum_i (prob_i / |p_i|)^2 per pixel, from its double sums."""
    pr, an = activated(d)
    H, W, k = d["H"], d["W"], d["k"]
    out, acc, qs = oracle.angmf_propagate(d["pred_norm"][None], pr[None], d["xy"][None],
                                          an[None], d["ray"], d["intr"], H, W, k, nthreads=8,
                                          return_acc=True, return_qs=True)
    ratio = (acc.reshape(3, -1) ** 2).sum(axis=0) / qs.reshape(-1)
    return np.asarray(out, np.float64).reshape(3, -1), ratio
