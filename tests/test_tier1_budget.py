"""The error budget behind the fast kernel's recompute threshold.

tier1_model.py rounds every fp32 operation of the kernel's tier 1 as the
kernel does; this compares its pixels with the oracle and checks that
err * |acc| / sqrt(sum wi^2) stays within the delta the kernel's threshold
kAccRatio2 is derived from (3.65e-7, from 1.2M emulated pixels), and that
delta / sqrt(kAccRatio2) is inside the 1e-5 parity bar.  CPU only."""
from __future__ import annotations

import os
import re

import numpy as np
import pytest

import oracle
from brovisionml_amd import workloads as wl
from tests import tier1_model as model

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DELTA = 3.65e-7
DELTA_LOGITS = 4.7e-7    # with the activations formed in fp32 (BVML_DSINE_LOGITS)


def kernel_constant(name: str) -> float:
    with open(os.path.join(ROOT, "brovisionml_amd", "csrc", "dsine_ops.hip")) as f:
        src = f.read()
    m = re.search(r"constexpr double %s = ([0-9.eE+-]+);" % name, src)
    assert m, name
    return float(m.group(1))


def test_threshold_inside_the_bar():
    t1 = kernel_constant("kAccRatio2")
    assert DELTA / np.sqrt(t1) <= 0.92e-5
    t1l = kernel_constant("kAccRatio2Logits")
    assert DELTA_LOGITS / np.sqrt(t1l) <= 0.92e-5


@pytest.mark.parametrize("H,W,fov,angle,normals,seed", [
    (48, 64, 60.0, "quarter", "sphere", 1),
    (40, 40, 140.0, "wide", "sphere", 2),
    (64, 48, 60.0, "wide", "zbias", 3),
])
def test_tier1_model_within_delta(H, W, fov, angle, normals, seed):
    rng = np.random.default_rng(seed)
    k, HW, K2 = 5, H * W, 25
    if normals == "sphere":
        n = rng.standard_normal((3, HW))
    else:
        n = np.vstack([rng.standard_normal((2, HW)), rng.uniform(0.5, 1.0, (1, HW))])
    n = (n / np.linalg.norm(n, axis=0)).astype(np.float32)
    th = (rng.uniform(0, np.pi / 4, (K2, HW)) if angle == "quarter"
          else rng.uniform(-3.2, 3.2, (K2, HW))).astype(np.float32)
    xy = rng.standard_normal((2 * K2, HW)).astype(np.float32)
    prob = (1 / (1 + np.exp(-rng.standard_normal((K2, HW))))).astype(np.float32)
    intr = wl.intrins_from_fov(8 * H, 8 * W, fov)
    fuv = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    ray = wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, HW)
    out, a2, qs = model.tier1(n, prob, xy, th, ray, fuv, H, W, k, rng)
    want = oracle.angmf_propagate(n[None], prob[None], xy[None], th[None], ray, fuv, H, W, k)
    want = np.asarray(want, np.float64).reshape(3, HW)
    err = np.abs(out.astype(np.float32).astype(np.float64) - want).max(axis=0)
    dpix = err * np.sqrt(a2 / qs)
    assert np.isfinite(dpix).all()
    assert dpix.max() <= DELTA
    # the pixels the kernel keeps are within the bar
    keep = a2 >= kernel_constant("kAccRatio2") * qs
    assert err[keep].max() <= 1e-5


def test_sigmoid_model_error():
    """The fp32 sigmoid (hardware exp2 and rcp at their error bounds) stays
    within 4 ulps of the correctly rounded float, or 3e-8 absolutely where
    the rounding of -x log2(e) dominates (large negative x, tiny sigmoid)."""
    rng = np.random.default_rng(0)
    x = rng.uniform(-30, 30, 200000).astype(np.float32)
    got = model.sigmoid(x, rng).astype(np.float64)
    want = (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)
    ulp = np.spacing(want).astype(np.float64)
    assert np.all(np.abs(got - want) <= np.maximum(4 * ulp, 3e-8))
    assert np.all(model.sigmoid(np.array([-np.inf, -1e30, -88.0], np.float32), rng) == 0)


@pytest.mark.parametrize("H,W,fov,scale,seed", [(64, 64, 60.0, 1.0, 1), (48, 48, 140.0, 3.0, 2)])
def test_tier1_model_logits_within_delta(H, W, fov, scale, seed):
    rng = np.random.default_rng(seed)
    k, HW, K2 = 5, H * W, 25
    n = rng.standard_normal((3, HW))
    n = (n / np.linalg.norm(n, axis=0)).astype(np.float32)
    lp = (rng.standard_normal((K2, HW)) * scale).astype(np.float32)
    la = (rng.standard_normal((K2, HW)) * scale).astype(np.float32)
    xy = rng.standard_normal((2 * K2, HW)).astype(np.float32)
    intr = wl.intrins_from_fov(8 * H, 8 * W, fov)
    fuv = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    ray = wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, HW)
    out, a2, qs = model.tier1(n, lp, xy, la, ray, fuv, H, W, k, rng, logits=True)
    sp = (1.0 / (1.0 + np.exp(-lp.astype(np.float64)))).astype(np.float32)
    sa = (1.0 / (1.0 + np.exp(-la.astype(np.float64)))).astype(np.float32)
    ang = (sa.astype(np.float64) * np.float64(model.K_PI)).astype(np.float32)
    want = oracle.angmf_propagate(n[None], sp[None], xy[None], ang[None], ray, fuv, H, W, k)
    want = np.asarray(want, np.float64).reshape(3, HW)
    err = np.abs(out.astype(np.float32).astype(np.float64) - want).max(axis=0)
    dpix = err * np.sqrt(a2 / qs)
    assert dpix.max() <= DELTA_LOGITS
    keep = a2 >= kernel_constant("kAccRatio2Logits") * qs
    assert err[keep].max() <= 1e-5
