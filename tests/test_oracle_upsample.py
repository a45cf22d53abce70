"""Pins of the CPU oracle's convex upsample + channel L2-normalise
(oracle_convex_upsample_f32), the restatement of the two calls the refiner
makes after each propagate (src/dsine_refine.cpp:276-282; arithmetic from the
spec at include/brovisionml/dsine_refine.h:91-97).  brotensor, which holds the
reference implementation, is not in the image, so each property is pinned by
an independent restatement and by what the mathematics fixes:
  independent  float64 torch: mask.view(N,1,9,s,s,H,W).softmax(2), F.pad
               (replicate) + F.unfold, permute onto the s-times grid,
               F.normalize (tests/golden/independent.py)
  one-hot      a mask that puts all weight on tap n gives the replicate-clamped
               neighbour (y-1+n//3, x-1+n%3), normalised
  uniform      an all-zero mask gives the normalised 3x3 mean
  constant     a constant field comes back unchanged (normalised)
  shift        adding a per-sub-pixel constant to its 9 taps changes nothing
  scale        the normalised output does not depend on |x| (above eps)
  partition    unnormalised, x = 1 gives 1: the weights sum to one
  NaN          a NaN tap makes its own sub-pixel NaN and no other
test_upsample_mutants_are_caught plants four plausible mistakes
(ORACLE_MUTATION 8-11) and checks that each fails at least one pin.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle
from tests.golden import independent as ind


def _field(rng, B, C, H, W, unit=True):
    x = rng.standard_normal((B, C, H, W))
    if unit:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
    return x.astype(np.float32)


def _mask(rng, B, H, W, s, sigma=2.0):
    return (sigma * rng.standard_normal((B, 9 * s * s, H, W))).astype(np.float32)


def _neighbour(x, y, xx, n):
    """x (C, H, W) at tap n of pixel (y, xx), replicate padding."""
    C, H, W = x.shape
    sy = min(max(y - 1 + n // 3, 0), H - 1)
    sx = min(max(xx - 1 + n % 3, 0), W - 1)
    return x[:, sy, sx].astype(np.float64)


def pin_up_independent(o):
    rng = np.random.default_rng(21)
    worst = 0.0
    for (B, C, H, W, s, norm) in [(1, 3, 4, 5, 8, True), (2, 3, 3, 4, 2, True), (1, 1, 5, 3, 3, False),
                                  (1, 4, 2, 6, 4, True), (1, 2, 3, 3, 1, False), (1, 3, 1, 1, 8, True)]:
        x = _field(rng, B, C, H, W, unit=(C == 3))
        m = _mask(rng, B, H, W, s)
        got = o.convex_upsample(x, m, H, W, s, normalize=norm)
        want = ind.convex_upsample(x.astype(np.float64), m.astype(np.float64), s, norm)
        worst = max(worst, float((np.abs(got - want) / np.maximum(1.0, np.abs(want))).max()))
    return worst < 1.2e-7, worst


def pin_up_one_hot(o):
    rng = np.random.default_rng(22)
    B, C, H, W, s = 1, 3, 3, 4, 2
    x = _field(rng, B, C, H, W)
    worst = 0.0
    for n in range(9):
        m = np.zeros((B, 9 * s * s, H, W), dtype=np.float32)
        m[0, n * s * s:(n + 1) * s * s] = 80.0
        out = o.convex_upsample(x, m, H, W, s)
        for y in range(H):
            for xx in range(W):
                v = _neighbour(x[0], y, xx, n)
                want = v / np.linalg.norm(v)
                for ky in range(s):
                    for kx in range(s):
                        worst = max(worst, np.abs(out[0, :, s * y + ky, s * xx + kx] - want).max())
    return worst < 1e-7, worst


def pin_up_uniform(o):
    rng = np.random.default_rng(23)
    B, C, H, W, s = 1, 3, 4, 3, 3
    x = _field(rng, B, C, H, W)
    m = np.zeros((B, 9 * s * s, H, W), dtype=np.float32)
    out = o.convex_upsample(x, m, H, W, s)
    pad = np.pad(x[0].astype(np.float64), ((0, 0), (1, 1), (1, 1)), mode="edge")
    worst = 0.0
    for y in range(H):
        for xx in range(W):
            v = pad[:, y:y + 3, xx:xx + 3].reshape(C, 9).mean(axis=1)
            want = v / np.linalg.norm(v)
            cell = out[0, :, s * y:s * y + s, s * xx:s * xx + s].reshape(C, -1)
            worst = max(worst, np.abs(cell - want[:, None]).max())
    return worst < 1e-7, worst


def pin_up_constant(o):
    rng = np.random.default_rng(24)
    H, W, s = 5, 4, 8
    c = np.array([0.3, -0.4, 0.8], dtype=np.float32)
    x = np.broadcast_to(c[None, :, None, None], (1, 3, H, W)).astype(np.float32)
    out = o.convex_upsample(x, _mask(rng, 1, H, W, s), H, W, s)
    want = c.astype(np.float64) / np.linalg.norm(c.astype(np.float64))
    worst = np.abs(out[0] - want[:, None, None]).max()
    return worst < 1e-7, worst


def pin_up_softmax_shift(o):
    """The oracle on a mask whose 9 taps are shifted by one constant per
    sub-pixel equals the independent restatement on the unshifted taps."""
    rng = np.random.default_rng(25)
    H, W, s = 3, 5, 4
    x = _field(rng, 1, 3, H, W)
    m = _mask(rng, 1, H, W, s)
    shift = rng.uniform(-20, 20, (1, 1, s * s, H, W))
    m2 = (m.reshape(1, 9, s * s, H, W) + shift).reshape(m.shape).astype(np.float32)
    a = o.convex_upsample(x, m2, H, W, s)
    m2_unshifted = (m2.astype(np.float64).reshape(1, 9, s * s, H, W) - shift).reshape(m.shape)
    c = ind.convex_upsample(x.astype(np.float64), m2_unshifted, s)
    worst = np.abs(a - c).max()
    return worst < 1.2e-7, worst


def pin_up_scale(o):
    rng = np.random.default_rng(26)
    H, W, s = 4, 4, 2
    x = _field(rng, 1, 3, H, W)
    m = _mask(rng, 1, H, W, s)
    a = o.convex_upsample(x, m, H, W, s)
    b = o.convex_upsample((x * np.float32(1e-7)).astype(np.float32), m, H, W, s)
    worst = np.abs(a - b).max()
    return worst < 2e-7, worst


def pin_up_partition(o):
    rng = np.random.default_rng(27)
    H, W, s = 3, 4, 8
    x = np.ones((1, 2, H, W), dtype=np.float32)
    out = o.convex_upsample(x, _mask(rng, 1, H, W, s, sigma=5.0), H, W, s, normalize=False)
    worst = np.abs(out - 1.0).max()
    return worst < 1e-7, worst


def pin_up_nan(o):
    rng = np.random.default_rng(28)
    H, W, s = 3, 3, 2
    x = _field(rng, 1, 3, H, W)
    m = _mask(rng, 1, H, W, s)
    n, ky, kx, y, xx = 4, 1, 0, 2, 1
    m[0, n * s * s + ky * s + kx, y, xx] = np.nan
    out = o.convex_upsample(x, m, H, W, s)
    bad = np.isnan(out[0]).any(axis=0)
    want = np.zeros_like(bad)
    want[s * y + ky, s * xx + kx] = True
    return np.array_equal(bad, want), int(bad.sum())


UP_PINS = [pin_up_independent, pin_up_one_hot, pin_up_uniform, pin_up_constant, pin_up_softmax_shift,
           pin_up_scale, pin_up_partition, pin_up_nan]


@pytest.mark.parametrize("pin", UP_PINS, ids=[p.__name__ for p in UP_PINS])
def test_up_pin(pin):
    ok, detail = pin(oracle.default())
    assert ok, detail


UP_MUTANTS = {
    8: "sub-pixel row and column swapped in the mask channel",
    9: "zero padding instead of replicate",
    10: "column-major taps",
    11: "eps inside the square root",
}


@pytest.mark.parametrize("mutation", sorted(UP_MUTANTS), ids=[UP_MUTANTS[m] for m in sorted(UP_MUTANTS)])
def test_upsample_mutants_are_caught(tmp_path, mutation):
    path = oracle.compile_variant(os.path.join(tmp_path, f"mut{mutation}.so"), mutation)
    o = oracle.Oracle(path)
    failed = [p.__name__ for p in UP_PINS if not p(o)[0]]
    assert failed, f"mutation {mutation} ({UP_MUTANTS[mutation]}) passed every pin"
