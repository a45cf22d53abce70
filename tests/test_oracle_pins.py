"""Pins of the CPU oracle (oracle/dsine_ops_oracle.c), the restatement of
src/dsine_ops.cpp that every GPU parity test checks against.

The reference's own source cannot be compiled here (it includes the absent
brotensor/tensor.h) and its tests hold no vectors for this op, so each part of
the oracle is pinned by what the mathematics and independent library routines
fix -- never by re-typing the oracle's formula:
  axis_angle_to_matrix  scipy Rotation.from_rotvec; R(z, pi/2) x = y;
                        R(0) == I exactly (Taylor branch); continuity at 1e-6
  axis                  ray-plane intersection geometry; axis . m == 0;
                        zero xy pair and dd == 0 give the identity
  RayReLU               torch F.cosine_similarity/F.relu/F.normalize;
                        identity when cos >= eps; cos(out, r) = eps /
                        sqrt(1 + eps^2 - c^2) when clamped; the float eps
  unfold / whole op     F.pad(replicate) + F.unfold based restatement
                        (tests/golden/independent.py); one-hot brute force;
                        fixed point, rescaling, zero prob, unit output
test_mutants_are_caught then plants seven plausible mistakes in the oracle
(ORACLE_MUTATION) and checks that each fails at least one pin.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch
from scipy.spatial.transform import Rotation

import oracle
from brovisionml_amd import workloads as wl
from tests.golden import independent as ind

EPS32 = float(np.float32(1e-2))


def _intr(H, W):
    i = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    return i, wl.scaled_intrinsics(i, H, W, 8 * H, 8 * W)


def _geometric_axis(m, pix, xy, intr):
    """Axis where the plane through P0 = ray(pix) with normal m meets the ray
    through pix + normalized xy."""
    fu, cu, fv, cv = intr
    m = np.asarray(m, dtype=np.float64)
    xn = np.asarray(xy, dtype=np.float64) / np.hypot(*xy)
    P0 = np.array([(pix[0] - cu) / fu, (pix[1] - cv) / fv, 1.0])
    d = np.array([(pix[0] + xn[0] - cu) / fu, (pix[1] + xn[1] - cv) / fv, 1.0])
    P1 = (P0 @ m) / (d @ m) * d
    v = P1 - P0
    return v / np.linalg.norm(v)


def _torch_ray_relu(n, r):
    t = lambda a: torch.as_tensor(np.asarray(a, dtype=np.float64))[:, None]
    return ind.ray_relu(t(n), t(r), dim=0)[:, 0].numpy()


def _random_grid(rng, B, H, W, k, scale_normals=False, per_sample_ray=False):
    HW, K2 = H * W, k * k
    n = rng.standard_normal((B, 3, HW))
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    if scale_normals:
        n *= rng.uniform(0.3, 3.0, (B, 1, HW))
    intr_, intr = _intr(H, W)
    ray = wl.build_ray8(intr_, H, W, 8 * H, 8 * W).reshape(3, HW)
    if per_sample_ray:
        ray = np.stack([ray * (1.0 + 0.05 * b) for b in range(B)])
    return dict(
        n=n.astype(np.float32),
        prob=(1 / (1 + np.exp(-rng.standard_normal((B, K2, HW))))).astype(np.float32),
        xy=rng.standard_normal((B, 2 * K2, HW)).astype(np.float32),
        angle=rng.uniform(-3.0, 3.0, (B, K2, HW)).astype(np.float32),
        ray=ray.astype(np.float32), intr=intr)


# ---------------------------------------------------------------- pins ------
# Each pin takes an Oracle and returns (ok, detail); the same pins run
# against the real oracle (must pass) and against mutants (some must fail).

def pin_rotation_vs_scipy(o):
    rng = np.random.default_rng(1)
    worst = 0.0
    for _ in range(300):
        v = rng.standard_normal(3)
        v *= rng.uniform(0, 3.5) / np.linalg.norm(v)
        worst = max(worst, np.abs(o.axis_angle_to_matrix(v) - Rotation.from_rotvec(v).as_matrix()).max())
    return worst < 1e-13, worst


def pin_rotation_known_answers(o):
    Rz = o.axis_angle_to_matrix([0, 0, math.pi / 2])
    Rx = o.axis_angle_to_matrix([math.pi / 2, 0, 0])
    e1 = np.abs(Rz @ [1, 0, 0] - np.array([0, 1, 0])).max()
    e2 = np.abs(Rx @ [0, 1, 0] - np.array([0, 0, 1])).max()
    ident = np.array_equal(o.axis_angle_to_matrix([0.0, 0.0, 0.0]), np.eye(3))
    return e1 < 1e-15 and e2 < 1e-15 and ident, (e1, e2, ident)


def pin_rotation_taylor_continuity(o):
    worst = 0.0
    a = np.array([0.3, -0.5, 0.81])
    a /= np.linalg.norm(a)
    for ang in (1e-6 * (1 - 1e-9), 1e-6, 1e-6 * (1 + 1e-9), 3e-7, 5e-9):
        v = a * ang
        worst = max(worst, np.abs(o.axis_angle_to_matrix(v) - Rotation.from_rotvec(v).as_matrix()).max())
    return worst < 1e-15, worst


def pin_axis_geometry(o):
    rng = np.random.default_rng(2)
    _, intr = _intr(32, 40)
    worst = perp = 0.0
    for _ in range(300):
        m = rng.standard_normal(3)
        m /= np.linalg.norm(m)
        pix = (rng.integers(0, 40) + 0.5, rng.integers(0, 32) + 0.5)
        xy = rng.standard_normal(2)
        g = _geometric_axis(m, pix, xy, intr)
        ax = o.axis(m, pix, xy, intr)
        worst = max(worst, np.abs(ax - g).max())
        perp = max(perp, abs(ax @ m))
    return worst < 1e-9 and perp < 1e-13, (worst, perp)


def pin_axis_special_cases(o):
    _, intr = _intr(16, 24)
    fu, cu, fv, cv = intr
    zero_xy = o.axis([0.3, 0.4, 0.866], (3.5, 4.5), (0.0, 0.0), intr)
    # dd == 0 exactly: m = (1,0,0) at a column centre equal to cu, xy = (0, 1)
    dd0 = o.axis([1.0, 0.0, 0.0], (cu, 4.5), (0.0, 1.0), (fu, cu, fv, cv))
    return (np.array_equal(zero_xy, np.zeros(3)) and np.array_equal(dd0, np.zeros(3)),
            (zero_xy, dd0))


def pin_ray_relu_torch(o):
    rng = np.random.default_rng(3)
    worst = 0.0
    for _ in range(300):
        n = rng.standard_normal(3) * rng.uniform(0.2, 3)
        r = rng.standard_normal(3)
        r /= np.linalg.norm(r)
        worst = max(worst, np.abs(o.ray_relu_vec(n, r) - _torch_ray_relu(n, r)).max())
    return worst < 1e-13, worst


def pin_ray_relu_closed_forms(o):
    rng = np.random.default_rng(4)
    worst_id = worst_cf = worst_plane = 0.0
    for _ in range(200):
        r = rng.standard_normal(3)
        r /= np.linalg.norm(r)
        n = rng.standard_normal(3)
        n /= np.linalg.norm(n)
        c = n @ r
        out = o.ray_relu_vec(n, r)
        if c >= EPS32:
            worst_id = max(worst_id, np.abs(out - n).max())
        else:
            worst_cf = max(worst_cf, abs(out @ r - EPS32 / math.sqrt(1 + EPS32 ** 2 - c * c)))
            worst_plane = max(worst_plane, abs(np.linalg.det(np.stack([n, r, out]))))
    return (worst_id < 1e-15 and worst_cf < 1e-13 and worst_plane < 1e-13,
            (worst_id, worst_cf, worst_plane))


def pin_ray_relu_eps_constant(o):
    """cos between float32(0.01) and 0.01: the float-widened eps clamps, the
    double one does not."""
    r = np.array([0.0, 0.0, 1.0])
    c = 0.5 * (EPS32 + 0.01)
    n = np.array([math.sqrt(1 - c * c), 0.0, c])
    out = o.ray_relu_vec(n, r)
    want = _torch_ray_relu(n, r)
    return np.abs(out - want).max() < 1e-15, np.abs(out - want).max()


def pin_unfold_one_hot(o):
    """prob one-hot at slot s, angle 0: out = RayReLU(normalize(N[clamp(y-P+ky),
    clamp(x-P+kx)])) -- the identity rotation, then the renormalise."""
    rng = np.random.default_rng(5)
    H, W, k = 5, 7, 5
    g = _random_grid(rng, 1, H, W, k)
    g["angle"][:] = 0
    worst = 0.0
    for s in (0, 3, 7, 12, 19, 24):
        prob = np.zeros_like(g["prob"])
        prob[0, s] = 1.0
        out = o.angmf_propagate(g["n"], prob, g["xy"], g["angle"], g["ray"], g["intr"], H, W, k)
        ky, kx = divmod(s, k)
        for y in range(H):
            for x in range(W):
                sy = min(max(y - 2 + ky, 0), H - 1)
                sx = min(max(x - 2 + kx, 0), W - 1)
                m = g["n"][0, :, sy * W + sx].astype(np.float64)
                want = _torch_ray_relu(m / np.linalg.norm(m), g["ray"][:, y * W + x])
                worst = max(worst, np.abs(out[0, :, y * W + x] - want).max())
    return worst < 1e-7, worst


def pin_whole_op_independent(o):
    rng = np.random.default_rng(6)
    worst = 0.0
    for (B, H, W, k, sc, ps) in [(2, 6, 9, 5, True, True), (1, 8, 7, 3, False, False),
                                 (1, 9, 10, 7, True, False), (2, 4, 5, 1, False, True)]:
        g = _random_grid(rng, B, H, W, k, scale_normals=sc, per_sample_ray=ps)
        K2 = k * k
        _, acc = o.angmf_propagate(g["n"], g["prob"], g["xy"], g["angle"], g["ray"], g["intr"],
                                   H, W, k, return_acc=True)
        _, iacc = ind.refine_step(g["n"].reshape(B, 3, H, W), g["prob"].reshape(B, K2, H, W),
                                  g["xy"].reshape(B, 2 * K2, H, W), g["angle"].reshape(B, K2, H, W),
                                  g["ray"].reshape(-1, 3, H, W), g["intr"], k)
        worst = max(worst, np.abs(acc.reshape(B, 3, H, W) - iacc).max())
    return worst < 1e-11, worst


PINS = [pin_rotation_vs_scipy, pin_rotation_known_answers, pin_rotation_taylor_continuity,
        pin_axis_geometry, pin_axis_special_cases, pin_ray_relu_torch, pin_ray_relu_closed_forms,
        pin_ray_relu_eps_constant, pin_unfold_one_hot, pin_whole_op_independent]


@pytest.mark.parametrize("pin", PINS, ids=[p.__name__ for p in PINS])
def test_pin(pin):
    ok, detail = pin(oracle.default())
    assert ok, detail


# ---------------------------------------------------------- invariants ------

def test_fixed_point_constant_field():
    """A constant camera-facing field with angle 0 reproduces itself,
    borders included."""
    H, W, k = 6, 8, 5
    rng = np.random.default_rng(7)
    g = _random_grid(rng, 1, H, W, k)
    c = np.array([0.1, -0.2, 0.97])
    c /= np.linalg.norm(c)
    n = np.repeat(c[:, None], H * W, axis=1)[None].astype(np.float32)
    # facing every ray: cos(n, ray) >= eps for this grid
    assert (np.einsum("c,cp->p", c, g["ray"]) > EPS32).all()
    out = oracle.angmf_propagate(n, g["prob"], g["xy"], np.zeros_like(g["angle"]), g["ray"],
                                 g["intr"], H, W, k)
    assert np.abs(out - n).max() < 2e-7


def test_prob_rescaling_zero_prob_unit_output():
    H, W, k = 7, 9, 5
    rng = np.random.default_rng(8)
    g = _random_grid(rng, 1, H, W, k)
    args = (g["xy"], g["angle"], g["ray"], g["intr"], H, W, k)
    o1 = oracle.angmf_propagate(g["n"], g["prob"], *args)
    o2 = oracle.angmf_propagate(g["n"], g["prob"] * np.float32(4.0), *args)
    assert np.abs(o1 - o2).max() < 1e-7
    z = oracle.angmf_propagate(g["n"], np.zeros_like(g["prob"]), *args)
    assert np.array_equal(z, np.zeros_like(z))
    assert np.abs(np.linalg.norm(o1.astype(np.float64), axis=1) - 1).max() < 1e-6


def test_rows_and_batch_reduce_to_whole_image():
    H, W, k = 10, 6, 3
    rng = np.random.default_rng(9)
    g = _random_grid(rng, 3, H, W, k, per_sample_ray=True)
    full = oracle.angmf_propagate(g["n"], g["prob"], g["xy"], g["angle"], g["ray"], g["intr"],
                                  H, W, k, nthreads=4)
    band = oracle.angmf_propagate(g["n"], g["prob"], g["xy"], g["angle"], g["ray"], g["intr"],
                                  H, W, k, rows=(3, 7))
    r = band.reshape(3, 3, H, W)
    f = full.reshape(3, 3, H, W)
    assert np.array_equal(r[:, :, 3:7], f[:, :, 3:7])
    assert np.isnan(r[:, :, :3]).all() and np.isnan(r[:, :, 7:]).all()
    for b in range(3):
        one = oracle.angmf_propagate(g["n"][b:b + 1], g["prob"][b:b + 1], g["xy"][b:b + 1],
                                     g["angle"][b:b + 1], g["ray"][b], g["intr"], H, W, k)
        assert np.array_equal(one[0], full[b])


def test_ray_relu_batch_matches_vec():
    rng = np.random.default_rng(10)
    H, W = 3, 5
    n = rng.standard_normal((2, 3, H * W)).astype(np.float32)
    r = rng.standard_normal((2, 3, H * W)).astype(np.float32)
    out = oracle.ray_relu(n, r, H, W)
    for b in range(2):
        for p in range(H * W):
            want = oracle.ray_relu_vec(n[b, :, p], r[b, :, p]).astype(np.float32)
            assert np.array_equal(out[b, :, p], want)


# ------------------------------------------------------------ mutants -------

MUTANTS = {
    1: "transposed rotation matrix",
    2: "sign of the axis numerator",
    3: "unclamped pixel centre at the border",
    4: "column-major window slots",
    5: "double eps (the CUDA twin's constant)",
    6: "sgn(0) = +1 in the dd clamp",
    7: "no renormalise after the rotation",
}


@pytest.mark.parametrize("mutation", sorted(MUTANTS), ids=[MUTANTS[m] for m in sorted(MUTANTS)])
def test_mutants_are_caught(tmp_path, mutation):
    path = oracle.compile_variant(os.path.join(tmp_path, f"mut{mutation}.so"), mutation)
    o = oracle.Oracle(path)
    failed = [p.__name__ for p in PINS if not p(o)[0]]
    assert failed, f"mutation {mutation} ({MUTANTS[mutation]}) passed every pin"
