"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bar: max-abs 1e-5 per component and 0.01 degrees of angular error against the
oracle's double-precision restatement of src/dsine_ops.cpp, on the same
seeded fp32 inputs; NaN patterns must match.  The double-precision kernel
(BVML_DSINE_FP64) must agree to a couple of float ulps.
"""
from __future__ import annotations

import glob
import os
import sys

import numpy as np
import pytest

import oracle
from brovisionml_amd import _lib, dsine, workloads as wl
from tests._util import TOL_ABS, TOL_DEG, Guarded, compare, to_dev

pytestmark = pytest.mark.gpu

NTHREADS = max(1, min(16, os.cpu_count() or 1))


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def run_gpu(inp, H, W, device, precise=False, ray=None):
    import torch
    t = {k: to_dev(inp[k], device) for k in ("pred_norm", "prob", "xy", "angle")}
    r = to_dev(inp["ray"] if ray is None else ray, device)
    fu, cu, fv, cv = inp["intrinsics"]
    g = Guarded(t["pred_norm"].numel(), device)
    out = dsine.angmf_propagate(t["pred_norm"], t["prob"], t["xy"], t["angle"], r,
                                fu, cu, fv, cv, H, W, g.out, precise=precise)
    torch.cuda.synchronize()
    assert out.data_ptr() == g.out.data_ptr()
    assert g.intact(), "angmf_propagate wrote outside its output"
    return out.cpu().numpy().reshape(t["pred_norm"].shape)


def run_oracle(inp, H, W, k, ray=None):
    return oracle.angmf_propagate(inp["pred_norm"], inp["prob"], inp["xy"], inp["angle"],
                                  inp["ray"] if ray is None else ray, inp["intrinsics"],
                                  H, W, k, nthreads=NTHREADS)


@pytest.mark.parametrize("idx", [0, 2, 3, 4])
def test_angmf_workload(cuda, idx):
    w = wl.WORKLOADS[idx]
    say(f"[gpu] angmf workload {w.name} B={w.B} {w.H}x{w.W} k={w.k}")
    inp = wl.make_inputs(w)
    got = run_gpu(inp, w.H, w.W, cuda)
    want = run_oracle(inp, w.H, w.W, w.k)
    max_abs, max_deg, nan_mm = compare(got.reshape(w.B, 3, -1), want.reshape(w.B, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG


@pytest.mark.parametrize("idx", [0, 2, 3])
def test_angmf_fp64_kernel(cuda, idx):
    w = wl.WORKLOADS[idx]
    say(f"[gpu] angmf fp64 kernel {w.name}")
    inp = wl.make_inputs(w)
    got = run_gpu(inp, w.H, w.W, cuda, precise=True)
    want = run_oracle(inp, w.H, w.W, w.k)
    max_abs, max_deg, nan_mm = compare(got.reshape(w.B, 3, -1), want.reshape(w.B, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
    assert nan_mm == 0
    assert max_abs <= 2.5e-7


def test_angmf_chain4(cuda):
    """Workload 1: four chained calls, each output feeds the next pred_norm."""
    w = wl.WORKLOADS[1]
    say(f"[gpu] angmf chained x{w.calls} {w.name}")
    inp = wl.make_inputs(w)
    g_inp = dict(inp)
    o_inp = dict(inp)
    for it in range(w.calls):
        got = run_gpu(g_inp, w.H, w.W, cuda)
        want = run_oracle(o_inp, w.H, w.W, w.k)
        max_abs, max_deg, nan_mm = compare(got.reshape(1, 3, -1), want.reshape(1, 3, -1))
        say(f"    call {it}: max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
        assert nan_mm == 0
        assert max_abs <= TOL_ABS and max_deg <= TOL_DEG
        g_inp = dict(g_inp, pred_norm=got)
        o_inp = dict(o_inp, pred_norm=want)


def _random_inputs(rng, B, H, W, k, theta_scale=1.0, per_sample_ray=False):
    HW, K2 = H * W, k * k
    n = rng.standard_normal((B, 3, HW))
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    fu, cu, fv, cv = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    ray = wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, HW)
    if per_sample_ray:
        ray = np.stack([ray * (1.0 + 0.01 * b) for b in range(B)]).astype(np.float32)
    return {
        "pred_norm": n.astype(np.float32),
        "prob": (1 / (1 + np.exp(-rng.standard_normal((B, K2, HW))))).astype(np.float32),
        "xy": rng.standard_normal((B, 2 * K2, HW)).astype(np.float32),
        "angle": (rng.uniform(-np.pi, np.pi, (B, K2, HW)) * theta_scale).astype(np.float32),
        "ray": ray,
        "intrinsics": (fu, cu, fv, cv),
    }


# Tiles: wide (64 x M) above 128 columns or 64 * M pixels; narrow full-width
# otherwise.  (1, 10, 64, 9) and (1, 5, 128, 7) stage two halo records per
# thread; (1, 6, 100, 9) is a row longer than one k = 9 workgroup.
# (2, 512, 512, 5) and (3, 500, 333, 7) are large enough for the whole-window
# kernel (one wave per 64 pixels runs every neighbour; 64 x 8 tiles), the
# second with ragged tiles on both edges.
SHAPES = [
    (1, 1, 1, 5), (1, 1, 9, 5), (1, 9, 1, 5), (1, 3, 4, 5), (1, 7, 130, 5),
    (1, 33, 65, 3), (2, 17, 200, 7), (1, 12, 20, 9), (3, 5, 6, 1), (1, 64, 64, 5),
    (1, 10, 64, 9), (1, 5, 128, 7), (1, 6, 100, 9), (2, 512, 512, 5), (3, 500, 333, 7),
    (1, 256, 256, 3), (4, 384, 80, 5), (1, 256, 256, 7), (4, 384, 40, 9), (1, 800, 800, 5),
    (16, 130, 70, 5),
]


@pytest.mark.parametrize("B,H,W,k", SHAPES)
def test_angmf_shapes(cuda, B, H, W, k):
    rng = np.random.default_rng(100 + B * 1000 + H * 10 + W + k)
    inp = _random_inputs(rng, B, H, W, k)
    fp32, g, tw, th = _lib.angmf_plan(B, H, W, k, *inp["intrinsics"])
    say(f"[gpu] angmf shape B={B} H={H} W={W} k={k}: G={g} tile {tw}x{th} fp32={fp32}")
    got = run_gpu(inp, H, W, cuda)
    want = run_oracle(inp, H, W, k)
    max_abs, max_deg, nan_mm = compare(got.reshape(B, 3, -1), want.reshape(B, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG


def test_angmf_per_sample_ray(cuda):
    B, H, W, k = 3, 20, 36, 5
    say(f"[gpu] angmf per-sample ray B={B} {H}x{W}")
    rng = np.random.default_rng(7)
    inp = _random_inputs(rng, B, H, W, k, per_sample_ray=True)
    got = run_gpu(inp, H, W, cuda)
    want = run_oracle(inp, H, W, k)
    max_abs, max_deg, nan_mm = compare(got.reshape(B, 3, -1), want.reshape(B, 3, -1))
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG


def test_angmf_xy_magnitudes(cuda):
    """xy pairs scaled log-uniformly over 1e-12 .. 1e21: |xy|^2 crosses the
    fast path's fp32 range (1e-20 .. 1e30) at both ends and overflows fp32
    above ~1.8e19; every pixel must match the oracle either way."""
    H, W, k = 12, 20, 5
    say("[gpu] angmf xy magnitudes")
    rng = np.random.default_rng(17)
    inp = _random_inputs(rng, 1, H, W, k)
    scale = 10.0 ** rng.uniform(-12.0, 21.0, size=inp["xy"].shape)
    inp["xy"] = (inp["xy"].astype(np.float64) * scale).astype(np.float32)
    got = run_gpu(inp, H, W, cuda)
    want = run_oracle(inp, H, W, k)
    max_abs, max_deg, nan_mm = compare(got.reshape(1, 3, -1), want.reshape(1, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg  nan-mismatch {nan_mm}")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG


def test_angmf_degenerate_inputs(cuda):
    """Zero xy pairs, zero / tiny normals, zero probs, dd == 0 exactly,
    non-finite values: every case the reference's clamps and isfinite guard
    decide must come out as the oracle says (NaN where it says NaN)."""
    H, W, k = 16, 24, 5
    HW, K2 = H * W, k * k
    say("[gpu] angmf degenerate inputs")
    rng = np.random.default_rng(11)
    inp = _random_inputs(rng, 1, H, W, k)
    pn, pr, xy, an = inp["pred_norm"], inp["prob"], inp["xy"], inp["angle"]
    fu, cu, fv, cv = inp["intrinsics"]
    # zero xy pairs
    xy[0, 3, 10:40] = 0
    xy[0, K2 + 3, 10:40] = 0
    # tiny xy pair (below the reference's 1e-12 clamp)
    xy[0, 5, 50:60] = 1e-13
    xy[0, K2 + 5, 50:60] = 0
    # zero and tiny normals
    pn[0, :, 70:75] = 0
    pn[0, :, 80:83] = 1e-20
    # all-zero prob at some pixels -> output exactly 0
    pr[0, :, 100:110] = 0
    # dd == 0 exactly: normal (1,0,0) at a pixel whose column centre equals cu,
    # xy pair (0, 1): tu = 0 there, so dd = 0 and num = 0 -> identity rotation.
    xc = 11
    cu = xc + 0.5
    inp["intrinsics"] = (fu, cu, fv, cv)
    y0 = 8
    sp = y0 * W + xc
    pn[0, :, sp] = (1.0, 0.0, 0.0)
    p_center = y0 * W + xc  # its own centre slot (ky = kx = 2)
    n_c = 2 * k + 2
    xy[0, n_c, p_center] = 0.0
    xy[0, K2 + n_c, p_center] = 1.0
    # non-finite values
    xy[0, 7, 200] = np.nan          # isfinite guard -> identity, finite output
    an[0, 8, 210] = np.nan          # NaN output
    pr[0, 9, 220] = np.inf          # NaN output
    pn[0, 0, 230] = np.nan          # NaN at every pixel that reads it
    inp["ray"][1, 240] = np.nan     # NaN output at that pixel
    got = run_gpu(inp, H, W, cuda)
    want = run_oracle(inp, H, W, k)
    max_abs, max_deg, nan_mm = compare(got.reshape(1, 3, -1), want.reshape(1, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg  nan-mismatch {nan_mm}")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG
    assert np.all(got.reshape(3, -1)[:, 100:110] == 0)


def test_angmf_large_angles_and_cancellation(cuda):
    """Angles beyond [0, pi] (negative, > pi, > 2 pi) and neighbour sets that
    nearly cancel (|acc| small), which the fast path must hand to the
    double-precision path."""
    H, W, k = 40, 48, 5
    say("[gpu] angmf large angles / cancellation")
    rng = np.random.default_rng(12)
    inp = _random_inputs(rng, 1, H, W, k)
    inp["angle"] = rng.uniform(-10, 10, inp["angle"].shape).astype(np.float32)
    # cancellation: pixels in the left half take probs 1 on two opposite
    # neighbours' normals -- the normal field alternates sign.
    pn = inp["pred_norm"].reshape(3, H, W)
    pn[:, :, ::2] *= -1
    got = run_gpu(inp, H, W, cuda)
    want = run_oracle(inp, H, W, k)
    max_abs, max_deg, nan_mm = compare(got.reshape(1, 3, -1), want.reshape(1, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG


def _cancel_count(inp, H, W, k, thresh):
    """Pixels whose prob-weighted sum nearly cancels: |acc|^2 < thresh *
    sum(prob^2), acc from the independent restatement.  sum(wi^2) >= sum(prob^2),
    so each of them is below the fast path's own |acc|^2 / sum(wi^2) test."""
    from tests.golden import independent as ind
    B = inp["pred_norm"].shape[0]
    shp = lambda a, c: np.asarray(a).reshape(-1, c, H, W)
    _, acc = ind.refine_step(shp(inp["pred_norm"], 3), shp(inp["prob"], k * k),
                             shp(inp["xy"], 2 * k * k), shp(inp["angle"], k * k),
                             shp(inp["ray"], 3), inp["intrinsics"], k)
    a2 = (acc ** 2).sum(axis=1)
    p2 = (shp(inp["prob"], k * k).astype(np.float64) ** 2).sum(axis=1)
    return int((a2 < thresh * p2).sum())


@pytest.mark.parametrize("far_angles", [False, True])
def test_angmf_recompute_tiers(cuda, far_angles):
    """Sums that nearly cancel, by construction: normals +-x alternating
    column by column, prob 1 on two horizontally adjacent slots (opposite
    normals) and 0 elsewhere, small angles.  Near the principal column both
    terms are RayReLU-clamped to ~ +-x + eps*r, so |acc|^2 / sum(wi^2) ~ 2e-4:
    tier 1 flags those pixels and tier 2 (the reduced form in double)
    recomputes them.  With far_angles a zero-prob slot of every pixel gets an
    angle of 5 rad, outside tier 2's domain, so every flagged pixel goes on
    to tier 3 (the reference-order body)."""
    H, W, k = 24, 64, 5
    K2 = k * k
    say(f"[gpu] angmf recompute tiers far_angles={far_angles}")
    rng = np.random.default_rng(21 + far_angles)
    inp = _random_inputs(rng, 1, H, W, k)
    pn = np.zeros((3, H, W), np.float32)
    pn[0] = 1.0
    pn[:, :, 1::2] *= -1
    inp["pred_norm"] = pn.reshape(1, 3, H * W)
    prob = np.zeros((1, K2, H * W), np.float32)
    prob[0, 2 * k + 2] = 0.8      # the pixel itself
    prob[0, 2 * k + 3] = 0.8      # its right-hand neighbour: the opposite normal
    inp["prob"] = prob
    inp["angle"] = rng.normal(0.0, 1e-3, inp["angle"].shape).astype(np.float32)
    if far_angles:
        inp["angle"][0, 0] = 5.0  # slot 0 has prob 0
    n_cancel = _cancel_count(inp, H, W, k, _lib.angmf_recompute_ratio(k))
    say(f"    pixels below the fast path's cancellation threshold: >= {n_cancel}")
    assert n_cancel >= 2 * H
    got = run_gpu(inp, H, W, cuda)
    want = run_oracle(inp, H, W, k)
    max_abs, max_deg, nan_mm = compare(got.reshape(1, 3, -1), want.reshape(1, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG


@pytest.mark.parametrize("fov", [100.0, 140.0, 170.0])
def test_angmf_wide_fields_of_view(cuda, fov):
    """The fp32 path's error bound holds up to |P0| = 4 over the image (about
    150 degrees diagonally); a 170-degree view runs the double kernel."""
    H, W, k = 40, 40, 5
    say(f"[gpu] angmf field of view {fov}")
    rng = np.random.default_rng(int(fov))
    inp = _random_inputs(rng, 1, H, W, k)
    intr = wl.intrins_from_fov(8 * H, 8 * W, fov)
    inp["intrinsics"] = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    inp["ray"] = wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, H * W)
    got = run_gpu(inp, H, W, cuda)
    want = run_oracle(inp, H, W, k)
    max_abs, max_deg, nan_mm = compare(got.reshape(1, 3, -1), want.reshape(1, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG


def test_angmf_odd_intrinsics_use_fp64(cuda):
    """Intrinsics outside the fp32 path's range run the double kernel."""
    H, W, k = 9, 11, 3
    say("[gpu] angmf extreme intrinsics")
    rng = np.random.default_rng(13)
    inp = _random_inputs(rng, 1, H, W, k)
    inp["intrinsics"] = (1e-5, 3.0, 2e8, -4.0)
    got = run_gpu(inp, H, W, cuda)
    want = run_oracle(inp, H, W, k)
    max_abs, max_deg, nan_mm = compare(got.reshape(1, 3, -1), want.reshape(1, 3, -1))
    assert nan_mm == 0
    assert max_abs <= 2.5e-7


# (4 pixels per lane where H*W is a multiple of 4 and the planes are 16-byte
# aligned; one otherwise: 33 x 17, and the shifted normal)
@pytest.mark.parametrize("B,H,W,shift", [(1, 60, 80, 0), (1, 256, 256, 0), (4, 33, 17, 0),
                                         (1, 1, 1, 0), (2, 64, 64, 1), (3, 16, 20, 0)])
def test_ray_relu(cuda, B, H, W, shift):
    import torch
    say(f"[gpu] ray_relu B={B} {H}x{W} shift={shift}")
    rng = np.random.default_rng(21 + H)
    HW = H * W
    intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    ray = wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, HW)
    n = rng.standard_normal((B, 3, HW)).astype(np.float32)
    # nearly antiparallel to the ray, the ill-conditioned end of the clamp
    m = min(HW, 50)
    n[0, :, :m] = -ray[:, :m] + 1e-4 * rng.standard_normal((3, m)).astype(np.float32)
    if B == 3:
        # one ray map per sample (ray_bstride 3*H*W)
        ray = np.stack([ray, ray[[1, 0, 2]], ray[[0, 2, 1]]]).astype(np.float32)
    g = Guarded(n.size, cuda, shift=shift, fill=n)
    dsine.ray_relu(g.out, to_dev(ray, cuda), H, W)
    torch.cuda.synchronize()
    assert g.intact(), "ray_relu wrote outside its tensor"
    got = g.out.cpu().numpy().reshape(n.shape)
    want = oracle.ray_relu(n, ray, H, W)
    max_abs, max_deg, nan_mm = compare(got, want)
    say(f"    max-abs {max_abs:.3e}")
    assert nan_mm == 0
    assert max_abs <= 2.5e-7


GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                       "angmf_*.npz")))


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_angmf_golden_fixture(cuda, path):
    d = np.load(path)
    H, W, k = int(d["H"]), int(d["W"]), int(d["k"])
    say(f"[gpu] angmf golden {os.path.basename(path)}")
    inp = {key: d[key] for key in ("pred_norm", "prob", "xy", "angle", "ray")}
    inp["intrinsics"] = tuple(d["intr"])
    B = inp["pred_norm"].shape[0]
    got = run_gpu(inp, H, W, cuda, ray=d["ray"].reshape(-1))
    max_abs, max_deg, nan_mm = compare(got.reshape(B, 3, -1), d["expect_out"])
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG


def test_cpp_dropin_on_device(cuda):
    """The C++ surface (include/brovisionml/dsine_ops.h) in the refiner's call
    pattern against the oracle (tests/cpp/test_dsine_ops.cpp, gpu mode)."""
    import subprocess
    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build", "test_dsine_ops")
    say("[gpu] C++ drop-in test_dsine_ops gpu")
    proc = subprocess.run([exe, "gpu"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                          timeout=110)
    say(proc.stdout)
    assert proc.returncode == 0, proc.stdout
