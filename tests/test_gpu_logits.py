"""GPU parity of BVML_DSINE_LOGITS: angmf_propagate on the prob and angle
heads' raw logits, the kernel applying the refiner's activations
(src/dsine_refine.cpp:262-267: apply_sigmoid(prob); apply_sigmoid(angle);
scale_inplace(angle, kPi), kPi the float pi of src/dsine_refine.cpp:26).

The expected output is the oracle's on the correctly rounded float
activations: sigmoid in double rounded once to float, the angle the float
product of that with float(pi).  Same bar as the plain op."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from brovisionml_amd import dsine, workloads as wl
from tests._util import TOL_ABS, TOL_DEG, Guarded, compare, to_dev

pytestmark = pytest.mark.gpu

F32_PI = np.float32(3.14159265358979323846)


def say(msg: str) -> None:
    print(msg, flush=True)


def activate(prob_logits, angle_logits):
    """The refiner's activations as correctly rounded floats."""
    with np.errstate(over="ignore"):
        sp = (1.0 / (1.0 + np.exp(-np.asarray(prob_logits, np.float64)))).astype(np.float32)
        sa = (1.0 / (1.0 + np.exp(-np.asarray(angle_logits, np.float64)))).astype(np.float32)
    ang = (sa.astype(np.float64) * np.float64(F32_PI)).astype(np.float32)
    return sp, ang


def logit(p):
    p = np.asarray(p, np.float64)
    return np.log(p / (1.0 - p))


def run(inp, lp, la, H, W, k, device, precise=False):
    import torch
    t = {key: to_dev(inp[key], device) for key in ("pred_norm", "xy", "ray")}
    fu, cu, fv, cv = inp["intrinsics"]
    g = Guarded(t["pred_norm"].numel(), device)
    out = dsine.angmf_propagate(t["pred_norm"], to_dev(lp, device), t["xy"], to_dev(la, device),
                                t["ray"], fu, cu, fv, cv, H, W, g.out, precise=precise,
                                logits=True)
    torch.cuda.synchronize()
    assert g.intact(), "angmf_propagate (logits) wrote outside its output"
    got = out.cpu().numpy().reshape(t["pred_norm"].shape)
    sp, ang = activate(lp, la)
    want = oracle.angmf_propagate(inp["pred_norm"], sp, inp["xy"], ang, inp["ray"],
                                  inp["intrinsics"], H, W, k, nthreads=16)
    return got, want


@pytest.mark.parametrize("idx", [0, 2, 3])
@pytest.mark.parametrize("precise", [False, True])
def test_logits_workload(cuda, idx, precise):
    """The workloads' prob and angle planes turned back into logits (the
    angle planes through angle / pi), so the activated inputs are the
    workloads' own up to rounding."""
    w = wl.WORKLOADS[idx]
    say(f"[gpu] angmf logits {w.name} precise={precise}")
    inp = wl.make_inputs(w)
    lp = logit(np.clip(inp["prob"], 1e-6, 1 - 1e-6)).astype(np.float32)
    la = logit(np.clip(inp["angle"] / np.pi, 1e-6, 1 - 1e-6)).astype(np.float32)
    got, want = run(inp, lp, la, w.H, w.W, w.k, cuda, precise)
    max_abs, max_deg, nan_mm = compare(got.reshape(w.B, 3, -1), want.reshape(w.B, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
    assert nan_mm == 0
    assert max_abs <= (2.5e-7 if precise else TOL_ABS) and max_deg <= TOL_DEG


@pytest.mark.parametrize("scale", [0.3, 3.0, 30.0])
def test_logits_scales(cuda, scale):
    """Random logits N(0, scale^2): from nearly-constant activations to
    saturated ones (sigmoid at 0 and 1, angles at 0 and pi)."""
    H, W, k = 40, 56, 5
    say(f"[gpu] angmf logits scale {scale}")
    rng = np.random.default_rng(int(scale * 10))
    w = wl.Workload(0, "logits", 1, H, W, k, 1, "normal:0.1", "sphere", 7)
    inp = wl.make_inputs(w)
    lp = (rng.standard_normal(inp["prob"].shape) * scale).astype(np.float32)
    la = (rng.standard_normal(inp["angle"].shape) * scale).astype(np.float32)
    got, want = run(inp, lp, la, H, W, k, cuda)
    max_abs, max_deg, nan_mm = compare(got.reshape(1, 3, -1), want.reshape(1, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG


def test_logits_special_values(cuda):
    """+-inf, NaN and extreme logits: sigmoid exactly 0 or 1 (a zero weight, a
    zero or pi angle), NaN propagating as the activated planes would."""
    H, W, k = 12, 16, 5
    say("[gpu] angmf logits special values")
    rng = np.random.default_rng(33)
    w = wl.Workload(0, "logits-special", 1, H, W, k, 1, "normal:0.1", "sphere", 8)
    inp = wl.make_inputs(w)
    lp = rng.standard_normal(inp["prob"].shape).astype(np.float32)
    la = rng.standard_normal(inp["angle"].shape).astype(np.float32)
    vals = np.array([np.inf, -np.inf, 100.0, -100.0, 87.5, -87.5, -200.0, 1e30, -1e30],
                    np.float32)
    for i, v in enumerate(vals):
        lp[0, i, 10 + i] = v
        la[0, (i + 3) % 25, 40 + i] = v
    lp[0, :, 60] = -np.inf          # every weight 0: output exactly 0
    lp[0, 5, 70] = np.nan           # NaN output
    la[0, 6, 80] = np.nan           # NaN output
    got, want = run(inp, lp, la, H, W, k, cuda)
    max_abs, max_deg, nan_mm = compare(got.reshape(1, 3, -1), want.reshape(1, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg  nan-mismatch {nan_mm}")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG
    assert np.all(got.reshape(3, -1)[:, 60] == 0)


def _random_logit_inputs(seed, B, H, W, k):
    rng = np.random.default_rng(seed + B * 1000 + H * 10 + W + k)
    HW, K2 = H * W, k * k
    n = rng.standard_normal((B, 3, HW))
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    fuv = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    inp = {
        "pred_norm": n.astype(np.float32),
        "xy": rng.standard_normal((B, 2 * K2, HW)).astype(np.float32),
        "ray": wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, HW),
        "intrinsics": fuv,
    }
    lp = (2.0 * rng.standard_normal((B, K2, HW))).astype(np.float32)
    la = (2.0 * rng.standard_normal((B, K2, HW))).astype(np.float32)
    return inp, lp, la


@pytest.mark.parametrize("B,H,W,k", [(2, 9, 13, 1), (1, 33, 65, 3), (1, 20, 140, 5),
                                     (2, 17, 70, 7), (1, 12, 20, 9), (1, 6, 100, 9),
                                     (2, 512, 512, 5), (3, 500, 333, 7), (1, 800, 800, 5)])
def test_logits_window_sizes(cuda, B, H, W, k):
    """Every window size's logits kernel (the workloads above are all k = 5):
    random logits N(0, 2^2) for prob and angle, so the activated angles
    span (0, pi), on narrow and wide tiles and (the last three) the
    whole-window kernel, with non-temporal plane loads at 3 x 500 x 333 and
    800 x 800."""
    say(f"[gpu] angmf logits shape B={B} H={H} W={W} k={k}")
    inp, lp, la = _random_logit_inputs(700, B, H, W, k)
    got, want = run(inp, lp, la, H, W, k, cuda)
    max_abs, max_deg, nan_mm = compare(got.reshape(B, 3, -1), want.reshape(B, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG


@pytest.mark.parametrize("B,H,W,k", [(1, 20, 200, 5), (2, 9, 13, 7), (2, 512, 512, 5),
                                     (1, 800, 800, 5)])
@pytest.mark.parametrize("precise", [False, True])
def test_logits_ray_from_intrinsics(cuda, B, H, W, k, precise):
    """Logits with the ray formed in the kernel (BVML_DSINE_LOGITS |
    BVML_DSINE_RAY_FROM_INTRINSICS): bit-identical to the same call on
    build_ray8's planes, which the oracle checks."""
    import torch
    say(f"[gpu] angmf logits, ray from intrinsics B={B} {H}x{W} k={k} precise={precise}")
    inp, lp, la = _random_logit_inputs(900, B, H, W, k)
    got, want = run(inp, lp, la, H, W, k, cuda, precise)
    fu, cu, fv, cv = inp["intrinsics"]
    synth = dsine.angmf_propagate(to_dev(inp["pred_norm"], cuda), to_dev(lp, cuda),
                                  to_dev(inp["xy"], cuda), to_dev(la, cuda), None,
                                  fu, cu, fv, cv, H, W, precise=precise, logits=True)
    torch.cuda.synchronize()
    synth = synth.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), synth.view(np.uint32))
    max_abs, max_deg, nan_mm = compare(got.reshape(B, 3, -1), want.reshape(B, 3, -1))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg")
    assert nan_mm == 0
    assert max_abs <= (2.5e-7 if precise else TOL_ABS) and max_deg <= TOL_DEG
