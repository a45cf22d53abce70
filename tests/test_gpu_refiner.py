"""The refiner loop on the device (brovisionml_amd/refiner.py: Refiner::forward,
src/dsine_refine.cpp:212-294, driving this package's kernels with the ConvGRU
and heads on torch's fp32 convolutions, MIOpen off) against its CPU
restatement (oracle/refiner.py: float64 convolutions, the C oracle's ops),
on synthetic weights and decoder outputs (no checkpoint ships here).

Two checks per iteration:
  * stepwise: the iteration's propagate against the C oracle on the device's
    own inputs (the previous iteration's device output and the device's
    heads, activated as correctly rounded floats): the op's bar, 1e-5;
  * end to end, against the float64 restatement: the returned map within
    5e-6 (the reference reports its whole pipeline "exact to FP32 round-off
    -- max-abs ~2-5e-6", docs/dsine.md:75-77), each iteration's up-sampled
    map within 2e-5, each iteration's propagated /8 normals within 1e-4.
    The heads are fp32 convolutions, here as in the reference, and where a
    pixel's window holds a small xy pair (|(xs, ys)| down to 1e-3 in these
    draws) their ~1e-7 rounding moves that neighbour's rotation axis by
    about 1e-7/|(xs, ys)| rad: measured up to 5.6e-5 on the /8 normals of
    such pixels (and of their neighbours in the next iteration), while every
    pixel whose pairs are all >= 0.05 stays within 4.8e-6.
The convolutions are a fixed algorithm per shape (im2col + an fp32 GEMM), so
the result does not depend on the process's history.  The closed-form pins
below, whose heads are exact, hold 1e-5 through the loop."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from brovisionml_amd import refiner as rf, workloads as wl
from oracle import refiner as oref

pytestmark = pytest.mark.gpu
TOL_STEP = 1e-5     # an iteration's propagate against the oracle on the device's own inputs
TOL_RESULT = 5e-6   # the returned map against the float64 restatement
TOL_UP = 2e-5       # each iteration's up-sampled map against the float64 restatement
TOL_COARSE = 1e-4   # each iteration's /8 normals against the float64 restatement


def say(msg: str) -> None:
    print(msg, flush=True)


def _inputs(H, W, seed):
    rng = np.random.default_rng(seed)
    n = rng.standard_normal((3, H, W))
    n[2] = np.abs(n[2]) + 0.5          # roughly camera-facing, as a decoder's
    n = (n / np.linalg.norm(n, axis=0)).astype(np.float32)
    feature = rng.standard_normal((64, H, W)).astype(np.float32)
    hidden = rng.uniform(-1, 1, (64, H, W)).astype(np.float32)
    return n, feature, hidden


@pytest.mark.parametrize("H,W,fov,seed", [(24, 32, 60.0, 0), (20, 20, 90.0, 1)])
def test_refiner_iterations(cuda, H, W, fov, seed):
    import torch
    say(f"[gpu] refiner {H}x{W} fov {fov}")
    weights = rf.random_weights(seed)
    n, feature, hidden = _inputs(H, W, seed)
    intr = wl.intrins_from_fov(8 * H, 8 * W, fov)
    fuv = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    dev = torch.device(cuda)
    model = rf.Refiner(weights, dev)
    dec = rf.DecoderOutput(*(torch.from_numpy(a)[None].to(dev) for a in (n, feature, hidden)))
    trace, heads = [], []
    out = model.forward(dec, intr, 8 * H, 8 * W, trace=trace, heads_trace=heads)
    torch.cuda.synchronize()
    ray8 = wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, H, W)
    uv8 = rf.uv_map(intr, H, W, 8 * H, 8 * W)
    want_trace = []
    want = oref.refine_forward(weights, n, feature, hidden, intr, fuv, ray8, uv8,
                               trace=want_trace, nthreads=16)
    assert len(trace) == len(heads) == len(want_trace) == rf.N_ITER
    for it, ((gp, gu), (wp, wu), (pin, prob, xy, angle)) in enumerate(
            zip(trace, want_trace, heads)):
        gp = gp.cpu().numpy().reshape(3, H, W)
        step = oracle.angmf_propagate(
            pin.cpu().numpy().reshape(1, 3, -1), oref._sigmoid_f32(prob.cpu().numpy()),
            xy.cpu().numpy(), oref.angle_from_logits(angle.cpu().numpy()), ray8.reshape(3, -1),
            fuv, H, W, rf.PS, nthreads=16).reshape(3, H, W)
        es = float(np.abs(gp.astype(np.float64) - step).max())
        ep = float(np.abs(gp.astype(np.float64) - wp).max())
        eu = float(np.abs(gu.cpu().numpy()[0].astype(np.float64) - wu).max())
        say(f"    iteration {it}: propagate stepwise max-abs {es:.3e}, against float64 "
            f"{ep:.3e}; upsample against float64 {eu:.3e}")
        assert es <= TOL_STEP and ep <= TOL_COARSE and eu <= TOL_UP
    er = float(np.abs(out.cpu().numpy()[0].astype(np.float64) - want).max())
    say(f"    result max-abs {er:.3e}")
    assert er <= TOL_RESULT
    assert out.shape == (1, 3, 8 * H, 8 * W)
    assert np.array_equal(out.cpu().numpy(), trace[-1][1].cpu().numpy())


def test_refiner_crop(cuda):
    """The result cropped to the unpadded image (src/dsine_refine.cpp:289-293)."""
    import torch
    H, W = 12, 16
    weights = rf.random_weights(5)
    n, feature, hidden = _inputs(H, W, 5)
    intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    dev = torch.device(cuda)
    model = rf.Refiner(weights, dev)
    dec = rf.DecoderOutput(*(torch.from_numpy(a)[None].to(dev) for a in (n, feature, hidden)))
    full = model.forward(dec, intr, 8 * H, 8 * W)
    crop = rf.Crop(orig_h=8 * H - 11, orig_w=8 * W - 6, pad_t=5, pad_l=3)
    part = model.forward(dec, intr, 8 * H, 8 * W, crop=crop)
    torch.cuda.synchronize()
    assert part.shape == (1, 3, crop.orig_h, crop.orig_w)
    assert np.array_equal(part.cpu().numpy(),
                          full.cpu().numpy()[:, :, 5:5 + crop.orig_h, 3:3 + crop.orig_w])


# ---- closed-form pins (tests/refiner_pins.py), independent of the restatement
def _gpu_run(pin, n0=0, H=24, W=32, fov=60.0, seed=7):
    import torch
    from tests import refiner_pins as pins
    n, feature, hidden, intr, fuv, ray8, uv8 = pins.setup(H, W, fov, seed)
    w, data = pins.pinned_weights(pin, seed, n0=n0)
    dev = torch.device("cuda:0")
    model = rf.Refiner(w, dev)
    dec = rf.DecoderOutput(*(torch.from_numpy(a)[None].to(dev) for a in (n, feature, hidden)))
    trace, htrace = [], []
    model.forward(dec, intr, 8 * H, 8 * W, trace=trace, hidden_trace=htrace)
    torch.cuda.synchronize()
    trace = [(p.cpu().numpy().reshape(3, H, W), u.cpu().numpy()[0]) for p, u in trace]
    htrace = [h.cpu().numpy()[0] for h in htrace]
    return trace, htrace, data, (n, hidden, fuv, ray8)


def test_pin_gate_closed(cuda):
    """convz saturated shut: every iteration's h_new is the decoder's hidden."""
    say("[gpu] refiner pin: gate closed")
    _, htrace, _, (_, hidden, _, _) = _gpu_run("gate_closed")
    err = max(float(np.abs(h - hidden).max()) for h in htrace)
    say(f"    max-abs {err:.3e}")
    assert err <= 1e-5


def test_pin_gate_open(cuda):
    """convz saturated open and convq weight 0: h_new = tanh(convq's bias)."""
    say("[gpu] refiner pin: gate open")
    _, htrace, data, _ = _gpu_run("gate_open")
    want = np.tanh(data["bq"].astype(np.float64))[:, None, None]
    err = max(float(np.abs(h - want).max()) for h in htrace)
    say(f"    max-abs {err:.3e}")
    assert err <= 1e-5


def test_pin_constant_heads(cuda):
    """Heads reduced to their biases: each iteration is one direct propagate
    of constant planes, as the C oracle computes it."""
    from tests import refiner_pins as pins
    say("[gpu] refiner pin: constant heads")
    trace, _, data, (n, _, fuv, ray8) = _gpu_run("const_heads")
    H, W = n.shape[1:]
    want = pins.const_heads_expected(data, n, ray8, fuv, H, W, chain=[p for p, _ in trace])
    for it, ((p, _), w) in enumerate(zip(trace, want)):
        err = float(np.abs(p.astype(np.float64) - w).max())
        say(f"    iteration {it}: max-abs {err:.3e}")
        assert err <= 1e-5


@pytest.mark.parametrize("n0", [0, 5, 7])
def test_pin_onehot_upsample(cuda, n0):
    """A one-hot up_prob_head bias: the up-sampled map is the normalised
    propagate output at each pixel's clamped tap."""
    from tests import refiner_pins as pins
    say(f"[gpu] refiner pin: one-hot up mask, tap {n0}")
    trace, _, _, _ = _gpu_run("onehot_up", n0=n0)
    err = max(float(np.abs(u - pins.onehot_up_expected(p, n0)).max()) for p, u in trace)
    say(f"    max-abs {err:.3e}")
    assert err <= 1e-5
