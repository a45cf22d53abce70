"""GPU parity of the fused convex upsample + L2-normalise
(bvml_dsine_convex_upsample_f32) against the CPU oracle's double-precision
restatement of the refiner's step (src/dsine_refine.cpp:276-282, arithmetic of
include/brovisionml/dsine_refine.h:91-97), on the same seeded fp32 inputs.

Bar: max-abs 1e-5 per component and 0.01 degrees (C = 3) for the fast path;
the double-precision kernel (BVML_DSINE_FP64) within 2 float ulps.  NaN
patterns must match exactly.  Unnormalised outputs: 1e-6 * max(1, max|x|).
"""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest

import oracle
from brovisionml_amd import dsine
from tests._util import Guarded, TOL_ABS, TOL_DEG, compare, to_dev
from tests.test_gpu_parity import NTHREADS, say

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
EPS = float(np.float32(1e-12))


def _inputs(rng, B, C, H, W, s, sigma=2.0, unit=True):
    x = rng.standard_normal((B, C, H, W))
    if unit:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
    mask = sigma * rng.standard_normal((B, 9 * s * s, H, W))
    return x.astype(np.float32), mask.astype(np.float32)


def run_gpu(x, mask, s, device, normalize=True, precise=False, eps=EPS, misalign=False):
    import torch
    B, C, H, W = x.shape
    xt, mt = to_dev(x, device), to_dev(mask, device)
    n = B * C * s * s * H * W
    # guarded out; misalign: its address 4 bytes past 16-byte alignment
    g = Guarded(n, device, shift=1 if misalign else 0)
    if normalize:
        r = dsine.convex_upsample_normalize(xt, mt, B, C, H, W, s, eps, g.out, precise=precise)
    else:
        r = dsine.convex_upsample(xt, mt, B, C, H, W, s, g.out, precise=precise)
    torch.cuda.synchronize()
    assert g.intact(), "convex upsample wrote outside its output"
    return r.cpu().numpy().reshape(B, C, s * H, s * W)


def run_oracle(x, mask, s, normalize=True, eps=EPS):
    B, C, H, W = x.shape
    return oracle.convex_upsample(x, mask, H, W, s, normalize=normalize, eps=eps,
                                  nthreads=NTHREADS)


def check(got, want, normalize=True, scale=1.0, exact=False):
    B, C = got.shape[:2]
    g, w = got.reshape(B, C, -1), want.reshape(B, C, -1)
    nan_mm = int((np.isnan(g) != np.isnan(w)).sum())
    fin = ~(np.isnan(g) | np.isnan(w))
    d = np.abs(g.astype(np.float64) - w.astype(np.float64))[fin]
    max_abs = float(d.max()) if d.size else 0.0
    msg = f"    max-abs {max_abs:.3e}  nan-mismatch {nan_mm}"
    if normalize and C == 3:
        _, max_deg, _ = compare(g, w.astype(np.float32))
        msg += f"  max-angle {max_deg:.3e} deg"
        assert max_deg <= TOL_DEG
    say(msg)
    assert nan_mm == 0
    if exact:
        ulp = np.spacing(np.abs(w.astype(np.float32)))[fin]
        assert (d <= 2 * ulp + 1e-45).all(), float((d / np.maximum(ulp, 1e-45)).max())
    elif normalize:
        assert max_abs <= TOL_ABS
    else:
        assert max_abs <= 1e-6 * max(1.0, scale)


# (B, C, H, W, s): the refiner's shapes (C = 3, s = 8, the /8 grid of 480x640
# and 2048x2048 images), ragged widths (pixel groups that straddle rows and
# partial last groups), other channel counts, a batch, and other scales
# (the generic kernel).  At s = 8, H*W a multiple of 4 takes the LDS-staged
# kernel (60x80: a partial last 128-pixel group; 3x4 and 2x2: fewer pixels
# than one group; 16x24: whole groups, B = 3), other H*W the register kernel.
CASES = [
    (1, 3, 60, 80, 8), (1, 3, 256, 256, 8), (2, 3, 7, 13, 8), (1, 1, 5, 3, 8),
    (1, 2, 33, 17, 8), (1, 4, 9, 65, 8), (3, 3, 1, 1, 8), (1, 3, 2, 31, 8),
    (1, 3, 3, 4, 8), (2, 1, 20, 20, 8), (1, 2, 12, 36, 8), (1, 4, 17, 12, 8),
    (3, 3, 16, 24, 8), (2, 3, 2, 2, 8),
    (1, 3, 10, 12, 4), (2, 2, 6, 7, 2), (1, 3, 5, 5, 1), (1, 3, 4, 6, 16), (1, 4, 3, 3, 3),
]


@pytest.mark.parametrize("B,C,H,W,s", CASES)
@pytest.mark.parametrize("normalize", [True, False])
def test_upsample_random(cuda, B, C, H, W, s, normalize):
    say(f"[gpu] upsample random B={B} C={C} {H}x{W} s={s} normalize={normalize}")
    rng = np.random.default_rng(1000 + 7 * H + W + s + C)
    x, mask = _inputs(rng, B, C, H, W, s)
    got = run_gpu(x, mask, s, cuda, normalize)
    want = run_oracle(x, mask, s, normalize)
    check(got, want, normalize)


@pytest.mark.parametrize("B,C,H,W,s", [(1, 3, 60, 80, 8), (2, 3, 7, 13, 8), (1, 2, 10, 12, 4)])
@pytest.mark.parametrize("normalize", [True, False])
def test_upsample_fp64_kernel(cuda, B, C, H, W, s, normalize):
    say(f"[gpu] upsample fp64 B={B} C={C} {H}x{W} s={s} normalize={normalize}")
    rng = np.random.default_rng(77 + H + s)
    x, mask = _inputs(rng, B, C, H, W, s)
    got = run_gpu(x, mask, s, cuda, normalize, precise=True)
    want = run_oracle(x, mask, s, normalize)
    check(got, want, normalize, exact=True)


@pytest.mark.parametrize("sigma", [0.0, 0.05, 8.0, 40.0])
def test_upsample_mask_scales(cuda, sigma):
    """Uniform weights (sigma 0), nearly uniform, peaked and one-hot-like."""
    say(f"[gpu] upsample mask sigma={sigma}")
    rng = np.random.default_rng(int(sigma * 10) + 5)
    x, mask = _inputs(rng, 1, 3, 24, 40, 8, sigma=sigma)
    check(run_gpu(x, mask, 8, cuda), run_oracle(x, mask, 8))


def test_upsample_cancellation(cuda):
    """Neighbours that nearly cancel (a checkerboard of +n / -n with small
    perturbations, and exactly antipodal pairs): the sub-pixels whose sum is
    small against the error bound take the double-precision body."""
    say("[gpu] upsample cancellation")
    rng = np.random.default_rng(9)
    H, W, s = 20, 24, 8
    n = np.array([0.3, -0.5, 0.81], dtype=np.float64)
    n /= np.linalg.norm(n)
    sign = np.where((np.add.outer(np.arange(H), np.arange(W)) % 2) == 0, 1.0, -1.0)
    x = sign[None, None] * n[None, :, None, None] + 1e-4 * rng.standard_normal((1, 3, H, W))
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    x = x.astype(np.float32)
    mask = (0.3 * rng.standard_normal((1, 9 * s * s, H, W))).astype(np.float32)
    mask[:, :, ::3, ::5] = 0.0  # exactly uniform weights at some pixels
    check(run_gpu(x, mask, s, cuda), run_oracle(x, mask, s))


def test_upsample_special_values(cuda):
    """NaN in the mask poisons exactly its sub-pixel; NaN in x poisons the
    sub-pixels that read it; +inf mask logits give NaN (inf - inf), -inf
    logits weigh zero; all as the oracle (torch softmax semantics)."""
    say("[gpu] upsample special values")
    rng = np.random.default_rng(10)
    H, W, s = 6, 7, 8
    x, mask = _inputs(rng, 1, 3, H, W, s)
    mask[0, 4 * 64 + 3 * 8 + 5, 2, 3] = np.nan
    mask[0, 0 * 64 + 1 * 8 + 0, 4, 4] = np.inf
    mask[0, 7 * 64 + 2 * 8 + 2, 1, 1] = -np.inf
    mask[0, 2 * 64 + 6 * 8 + 7, 5, 6] = -np.inf
    x[0, 1, 3, 2] = np.nan
    # exact cancellation: sub-pixel (0, 0) of pixel (1, 5) weighs only its left
    # and right taps, equally, and they are opposite: |v| = 0, out = 0 / eps
    mask[0, 0:9 * 64:64, 1, 5] = -np.inf
    mask[0, 3 * 64, 1, 5] = mask[0, 5 * 64, 1, 5] = 0.0
    x[0, :, 1, 6] = -x[0, :, 1, 4]
    for normalize in (True, False):
        got = run_gpu(x, mask, s, cuda, normalize)
        want = run_oracle(x, mask, s, normalize)
        assert np.isnan(want).any()
        assert (want[0, :, 1 * s, 5 * s] == 0).all()
        check(got, want, normalize)


@pytest.mark.parametrize("scale", [1e-14, 1e-7, 1e18])
def test_upsample_magnitudes(cuda, scale):
    """Inputs scaled far from unit length: below eps the normalise divides by
    eps (the output is not unit length); large ones leave fp32's |v|^2 range."""
    say(f"[gpu] upsample magnitude {scale:g}")
    rng = np.random.default_rng(11)
    x, mask = _inputs(rng, 1, 3, 9, 10, 8)
    x = (x.astype(np.float64) * scale).astype(np.float32)
    check(run_gpu(x, mask, 8, cuda), run_oracle(x, mask, 8))
    check(run_gpu(x, mask, 8, cuda, normalize=False), run_oracle(x, mask, 8, normalize=False),
          normalize=False, scale=scale)


@pytest.mark.parametrize("eps", [0.0, 0.5, 1e30])
def test_upsample_eps(cuda, eps):
    say(f"[gpu] upsample eps={eps:g}")
    rng = np.random.default_rng(12)
    x, mask = _inputs(rng, 1, 3, 8, 8, 8)
    eps32 = float(np.float32(eps))
    check(run_gpu(x, mask, 8, cuda, eps=eps32), run_oracle(x, mask, 8, eps=eps32))


def test_upsample_unaligned_out(cuda):
    """An `out` 4 bytes past 16-byte alignment takes the any-scale kernel at
    s = 8; its result equals the aligned call's to the bit."""
    say("[gpu] upsample unaligned out")
    rng = np.random.default_rng(13)
    x, mask = _inputs(rng, 2, 3, 11, 37, 8)
    a = run_gpu(x, mask, 8, cuda)
    b = run_gpu(x, mask, 8, cuda, misalign=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    check(b, run_oracle(x, mask, 8))


@pytest.mark.parametrize("B,C,H,W", [(1, 3, 60, 80), (2, 1, 20, 20), (1, 4, 17, 12), (2, 3, 2, 2)])
@pytest.mark.parametrize("normalize,precise,bias", [(True, False, False), (False, False, False),
                                                    (True, True, False), (True, False, True)])
def test_upsample_staged_matches_register_kernel(cuda, B, C, H, W, normalize, precise, bias):
    """At s = 8 the LDS-staged kernel (a 16-byte-aligned mask and H*W a
    multiple of 4) and the register kernel (the same mask 4 bytes past
    16-byte alignment) compute every sub-pixel in the same order: the same
    bits, fast and double paths, with and without a mask bias."""
    import torch
    say(f"[gpu] upsample staged vs register kernel B={B} C={C} {H}x{W} normalize={normalize} "
        f"precise={precise} bias={bias}")
    rng = np.random.default_rng(400 + H + W + C + 3 * precise + 5 * bias)
    x, mask = _inputs(rng, B, C, H, W, 8)
    xt = to_dev(x, cuda)
    n = mask.size
    buf = torch.empty(n + 4, dtype=torch.float32, device=cuda)
    assert buf.data_ptr() % 16 == 0
    aligned = buf[:n].view(mask.shape)
    shifted = buf[1:n + 1].view(mask.shape)
    bt = to_dev((3.0 * rng.standard_normal(576)).astype(np.float32), cuda) if bias else None
    outs = []
    for m in (aligned, shifted):
        m.copy_(torch.from_numpy(mask))
        g = Guarded(B * C * 64 * H * W, cuda)
        if normalize:
            r = dsine.convex_upsample_normalize(xt, m, B, C, H, W, 8, EPS, g.out,
                                                precise=precise, mask_bias=bt)
        else:
            r = dsine.convex_upsample(xt, m, B, C, H, W, 8, g.out, precise=precise, mask_bias=bt)
        torch.cuda.synchronize()
        assert g.intact(), "convex upsample wrote outside its output"
        outs.append(r.cpu().numpy().reshape(B, C, 8 * H, 8 * W))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    if not bias:
        check(outs[0], run_oracle(x, mask, 8, normalize), normalize, exact=precise)


def test_upsample_many_samples(cuda):
    """More samples than one launch's grid y holds (65535): the second launch
    starts at the right sample."""
    B = 65537
    say(f"[gpu] upsample B={B} 1x1")
    rng = np.random.default_rng(14)
    x, mask = _inputs(rng, B, 3, 1, 1, 8)
    check(run_gpu(x, mask, 8, cuda), run_oracle(x, mask, 8))


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "upsample_*.npz"))),
                         ids=lambda p: os.path.basename(p)[:-4])
def test_upsample_golden(cuda, path):
    """The committed fixtures (inputs and the independent float64 torch
    restatement's outputs)."""
    say(f"[gpu] upsample golden {os.path.basename(path)}")
    d = np.load(path)
    s, normalize = int(d["s"]), bool(int(d["normalize"]))
    got = run_gpu(d["x"], d["mask"], s, cuda, normalize)
    check(got, d["expect"], normalize, scale=float(np.abs(d["x"]).max()))


@pytest.mark.parametrize("s,misalign", [(8, False), (8, True), (4, False)])
@pytest.mark.parametrize("normalize,precise", [(True, False), (False, False), (True, True)])
def test_upsample_mask_bias(cuda, s, misalign, normalize, precise):
    """A per-channel mask bias added in the kernel (the up-mask head's last
    bias, bvml_dsine_convex_upsample_bias_f32) equals the call on the mask
    with the bias added beforehand in fp32, bit for bit: the s = 8 kernel, its
    unaligned-out fallback and another scale, fast and double paths; the
    result is also within the bar of the oracle on the biased mask."""
    import torch
    say(f"[gpu] upsample mask bias s={s} misalign={misalign} normalize={normalize} "
        f"precise={precise}")
    rng = np.random.default_rng(300 + s + 2 * misalign + 4 * normalize + 8 * precise)
    B, C, H, W = 2, 3, 7, 13
    x, mask = _inputs(rng, B, C, H, W, s)
    bias = (3.0 * rng.standard_normal(9 * s * s)).astype(np.float32)
    biased = (mask + bias[None, :, None, None]).astype(np.float32)
    want = run_gpu(x, biased, s, cuda, normalize, precise, misalign=misalign)
    xt, mt, bt = to_dev(x, cuda), to_dev(mask, cuda), to_dev(bias, cuda)
    g = Guarded(B * C * s * s * H * W, cuda, shift=1 if misalign else 0)
    if normalize:
        r = dsine.convex_upsample_normalize(xt, mt, B, C, H, W, s, EPS, g.out, precise=precise,
                                            mask_bias=bt)
    else:
        r = dsine.convex_upsample(xt, mt, B, C, H, W, s, g.out, precise=precise, mask_bias=bt)
    torch.cuda.synchronize()
    assert g.intact(), "convex upsample wrote outside its output"
    got = r.cpu().numpy().reshape(B, C, s * H, s * W)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    check(got, run_oracle(x, biased, s, normalize), normalize, exact=precise)
