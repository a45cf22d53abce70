"""bvml_dsine_refiner_forward_noalloc (include/bvml_dsine_refine.h: the native
refiner's forward on maps in a fixed device array, for callers that cannot
allocate) against bvml_dsine_refiner_forward on the same weights and maps:
two allocation-free calls in a row, the second on a smaller grid with a crop,
each within the refiner's bar (1e-4 per component: the two differ only in
the heads' 3x3 convolution, MIOpen's against this library's), the first also
against the float64 restatement; then its refusals (a grid beyond the
array, weights not on the device)."""
from __future__ import annotations

import numpy as np
import pytest

from brovisionml_amd import _lib, refiner as rf, workloads as wl
from oracle import refiner as oref
from tests import refiner_pins as pins

pytestmark = pytest.mark.gpu
TOL = 1e-4


def say(msg: str) -> None:
    print(msg, flush=True)


def _dec(arrays):
    import torch
    return rf.DecoderOutput(*(torch.from_numpy(a)[None].to("cuda:0") for a in arrays))


def _noalloc(model, dec, intr, orig_h, orig_w, crop, out, coarse=None):
    import torch
    _, _, H, W = dec.normal.shape
    return model._lib.bvml_dsine_refiner_forward_noalloc(
        model._h, dec.normal.data_ptr(), dec.feature.data_ptr(), dec.hidden.data_ptr(), H, W,
        intr.fx, intr.fy, intr.cx, intr.cy, orig_h, orig_w, crop.pad_t, crop.pad_l, crop.orig_h,
        crop.orig_w, out.data_ptr(), coarse.data_ptr() if coarse is not None else None,
        torch.cuda.current_stream().cuda_stream)


def test_noalloc_matches_forward(cuda):
    import torch
    weights = rf.random_weights(17)
    model = rf.NativeRefiner(weights)
    cases = []
    for H, W, seed, crop in ((60, 80, 17, None), (24, 32, 18, rf.Crop(181, 250, 5, 3))):
        arrays = pins.inputs(H, W, seed)
        intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
        c = crop or rf.Crop(8 * H, 8 * W)
        cases.append((H, W, arrays, _dec(arrays), intr, c))
    # the allocating forward first (it also uploads the weights)
    want = [model.forward(dec, intr, 8 * H, 8 * W, crop=c, coarse=True)
            for H, W, _, dec, intr, c in cases]
    torch.cuda.synchronize()
    # two allocation-free calls in a row, the second smaller
    got = []
    for H, W, _, dec, intr, c in cases:
        say(f"[gpu] refiner forward_noalloc {H}x{W} crop {c}")
        out = torch.full((1, 3, c.orig_h, c.orig_w), float("nan"), device=cuda)
        coarse = torch.full((rf.N_ITER, 3, H, W), float("nan"), device=cuda)
        st = _noalloc(model, dec, intr, 8 * H, 8 * W, c, out, coarse)
        assert st == _lib.OK, _lib.refine_last_error()
        got.append((out, coarse))
    torch.cuda.synchronize()
    for (H, W, arrays, _, intr, c), (wo, wc), (go, gc) in zip(cases, want, got):
        eo = float((go - wo).abs().max())
        ec = float((gc - wc).abs().max())
        say(f"    {H}x{W}: result max-abs {eo:.3e}, coarse max-abs {ec:.3e} against forward")
        assert eo <= TOL and ec <= TOL
    # the first against the float64 restatement
    H, W, arrays, _, intr, _ = cases[0]
    fuv = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    trace = []
    oref.refine_forward(weights, *arrays, intr, fuv,
                        wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, H, W),
                        rf.uv_map(intr, H, W, 8 * H, 8 * W), trace=trace, nthreads=16)
    gc = got[0][1].cpu().numpy()
    for it, (wp, _) in enumerate(trace):
        assert np.abs(gc[it].astype(np.float64) - wp).max() <= TOL, it
    eu = float(np.abs(got[0][0].cpu().numpy()[0].astype(np.float64) - trace[-1][1]).max())
    say(f"    60x80 against the float64 restatement: result max-abs {eu:.3e}")
    assert eu <= TOL


def test_noalloc_refusals(cuda):
    import torch
    weights = rf.random_weights(19)
    model = rf.NativeRefiner(weights)
    H, W = 16, 16
    dec = _dec(pins.inputs(H, W, 19))
    intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    c = rf.Crop(8 * H, 8 * W)
    out = torch.empty((1, 3, 8 * H, 8 * W), device=cuda)
    # before any forward: the weights are not on the device
    assert _noalloc(model, dec, intr, 8 * H, 8 * W, c, out) == _lib.EWEIGHTS
    assert "not on the device" in _lib.refine_last_error()
    model.forward(dec, intr, 8 * H, 8 * W)
    assert _noalloc(model, dec, intr, 8 * H, 8 * W, c, out) == _lib.OK
    # a weight changed since: refused until a forward uploads it
    model.set_tensor("gru.convq.bias", weights["gru.convq.bias"] * 0.5)
    assert _noalloc(model, dec, intr, 8 * H, 8 * W, c, out) == _lib.EWEIGHTS
    # a grid beyond the array (no launch: refused before the device is touched)
    model.forward(dec, intr, 8 * H, 8 * W)
    big = _dec(pins.inputs(100, 100, 20))
    intr_big = wl.intrins_from_fov(800, 800, 60.0)
    out_big = torch.empty((1, 3, 800, 800), device=cuda)
    assert _noalloc(model, big, intr_big, 800, 800, rf.Crop(800, 800), out_big) == _lib.ESIZE
    assert "floats of scratch" in _lib.refine_last_error()
    torch.cuda.synchronize()
