"""bvml_dsine_refiner_forward_noalloc (include/bvml_dsine_refine.h: the native
refiner's forward on maps in a fixed device array, for callers that cannot
allocate) against bvml_dsine_refiner_forward on the same weights and maps:
two allocation-free calls in a row, the second on a smaller grid with a crop,
each bit-identical to the allocating forward (the same kernels at the same
launch shapes), the first also against the float64 restatement (the result
within 5e-6, each iteration's /8 normals within 1e-4, the refiner's bars,
tests/test_gpu_refiner.py); two
calls on two streams with no synchronisation between them (the library puts
calls on one GPU in order); then its refusals (a grid beyond the array,
weights not on the device)."""
from __future__ import annotations

import numpy as np
import pytest

from brovisionml_amd import _lib, refiner as rf, workloads as wl
from oracle import refiner as oref
from tests import refiner_pins as pins

pytestmark = pytest.mark.gpu
TOL_RESULT = 5e-6   # the returned map against the float64 restatement
TOL_COARSE = 1e-4   # each iteration's /8 normals against the float64 restatement


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
        assert torch.equal(go, wo) and torch.equal(gc, wc)
    # the first against the float64 restatement
    H, W, arrays, _, intr, _ = cases[0]
    fuv = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    trace = []
    oref.refine_forward(weights, *arrays, intr, fuv,
                        wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, H, W),
                        rf.uv_map(intr, H, W, 8 * H, 8 * W), trace=trace, nthreads=16)
    gc = got[0][1].cpu().numpy()
    for it, (wp, _) in enumerate(trace):
        assert np.abs(gc[it].astype(np.float64) - wp).max() <= TOL_COARSE, it
    eu = float(np.abs(got[0][0].cpu().numpy()[0].astype(np.float64) - trace[-1][1]).max())
    say(f"    60x80 against the float64 restatement: result max-abs {eu:.3e}")
    assert eu <= TOL_RESULT


def test_noalloc_calls_on_two_streams(cuda):
    """Two allocation-free calls on two streams, enqueued back to back with no
    synchronisation between them: both use the GPU's one scratch array, so
    the second waits for the first, and each gives the allocating forward's
    result, bit for bit."""
    import torch
    weights = rf.random_weights(23)
    model = rf.NativeRefiner(weights)
    H, W = 40, 48
    cases = []
    for seed, fov in ((23, 60.0), (24, 75.0)):
        cases.append((_dec(pins.inputs(H, W, seed)), wl.intrins_from_fov(8 * H, 8 * W, fov)))
    c = rf.Crop(8 * H, 8 * W)
    want = [model.forward(dec, intr, 8 * H, 8 * W) for dec, intr in cases]
    outs = [torch.full((1, 3, 8 * H, 8 * W), float("nan"), device=cuda) for _ in cases]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for (dec, intr), out, s in zip(cases, outs, streams):
        say(f"[gpu] refiner forward_noalloc {H}x{W} on stream {s.cuda_stream:#x}")
        with torch.cuda.stream(s):
            st = _noalloc(model, dec, intr, 8 * H, 8 * W, c, out)
        assert st == _lib.OK, _lib.refine_last_error()
    torch.cuda.synchronize()
    for out, w in zip(outs, want):
        assert torch.equal(out, w)


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
