"""The native refiner (libbvml_dsine_refine.so, include/bvml_dsine_refine.h:
Refiner::forward of src/dsine_refine.cpp:212-294 in C++) on the device,
against the CPU restatement (oracle/refiner.py: float64 convolutions, the C
oracle's ops), the closed-form pins of tests/refiner_pins.py and the Python
driver (brovisionml_amd/refiner.py), on synthetic weights and decoder maps.

The bars against the float64 restatement are those of
tests/test_gpu_refiner.py: the returned map within 5e-6 (the reference's
"exact to FP32 round-off -- max-abs ~2-5e-6", docs/dsine.md:75-77), each
iteration's propagated /8 normals within 1e-4 (fp32 heads whose rounding a
small xy pair amplifies), 1e-5 where the pins' heads are exact.  Every
convolution of the
native refiner is this library's kernel, whose launch shape depends on the
grid size only, so forwards of the same weights and maps are bit-identical:
in one process, across a change of grid size and back, from a checkpoint
file, and in another process (the C++ class's test binary)."""
from __future__ import annotations

import os

import numpy as np
import pytest

from brovisionml_amd import refiner as rf, workloads as wl
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


@pytest.mark.parametrize("H,W,fov,seed", [(24, 32, 60.0, 0), (20, 20, 90.0, 1), (13, 19, 75.0, 2)])
def test_native_matches_oracle(cuda, H, W, fov, seed):
    import torch
    say(f"[gpu] native refiner {H}x{W} fov {fov}")
    weights = rf.random_weights(seed)
    n, feature, hidden = pins.inputs(H, W, seed)
    intr = wl.intrins_from_fov(8 * H, 8 * W, fov)
    fuv = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    model = rf.NativeRefiner(weights)
    out, coarse = model.forward(_dec((n, feature, hidden)), intr, 8 * H, 8 * W, coarse=True)
    torch.cuda.synchronize()
    ray8 = wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, H, W)
    uv8 = rf.uv_map(intr, H, W, 8 * H, 8 * W)
    want = []
    oref.refine_forward(weights, n, feature, hidden, intr, fuv, ray8, uv8, trace=want,
                        nthreads=16)
    coarse = coarse.cpu().numpy()
    for it, (wp, _) in enumerate(want):
        ep = float(np.abs(coarse[it].astype(np.float64) - wp).max())
        say(f"    iteration {it}: propagate max-abs {ep:.3e}")
        assert ep <= TOL_COARSE
    eu = float(np.abs(out.cpu().numpy()[0].astype(np.float64) - want[-1][1]).max())
    say(f"    result max-abs {eu:.3e}")
    assert eu <= TOL_RESULT
    assert out.shape == (1, 3, 8 * H, 8 * W)


def test_native_matches_python_driver(cuda):
    """The C++ loop and the Python loop on the same weights and maps (fp32
    convolutions of two algorithms: their results, each within a few 1e-6 of
    the float64 restatement, within 1e-5 of each other)."""
    import torch
    H, W = 32, 40
    say(f"[gpu] native refiner vs Python driver {H}x{W}")
    weights = rf.random_weights(11)
    dec = _dec(pins.inputs(H, W, 11))
    intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    trace = []
    py = rf.Refiner(weights, "cuda:0").forward(dec, intr, 8 * H, 8 * W, trace=trace)
    nat, coarse = rf.NativeRefiner(weights).forward(dec, intr, 8 * H, 8 * W, coarse=True)
    torch.cuda.synchronize()
    ep = max(float((coarse[i] - trace[i][0].reshape(3, H, W)).abs().max()) for i in range(rf.N_ITER))
    eu = float((nat - py).abs().max())
    say(f"    propagate max-abs {ep:.3e}  result max-abs {eu:.3e}")
    assert ep <= TOL_COARSE and eu <= 1e-5


def test_native_crop_and_grid_change(cuda):
    """The crop (src/dsine_refine.cpp:289-293) is the slice of the whole map,
    and a refiner re-planned for another grid size gives what a fresh one
    gives, bit for bit."""
    import torch
    weights = rf.random_weights(5)
    model = rf.NativeRefiner(weights)
    H, W = 12, 16
    say(f"[gpu] native refiner crop {H}x{W}")
    dec = _dec(pins.inputs(H, W, 5))
    intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    full = model.forward(dec, intr, 8 * H, 8 * W)
    crop = rf.Crop(orig_h=8 * H - 11, orig_w=8 * W - 6, pad_t=5, pad_l=3)
    part = model.forward(dec, intr, 8 * H, 8 * W, crop=crop)
    torch.cuda.synchronize()
    assert part.shape == (1, 3, crop.orig_h, crop.orig_w)
    assert torch.equal(part, full[:, :, 5:5 + crop.orig_h, 3:3 + crop.orig_w])
    # another grid, then back
    dec2 = _dec(pins.inputs(9, 14, 6))
    intr2 = wl.intrins_from_fov(72, 112, 70.0)
    other = model.forward(dec2, intr2, 72, 112)
    again = model.forward(dec, intr, 8 * H, 8 * W)
    fresh = rf.NativeRefiner(weights).forward(dec2, intr2, 72, 112)
    torch.cuda.synchronize()
    assert torch.equal(again, full)
    assert torch.equal(other, fresh)


def test_native_pin_constant_heads(cuda):
    """Heads reduced to their biases: each iteration is one direct propagate
    of constant planes, as the C oracle computes it."""
    import torch
    H, W = 24, 32
    say("[gpu] native refiner pin: constant heads")
    n, feature, hidden, intr, fuv, ray8, _ = pins.setup(H, W, 60.0, 7)
    w, data = pins.pinned_weights("const_heads", 7)
    _, coarse = rf.NativeRefiner(w).forward(_dec((n, feature, hidden)), intr, 8 * H, 8 * W,
                                            coarse=True)
    torch.cuda.synchronize()
    chain = list(coarse.cpu().numpy())
    want = pins.const_heads_expected(data, n, ray8, fuv, H, W, chain=chain)
    for it, (p, wp) in enumerate(zip(chain, want)):
        err = float(np.abs(p.astype(np.float64) - wp).max())
        say(f"    iteration {it}: max-abs {err:.3e}")
        assert err <= 1e-5


@pytest.mark.parametrize("n0", [0, 5, 7])
def test_native_pin_onehot_upsample(cuda, n0):
    """A one-hot up_prob_head bias: the result is the normalised last
    propagate output at each pixel's clamped tap."""
    import torch
    H, W = 24, 32
    say(f"[gpu] native refiner pin: one-hot up mask, tap {n0}")
    n, feature, hidden, intr, _, _, _ = pins.setup(H, W, 60.0, 7)
    w, _ = pins.pinned_weights("onehot_up", 7, n0=n0)
    out, coarse = rf.NativeRefiner(w).forward(_dec((n, feature, hidden)), intr, 8 * H, 8 * W,
                                              coarse=True)
    torch.cuda.synchronize()
    err = float(np.abs(out.cpu().numpy()[0] -
                       pins.onehot_up_expected(coarse[-1].cpu().numpy(), n0)).max())
    say(f"    max-abs {err:.3e}")
    assert err <= 1e-5


@pytest.mark.parametrize("dtype", ["F32", "F16"])
def test_native_load_file(cuda, tmp_path, dtype):
    """Weights read from a safetensors file give the forward of the same
    weights set from memory (F16 files: the F16-rounded weights), bit for
    bit."""
    import torch
    from safetensors.numpy import save_file
    say(f"[gpu] native refiner load_file {dtype}")
    weights = rf.random_weights(3)
    if dtype == "F16":
        weights = {k: v.astype(np.float16) for k, v in weights.items()}
    path = os.path.join(str(tmp_path), "model.safetensors")
    save_file({k: np.ascontiguousarray(v) for k, v in weights.items()}, path)
    H, W = 10, 12
    dec = _dec(pins.inputs(H, W, 3))
    intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    a = rf.NativeRefiner(path=path).forward(dec, intr, 8 * H, 8 * W)
    b = rf.NativeRefiner({k: v.astype(np.float32) for k, v in weights.items()}).forward(
        dec, intr, 8 * H, 8 * W)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_cpp_refiner_on_device(cuda, tmp_path):
    """brovisionml::dsine::Refiner (tests/cpp/test_dsine_refine.cpp, run on
    brotensor's CUDA tag, in its own process) against the native refiner's
    device forward in this process, bit for bit, and its host path against
    its device path."""
    import torch
    from tests.test_refiner_native_host import _cpu_dec, cpp_case, run_cpp_refine
    wpath, cpath, weights, maps, intr, crop = cpp_case(tmp_path)
    say("[gpu] C++ Refiner class, run gpu")
    opath = str(tmp_path / "out.bin")
    rc, out = run_cpp_refine("run", "gpu", wpath, cpath, opath, timeout=110)
    say(out)
    assert rc == 0 and "OK" in out, out
    got = np.fromfile(opath, np.float32).reshape(1, 3, crop.orig_h, crop.orig_w)
    H, W = maps[0].shape[1:]
    dev = rf.NativeRefiner(weights).forward(_dec(maps), intr, 8 * H, 8 * W, crop=crop)
    host = rf.NativeRefiner(weights).forward(_cpu_dec(maps), intr, 8 * H, 8 * W, crop=crop)
    torch.cuda.synchronize()
    dev = dev.cpu().numpy()
    e_cpp = float(np.abs(got - dev).max())
    e_host = float(np.abs(host.numpy() - dev).max())
    say(f"    C++ class vs device forward max-abs {e_cpp:.3e}; host vs device {e_host:.3e}")
    assert np.array_equal(got, dev), e_cpp
    assert e_host <= 1e-5
