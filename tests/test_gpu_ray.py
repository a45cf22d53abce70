"""GPU tests of the ray map formed from the intrinsics: bvml_dsine_build_ray8_f32
against the host restatement of build_ray8 (src/dsine_decoder.cpp:242-293),
bit for bit, and angmf_propagate's RAY_FROM_INTRINSICS mode against the same
call given that ray, bit for bit, on the fp32 path, its reference-order
recompute and the double-precision kernel."""
from __future__ import annotations

import numpy as np
import pytest

from brovisionml_amd import dsine, workloads as wl
from tests._util import TOL_ABS, TOL_DEG, compare, to_dev
from tests.test_gpu_parity import _random_inputs, run_oracle, say

pytestmark = pytest.mark.gpu

# (H, W, intrinsics): the refiner's own (intrins_from_fov on the padded
# image), and off-centre principal points with unequal focal lengths.
RAY_CASES = [
    (60, 80, None),
    (256, 256, None),
    (1, 1, None),
    (33, 17, wl.Intrinsics(fx=311.7, fy=287.25, cx=101.3, cy=140.9)),
    (7, 130, wl.Intrinsics(fx=1234.5, fy=1190.0, cx=700.0, cy=20.0)),
    (40, 40, wl.Intrinsics(fx=50.0, fy=50.0, cx=-30.0, cy=400.0)),
]


def _intrinsics(H, W, intr):
    intr = intr or wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    return intr, wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)


@pytest.mark.parametrize("H,W,intr", RAY_CASES)
def test_build_ray8_bit_exact(cuda, H, W, intr):
    intr, (fu, cu, fv, cv) = _intrinsics(H, W, intr)
    say(f"[gpu] build_ray8 {H}x{W}")
    got = dsine.build_ray8(fu, cu, fv, cv, H, W, device=cuda).cpu().numpy()
    want = wl.build_ray8(intr, H, W, 8 * H, 8 * W)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("H,W,intr", RAY_CASES)
def test_build_uv8_bit_exact(cuda, H, W, intr):
    """bvml_dsine_build_uv8_f32 against the host restatement of build_uv
    (src/dsine_decoder.cpp:242-274)."""
    import torch
    from brovisionml_amd import _lib, refiner as rf
    intr, (fu, cu, fv, cv) = _intrinsics(H, W, intr)
    say(f"[gpu] build_uv8 {H}x{W}")
    uv = torch.empty((2, H, W), dtype=torch.float32, device=cuda)
    assert _lib.build_uv8_f32(uv.data_ptr(), fu, cu, fv, cv, H, W,
                              torch.cuda.current_stream().cuda_stream) == _lib.OK
    torch.cuda.synchronize()
    want = rf.uv_map(intr, H, W, 8 * H, 8 * W)
    assert np.array_equal(uv.cpu().numpy().view(np.uint32), want.view(np.uint32))


def _run(inp, H, W, device, ray, precise):
    import torch
    t = {k: to_dev(inp[k], device) for k in ("pred_norm", "prob", "xy", "angle")}
    fu, cu, fv, cv = inp["intrinsics"]
    r = None if ray is None else to_dev(ray, device)
    out = dsine.angmf_propagate(t["pred_norm"], t["prob"], t["xy"], t["angle"], r,
                                fu, cu, fv, cv, H, W, precise=precise)
    torch.cuda.synchronize()
    return out.cpu().numpy()


# wide and narrow tiles, k = 3, 5, 7, a batch, the whole-window kernel
# (2 x 512 x 512, k = 5; 800 x 800 with non-temporal plane loads); flagged
# pixels (zero xy pairs, large angles) take the reference-order recompute
@pytest.mark.parametrize("B,H,W,k", [(1, 20, 200, 5), (2, 9, 13, 7), (1, 33, 65, 3), (1, 64, 64, 5),
                                     (2, 512, 512, 5), (1, 800, 800, 5)])
@pytest.mark.parametrize("precise", [False, True])
def test_angmf_ray_from_intrinsics(cuda, B, H, W, k, precise):
    say(f"[gpu] angmf ray from intrinsics B={B} {H}x{W} k={k} precise={precise}")
    rng = np.random.default_rng(100 + H + W + k)
    inp = _random_inputs(rng, B, H, W, k, theta_scale=1.3)
    K2, HW = k * k, H * W
    inp["xy"][:, 1, :: 7] = 0.0
    inp["xy"][:, K2 + 1, :: 7] = 0.0
    explicit = _run(inp, H, W, cuda, inp["ray"], precise)
    synth = _run(inp, H, W, cuda, None, precise)
    assert np.array_equal(explicit.view(np.uint32), synth.view(np.uint32))
    want = run_oracle(inp, H, W, k)
    max_abs, max_deg, nan_mm = compare(synth.reshape(B, 3, HW), want.reshape(B, 3, HW))
    say(f"    max-abs {max_abs:.3e}  max-angle {max_deg:.3e} deg  nan-mismatch {nan_mm}")
    assert nan_mm == 0
    assert max_abs <= TOL_ABS and max_deg <= TOL_DEG
