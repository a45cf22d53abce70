"""The CPU branch of the public dispatch (brovisionml_amd.dsine and the C ABI's
*_cpu_f32 entry points): CPU tensors take the path of the reference's CPU
twin (src/dsine_ops.cpp:55-172 via the dispatch at :178-215) and must equal
the oracle's restatement of it bit for bit, over the extensions the device
entry points carry (B > 1, odd k, per-sample rays, rays formed from the
intrinsics, logits) and the edge cases (empty maps, one-pixel maps)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from brovisionml_amd import _lib, dsine
from brovisionml_amd import workloads as wl


def inputs(rng, B, H, W, k, per_sample_ray=False):
    HW, K2 = H * W, k * k
    n = rng.standard_normal((B, 3, HW))
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    intr_full = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    fu, cu, fv, cv = wl.scaled_intrinsics(intr_full, H, W, 8 * H, 8 * W)
    ray = wl.build_ray8(intr_full, H, W, 8 * H, 8 * W).reshape(3, HW)
    if per_sample_ray:
        r = rng.standard_normal((B, 3, HW))
        ray = (r / np.linalg.norm(r, axis=1, keepdims=True)).astype(np.float32)
    return dict(
        pred_norm=n.astype(np.float32),
        prob=(1 / (1 + np.exp(-rng.standard_normal((B, K2, HW))))).astype(np.float32),
        xy=rng.standard_normal((B, 2 * K2, HW)).astype(np.float32),
        angle=rng.uniform(0, np.pi, (B, K2, HW)).astype(np.float32),
        ray=np.ascontiguousarray(ray, dtype=np.float32),
        intr=(fu, cu, fv, cv))


def run_cpu(d, H, W, logits=False, synth=False):
    t = {key: torch.from_numpy(d[key]) for key in ("pred_norm", "prob", "xy", "angle", "ray")}
    out = dsine.angmf_propagate(t["pred_norm"], t["prob"], t["xy"], t["angle"],
                                None if synth else t["ray"], *d["intr"], H, W, logits=logits)
    assert out.device.type == "cpu"
    return out.numpy()


@pytest.mark.parametrize("B,H,W,k", [(1, 23, 31, 5), (2, 17, 19, 3), (1, 9, 40, 7),
                                     (2, 12, 11, 9), (1, 5, 6, 1), (1, 1, 1, 5), (1, 2, 33, 5)])
def test_angmf_cpu_bit_exact(B, H, W, k):
    rng = np.random.default_rng(100 + 7 * k + H)
    d = inputs(rng, B, H, W, k)
    got = run_cpu(d, H, W)
    want = oracle.angmf_propagate(d["pred_norm"], d["prob"], d["xy"], d["angle"], d["ray"],
                                  d["intr"], H, W, k)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_angmf_cpu_per_sample_ray_and_synth_ray():
    rng = np.random.default_rng(3)
    B, H, W = 2, 15, 21
    d = inputs(rng, B, H, W, 5, per_sample_ray=True)
    got = run_cpu(d, H, W)
    want = oracle.angmf_propagate(d["pred_norm"], d["prob"], d["xy"], d["angle"], d["ray"],
                                  d["intr"], H, W, 5)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # rays formed from the intrinsics equal build_ray8's map (src/dsine_decoder.cpp:242-293)
    d1 = inputs(rng, 1, H, W, 5)
    np.testing.assert_array_equal(run_cpu(d1, H, W, synth=True).view(np.uint32),
                                  run_cpu(d1, H, W).view(np.uint32))


def test_angmf_cpu_logits_apply_the_refiners_activations():
    rng = np.random.default_rng(4)
    H, W = 14, 18
    d = inputs(rng, 1, H, W, 5)
    lp = (3 * rng.standard_normal(d["prob"].shape)).astype(np.float32)
    la = (3 * rng.standard_normal(d["angle"].shape)).astype(np.float32)
    sig = lambda x: (1 / (1 + np.exp(-x.astype(np.float64)))).astype(np.float32)  # noqa: E731
    want = oracle.angmf_propagate(d["pred_norm"], sig(lp), d["xy"], sig(la) * np.float32(np.pi),
                                  d["ray"], d["intr"], H, W, 5)
    d2 = dict(d, prob=lp, angle=la)
    np.testing.assert_array_equal(run_cpu(d2, H, W, logits=True).view(np.uint32),
                                  want.view(np.uint32))


def test_ray_relu_cpu_bit_exact_in_place():
    rng = np.random.default_rng(6)
    B, H, W = 2, 19, 27
    d = inputs(rng, B, H, W, 5)
    # include antipodal and exactly-on-the-boundary normals
    d["pred_norm"][0, :, 0] = -d["ray"][:, 0]
    n = torch.from_numpy(d["pred_norm"].copy())
    dsine.ray_relu(n, torch.from_numpy(d["ray"]), H, W)
    want = oracle.ray_relu(d["pred_norm"], d["ray"], H, W)
    np.testing.assert_array_equal(n.numpy().view(np.uint32), want.view(np.uint32))


def test_cpu_threads_change_no_result():
    rng = np.random.default_rng(8)
    H, W = 70, 33
    d = inputs(rng, 1, H, W, 5)
    outs = []
    for nt in (1, 3, 8):
        o = np.empty_like(d["pred_norm"])
        st = _lib.angmf_propagate_cpu_f32(
            d["pred_norm"].ctypes.data, d["prob"].ctypes.data, d["xy"].ctypes.data,
            d["angle"].ctypes.data, d["ray"].ctypes.data, *d["intr"], 1, H, W, 5, 0,
            o.ctypes.data, _lib.DEFAULT, nt)
        assert st == _lib.OK
        outs.append(o)
    for o in outs[1:]:
        np.testing.assert_array_equal(o.view(np.uint32), outs[0].view(np.uint32))


def test_cpu_empty_and_errors():
    z = torch.zeros(0)
    out = dsine.angmf_propagate(z, z, z, z, z, 1.0, 0.5, 1.0, 0.5, 0, 4)
    assert out.numel() == 0
    n = torch.zeros(3 * 4 * 5)
    with pytest.raises(RuntimeError, match="^dsine ops: ray_relu"):
        dsine.ray_relu(n, torch.zeros(3 * 4 * 4), 4, 5)
    assert _lib.angmf_propagate_cpu_f32(1, 1, 1, 1, 1, 1.0, 0.5, 1.0, 0.5, 1, 4, 4, 4, 0, 2,
                                        _lib.DEFAULT, 1) == _lib.EK
    assert _lib.angmf_propagate_cpu_f32(0, 1, 1, 1, 1, 1.0, 0.5, 1.0, 0.5, 1, 4, 4, 5, 0, 2,
                                        _lib.DEFAULT, 1) == _lib.ENULL
    assert _lib.angmf_propagate_cpu_f32(1, 1, 1, 1, 1, 1.0, 0.5, 1.0, 0.5, 1, 4, 4, 5, 0, 2,
                                        8, 1) == _lib.EFLAGS
    # out overlapping an input
    buf = np.zeros(1000, np.float32)
    p = buf.ctypes.data
    assert _lib.angmf_propagate_cpu_f32(p, p + 4000, p + 4000, p + 4000, p + 4000, 1.0, 0.5, 1.0,
                                        0.5, 1, 2, 2, 1, 0, p + 8, _lib.DEFAULT, 1) == _lib.EALIAS
    with pytest.raises(RuntimeError, match="CPU"):
        dsine.convex_upsample(torch.zeros(3), torch.zeros(9), 1, 3, 1, 1, 1)
