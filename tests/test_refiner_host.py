"""Host-side parts of the refiner driver (no GPU): checkpoint tensor names and
shapes (src/dsine_refine.cpp:46-94, 161-180), the safetensors round trip,
and build_uv's float semantics (src/dsine_decoder.cpp:242-274)."""
from __future__ import annotations

import numpy as np

from brovisionml_amd import refiner as rf, workloads as wl


def test_weight_names_and_shapes():
    s = rf.weight_shapes()
    assert s["gru.convz.weight"] == (64, 130, 5, 5) and s["gru.convq.bias"] == (64,)
    assert s["prob_head.0.weight"] == (64, 66, 3, 3)
    assert s["xy_head.4.weight"] == (50, 64, 1, 1)
    assert s["angle_head.4.weight"] == (25, 64, 1, 1)
    assert s["up_prob_head.4.weight"] == (576, 64, 1, 1)
    assert len(s) == 2 * (3 + 4 * 3)


def test_random_weights_bounds():
    w = rf.random_weights(3)
    assert set(w) == set(rf.weight_shapes())
    for name, a in w.items():
        conv = name.rsplit(".", 1)[0]
        fan_in = np.prod(rf.weight_shapes()[conv + ".weight"][1:])
        assert a.dtype == np.float32 and np.abs(a).max() <= 1 / np.sqrt(fan_in)


def test_safetensors_round_trip(tmp_path):
    from safetensors.numpy import save_file
    w = rf.random_weights(4)
    # the reference's checkpoint layout: (C_out, C_in*k*k) weights, (C_out, 1) biases
    flat = {k: (v.reshape(v.shape[0], -1) if v.ndim == 4 else v.reshape(-1, 1)) for k, v in w.items()}
    path = str(tmp_path / "model.safetensors")
    save_file(flat, path)
    back = rf.load_safetensors(path)
    for k in w:
        assert np.array_equal(back[k], w[k])


def test_uv_map_matches_build_ray8_before_normalising():
    H, W = 9, 14
    intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    uv = rf.uv_map(intr, H, W, 8 * H, 8 * W)
    ray = wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, H, W).astype(np.float64)
    # build_ray8 = normalize([uv_x, uv_y, 1]) per pixel
    v = np.stack([uv[0].astype(np.float64), uv[1].astype(np.float64), np.ones((H, W))])
    v /= np.linalg.norm(v, axis=0)
    assert np.array_equal(v.astype(np.float32), ray.astype(np.float32))
