"""Camera closed forms that feed the ops and the benchmark workloads."""
from __future__ import annotations

import math

import numpy as np

from brovisionml_amd import workloads as wl


def approx(a, b, tol):
    return abs(a - b) <= tol


def test_intrins_from_fov_known_answers():
    # the reference's own checks, tests/test_dsine_preprocess.cpp:74-90
    half = (60.0 / 2.0) * 3.14159265358979323846 / 180.0
    k = wl.intrins_from_fov(256, 256, 60.0)
    f = (256.0 / 2.0) / math.tan(half)
    assert approx(k.fx, f, 1e-3) and approx(k.fy, f, 1e-3)
    assert approx(k.cx, 256.0 / 2.0 - 0.5, 1e-5) and approx(k.cy, 256.0 / 2.0 - 0.5, 1e-5)
    k2 = wl.intrins_from_fov(348, 500, 60.0)
    f2 = (500.0 / 2.0) / math.tan(half)
    assert approx(k2.fx, f2, 1e-3)
    assert approx(k2.cx, 500.0 / 2.0 - 0.5, 1e-5) and approx(k2.cy, 348.0 / 2.0 - 0.5, 1e-5)
    # every field is a float
    for v in (k.fx, k.fy, k.cx, k.cy):
        assert float(np.float32(v)) == v


def test_scaled_intrinsics_of_the_workloads():
    # fu = fv = f/8, cu = W/2, cv = H/2 on the /8 grid of an image with a 60 degree FOV
    want = {0: (69.282036, 40.0, 30.0), 2: (221.702499, 128.0, 128.0), 4: (443.404999, 256.0, 256.0)}
    for i, (f, cu, cv) in want.items():
        _, (fu, cu_, fv, cv_) = wl.WORKLOADS[i].intrinsics()
        assert approx(fu, f, 1e-5) and fu == fv
        assert cu_ == cu and cv_ == cv


def test_build_ray8_unit_and_central_ray():
    intr = wl.intrins_from_fov(64, 96, 60.0)
    ray = wl.build_ray8(intr, 8, 12, 64, 96)
    n = np.sqrt((ray.astype(np.float64) ** 2).sum(axis=0))
    assert np.abs(n - 1).max() < 1e-7
    assert (ray[2] > 0).all()
    # the principal point sits between the centre pixels: symmetric rays
    assert np.allclose(ray[0], -ray[0][:, ::-1], atol=1e-7)
    assert np.allclose(ray[1], -ray[1][::-1, :], atol=1e-7)
    # closed form at one pixel: ray_x = float((x + 0.5 - cu)/fu)
    fu, cu, fv, cv = wl.scaled_intrinsics(intr, 8, 12, 64, 96)
    rx = float(np.float32((3 + 0.5 - cu) / fu))
    ry = float(np.float32((5 + 0.5 - cv) / fv))
    inv = 1.0 / math.sqrt(rx * rx + ry * ry + 1.0)
    assert ray[0, 5, 3] == np.float32(rx * inv) and ray[2, 5, 3] == np.float32(inv)


def test_workload_bytes_match_the_measurement_plan():
    # algorithmic bytes per step (shared ray; per-sample in parentheses)
    assert wl.WORKLOADS[0].algorithmic_bytes() == 2092800
    assert wl.WORKLOADS[1].algorithmic_bytes() == 4 * 7143424
    assert wl.WORKLOADS[2].algorithmic_bytes() == 28573696
    assert wl.WORKLOADS[3].algorithmic_bytes() == 65184000
    assert wl.WORKLOADS[3].algorithmic_bytes(shared_ray=False) == 66969600
    assert wl.WORKLOADS[4].algorithmic_bytes() == 850395136
    assert wl.WORKLOADS[4].algorithmic_bytes(shared_ray=False) == 859832320


def test_make_sample_distributions():
    s = wl.make_sample(wl.WORKLOADS[2])
    n = np.sqrt((s["pred_norm"].astype(np.float64) ** 2).sum(axis=0))
    assert np.abs(n - 1).max() < 1e-6
    assert s["angle"].min() >= 0 and s["angle"].max() <= math.pi / 4
    assert (s["prob"] > 0).all() and (s["prob"] < 1).all()
    z = wl.make_sample(wl.WORKLOADS[4])["pred_norm"]
    zn = z[2] / np.sqrt((z.astype(np.float64) ** 2).sum(axis=0))
    assert (zn > 0).all()
    # deterministic
    assert np.array_equal(wl.make_sample(wl.WORKLOADS[0])["xy"], wl.make_sample(wl.WORKLOADS[0])["xy"])


def test_every_workload_finds_its_traffic_profile():
    # the bench line's roofline.traffic comes from the committed rocprofv3
    # summary whose workload field names the workload exactly
    import os
    import sys
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench
    for w in wl.WORKLOADS:
        t = bench.traffic_from_profile("angmf", w.name)
        assert t is not None, w.name
        algo = w.algorithmic_bytes(shared_ray=True) // w.calls
        assert algo <= t <= 1.2 * algo, (w.name, t, algo)
    up = bench.traffic_from_profile("upsample", "dsine-upsample-256x256-s8")
    assert up is not None
