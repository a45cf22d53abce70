"""Writes the golden fixtures tests/golden/*.npz from the independent float64
restatement (tests/golden/independent.py) -- not from the oracle, so they pin
the oracle as well as the HIP path.  Inputs are float32 as the ops take them;
expected values are float64.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from brovisionml_amd import workloads as wl  # noqa: E402
from tests.golden import independent as ind  # noqa: E402


def random_case(seed, B, H, W, k, angle_range, per_sample_ray=False):
    rng = np.random.default_rng(seed)
    HW, K2 = H * W, k * k
    n = rng.standard_normal((B, 3, HW))
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    intr_ = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    intr = wl.scaled_intrinsics(intr_, H, W, 8 * H, 8 * W)
    ray = wl.build_ray8(intr_, H, W, 8 * H, 8 * W).reshape(1, 3, HW)
    if per_sample_ray:
        ray = np.concatenate([ray * np.float32(1.0 + 0.02 * b) for b in range(B)]).astype(np.float32)
    return dict(pred_norm=n.astype(np.float32),
                prob=(1 / (1 + np.exp(-rng.standard_normal((B, K2, HW))))).astype(np.float32),
                xy=rng.standard_normal((B, 2 * K2, HW)).astype(np.float32),
                angle=rng.uniform(*angle_range, (B, K2, HW)).astype(np.float32),
                ray=ray.astype(np.float32), intr=np.array(intr), k=np.int32(k),
                H=np.int32(H), W=np.int32(W))


def smooth_case(seed, H, W):
    """A camera-facing, slowly varying normal field with head-like
    activations: prob = sigmoid(.), angle = sigmoid(.) * pi."""
    rng = np.random.default_rng(seed)
    k, HW, K2 = 5, H * W, 25
    ys, xs = np.meshgrid(np.linspace(-1, 1, H), np.linspace(-1, 1, W), indexing="ij")
    n = np.stack([0.4 * np.sin(2 * xs + ys), 0.3 * np.cos(3 * ys), -np.ones_like(xs)]).reshape(1, 3, HW)
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    intr_ = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    intr = wl.scaled_intrinsics(intr_, H, W, 8 * H, 8 * W)
    ray = wl.build_ray8(intr_, H, W, 8 * H, 8 * W).reshape(1, 3, HW)
    sig = lambda a: 1 / (1 + np.exp(-a))
    return dict(pred_norm=n.astype(np.float32),
                prob=sig(2 * rng.standard_normal((1, K2, HW))).astype(np.float32),
                xy=rng.standard_normal((1, 2 * K2, HW)).astype(np.float32),
                angle=(sig(rng.standard_normal((1, K2, HW)) - 2) * np.pi).astype(np.float32),
                ray=ray.astype(np.float32), intr=np.array(intr), k=np.int32(k),
                H=np.int32(H), W=np.int32(W))


def finish(case):
    B = case["pred_norm"].shape[0]
    H, W, k = int(case["H"]), int(case["W"]), int(case["k"])
    K2 = k * k
    out, acc = ind.refine_step(case["pred_norm"].reshape(B, 3, H, W),
                               case["prob"].reshape(B, K2, H, W),
                               case["xy"].reshape(B, 2 * K2, H, W),
                               case["angle"].reshape(B, K2, H, W),
                               case["ray"].reshape(-1, 3, H, W), tuple(case["intr"]), k)
    case["expect_out"] = out.reshape(B, 3, H * W)
    case["expect_acc"] = acc.reshape(B, 3, H * W)
    return case


def ray_relu_case(seed, H, W):
    rng = np.random.default_rng(seed)
    import torch
    HW = H * W
    intr_ = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    ray = wl.build_ray8(intr_, H, W, 8 * H, 8 * W).reshape(3, HW)
    n = rng.standard_normal((3, HW)).astype(np.float32)
    n[:, :20] = -ray[:, :20] + np.float32(1e-3) * rng.standard_normal((3, 20)).astype(np.float32)
    want = ind.ray_relu(torch.from_numpy(n.astype(np.float64)),
                        torch.from_numpy(ray.astype(np.float64)), dim=0).numpy()
    return dict(normal=n, ray=ray, H=np.int32(H), W=np.int32(W), expect=want)


def upsample_case(seed, B, C, H, W, s, normalize, smooth=False):
    """Convex-upsample inputs: x a field of C-vectors (unit normals when
    C == 3), the 9*s*s-channel mask ~ N(0, 2^2)."""
    rng = np.random.default_rng(seed)
    if smooth:
        ys, xs = np.meshgrid(np.linspace(0, 1, H), np.linspace(0, 1, W), indexing="ij")
        x = np.stack([0.5 * np.sin(3 * xs + ys), 0.4 * np.cos(2 * ys), -np.ones_like(xs)])[None]
        x = np.repeat(x, B, axis=0)
    else:
        x = rng.standard_normal((B, C, H, W))
    if C == 3:
        x = x / np.linalg.norm(x, axis=1, keepdims=True)
    x = x.astype(np.float32)
    mask = (2.0 * rng.standard_normal((B, 9 * s * s, H, W))).astype(np.float32)
    want = ind.convex_upsample(x.astype(np.float64), mask.astype(np.float64), s, normalize)
    return dict(x=x, mask=mask, H=np.int32(H), W=np.int32(W), s=np.int32(s),
                normalize=np.int32(normalize), expect=want)


CASES = {
    "angmf_8x10_k5": lambda: finish(random_case(101, 1, 8, 10, 5, (0.0, np.pi))),
    "angmf_b2_12x16_k3_raystride": lambda: finish(random_case(102, 2, 12, 16, 3, (-1.0, 1.0), True)),
    "angmf_9x13_k7": lambda: finish(random_case(103, 1, 9, 13, 7, (0.0, np.pi / 4))),
    "angmf_smooth_16x20_k5": lambda: finish(smooth_case(104, 16, 20)),
    "ray_relu_12x20": lambda: ray_relu_case(105, 12, 20),
    "upsample_4x5_s8": lambda: upsample_case(106, 1, 3, 4, 5, 8, True),
    "upsample_4x6_s4_c2_raw": lambda: upsample_case(107, 1, 2, 4, 6, 4, False),
    "upsample_smooth_5x6_s8": lambda: upsample_case(108, 1, 3, 5, 6, 8, True, smooth=True),
    "upsample_b2_3x5_s2_c4": lambda: upsample_case(109, 2, 4, 3, 5, 2, True),
}


def main():
    for name, make in CASES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **make())
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
