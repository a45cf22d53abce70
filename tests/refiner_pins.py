"""Closed-form pins of the refiner loop (src/dsine_refine.cpp:212-294), shared
by the CPU tests of its restatement (oracle/refiner.py, with planted
mistakes) and the GPU tests of brovisionml_amd/refiner.py.  Each pin sets
some weights so that a step's result has a form that does not need the
refiner to compute:

  gate_closed   convz weight 0, bias -100: z = sigmoid(-100) = 0, so every
                iteration's h_new = (1 - z) h + z q is the decoder's hidden h
  gate_open     convz weight 0, bias +100 (z = 1) and convq weight 0, bias b:
                h_new = q = tanh(b), per channel, everywhere
  const_heads   the prob, xy and angle heads' last convolutions weight 0,
                biases chosen: each iteration propagates with planes constant
                per channel, activated as the refiner activates the logits;
                the pin is that propagate (and RayReLU) from the C oracle,
                one step from each iteration's input
  onehot_up     up_prob_head's last convolution weight 0, its bias +60 on
                tap n0 of every sub-pixel and 0 on the others: the softmax is
                one-hot, so up(8y + ky, 8x + kx) = normalize(pred_norm at
                (clamp(y + dy0), clamp(x + dx0))), n0 = 3 (dy0 + 1) + (dx0 + 1)
"""
from __future__ import annotations

import numpy as np

from brovisionml_amd import refiner as rf, workloads as wl

PS, K_UP = 5, 8
K_PI32 = np.float32(3.14159265358979323846)


def inputs(H, W, seed):
    rng = np.random.default_rng(seed)
    n = rng.standard_normal((3, H, W))
    n[2] = np.abs(n[2]) + 0.5
    n = (n / np.linalg.norm(n, axis=0)).astype(np.float32)
    feature = rng.standard_normal((64, H, W)).astype(np.float32)
    hidden = rng.uniform(-1, 1, (64, H, W)).astype(np.float32)
    return n, feature, hidden


def pinned_weights(pin: str, seed: int, n0: int = 0):
    """Random weights with the pin's weights and biases set; returns
    (weights, data) where data holds the pin's chosen values."""
    w = rf.random_weights(seed)
    rng = np.random.default_rng(seed + 77)
    data = {}
    if pin == "gate_closed":
        w["gru.convz.weight"][:] = 0.0
        w["gru.convz.bias"][:] = -100.0
    elif pin == "gate_open":
        w["gru.convz.weight"][:] = 0.0
        w["gru.convz.bias"][:] = 100.0
        w["gru.convq.weight"][:] = 0.0
        b = rng.uniform(-2, 2, 64).astype(np.float32)
        w["gru.convq.bias"][:] = b
        data["bq"] = b
    elif pin == "const_heads":
        for head, nch, lo, hi in (("prob_head", PS * PS, -2, 2), ("xy_head", 2 * PS * PS, -2, 2),
                                  ("angle_head", PS * PS, -1, 1)):
            w[f"{head}.4.weight"][:] = 0.0
            b = rng.uniform(lo, hi, nch).astype(np.float32)
            w[f"{head}.4.bias"][:] = b
            data[head] = b
    elif pin == "onehot_up":
        w["up_prob_head.4.weight"][:] = 0.0
        b = np.zeros(9 * K_UP * K_UP, np.float32)
        b[n0 * K_UP * K_UP:(n0 + 1) * K_UP * K_UP] = 60.0
        w["up_prob_head.4.bias"][:] = b
        data["n0"] = n0
    else:
        raise ValueError(pin)
    return w, data


def const_heads_expected(data, normal, ray8, fuv, H, W, chain=None, n_iter=rf.N_ITER):
    """Each iteration's propagated normals under const_heads, from the C
    oracle's RayReLU and angmf_propagate alone.  Iteration i propagates the
    oracle's own iteration i - 1 output, or, when chain (the refiner's
    per-iteration outputs, (3, H, W) each) is given, chain[i - 1]: one step
    from the refiner's own input, so errors do not compound over the chain."""
    import oracle
    HW = H * W
    sig = lambda v: (1.0 / (1.0 + np.exp(-v.astype(np.float64)))).astype(np.float32)  # noqa: E731
    prob = np.repeat(sig(data["prob_head"])[:, None], HW, axis=1)
    xy = np.repeat(data["xy_head"][:, None], HW, axis=1)
    angle = np.repeat((sig(data["angle_head"]).astype(np.float64) * np.float64(K_PI32))
                      .astype(np.float32)[:, None], HW, axis=1)
    pred = oracle.ray_relu(normal.reshape(3, HW), ray8.reshape(3, HW), H, W)
    out = []
    for i in range(n_iter):
        if chain is not None and i > 0:
            pred = np.asarray(chain[i - 1], np.float32).reshape(3, HW)
        pred = oracle.angmf_propagate(pred.reshape(1, 3, HW), prob[None], xy[None], angle[None],
                                      ray8.reshape(3, HW), fuv, H, W, PS, nthreads=8)
        pred = pred.reshape(3, HW)
        out.append(pred.reshape(3, H, W).copy())
    return out


def onehot_up_expected(pred, n0):
    """up under onehot_up from pred (3, H, W): each output pixel the
    normalised pred at its tap's clamped neighbour."""
    _, H, W = pred.shape
    dy, dx = n0 // 3 - 1, n0 % 3 - 1
    ys = np.clip(np.arange(H) + dy, 0, H - 1)
    xs = np.clip(np.arange(W) + dx, 0, W - 1)
    src = pred.astype(np.float64)[:, ys][:, :, xs]
    src = src / np.maximum(np.linalg.norm(src, axis=0), 1e-12)
    return np.repeat(np.repeat(src, K_UP, axis=1), K_UP, axis=2)


def setup(H, W, fov, seed):
    n, feature, hidden = inputs(H, W, seed)
    intr = wl.intrins_from_fov(8 * H, 8 * W, fov)
    fuv = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    ray8 = wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, H, W)
    uv8 = rf.uv_map(intr, H, W, 8 * H, 8 * W)
    return n, feature, hidden, intr, fuv, ray8, uv8
