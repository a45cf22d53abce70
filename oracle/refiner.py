"""CPU restatement of the DSINE NRN refiner loop -- TEST INFRASTRUCTURE ONLY.

Refiner::forward (src/dsine_refine.cpp:212-294) on the CPU: the ConvGRU and
the four heads as float64 torch convolutions (the reference's brotensor
conv2d_forward, :94-101, in higher precision), each head's output rounded to
float as the reference's fp32 tensors are; the activations of :262-267 as
correctly rounded floats; RayReLU, angmf_propagate and the convex upsample +
normalise from this directory's C oracle.  The tests check
brovisionml_amd/refiner.py against it; the product never imports it.
"""
from __future__ import annotations

import numpy as np

from . import angmf_propagate, convex_upsample, ray_relu

K_UP, N_ITER, PS = 8, 5, 5
K_PI32 = np.float32(3.14159265358979323846)   # src/dsine_refine.cpp:26


def _sigmoid_f32(x):
    return (1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))).astype(np.float32)


def angle_from_logits(x):
    """The angle head's activation, sigmoid(x) * pi (src/dsine_refine.cpp:265-267),
    each step rounded to float."""
    return (_sigmoid_f32(x).astype(np.float64) * np.float64(K_PI32)).astype(np.float32)


MUTATIONS = (None, "swap_zr", "swap_xy")


def refine_forward(weights, normal, feature, hidden, intr, fuv, ray8, uv8, trace=None,
                   nthreads: int = 1, hidden_trace=None, mutation=None, cond_trace=None):
    """weights: name -> OIHW / (C,) float32 arrays; normal (3, H, W), feature
    and hidden (C, H, W) float32; intr unused beyond fuv = (fu, cu, fv, cv);
    ray8 (3, H, W) and uv8 (2, H, W) float32 as build_ray8 / build_uv give
    them.  Returns the last up-sampled map (3, 8H, 8W) float32; trace, when
    given, receives each iteration's (pred_norm, up), hidden_trace each
    iteration's h_new (C, H, W) float64, cond_trace each iteration's
    propagate conditioning per pixel, a dict of (H, W) maps: "ratio",
    |acc| / sqrt(sum (prob/|p|)^2) from the oracle's double sums (small where
    the sum cancels: the output then moves by about 1/ratio times a relative
    change of the terms), and "min_xy", the smallest |(xs, ys)| of the
    pixel's k*k pairs (the rotation axis's direction moves by about an
    absolute change of the pair over |(xs, ys)|).  mutation plants a mistake,
    for the
    tests that show the checks catch one: "swap_zr" exchanges the GRU's z and
    r gates, "swap_xy" the propagate's xs and ys planes."""
    assert mutation in MUTATIONS
    import torch
    import torch.nn.functional as F

    del intr
    _, H, W = normal.shape
    t64 = lambda a: torch.as_tensor(np.asarray(a, np.float64))[None]
    w = {k: torch.as_tensor(np.asarray(v, np.float64)) for k, v in weights.items()}

    def conv(x, name, pad):
        return F.conv2d(x, w[name + ".weight"], w[name + ".bias"], padding=pad)

    def head(name, x):
        h = torch.relu(conv(x, name + ".0", 1))
        h = torch.relu(conv(h, name + ".2", 0))
        return conv(h, name + ".4", 0)[0].numpy().astype(np.float32)

    uv = t64(uv8)
    pred = ray_relu(np.asarray(normal, np.float32).reshape(3, -1), ray8.reshape(3, -1), H, W)
    feat_map = torch.cat([t64(feature), uv], dim=1)
    h = t64(hidden)
    up = None
    for _ in range(N_ITER):
        hx = torch.cat([h, feat_map], dim=1)
        z = torch.sigmoid(conv(hx, "gru.convz", 2))
        r = torch.sigmoid(conv(hx, "gru.convr", 2))
        if mutation == "swap_zr":
            z, r = r, z
        q = torch.tanh(conv(torch.cat([r * h, feat_map], dim=1), "gru.convq", 2))
        h_new = (1 - z) * h + z * q
        hin = torch.cat([h_new, uv], dim=1)
        prob = _sigmoid_f32(head("prob_head", hin))
        xy = head("xy_head", hin)
        if mutation == "swap_xy":
            xy = np.concatenate([xy[PS * PS:], xy[:PS * PS]])
        angle = angle_from_logits(head("angle_head", hin))
        res = angmf_propagate(pred.reshape(1, 3, -1), prob.reshape(1, PS * PS, -1),
                              xy.reshape(1, 2 * PS * PS, -1), angle.reshape(1, PS * PS, -1),
                              ray8.reshape(3, -1), fuv, H, W, PS, nthreads=nthreads,
                              return_acc=cond_trace is not None,
                              return_qs=cond_trace is not None)
        if cond_trace is not None:
            res, acc, qs = res
            a2 = (np.asarray(acc, np.float64).reshape(3, -1) ** 2).sum(axis=0)
            ratio = np.sqrt(a2 / np.maximum(np.asarray(qs, np.float64).reshape(-1), 1e-300))
            xy64 = xy.astype(np.float64).reshape(2, PS * PS, H, W)
            cond_trace.append({"ratio": ratio.reshape(H, W),
                               "min_xy": np.sqrt((xy64 ** 2).sum(axis=0)).min(axis=0)})
        pred = res.reshape(3, -1)
        mask = head("up_prob_head", hin)
        up = convex_upsample(pred.reshape(1, 3, H, W), mask[None], H, W, K_UP, normalize=True,
                             eps=float(np.float32(1e-12)), nthreads=nthreads)[0]
        if trace is not None:
            trace.append((pred.reshape(3, H, W).copy(), up))
        if hidden_trace is not None:
            hidden_trace.append(h_new[0].numpy().copy())
        h = h_new
    return up
