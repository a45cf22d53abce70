"""An independent float64 restatement of DSINE's AngMF refine step, built from
library routines and geometry rather than from the reference's formula, used
to pin the oracle and to generate the golden fixtures.

It follows the PyTorch structure the reference ports (the spec comments in
include/brovisionml/dsine_refine.h:45-111):
  get_unfold         F.pad(mode="replicate") + F.unfold (row-major slots)
  xy normalise       F.normalize over the (xs, ys) pair
  rotation axis      the line where the neighbour's surface plane (normal m,
                     through P0 = its pixel ray at depth 1) meets the ray
                     through the offset pixel: P1 = t d, t = (P0.m)/(d.m),
                     axis = normalize(P1 - P0) -- geometry, not the
                     reference's num/dd algebra
  axis_angle_to_matrix  scipy.spatial.transform.Rotation.from_rotvec
  RayReLU            F.cosine_similarity(eps 1e-8) + F.relu + F.normalize
  weighted sum       prob-weighted sum over slots, F.normalize
Valid for regular inputs only (no zero xy pairs, no d.m == 0, finite
values): the reference's clamps and isfinite fallback are pinned by the
special-case tests instead.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F
from scipy.spatial.transform import Rotation

RAY_EPS = float(np.float32(1e-2))  # the reference's float constant, widened


def unfold(t: torch.Tensor, k: int) -> torch.Tensor:
    """(B, C, H, W) -> (B, C, k*k, H, W), replicate padding."""
    B, C, H, W = t.shape
    P = k // 2
    tp = F.pad(t, (P, P, P, P), mode="replicate")
    return F.unfold(tp, kernel_size=k).view(B, C, k * k, H, W)


def ray_relu(n: torch.Tensor, r: torch.Tensor, dim: int = 1) -> torch.Tensor:
    cos = F.cosine_similarity(n, r, dim=dim, eps=1e-8).unsqueeze(dim)
    diff = r * (F.relu(cos - RAY_EPS) + RAY_EPS) - r * cos
    return F.normalize(n + diff, dim=dim)


def refine_step(pred_norm, prob, xy, angle, ray, intr, k: int):
    """pred_norm (B,3,H,W), prob (B,K2,H,W), xy (B,2K2,H,W) = [xs, ys],
    angle (B,K2,H,W), ray (B or 1,3,H,W); numpy or torch, any float dtype.
    Returns (normalised output, pre-normalisation sum), both (B,3,H,W) float64."""
    t = lambda a: torch.as_tensor(np.asarray(a), dtype=torch.float64)
    pred_norm, prob, xy, angle, ray = (t(a) for a in (pred_norm, prob, xy, angle, ray))
    fu, cu, fv, cv = intr
    B, _, H, W = pred_norm.shape
    K2 = k * k
    m = unfold(pred_norm, k)                                    # (B,3,K2,H,W)
    ys, xs = torch.meshgrid(torch.arange(H, dtype=torch.float64),
                            torch.arange(W, dtype=torch.float64), indexing="ij")
    pix = torch.stack([xs + 0.5, ys + 0.5])[None].expand(B, 2, H, W).contiguous()
    npix = unfold(pix, k)                                       # (B,2,K2,H,W)
    nxy = F.normalize(xy.view(B, 2, K2, H, W), dim=1)
    one = torch.ones_like(npix[:, 0])
    P0 = torch.stack([(npix[:, 0] - cu) / fu, (npix[:, 1] - cv) / fv, one], dim=1)
    d = torch.stack([(npix[:, 0] + nxy[:, 0] - cu) / fu, (npix[:, 1] + nxy[:, 1] - cv) / fv,
                     one], dim=1)
    tpar = (P0 * m).sum(1, keepdim=True) / (d * m).sum(1, keepdim=True)
    axis = F.normalize(tpar * d - P0, dim=1)
    rotvec = (axis * angle[:, None]).permute(0, 2, 3, 4, 1).reshape(-1, 3).numpy()
    R = torch.from_numpy(Rotation.from_rotvec(rotvec).as_matrix())      # (N,3,3)
    mv = m.permute(0, 2, 3, 4, 1).reshape(-1, 3, 1)
    rot = (R @ mv).reshape(B, K2, H, W, 3).permute(0, 4, 1, 2, 3)
    rot = F.normalize(rot, dim=1)
    rb = ray.view(-1, 3, 1, H, W).expand(B, 3, K2, H, W)
    v = ray_relu(rot, rb, dim=1)
    acc = (prob[:, None] * v).sum(2)
    return F.normalize(acc, dim=1).numpy(), acc.numpy()


def convex_upsample(x, mask, s: int = 8, normalize: bool = True, eps: float = 1e-12):
    """DSINE's upsample_via_mask with replicate padding (the structure
    include/brovisionml/dsine_refine.h:91-97 specifies), then F.normalize over
    channels: the mask viewed as (N, 1, 9, s, s, H, W) and softmaxed over the
    9 taps, the 3x3 replicate-padded unfold of x weighted and summed, the
    (s, s) sub-cells permuted onto the s-times grid.  float64 torch;
    x (N, C, H, W), mask (N, 9*s*s, H, W) -> (N, C, s*H, s*W)."""
    xt = torch.as_tensor(np.asarray(x), dtype=torch.float64)
    mt = torch.as_tensor(np.asarray(mask), dtype=torch.float64)
    N, C, H, W = xt.shape
    w = mt.view(N, 1, 9, s, s, H, W).softmax(dim=2)
    taps = F.unfold(F.pad(xt, (1, 1, 1, 1), mode="replicate"), [3, 3], padding=0)
    taps = taps.view(N, C, 9, 1, 1, H, W)
    up = (w * taps).sum(dim=2)                              # (N, C, s, s, H, W)
    up = up.permute(0, 1, 4, 2, 5, 3).reshape(N, C, s * H, s * W)
    if normalize:
        up = F.normalize(up, dim=1, eps=eps)
    return up.numpy()
