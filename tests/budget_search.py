"""Adversarial search for the fast kernel's largest cancellation-scaled error
(test infrastructure: nothing in the library imports it).

The recompute threshold t rests on delta = err * sqrt(ratio), ratio =
|acc|^2 / sum (prob/|p|)^2 from the oracle's double sums: a kept pixel
(ratio >= t) has an error of at most delta / sqrt(t).  The families of
tests/budget_families.py sample each mechanism that stresses tier 1; this
module climbs from them toward the inputs that maximise the error of a kept
pixel, pressing pixels toward cancellation up to the threshold.

Hill climbing, per pixel: each step perturbs every pixel's own planes at once
(its k*k xy pairs, angles and weights; the normals, shared between windows,
stay), evaluates the whole image, and keeps a pixel's new planes where its
score grew.  A pixel's output depends only on its own planes and the shared
normals and ray, so the pixels climb independently.  Only pixels the fast
path keeps score: ratio at or above the threshold and, for the CPU model,
not flagged by domain (|dd| below the kernel's floor, |t| > 3.2, ...), so
the search presses against those edges from the side the fast path keeps.

The seeds, one per mechanism: q cancelling (xy pairs perpendicular to m) with
grazing normals, wide angles, a 140-degree field of view (|P0| toward 4 at
the corners), saturated logits, and normals facing away from the ray."""
from __future__ import annotations

import numpy as np

from tests import budget_families as fam

SEEDS = ("grazing_qcancel", "qcancel", "wideangle", "widefov", "logits", "antipode")


def _perturb(d: dict, rng: np.random.Generator, step: float) -> dict:
    """A copy of d with every pixel's own planes moved by a random step."""
    c = dict(d)
    K2 = d["k"] * d["k"]
    xy = d["xy"].astype(np.float64)
    scale = np.sqrt((xy[:K2] ** 2 + xy[K2:] ** 2).mean(axis=0, keepdims=True))
    c["xy"] = (xy + step * scale * rng.standard_normal(xy.shape)).astype(np.float32)
    if d["logits"]:
        c["prob"] = (d["prob"] + 3.0 * step * rng.standard_normal(d["prob"].shape)).astype(
            np.float32)
        c["angle"] = (d["angle"] + 3.0 * step * rng.standard_normal(d["angle"].shape)).astype(
            np.float32)
    else:
        p = d["prob"].astype(np.float64) * np.exp(2.0 * step * rng.standard_normal(d["prob"].shape))
        c["prob"] = np.clip(p, 1e-6, 1.0).astype(np.float32)
        t = d["angle"].astype(np.float64) + step * rng.standard_normal(d["angle"].shape)
        c["angle"] = np.clip(t, -3.2, 3.2).astype(np.float32)
    return c


def _take(d: dict, c: dict, better: np.ndarray) -> dict:
    """d with the pixels in `better` taken from c."""
    out = dict(d)
    for key in ("xy", "prob", "angle"):
        a = d[key].copy()
        a[:, better] = c[key][:, better]
        out[key] = a
    return out


def climb(evaluate, d: dict, steps: int, rng: np.random.Generator, step: float = 0.1):
    """Climb from draw d.  evaluate(d) -> score per pixel (HW,): the pixel's
    error where the fast path keeps it, 0 elsewhere.  Returns (best score
    per pixel, the climbed draw)."""
    score = evaluate(d)
    for _ in range(steps):
        c = _perturb(d, rng, step)
        s = evaluate(c)
        better = s > score
        if better.any():
            d = _take(d, c, better)
            score = np.where(better, s, score)
    return score, d


def model_evaluator(oracle, model, lib, threshold: float, rng_seed: int = 0):
    """The CPU model's error per pixel (the runs summed as the kernel's
    launch plan splits them; lib is brovisionml_amd._lib), on the pixels the
    kernel would keep in fp32 (not flagged by domain, ratio at or above
    `threshold`), 0 elsewhere.  Every hardware function sits at its error bound with a fixed
    random sign pattern, so the score is a deterministic function of the
    inputs.  Also returns, through .last, the last call's (err, ratio,
    flags)."""
    def evaluate(d):
        H, W, k = d["H"], d["W"], d["k"]
        flags = np.zeros(H * W, bool)
        out, _, _ = model.tier1(d["pred_norm"], d["prob"], d["xy"], d["angle"], d["ray"],
                                d["intr"], H, W, k, np.random.default_rng(rng_seed),
                                logits=d["logits"], flags=flags, G=model.kernel_waves(lib, d))
        want, ratio = fam.exact_terms(oracle, d)
        err = np.abs(out.astype(np.float32).astype(np.float64) - want).max(axis=0)
        evaluate.last = (err, ratio, flags)
        keep = ~flags & (ratio >= threshold) & np.isfinite(err)
        return np.where(keep, err, 0.0)
    return evaluate


def kernel_evaluator(oracle, lib, device, threshold: float):
    """The fast kernel's error per pixel through the C ABI (lib is
    brovisionml_amd._lib) on `device`, on the pixels it keeps in fp32 (ratio
    at or above `threshold`; it recomputes the rest), 0 elsewhere.  .last
    holds the last call's (err, ratio)."""
    import torch

    def evaluate(d):
        H, W, k = d["H"], d["W"], d["k"]
        t = {key: torch.from_numpy(np.ascontiguousarray(d[key])).to(device)
             for key in ("pred_norm", "prob", "xy", "angle", "ray")}
        out = torch.full_like(t["pred_norm"], float("nan"))
        fu, cu, fv, cv = d["intr"]
        st = lib.angmf_propagate_f32(t["pred_norm"].data_ptr(), t["prob"].data_ptr(),
                                     t["xy"].data_ptr(), t["angle"].data_ptr(),
                                     t["ray"].data_ptr(), fu, cu, fv, cv, 1, H, W, k, 0,
                                     out.data_ptr(), lib.LOGITS if d["logits"] else lib.DEFAULT)
        assert st == 0, lib.last_error()
        got = out.cpu().numpy().reshape(3, -1).astype(np.float64)
        want, ratio = fam.exact_terms(oracle, d)
        err = np.abs(got - want).max(axis=0)
        evaluate.last = (err, ratio)
        keep = (ratio >= threshold) & np.isfinite(err)
        return np.where(keep, err, 0.0)
    return evaluate
