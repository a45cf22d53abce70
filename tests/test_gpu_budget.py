"""The fast kernel against the error budget of its recompute threshold, on
the GPU: every input family of tests/budget_families.py, through the C ABI,
in both work layouts (two 128 x 128 draws at k = 3, 5, 7 and 9: G > 1 waves
per 64-pixel group; one 768 x 768 draw at k = 5 and 7: the whole-window
layout).  For the pixels the kernel keeps (cancellation ratio |acc|^2 /
sum (prob/|p|)^2 at or above its threshold, from the oracle's double sums)
the error stays within 75% of the 1e-5 bar and, in the cancellation band,
err * sqrt(ratio) within DELTA_KERNEL, the delta the threshold is derived
from (tests/test_tier1_budget.py); every pixel, recomputed ones included, is
within the bar.  A hill-climbing search from each family toward the largest
kept error (tests/budget_search.py) holds the same bounds."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from brovisionml_amd import _lib
from tests import budget_families as fam
from tests._util import TOL_ABS
from tests.test_tier1_budget import BAR, DELTA_KERNEL, HEADROOM


def _check(cuda, name, H, W, k, seeds, whole):
    import torch
    worst_kept, worst_delta = 0.0, 0.0
    for seed in seeds:
        rng = np.random.default_rng(seed)
        d = fam.family(name, rng, H, W, k)
        want, ratio = fam.exact_terms(oracle, d)
        flags = _lib.LOGITS if d["logits"] else _lib.DEFAULT
        fu, cu, fv, cv = d["intr"]
        fp32, g, _, _ = _lib.angmf_plan(1, H, W, k, fu, cu, fv, cv, flags)
        # (the 140-degree family's corner rays exceed the fast path's |P0| at
        # 768 x 768: the double-precision kernel runs it, within the bar)
        assert (fp32 and (g == 1) == whole) or (name == "widefov" and H > 128), (fp32, g)
        t = {key: torch.from_numpy(np.ascontiguousarray(d[key])).to(cuda)
             for key in ("pred_norm", "prob", "xy", "angle", "ray")}
        out = torch.full_like(t["pred_norm"], float("nan"))
        st = _lib.angmf_propagate_f32(t["pred_norm"].data_ptr(), t["prob"].data_ptr(),
                                      t["xy"].data_ptr(), t["angle"].data_ptr(),
                                      t["ray"].data_ptr(), fu, cu, fv, cv, 1, H, W, k, 0,
                                      out.data_ptr(), flags)
        assert st == 0, _lib.last_error()
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(3, -1).astype(np.float64)
        err = np.abs(got - want).max(axis=0)
        assert np.isfinite(err).all()
        assert err.max() <= TOL_ABS
        keep = ratio >= _lib.angmf_recompute_ratio(k, flags)
        band = keep & (ratio < 0.05)
        worst_kept = max(worst_kept, float(err[keep].max()))
        if band.any():
            worst_delta = max(worst_delta, float((err[band] * np.sqrt(ratio[band])).max()))
    print(f"{name} {H}x{W} k={k}: worst kept error {worst_kept:.3e}, worst band delta "
          f"{worst_delta:.3e}", flush=True)
    assert worst_kept <= HEADROOM * BAR
    assert worst_delta <= DELTA_KERNEL[k]


@pytest.mark.gpu
@pytest.mark.parametrize("name", fam.FAMILIES)
@pytest.mark.parametrize("k", [3, 5, 7, 9])
def test_kernel_budget(cuda, name, k):
    """The run-split layout (128 x 128: G > 1 waves per 64-pixel group, each
    run summed in fp32, the runs in double)."""
    _check(cuda, name, 128, 128, k, (11, 12), whole=False)


@pytest.mark.gpu
@pytest.mark.parametrize("name", fam.FAMILIES)
@pytest.mark.parametrize("k", [5, 7])
def test_kernel_budget_whole_window(cuda, name, k):
    """The whole-window layout (768 x 768: one wave sums all k*k neighbours
    of its pixels in fp32)."""
    _check(cuda, name, 768, 768, k, (13,), whole=True)


@pytest.mark.gpu
@pytest.mark.parametrize("H,W,k,steps", [(64, 64, 3, 30), (64, 64, 5, 30), (64, 64, 7, 30),
                                         (64, 64, 9, 20), (768, 768, 5, 5), (768, 768, 7, 4)])
def test_kernel_adversarial_search(cuda, H, W, k, steps):
    """A hill-climbing search (tests/budget_search.py) over the kernel's own
    inputs, from each family that stresses a mechanism, toward the largest
    error of a pixel the kernel keeps in fp32 (64 x 64: the run-split layout;
    768 x 768: the whole-window layout): the worst found stays 25% inside the
    bar, and the climbed inputs' cancellation-band delta within DELTA_KERNEL."""
    from tests import budget_search as bs
    t = _lib.angmf_recompute_ratio(k)
    evaluate = bs.kernel_evaluator(oracle, _lib, cuda, t)
    worst, worst_delta = 0.0, 0.0
    for name in bs.SEEDS:
        if name == "widefov" and H > 128:
            continue   # the double-precision kernel runs it at this size
        rng = np.random.default_rng(7)
        d = fam.family(name, rng, H, W, k)
        score, climbed = bs.climb(evaluate, d, steps, rng)
        evaluate(climbed)
        err, ratio = evaluate.last
        band = (ratio >= t) & (ratio < 0.05)
        worst = max(worst, float(score.max()))
        if band.any():
            worst_delta = max(worst_delta, float((err[band] * np.sqrt(ratio[band])).max()))
    print(f"{H}x{W} k={k}: worst kept error found {worst:.3e}, band delta {worst_delta:.3e}",
          flush=True)
    assert 0.0 < worst <= HEADROOM * BAR
    assert worst_delta <= DELTA_KERNEL[k]
