"""The error bounds of the gfx950 hardware functions the fast kernels rely on,
measured over every float argument of the range each kernel feeds them, against
double-precision references (tests/hw/probe.hip).  These are the constants of
the tier-1 model (tests/tier1_model.py), hence of the propagate's recompute
threshold, and the upsample's kExpRel (brovisionml_amd/csrc/upsample.hip)."""
from __future__ import annotations

import os
import re

import numpy as np
import pytest

from tests import tier1_model as model
from tests.hw import probe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def upsample_exp_rel() -> float:
    src = open(os.path.join(ROOT, "brovisionml_amd", "csrc", "upsample.hip")).read()
    m = re.search(r"constexpr (?:float|double) kExpRel = ([0-9.eE+-]+)f?;", src)
    assert m, "kExpRel not found"
    return float(m.group(1))


# (function, magnitudes lo..hi, negative arguments, absolute or relative, bound)
CASES = [
    # sincos_hw: a = t / (2 pi) for |t| <= 3.2, both signs
    ("sin", 0.0, 0.51, False, "abs", model.SIN_ABS),
    ("sin", 0.0, 0.51, True, "abs", model.SIN_ABS),
    ("cos", 0.0, 0.51, False, "abs", model.SIN_ABS),
    ("cos", 0.0, 0.51, True, "abs", model.SIN_ABS),
    # rsq: |xy|^2 in [1e-20, 1e30], |c|^2 >= 1e-30, |p|^2 up to ~(1 + 2.02)^2, |r|^2 ~ 1
    ("rsq", 1e-30, 1e30, False, "rel", model.RSQ_REL),
    # rcp: d = 1 + exp(-L) for L >= -87 (sigmoid_f32 returns 0 below), so
    # d in [1, 1 + e^87 = 6.08e37]; beyond 8.5e37 the reciprocal is below the
    # normal range and the hardware returns 0
    ("rcp", 1.0, 6.1e37, False, "rel", model.RCP_REL),
    # exp2: the upsample's weights on [-126, 0]; the logits' exp(-L) on [-126, 126]
    ("exp2", 0.0, 126.0, True, "rel", model.EXP2_REL),
    ("exp2", 0.0, 126.0, False, "rel", model.EXP2_REL),
]


@pytest.mark.gpu
@pytest.mark.parametrize("op,lo,hi,neg,kind,bound", CASES)
def test_hardware_function_bound(cuda, op, lo, hi, neg, kind, bound):
    a, r, arg = probe.hw_error(op, lo, hi, neg)
    got = a if kind == "abs" else r
    print(f"{op} [{'-' if neg else ''}{lo}, {hi}]: max abs {a:.4e} max rel {r:.4e} at {arg!r}",
          flush=True)
    assert got <= bound
    # the bound is tight: within 15% of the measured maximum
    assert got >= 0.85 * bound


@pytest.mark.gpu
def test_upsample_exp_constant(cuda):
    """The upsample's kExpRel covers v_exp_f32 on its [-126, 0] weights."""
    _, r, _ = probe.hw_error("exp2", 0.0, 126.0, True)
    assert r <= upsample_exp_rel()


@pytest.mark.gpu
@pytest.mark.parametrize("unroll", [1, 2, 4, 8])
def test_stream_read_reads_every_element(cuda, unroll):
    """The read ceiling's probe touches each float of the buffer once: its
    partials add up to the buffer's sum (odd length: a float tail)."""
    import torch
    from tests.hw import probe
    n = 1_000_003
    rng = np.random.default_rng(unroll)
    x = rng.integers(-8, 8, n).astype(np.float32)   # small integers: exact float sums
    buf = torch.from_numpy(x).to(cuda)
    n_part = probe.read_partials(n, unroll)
    part = torch.full((n_part + 64,), 12345.0, dtype=torch.float32, device=cuda)
    probe.stream_read(buf.data_ptr(), n, unroll, part.data_ptr(), n_part)
    torch.cuda.synchronize()
    p = part.cpu().numpy()
    assert (p[n_part:] == 12345.0).all()
    assert float(p[:n_part].astype(np.float64).sum()) == float(x.astype(np.float64).sum())
