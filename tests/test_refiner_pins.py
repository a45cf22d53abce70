"""The refiner restatement (oracle/refiner.py) against the closed-form pins of
tests/refiner_pins.py, and the same pins catching planted mistakes in it
(the GPU refiner meets the same pins in tests/test_gpu_refiner.py).  CPU
only: float64 convolutions on a 12 x 16 grid."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import refiner as oref
from tests import refiner_pins as pins

H, W, FOV, SEED = 12, 16, 60.0, 3


def run(pin, mutation=None, n0=0):
    n, feature, hidden, intr, fuv, ray8, uv8 = pins.setup(H, W, FOV, SEED)
    w, data = pins.pinned_weights(pin, SEED, n0=n0)
    trace, htrace = [], []
    oref.refine_forward(w, n, feature, hidden, intr, fuv, ray8, uv8, trace=trace,
                        hidden_trace=htrace, nthreads=8, mutation=mutation)
    return trace, htrace, data, (n, hidden, fuv, ray8)


def gate_closed_err(htrace, hidden):
    return max(float(np.abs(h - hidden).max()) for h in htrace)


def gate_open_err(htrace, bq):
    want = np.tanh(bq.astype(np.float64))[:, None, None]
    return max(float(np.abs(h - want).max()) for h in htrace)


def test_gate_closed_keeps_the_hidden_state():
    _, htrace, _, (_, hidden, _, _) = run("gate_closed")
    assert gate_closed_err(htrace, hidden) <= 1e-12
    _, htrace, _, _ = run("gate_closed", mutation="swap_zr")
    assert gate_closed_err(htrace, hidden) > 1e-2


def test_gate_open_is_tanh_of_the_bias():
    _, htrace, data, _ = run("gate_open")
    assert gate_open_err(htrace, data["bq"]) <= 1e-12
    _, htrace, data, _ = run("gate_open", mutation="swap_zr")
    assert gate_open_err(htrace, data["bq"]) > 1e-2


def test_constant_heads_propagate_directly():
    trace, _, data, (n, _, fuv, ray8) = run("const_heads")
    want = pins.const_heads_expected(data, n, ray8, fuv, H, W)
    for (p, _), w in zip(trace, want):
        assert np.array_equal(p.view(np.uint32), w.view(np.uint32))
    trace, _, data, _ = run("const_heads", mutation="swap_xy")
    errs = [float(np.abs(p.astype(np.float64) - w).max()) for (p, _), w in zip(trace, want)]
    assert max(errs) > 1e-3


@pytest.mark.parametrize("n0", [0, 5, 7])
def test_onehot_mask_picks_the_clamped_tap(n0):
    trace, _, _, _ = run("onehot_up", n0=n0)
    for p, up in trace:
        assert np.abs(up - pins.onehot_up_expected(p, n0)).max() <= 1e-6
    # the tap layout matters: the transposed tap (dy and dx exchanged) is off
    t = 3 * (n0 % 3) + n0 // 3
    if t != n0:
        p, up = trace[-1]
        assert np.abs(up - pins.onehot_up_expected(p, t)).max() > 1e-2
