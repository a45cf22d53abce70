"""The CPU oracle against the golden fixtures (tests/golden/*.npz), which the
independent library-based restatement (tests/golden/independent.py)
generated; see tests/golden/make_golden.py."""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest

import oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ANGMF = sorted(glob.glob(os.path.join(HERE, "angmf_*.npz")))
UPSAMPLE = sorted(glob.glob(os.path.join(HERE, "upsample_*.npz")))


def test_fixtures_present():
    assert len(ANGMF) >= 4
    assert len(UPSAMPLE) >= 4
    assert os.path.exists(os.path.join(HERE, "ray_relu_12x20.npz"))


@pytest.mark.parametrize("path", ANGMF, ids=[os.path.basename(p) for p in ANGMF])
def test_oracle_matches_fixture(path):
    d = np.load(path)
    H, W, k = int(d["H"]), int(d["W"]), int(d["k"])
    out, acc = oracle.angmf_propagate(d["pred_norm"], d["prob"], d["xy"], d["angle"], d["ray"],
                                      tuple(d["intr"]), H, W, k, return_acc=True)
    assert np.abs(acc - d["expect_acc"]).max() < 1e-11
    assert np.abs(out - d["expect_out"]).max() < 1e-7


def test_oracle_ray_relu_matches_fixture():
    d = np.load(os.path.join(HERE, "ray_relu_12x20.npz"))
    out = oracle.ray_relu(d["normal"], d["ray"], int(d["H"]), int(d["W"]))
    assert np.abs(out - d["expect"]).max() < 1e-7


@pytest.mark.parametrize("path", UPSAMPLE, ids=[os.path.basename(p) for p in UPSAMPLE])
def test_oracle_upsample_matches_fixture(path):
    d = np.load(path)
    out = oracle.convex_upsample(d["x"], d["mask"], int(d["H"]), int(d["W"]), int(d["s"]),
                                 normalize=bool(d["normalize"]))
    want = d["expect"]
    assert out.shape == want.shape
    assert (np.abs(out - want) / np.maximum(1.0, np.abs(want))).max() < 1.2e-7
