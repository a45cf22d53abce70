"""The refiner's fused elementwise kernels (brovisionml_amd/csrc/gru.hip,
through the C ABI) against plain PyTorch fp32 of the same steps
(src/dsine_refine.cpp:119-159): the ConvGRU's gates and update, a
convolution's bias + ReLU.  Channel slices of larger maps as arguments (as
the refiner passes them), odd plane sizes (the one-float-per-lane kernels)
and in-place updates; outputs inside canary-guarded buffers."""
from __future__ import annotations

import numpy as np
import pytest

from brovisionml_amd import dsine
from tests._util import Guarded

pytestmark = pytest.mark.gpu
TOL = 2e-6   # expf / tanhf of the device library against torch's, a few ulp


def _t(rng, shape, cuda, scale=3.0):
    import torch
    return torch.from_numpy((scale * rng.standard_normal(shape)).astype(np.float32)).to(cuda)


@pytest.mark.parametrize("C,H,W", [(64, 24, 32), (64, 7, 9), (5, 1, 3)])
def test_gru_gates_and_update(cuda, C, H, W):
    import torch
    rng = np.random.default_rng(C + H + W)
    HW = H * W
    zr = _t(rng, (1, 2 * C, H, W), cuda)
    h = _t(rng, (1, C, H, W), cuda, 1.0)
    bz, br, bq = _t(rng, (C,), cuda), _t(rng, (C,), cuda), _t(rng, (C,), cuda)
    qp = _t(rng, (1, C, H, W), cuda)
    # rh into a channel slice of a wider map, z and the copy into guarded buffers
    rhx = torch.full((1, C + 3, H, W), 7.0, device=cuda)
    gz = Guarded(C * HW, cuda)
    dsine.gru_gates(zr, bz, br, h, C, HW, gz.out, rhx[:, :C])
    torch.cuda.synchronize()
    z_want = torch.sigmoid(zr[:, :C] + bz[None, :, None, None])
    r_want = torch.sigmoid(zr[:, C:] + br[None, :, None, None])
    assert gz.intact()
    assert (gz.out.view(1, C, H, W) - z_want).abs().max().item() <= TOL
    assert (rhx[:, :C] - r_want * h).abs().max().item() <= TOL
    assert (rhx[:, C:] == 7.0).all()
    # update in place on h, and a copy into a slice of [h_new | uv]
    q_want = torch.tanh(qp + bq[None, :, None, None])
    hn_want = (1 - z_want) * h + z_want * q_want
    hin = torch.full((1, C + 2, H, W), 5.0, device=cuda)
    hh = h.clone()
    dsine.gru_update(qp, bq, gz.out.view(1, C, H, W), hh, C, HW, hh, hin[:, :C])
    torch.cuda.synchronize()
    assert (hh - hn_want).abs().max().item() <= 2 * TOL
    assert torch.equal(hin[:, :C], hh)
    assert (hin[:, C:] == 5.0).all()


@pytest.mark.parametrize("C,H,W,relu", [(256, 24, 32, True), (3, 5, 7, True), (64, 8, 8, False)])
def test_bias_act(cuda, C, H, W, relu):
    import torch
    rng = np.random.default_rng(C * 7 + H)
    x = _t(rng, (1, C, H, W), cuda)
    b = _t(rng, (C,), cuda)
    want = x + b[None, :, None, None]
    if relu:
        want = torch.relu(want)
    g = Guarded(C * H * W, cuda, fill=x.cpu().numpy())
    dsine.bias_act(g.out, b, C, H * W, relu=relu)
    torch.cuda.synchronize()
    assert g.intact()
    assert torch.equal(g.out.view(1, C, H, W), want)


def test_fused_kernels_reject_bad_arguments(cuda):
    import torch
    C, HW = 4, 16
    a = torch.zeros(2 * C * HW, device=cuda)
    h = torch.zeros(C * HW, device=cuda)
    b = torch.zeros(C, device=cuda)
    with pytest.raises(RuntimeError, match="^dsine ops: gru_gates"):
        dsine.gru_gates(a, b, b, h, C, HW, h, h)     # z and rh overlap h
    with pytest.raises(RuntimeError, match="holds"):
        dsine.bias_act(h, torch.zeros(C + 1, device=cuda), C, HW, relu=True)
    with pytest.raises(RuntimeError, match="HIP device"):
        dsine.bias_act(h.cpu(), b.cpu(), C, HW, relu=True)
