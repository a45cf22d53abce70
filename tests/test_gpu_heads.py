"""bvml_dsine_heads_mlp_f32 (brovisionml_amd/csrc/heads.hip: the refiner's
heads after their 3x3 layer, src/dsine_refine.cpp:119-127, on the fp32
matrix cores) against a float64 restatement of the same two 1x1 layers, on
synthetic weights at the checkpoint's widths, with ragged pixel counts and
guard regions around every output.

The kernel's sums are fp32 in the matrix instruction's order, so the bar is
a rounding bound, per output: 4 x (64 u sum |W4| |t| + sum |W4| e_t + u |out|)
with e_t = 64 u sum |W2| |a| + u |t| the middle layer's bound and u = 2^-24,
twice the worst case of a sequential sum, times two for slack."""
from __future__ import annotations

import numpy as np
import pytest

from brovisionml_amd import _lib, refiner as rf
from tests._util import Guarded

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


def say(msg: str) -> None:
    print(msg, flush=True)


def reference(t0, b0, w2, b2, w4s, b4s):
    """float64 restatement and its rounding bound, per head."""
    nh = len(w4s)
    outs, bounds = [], []
    for h in range(nh):
        a = np.maximum(t0[64 * h:64 * (h + 1)] + b0[64 * h:64 * (h + 1), None], 0)  # fp32 ops
        a = np.where(a < 0, 0, a).astype(np.float64)
        W2 = w2[h].astype(np.float64)
        s = W2 @ a + b2[64 * h:64 * (h + 1), None].astype(np.float64)
        t = np.maximum(s, 0)
        et = 64 * U * (np.abs(W2) @ np.abs(a)) + U * np.abs(s)
        W4 = w4s[h].astype(np.float64)
        o = W4 @ t
        if b4s[h] is not None:
            o = o + b4s[h].astype(np.float64)[:, None]
        eo = 64 * U * (np.abs(W4) @ t) + np.abs(W4) @ et + U * np.abs(o)
        outs.append(o)
        bounds.append(4 * eo + 1e-30)
    return outs, bounds


@pytest.mark.parametrize("H,W,outs,with_bias", [
    (24, 32, (25, 50, 25), True),
    (13, 19, (25, 50, 25), True),
    (16, 20, (25, 50, 25, 576), True),
    (7, 9, (1, 17, 33, 64), False),
    (1, 1, (25,), True),
    (256, 256, (25, 50, 25), True),
])
def test_heads_mlp(cuda, H, W, outs, with_bias):
    import torch
    nh = len(outs)
    say(f"[gpu] heads_mlp {H}x{W} outs {outs}")
    rng = np.random.default_rng(H * 1000 + W + nh)
    HW = H * W
    t0 = rng.standard_normal((64 * nh, HW)).astype(np.float32)
    b0 = rng.uniform(-0.5, 0.5, 64 * nh).astype(np.float32)
    w2 = rng.uniform(-1 / 8, 1 / 8, (nh, 64, 64)).astype(np.float32)
    b2 = rng.uniform(-1 / 8, 1 / 8, 64 * nh).astype(np.float32)
    w4s = [rng.uniform(-1 / 8, 1 / 8, (n, 64)).astype(np.float32) for n in outs]
    b4s = [rng.uniform(-1 / 8, 1 / 8, n).astype(np.float32) if with_bias else None for n in outs]
    w2p, w4p = _lib.heads_pack_f32(w2, w4s)
    dev = torch.device(cuda)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    t0d, b0d, b2d, w2pd = T(t0), T(b0), T(b2), T(w2p)
    w4pd = [T(w) for w in w4p]
    b4d = [T(b) if b is not None else None for b in b4s]
    outd = [Guarded(n * HW, dev, shift=h) for h, n in enumerate(outs)]
    st = _lib.heads_mlp_f32(t0d.data_ptr(), b0d.data_ptr(), w2pd.data_ptr(), b2d.data_ptr(),
                            [w.data_ptr() for w in w4pd],
                            [b.data_ptr() if b is not None else 0 for b in b4d], list(outs), H, W,
                            [o.out.data_ptr() for o in outd],
                            torch.cuda.current_stream(dev).cuda_stream)
    assert st == _lib.OK, _lib.last_error()
    torch.cuda.synchronize()
    want, bound = reference(t0, b0, w2, b2, w4s, b4s)
    for h in range(nh):
        assert outd[h].intact(), f"head {h} wrote outside its output"
        got = outd[h].out.cpu().numpy().reshape(outs[h], HW).astype(np.float64)
        err = np.abs(got - want[h])
        say(f"    head {h}: max-abs {err.max():.3e}, max err/bound {(err / bound[h]).max():.3f}")
        assert (err <= bound[h]).all()


def test_heads_mlp_relu_and_nan(cuda):
    """ReLU is v < 0 ? 0 : v at both layers: a NaN in t0 reaches every output
    of that pixel; -0.0 and negative inputs give exactly the bias path."""
    import torch
    H, W, outs = 4, 8, (25, 50, 25)
    rng = np.random.default_rng(3)
    t0 = -np.abs(rng.standard_normal((192, H * W))).astype(np.float32) - 10  # all clamp to 0
    t0[5, 3] = np.nan
    b0 = np.zeros(192, np.float32)
    w2 = rng.uniform(-1 / 8, 1 / 8, (3, 64, 64)).astype(np.float32)
    b2 = rng.uniform(-1, 1, 192).astype(np.float32)
    w4s = [rng.uniform(-1 / 8, 1 / 8, (n, 64)).astype(np.float32) for n in outs]
    b4s = [rng.uniform(-1, 1, n).astype(np.float32) for n in outs]
    w2p, w4p = _lib.heads_pack_f32(w2, w4s)
    dev = torch.device(cuda)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    out = [torch.empty(n * H * W, device=dev) for n in outs]
    keep = [T(x) for x in (t0, b0, w2p, b2)] + [T(w) for w in w4p] + [T(b) for b in b4s]
    st = _lib.heads_mlp_f32(keep[0].data_ptr(), keep[1].data_ptr(), keep[2].data_ptr(),
                            keep[3].data_ptr(), [w.data_ptr() for w in keep[4:7]],
                            [b.data_ptr() for b in keep[7:10]], list(outs), H, W,
                            [o.data_ptr() for o in out], torch.cuda.current_stream(dev).cuda_stream)
    assert st == _lib.OK
    torch.cuda.synchronize()
    for h, n in enumerate(outs):
        got = out[h].cpu().numpy().reshape(n, H * W)
        # head 0 holds the NaN channel: its pixel 3 is NaN everywhere, as torch's relu passes NaN
        if h == 0:
            assert np.isnan(got[:, 3]).all()
            got = np.delete(got, 3, axis=1)
        t = np.maximum(b2[64 * h:64 * (h + 1)].astype(np.float64), 0)
        want = w4s[h].astype(np.float64) @ t + b4s[h]
        assert np.abs(got - want[:, None]).max() <= 1e-5


def test_heads_mlp_rejects(cuda):
    import torch
    dev = torch.device(cuda)
    x = torch.zeros(64 * 3 * 16, device=dev)
    p = x.data_ptr()
    assert _lib.heads_mlp_f32(p, p, p, p, [p], [0], [25], 4, 4, [p]) == _lib.EALIAS
    assert _lib.heads_mlp_f32(p, p, p, p, [p] * 5, [0] * 5, [1] * 5, 4, 4, [p] * 5) == _lib.EPARAM
    assert _lib.heads_mlp_f32(p, p, p, p, [p], [0], [0], 4, 4, [p]) == _lib.EPARAM
    assert _lib.heads_mlp_f32(0, p, p, p, [p], [0], [25], 4, 4, [p]) == _lib.ENULL
    assert _lib.heads_mlp_f32(p, p, p, p, [p], [0], [25], -1, 4, [p]) == _lib.ESHAPE
    assert rf.N_ITER == 5


def reference_fused(x, w3, b0, w2, b2, w4s, b4s):
    """float64 restatement of the 3x3 layer and the heads after it, with the
    rounding bound carried through: the convolution's own bound (conv64), the
    bias adds, then the two 1x1 layers as in reference() with the middle
    layer's inputs uncertain by the 3x3 layer's bound."""
    from tests.test_gpu_conv import conv64
    s3, e3 = conv64(x, w3)
    nh = len(w4s)
    s3 = s3.reshape(64 * nh, -1)
    e3 = e3.reshape(64 * nh, -1)
    outs, bounds = [], []
    for h in range(nh):
        pre = s3[64 * h:64 * (h + 1)] + b0[64 * h:64 * (h + 1), None]
        a = np.maximum(pre, 0)
        ea = e3[64 * h:64 * (h + 1)] + U * np.abs(pre)
        W2 = w2[h].astype(np.float64)
        s = W2 @ a + b2[64 * h:64 * (h + 1), None].astype(np.float64)
        t = np.maximum(s, 0)
        et = 64 * U * (np.abs(W2) @ a) + np.abs(W2) @ ea + U * np.abs(s)
        W4 = w4s[h].astype(np.float64)
        o = W4 @ t
        if b4s[h] is not None:
            o = o + b4s[h].astype(np.float64)[:, None]
        eo = 64 * U * (np.abs(W4) @ t) + np.abs(W4) @ et + U * np.abs(o)
        outs.append(o)
        bounds.append(4 * eo + 1e-30)
    return outs, bounds


@pytest.mark.parametrize("H,W,outs,with_bias", [
    (24, 32, (25, 50, 25), True),       # two wave groups per workgroup (a small grid)
    (13, 19, (25, 50, 25), True),       # ragged tiles
    (224, 240, (25, 50, 25), True),     # one wave group, three workgroups per CU
    (16, 20, (25, 50, 25, 576), True),  # the up-mask head too
    (7, 9, (1, 17, 33, 64), False),
])
def test_conv_heads(cuda, H, W, outs, with_bias):
    """bvml_dsine_conv_heads_f32 (the 3x3 layer with the heads in its
    epilogue) against the float64 restatement, and against the unfused
    bvml_dsine_conv_f32 + bvml_dsine_heads_mlp_f32 to the same bound."""
    import torch
    nh = len(outs)
    say(f"[gpu] conv_heads {H}x{W} outs {outs}")
    rng = np.random.default_rng(H * 7 + W + nh)
    HW, cin = H * W, 66
    x = rng.standard_normal((cin, H, W)).astype(np.float32)
    w3 = rng.uniform(-1, 1, (64 * nh, cin, 3, 3)).astype(np.float32) / np.sqrt(cin * 9)
    b0 = rng.uniform(-0.5, 0.5, 64 * nh).astype(np.float32)
    w2 = rng.uniform(-1 / 8, 1 / 8, (nh, 64, 64)).astype(np.float32)
    b2 = rng.uniform(-1 / 8, 1 / 8, 64 * nh).astype(np.float32)
    w4s = [rng.uniform(-1 / 8, 1 / 8, (n, 64)).astype(np.float32) for n in outs]
    b4s = [rng.uniform(-1 / 8, 1 / 8, n).astype(np.float32) if with_bias else None for n in outs]
    w2p, w4p = _lib.heads_pack_f32(w2, w4s)
    dev = torch.device(cuda)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    xd, w3d = T(x), T(_lib.conv_pack_f32(w3))
    b0d, b2d, w2pd, w2qd = T(b0), T(b2), T(w2p), T(_lib.heads_w2q_f32(w2))
    w4pd = [T(w) for w in w4p]
    b4d = [T(b) if b is not None else None for b in b4s]
    b4p = [b.data_ptr() if b is not None else 0 for b in b4d]
    stream = torch.cuda.current_stream(dev).cuda_stream
    outd = [Guarded(n * HW, dev, shift=h + 1) for h, n in enumerate(outs)]
    st = _lib.conv_heads_f32(xd.data_ptr(), cin, H, W, w3d.data_ptr(), b0d.data_ptr(),
                             w2qd.data_ptr(), b2d.data_ptr(), [w.data_ptr() for w in w4pd], b4p,
                             list(outs), [o.out.data_ptr() for o in outd], stream)
    assert st == _lib.OK, _lib.last_error()
    # the unfused path
    t0 = torch.empty(64 * nh * HW, device=dev)
    lib = _lib.load()
    assert lib.bvml_dsine_conv_f32(xd.data_ptr(), cin, H, W, w3d.data_ptr(), 64 * nh, 3,
                                   t0.data_ptr(), stream) == _lib.OK, _lib.last_error()
    unf = [torch.empty(n * HW, device=dev) for n in outs]
    assert _lib.heads_mlp_f32(t0.data_ptr(), b0d.data_ptr(), w2pd.data_ptr(), b2d.data_ptr(),
                              [w.data_ptr() for w in w4pd], b4p, list(outs), H, W,
                              [u.data_ptr() for u in unf], stream) == _lib.OK, _lib.last_error()
    torch.cuda.synchronize()
    want, bound = reference_fused(x, w3, b0, w2, b2, w4s, b4s)
    for h in range(nh):
        assert outd[h].intact(), f"head {h} wrote outside its output"
        got = outd[h].out.cpu().numpy().reshape(outs[h], HW).astype(np.float64)
        ref = unf[h].cpu().numpy().reshape(outs[h], HW).astype(np.float64)
        err = np.abs(got - want[h])
        say(f"    head {h}: max-abs {err.max():.3e}, max err/bound {(err / bound[h]).max():.3f}, "
            f"against the unfused path {np.abs(got - ref).max():.3e}")
        assert (err <= bound[h]).all()
        assert (np.abs(ref - want[h]) <= bound[h]).all()


def test_conv_heads_rejects(cuda):
    import torch
    dev = torch.device(cuda)
    x = torch.zeros(66 * 16 * 4, device=dev)
    p = x.data_ptr()
    f = _lib.conv_heads_f32
    assert f(p, 66, 4, 4, p, p, p, p, [p], [0], [25], [p]) == _lib.EALIAS
    assert f(p, 66, 4, 4, p, p, p, p, [p] * 5, [0] * 5, [1] * 5, [p] * 5) == _lib.EPARAM
    assert f(p, 66, 4, 4, p, p, p, p, [p], [0], [0], [p]) == _lib.EPARAM
    assert f(0, 66, 4, 4, p, p, p, p, [p], [0], [25], [p]) == _lib.ENULL
    assert f(p, 66, -1, 4, p, p, p, p, [p], [0], [25], [p]) == _lib.ESHAPE
    assert f(p, 66, 8193, 8193, p, p, p, p, [p], [0], [25], [p]) == _lib.ESIZE


def test_conv_heads_nan_pattern(cuda):
    """A NaN in the 3x3 layer's input reaches exactly the outputs of the
    pixels whose 3x3 window holds it, in the fused and the unfused path
    alike; every other output of the two paths agrees."""
    import torch
    H, W, outs, cin = 20, 24, (25, 50, 25), 66
    nh = len(outs)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((cin, H, W)).astype(np.float32)
    x[7, 9, 13] = np.nan
    w3 = rng.uniform(-1, 1, (64 * nh, cin, 3, 3)).astype(np.float32) / np.sqrt(cin * 9)
    b0 = rng.uniform(-0.5, 0.5, 64 * nh).astype(np.float32)
    w2 = rng.uniform(-1 / 8, 1 / 8, (nh, 64, 64)).astype(np.float32)
    b2 = rng.uniform(-1 / 8, 1 / 8, 64 * nh).astype(np.float32)
    w4s = [rng.uniform(-1 / 8, 1 / 8, (n, 64)).astype(np.float32) for n in outs]
    b4s = [rng.uniform(-1 / 8, 1 / 8, n).astype(np.float32) for n in outs]
    w2p, w4p = _lib.heads_pack_f32(w2, w4s)
    dev = torch.device(cuda)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    xd, w3d = T(x), T(_lib.conv_pack_f32(w3))
    b0d, b2d, w2pd, w2qd = T(b0), T(b2), T(w2p), T(_lib.heads_w2q_f32(w2))
    w4pd = [T(w) for w in w4p]
    b4d = [T(b) for b in b4s]
    stream = torch.cuda.current_stream(dev).cuda_stream
    fused = [torch.empty(n * H * W, device=dev) for n in outs]
    assert _lib.conv_heads_f32(xd.data_ptr(), cin, H, W, w3d.data_ptr(), b0d.data_ptr(),
                               w2qd.data_ptr(), b2d.data_ptr(), [w.data_ptr() for w in w4pd],
                               [b.data_ptr() for b in b4d], list(outs),
                               [o.data_ptr() for o in fused], stream) == _lib.OK
    t0 = torch.empty(64 * nh * H * W, device=dev)
    assert _lib.load().bvml_dsine_conv_f32(xd.data_ptr(), cin, H, W, w3d.data_ptr(), 64 * nh, 3,
                                           t0.data_ptr(), stream) == _lib.OK
    unf = [torch.empty(n * H * W, device=dev) for n in outs]
    assert _lib.heads_mlp_f32(t0.data_ptr(), b0d.data_ptr(), w2pd.data_ptr(), b2d.data_ptr(),
                              [w.data_ptr() for w in w4pd], [b.data_ptr() for b in b4d],
                              list(outs), H, W, [u.data_ptr() for u in unf], stream) == _lib.OK
    torch.cuda.synchronize()
    window = np.zeros((H, W), bool)
    window[8:11, 12:15] = True
    for h, n in enumerate(outs):
        f = fused[h].cpu().numpy().reshape(n, H, W)
        u = unf[h].cpu().numpy().reshape(n, H, W)
        assert np.isnan(f[:, window]).all() and np.isnan(u[:, window]).all()
        assert np.isfinite(f[:, ~window]).all()
        assert np.abs(f[:, ~window] - u[:, ~window]).max() <= 1e-5
