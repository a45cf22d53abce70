"""bvml_dsine_conv_* (brovisionml_amd/csrc/conv.hip: the refiner's 5x5 and 3x3
convolutions as implicit GEMMs on the fp32 matrix cores, with the ConvGRU's
gates and update fused into their epilogues; src/dsine_refine.cpp:94-101,
:138-159) against a float64 restatement (torch's conv2d in float64 on the
CPU), at the refiner's channel counts and on ragged maps, with guard regions
around every output.

The sums are fp32 in the matrix instruction's order: the bar for a
convolution output is a rounding bound, 4 * (n u sum |w| |x| + u |s|) with n
the reduction length and u = 2^-24 (twice the worst case of a sequential sum,
times two).  The fused gates and update then round as the elementwise
kernels do; their bar adds the activations' few ulps."""
from __future__ import annotations

import numpy as np
import pytest

from brovisionml_amd import _lib
from tests._util import Guarded

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


def say(msg: str) -> None:
    print(msg, flush=True)


def conv64(x, w):
    """float64 conv, zero 'same' padding, and its rounding bound."""
    import torch
    import torch.nn.functional as F
    k = w.shape[-1]
    xt = torch.from_numpy(x.astype(np.float64))[None]
    wt = torch.from_numpy(w.astype(np.float64))
    s = F.conv2d(xt, wt, padding=k // 2)[0].numpy()
    mag = F.conv2d(xt.abs(), wt.abs(), padding=k // 2)[0].numpy()
    n = w.shape[1] * k * k
    return s, 4 * (n * U * mag + U * np.abs(s)) + 1e-30


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("cin,cout,k,H,W", [
    (130, 64, 5, 24, 32), (66, 256, 3, 20, 36), (66, 192, 3, 13, 19), (7, 20, 5, 9, 5),
    (130, 128, 5, 1, 1), (66, 192, 3, 64, 80),
    # one chunk of input channels: the second wave group of a split launch has none
    (3, 20, 5, 9, 5), (4, 64, 5, 17, 33),
])
def test_conv_plain(cuda, cin, cout, k, H, W):
    import torch
    say(f"[gpu] conv {cin}->{cout} k{k} {H}x{W}")
    rng = np.random.default_rng(cin * 7 + cout + k + H)
    x = rng.standard_normal((cin, H, W)).astype(np.float32)
    w = rng.uniform(-1, 1, (cout, cin, k, k)).astype(np.float32) / np.sqrt(cin * k * k)
    dev = torch.device(cuda)
    wp = _dev(_lib.conv_pack_f32(w), dev)
    xd = _dev(x, dev)
    out = Guarded(cout * H * W, dev, shift=1)
    st = _lib.load().bvml_dsine_conv_f32(xd.data_ptr(), cin, H, W, wp.data_ptr(), cout, k,
                                         out.out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert st == _lib.OK, _lib.last_error()
    torch.cuda.synchronize()
    assert out.intact()
    want, bound = conv64(x, w)
    err = np.abs(out.out.cpu().numpy().reshape(cout, H, W) - want)
    say(f"    max-abs {err.max():.3e}, max err/bound {(err / bound).max():.3f}")
    assert (err <= bound).all()


def _sig(v):
    return 1.0 / (1.0 + np.exp(-v))


# (256 x 520: 528 tiles, so convq runs with one wave group, the launch for
# maps of two or more workgroups per CU)
@pytest.mark.parametrize("H,W", [(24, 32), (13, 19), (64, 64), (256, 520)])
def test_conv_gru(cuda, H, W):
    """The fused gates (convz + convr) and update (convq) against the float64
    restatement of src/dsine_refine.cpp:145-157."""
    import torch
    say(f"[gpu] conv gru {H}x{W}")
    C, cin = 64, 130
    rng = np.random.default_rng(H + W)
    hx = rng.standard_normal((cin, H, W)).astype(np.float32)
    h = hx[:C].copy()
    wz, wr, wq = (rng.uniform(-1, 1, (C, cin, 5, 5)).astype(np.float32) / np.sqrt(cin * 25)
                  for _ in range(3))
    bz, br, bq = (rng.uniform(-0.3, 0.3, C).astype(np.float32) for _ in range(3))
    dev = torch.device(cuda)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    wzr = _dev(_lib.conv_pack_f32(np.concatenate([wz, wr]), interleave=True), dev)
    wqp = _dev(_lib.conv_pack_f32(wq), dev)
    hxd, hd = _dev(hx, dev), _dev(h, dev)
    bzd, brd, bqd = _dev(bz, dev), _dev(br, dev), _dev(bq, dev)
    z = Guarded(C * H * W, dev)
    rh = Guarded(C * H * W, dev, shift=3)
    st = lib.bvml_dsine_conv_gru_gates_f32(hxd.data_ptr(), cin, H, W, wzr.data_ptr(), C,
                                           bzd.data_ptr(), brd.data_ptr(), hd.data_ptr(),
                                           z.out.data_ptr(), rh.out.data_ptr(), stream)
    assert st == _lib.OK, _lib.last_error()
    # update on x = [rh | hx[C:]] as the refiner feeds it
    rhx = torch.cat([rh.out.view(C, H, W), hxd[C:]]).contiguous()
    hn = Guarded(C * H * W, dev, shift=2)
    hc = Guarded(C * H * W, dev, shift=5)
    st = lib.bvml_dsine_conv_gru_update_f32(rhx.data_ptr(), cin, H, W, wqp.data_ptr(), C,
                                            bqd.data_ptr(), z.out.data_ptr(), hd.data_ptr(),
                                            hn.out.data_ptr(), hc.out.data_ptr(), stream)
    assert st == _lib.OK, _lib.last_error()
    torch.cuda.synchronize()
    assert z.intact() and rh.intact() and hn.intact() and hc.intact()
    sz, ez = conv64(hx, wz)
    sr, er = conv64(hx, wr)
    want_z = _sig(sz + bz[:, None, None])
    want_rh = _sig(sr + br[:, None, None]) * h
    # sigmoid' <= 1/4: the sum's bound carries through, plus a few ulps of the activation
    gz = z.out.cpu().numpy().reshape(C, H, W)
    grh = rh.out.cpu().numpy().reshape(C, H, W)
    e1 = np.abs(gz - want_z) - (ez / 4 + 8 * U)
    e2 = np.abs(grh - want_rh) - (np.abs(h) * (er / 4 + 8 * U))
    say(f"    gates: z max-abs {np.abs(gz - want_z).max():.3e}, rh max-abs "
        f"{np.abs(grh - want_rh).max():.3e}")
    assert (e1 <= 0).all() and (e2 <= 0).all()
    # the update from the device's own z and rh (so the gates' rounding does not enter)
    rhx_h = rhx.cpu().numpy()
    sq, eq = conv64(rhx_h, wq)
    q = np.tanh(sq + bq[:, None, None])
    want_h = (1 - gz.astype(np.float64)) * h + gz * q
    ghn = hn.out.cpu().numpy().reshape(C, H, W)
    bound_h = np.abs(gz) * eq + 16 * U * (np.abs(h) + np.abs(q))
    say(f"    update: max-abs {np.abs(ghn - want_h).max():.3e}")
    assert (np.abs(ghn - want_h) <= bound_h).all()
    assert np.array_equal(ghn, hc.out.cpu().numpy().reshape(C, H, W))


@pytest.mark.parametrize("H,W", [(24, 32), (13, 19)])
def test_conv_gru_split_sums(cuda, H, W):
    """The _sum entry points: convz + convr and convq over the hidden state's
    64 channels, with the part over the other 66 (feature, uv) computed by
    bvml_dsine_conv_f32 from the same split weights and passed as sum0, as
    the refiner runs them; against the float64 restatement of the whole
    130-channel convolutions, to the whole convolutions' bars."""
    import torch
    say(f"[gpu] conv gru split sums {H}x{W}")
    C, cin, ch = 64, 130, 64
    rng = np.random.default_rng(7 * H + W)
    hx = rng.standard_normal((cin, H, W)).astype(np.float32)
    h = hx[:C].copy()
    wz, wr, wq = (rng.uniform(-1, 1, (C, cin, 5, 5)).astype(np.float32) / np.sqrt(cin * 25)
                  for _ in range(3))
    bz, br, bq = (rng.uniform(-0.3, 0.3, C).astype(np.float32) for _ in range(3))
    dev = torch.device(cuda)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    wzr = np.concatenate([wz, wr])
    wzr_h = _dev(_lib.conv_pack_f32(wzr[:, :ch], interleave=True), dev)
    wzr_f = _dev(_lib.conv_pack_f32(wzr[:, ch:], interleave=True), dev)
    wq_h = _dev(_lib.conv_pack_f32(wq[:, :ch]), dev)
    wq_f = _dev(_lib.conv_pack_f32(wq[:, ch:]), dev)
    hxd, hd = _dev(hx, dev), _dev(h, dev)
    bzd, brd, bqd = _dev(bz, dev), _dev(br, dev), _dev(bq, dev)
    s_zr = torch.empty(2 * C * H * W, device=dev)
    s_q = torch.empty(C * H * W, device=dev)
    xf = hxd[ch:]
    assert lib.bvml_dsine_conv_f32(xf.data_ptr(), cin - ch, H, W, wzr_f.data_ptr(), 2 * C, 5,
                                   s_zr.data_ptr(), stream) == _lib.OK, _lib.last_error()
    assert lib.bvml_dsine_conv_f32(xf.data_ptr(), cin - ch, H, W, wq_f.data_ptr(), C, 5,
                                   s_q.data_ptr(), stream) == _lib.OK, _lib.last_error()
    z = Guarded(C * H * W, dev)
    rh = Guarded(C * H * W, dev, shift=3)
    st = lib.bvml_dsine_conv_gru_gates_sum_f32(hxd.data_ptr(), ch, H, W, wzr_h.data_ptr(), C,
                                               s_zr.data_ptr(), bzd.data_ptr(), brd.data_ptr(),
                                               hd.data_ptr(), z.out.data_ptr(), rh.out.data_ptr(),
                                               stream)
    assert st == _lib.OK, _lib.last_error()
    hn = Guarded(C * H * W, dev, shift=2)
    st = lib.bvml_dsine_conv_gru_update_sum_f32(rh.out.data_ptr(), ch, H, W, wq_h.data_ptr(), C,
                                                s_q.data_ptr(), bqd.data_ptr(), z.out.data_ptr(),
                                                hd.data_ptr(), hn.out.data_ptr(), None, stream)
    assert st == _lib.OK, _lib.last_error()
    torch.cuda.synchronize()
    assert z.intact() and rh.intact() and hn.intact()
    sz, ez = conv64(hx, wz)
    sr, er = conv64(hx, wr)
    gz = z.out.cpu().numpy().reshape(C, H, W)
    grh = rh.out.cpu().numpy().reshape(C, H, W)
    want_z = _sig(sz + bz[:, None, None])
    want_rh = _sig(sr + br[:, None, None]) * h
    say(f"    gates: z max-abs {np.abs(gz - want_z).max():.3e}, rh max-abs "
        f"{np.abs(grh - want_rh).max():.3e}")
    assert (np.abs(gz - want_z) <= ez / 4 + 8 * U).all()
    assert (np.abs(grh - want_rh) <= np.abs(h) * (er / 4 + 8 * U)).all()
    rhx_h = np.concatenate([grh, hx[C:]])
    sq, eq = conv64(rhx_h, wq)
    q = np.tanh(sq + bq[:, None, None])
    want_h = (1 - gz.astype(np.float64)) * h + gz * q
    ghn = hn.out.cpu().numpy().reshape(C, H, W)
    say(f"    update: max-abs {np.abs(ghn - want_h).max():.3e}")
    assert (np.abs(ghn - want_h) <= np.abs(gz) * eq + 16 * U * (np.abs(h) + np.abs(q))).all()
    # sum0 must not overlap an output
    assert lib.bvml_dsine_conv_gru_gates_sum_f32(hxd.data_ptr(), ch, H, W, wzr_h.data_ptr(), C,
                                                 z.out.data_ptr(), bzd.data_ptr(),
                                                 brd.data_ptr(), hd.data_ptr(), z.out.data_ptr(),
                                                 rh.out.data_ptr(), stream) == _lib.EALIAS


def test_conv_rejects(cuda):
    import torch
    lib = _lib.load()
    x = torch.zeros(130 * 16, device=cuda)
    p = x.data_ptr()
    assert lib.bvml_dsine_conv_f32(p, 130, 4, 4, p, 64, 4, p, None) == _lib.EK
    assert lib.bvml_dsine_conv_f32(p, 130, 4, 4, p, 64, 5, p, None) == _lib.EALIAS
    assert lib.bvml_dsine_conv_f32(0, 130, 4, 4, p, 64, 5, p, None) == _lib.ENULL
    assert lib.bvml_dsine_conv_gru_update_f32(p, 130, 4, 4, p, 48, p, p, p, p, None, None) == \
        _lib.ESHAPE
    # h_new partly over h (one plane on): another lane's write would race this
    # lane's read, so it is refused before any launch (h_new == h is allowed)
    xs = torch.zeros(130 * 16, device=cuda)
    zs = torch.zeros(64 * 16, device=cuda)
    hs = torch.zeros(65 * 16, device=cuda)
    bq = torch.zeros(64, device=cuda)
    assert lib.bvml_dsine_conv_gru_update_f32(
        xs.data_ptr(), 130, 4, 4, p, 64, bq.data_ptr(), zs.data_ptr(), hs.data_ptr(),
        hs.data_ptr() + 16 * 4, None, None) == _lib.EALIAS
    assert lib.bvml_dsine_conv_packed_size(64, 130, 5) == 33 * 25 * 4 * 64
    assert lib.bvml_dsine_conv_packed_size(192, 66, 3) == 17 * 9 * 12 * 64
