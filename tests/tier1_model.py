"""A numpy model of the fast kernel's tier-1 arithmetic (the fp32 neighbour
terms of brovisionml_amd/csrc/dsine_ops.hip, angmf_f32_kernel), used by
test_tier1_budget.py to check the error budget its recompute threshold
assumes.  Test infrastructure: nothing in the library imports it.

Every fp32 operation is rounded as the kernel rounds it: a fused
multiply-add is one rounding of the exact product of two floats plus the
third (formed in float64, where the product of two floats is exact; the
second rounding to float32 can differ from a true fma only on exact ties of
the double, which do not matter to the statistics here).  The hardware
functions are modelled at the error bounds measured on gfx950 over every
float argument in their domains (tests/test_gpu_hw_bounds.py pins them): each
result is the exact value moved by the bound with a random sign, so the
model's errors are at least as large as the kernel's:
  v_rsq_f32  relative  RSQ_REL
  v_sin_f32, v_cos_f32 (argument in revolutions, |a| <= 0.51)  absolute  SIN_ABS
  v_exp_f32  relative  EXP2_REL
  v_rcp_f32  relative  RCP_REL
"""
from __future__ import annotations

import numpy as np

f32, f64 = np.float32, np.float64

RSQ_REL = 9.4e-8
SIN_ABS = 1.26e-7
EXP2_REL = 8.5e-8
RCP_REL = 9.2e-8

EPS = f32(1e-2)
K_PI = f32(3.14159265358979323846)
L2E = f32(1.44269502)
INV_2PI = f32(0.159154943091895335768883763)
TWO_PI_HI = f32(6.28318548202514648438)
TWO_PI_LO = f32(-1.74845553146951715e-07)


def fma(a, b, c):
    return (np.asarray(a, f32).astype(f64) * np.asarray(b, f32).astype(f64)
            + np.asarray(c, f32).astype(f64)).astype(f32)


def _bounded(y, bound, rng, relative=True):
    y = np.asarray(y, f64)
    s = rng.choice([-1.0, 1.0], size=y.shape)
    with np.errstate(over="ignore", invalid="ignore"):
        return (y * (1.0 + s * bound) if relative else y + s * bound).astype(f32)


def rsq(x, rng):
    with np.errstate(divide="ignore"):
        return _bounded(1.0 / np.sqrt(np.asarray(x, f32).astype(f64)), RSQ_REL, rng)


def rcp(x, rng):
    with np.errstate(divide="ignore"):
        return _bounded(1.0 / np.asarray(x, f32).astype(f64), RCP_REL, rng)


def exp2(x, rng):
    with np.errstate(over="ignore"):
        return _bounded(np.exp2(np.asarray(x, f32).astype(f64)), EXP2_REL, rng)


def sincos(t, rng):
    """sincos_hw: the hardware sine and cosine of a = t/(2 pi) rounded to
    float, then the first-order correction by e = t - 2 pi a."""
    t = np.asarray(t, f32)
    a = (t * INV_2PI).astype(f32)
    x = 2.0 * np.pi * a.astype(f64)
    s = _bounded(np.sin(x), SIN_ABS, rng, relative=False)
    c = _bounded(np.cos(x), SIN_ABS, rng, relative=False)
    e = fma(-a, TWO_PI_LO, fma(-a, TWO_PI_HI, t))
    return fma(e, c, s), fma(-e, s, c)


def one_plus_exp_neg(x, rng):
    """1 + exp(-x) from the hardware exp2 of the rounded -x log2(e)."""
    with np.errstate(over="ignore"):
        return f32(1.0) + exp2(-np.asarray(x, f32) * L2E, rng)


def sigmoid(x, rng):
    """sigmoid_f32: 1/(1 + exp(-x)) from the hardware rcp and one Newton
    step; 0 below x = -87."""
    x = np.asarray(x, f32)
    tiny = x < f32(-87.0)
    d = one_plus_exp_neg(np.where(tiny, f32(0.0), x), rng)
    r = rcp(d, rng)
    return np.where(tiny, f32(0.0), fma(r, fma(-d, r, f32(1.0)), r))


def runs(K2: int, G: int):
    """The kernel's split of the window into G runs of consecutive neighbours
    (lengths differ by at most one, the longer ones first)."""
    run, rem = divmod(K2, G)
    out, n0 = [], 0
    for g in range(G):
        n1 = n0 + run + (1 if g < rem else 0)
        out.append((n0, n1))
        n0 = n1
    return out


def kernel_waves(lib, d: dict) -> int:
    """The waves per 64-pixel group the kernel's launch plan takes for draw d
    (lib is brovisionml_amd._lib): the G of its run split, so the model sums
    the runs as that launch does."""
    fu, cu, fv, cv = d["intr"]
    flags = lib.LOGITS if d["logits"] else lib.DEFAULT
    return lib.angmf_plan(1, d["H"], d["W"], d["k"], fu, cu, fv, cv, flags)[1]


def dd_min(intr, H, W) -> float:
    """The fast kernel's |dd| floor for an H x W image (plan_angmf in
    brovisionml_amd/csrc/dsine_ops.hip): the reference's clamp plus dd's
    error bound, from the largest |P0| over the image's corners times the
    largest accepted |m|."""
    fu, cu, fv, cv = intr
    gmax = 0.0
    for cy in (0, H - 1):
        for cx in (0, W - 1):
            tu, tv = (cx + 0.5 - cu) / fu, (cy + 0.5 - cv) / fv
            gmax = max(gmax, np.sqrt(1.0 + tu * tu + tv * tv))
    gmax *= np.sqrt(1.0 + 1e-5)
    return 1.02e-8 + 1e-7 * gmax + 3e-7 / min(abs(fu), abs(fv))


def tier1(pred_norm, prob, xy, angle, ray, intr, H, W, k, rng, logits=False, G=4,
          q_double=True, flags=None):
    """One sample: planes as the op takes them (with logits, prob and angle
    hold the heads' raw logits and the kernel applies sigmoid and
    sigmoid * pi itself).  Returns the pixel outputs (3, HW) float64
    (normalised in double, as phase B does), |acc|^2 and sum(wi^2) per pixel.
    The window is split into G runs as the kernel splits it, each run's sums
    in fp32, the runs' partials summed in double.  q_double=False forms q in
    fp32 instead (a planted weakness the budget test must detect).  flags,
    when given (a bool array of HW), receives the pixels the kernel sends to
    the recompute for a neighbour outside the fp32 form's domain: |xy|^2
    outside [1e-20, 1e30], |t| > 3.2, |dd| < dd_min, |V x m'|^2 < 1e-30, or a
    non-finite value in any of them."""
    fu, cu, fv, cv = intr
    HW, K2, P = H * W, k * k, k // 2
    pn = np.asarray(pred_norm, f32).reshape(3, H, W)
    ray = np.asarray(ray, f32).reshape(3, HW)
    ifu, ifv = 1.0 / fu, 1.0 / fv
    yy, xx = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
    rx, ry, rz = ray
    # 1/|r| from rsq and one Newton step; -r-hat/2 and 2r
    r2 = fma(rx, rx, fma(ry, ry, rz * rz))
    ir0 = rsq(r2, rng)
    ir1 = fma(f32(0.5) * ir0, fma(-(r2 * ir0), ir0, f32(1.0)), ir0)
    ir = np.where(r2 < f32(1e-16), f32(1e8), ir1)
    nhx, nhy, nhz = (f32(-0.5) * (c * ir) for c in (rx, ry, rz))
    r2x, r2y, r2z = (f32(2.0) * c for c in (rx, ry, rz))
    ddf = f32(dd_min(intr, H, W))
    bad = np.zeros(HW, bool)
    acc = np.zeros((3, HW))
    qs = np.zeros(HW)
    for a, b in runs(K2, G):
        pa = np.zeros((3, HW), f32)
        pq = np.zeros(HW, f32)
        for n in range(a, b):
            ky, kx = divmod(n, k)
            sy = np.clip(yy - P + ky, 0, H - 1).ravel()
            sx = np.clip(xx - P + kx, 0, W - 1).ravel()
            mx, my, mz = pn[:, sy, sx]
            # the halo record (stage_halo)
            tu0 = sx * ifu + (0.5 - cu) / fu
            tv0 = sy * ifv + (0.5 - cv) / fv
            m2 = fma(mx, mx, fma(my, my, mz * mz))
            im = fma(f32(-0.5), m2, f32(1.5))
            mpx, mpy, mpz = mx * im, my * im, mz * im
            g = tu0 * mx.astype(f64) + tv0 * my.astype(f64) + mz.astype(f64)
            gf = g.astype(f32)
            gu, gv = (g * ifu).astype(f32), (g * ifv).astype(f32)
            tu, tv = tu0.astype(f32), tv0.astype(f32)
            e1y, e1z, e2x, e2z = -(gu * mpz), gu * mpy, gv * mpz, -(gv * mpx)
            fx, fy, fz = fma(tv, mpz, -mpy), fma(-tu, mpz, mpx), fma(tu, mpy, -(tv * mpx))
            # the neighbour
            xs = np.asarray(xy[n], f32)
            ys = np.asarray(xy[K2 + n], f32)
            t = np.asarray(angle[n], f32)
            w = np.asarray(prob[n], f32)
            if logits:
                t = sigmoid(t, rng) * K_PI
            if q_double:
                q = (xs.astype(f64) * (mx.astype(f64) * ifu)
                     + ys.astype(f64) * (my.astype(f64) * ifv)).astype(f32)
            else:
                q = fma(xs, (mx.astype(f64) * ifu).astype(f32),
                        ys * (my.astype(f64) * ifv).astype(f32))
            s = fma(xs, xs, ys * ys)
            dd = fma(q, rsq(s, rng), gf)
            cx = fma(ys, e2x, -(q * fx))
            cy = fma(xs, e1y, -(q * fy))
            cz = fma(xs, e1z, fma(ys, e2z, -(q * fz)))
            n2 = fma(cx, cx, fma(cy, cy, cz * cz))
            with np.errstate(invalid="ignore"):
                bad |= ~((s >= f32(1e-20)) & (s <= f32(1e30)) & (np.abs(t) <= f32(3.2))
                         & (np.abs(dd) >= ddf) & (n2 >= f32(1e-30)))
            st, ct = sincos(t, rng)
            S = st * np.copysign(rsq(n2, rng), dd)
            vx = fma(cx, S, mpx * ct)
            vy = fma(cy, S, mpy * ct)
            vz = fma(cz, S, mpz * ct)
            h = np.clip(fma(vz, nhz, fma(vy, nhy, fma(vx, nhx, f32(0.5) * EPS))), f32(0), f32(1))
            px, py, pz = fma(r2x, h, vx), fma(r2y, h, vy), fma(r2z, h, vz)
            p2 = fma(px, px, fma(py, py, pz * pz))
            if logits:
                d = one_plus_exp_neg(w, rng)
                with np.errstate(over="ignore", invalid="ignore"):
                    wi = rsq(p2 * d * d, rng)
            else:
                wi = w * rsq(p2, rng)
            pa = np.stack([fma(px, wi, pa[0]), fma(py, wi, pa[1]), fma(pz, wi, pa[2])])
            pq = fma(wi, wi, pq)
        acc += pa.astype(f64)
        qs += pq.astype(f64)
    a2 = (acc ** 2).sum(axis=0)
    out = acc / np.sqrt(np.maximum(a2, 1e-300))
    if flags is not None:
        flags[...] = bad
    return out, a2, qs
