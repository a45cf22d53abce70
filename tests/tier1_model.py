"""A numpy model of the fast kernel's tier-1 arithmetic (the fp32 neighbour
terms of brovisionml_amd/csrc/dsine_ops.hip, angmf_f32_kernel), used by
test_tier1_budget.py to check the error budget its recompute threshold
assumes.  Test infrastructure: nothing in the library imports it.

Every fp32 operation is rounded as the kernel rounds it (a fused multiply-add
as one rounding: the exact double product of two floats plus the third,
rounded once -- double rounding through float64 aside); the hardware rsq is
modelled as the exact value times (1 +- 9.4e-8), its largest relative error
measured on gfx950, with a random sign; the sin/cos polynomials are the
kernel's."""
from __future__ import annotations

import numpy as np

f32, f64 = np.float32, np.float64
RSQ_REL = 9.4e-8
EPS = f32(1e-2)


def fma(a, b, c):
    return (np.asarray(a, f32).astype(f64) * np.asarray(b, f32).astype(f64)
            + np.asarray(c, f32).astype(f64)).astype(f32)


def rsq(x, rng):
    y = 1.0 / np.sqrt(np.asarray(x, f32).astype(f64))
    return (y * (1.0 + rng.choice([-RSQ_REL, RSQ_REL], size=y.shape))).astype(f32)


def sincos(t):
    """sincos_small: half-angle polynomials, then the double-angle forms."""
    t = np.asarray(t, f32)
    h = f32(0.5) * t
    u = h * h
    p = fma(u, f32(2.630318e-06), f32(-0.00019821344))
    p = fma(u, p, f32(0.008333231))
    p = fma(u, p, f32(-0.16666666))
    s = fma(h * u, p, h)
    q = fma(u, f32(-2.625131e-07), f32(2.4772546e-05))
    q = fma(u, q, f32(-0.0013888624))
    q = fma(u, q, f32(0.041666657))
    q = fma(u, q, f32(-0.5))
    c = fma(u, q, f32(1.0))
    sc = s * c
    return sc + sc, fma(c, c, -(s * s))


K_PI = f32(3.14159265358979323846)
L2E = f32(1.44269502)


def exp2(x, rng):
    """The hardware exp2 (v_exp_f32), at its measured relative error bound."""
    y = np.exp2(np.asarray(x, f32).astype(f64))
    with np.errstate(over="ignore"):
        return (y * (1.0 + rng.choice([-8.5e-8, 8.5e-8], size=y.shape))).astype(f32)


def rcp(x, rng):
    y = 1.0 / np.asarray(x, f32).astype(f64)
    return (y * (1.0 + rng.choice([-RSQ_REL, RSQ_REL], size=y.shape))).astype(f32)


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


def tier1(pred_norm, prob, xy, angle, ray, intr, H, W, k, rng, logits=False):
    """One sample: (B=1) planes as the op takes them (with logits, prob and
    angle hold the heads' raw logits and the kernel applies sigmoid and
    sigmoid * pi itself).  Returns the pixel
    outputs (3, HW) float64 (normalised in double, as phase B does), |acc|^2
    and sum(wi^2) per pixel.  Runs of the window split as the kernel splits
    them (k = 5: 7, 6, 6, 6), each run's sums in fp32."""
    fu, cu, fv, cv = intr
    HW, K2, P = H * W, k * k, k // 2
    pn = np.asarray(pred_norm, f32).reshape(3, H, W)
    ray = np.asarray(ray, f32).reshape(3, HW)
    ifu, ifv = 1.0 / fu, 1.0 / fv
    yy, xx = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
    rx, ry, rz = ray
    r2 = fma(rx, rx, fma(ry, ry, rz * rz))
    ir = np.where(r2 < f32(1e-16), f32(1e8), rsq(r2, rng))
    rhx, rhy, rhz = rx * ir, ry * ir, rz * ir
    G = 4 if k in (5, 7) else (2 if k == 3 else (1 if k == 1 else 8))
    run, rem = divmod(K2, G)
    bounds, n0 = [], 0
    for g in range(G):
        n1 = n0 + run + (1 if g < rem else 0)
        bounds.append((n0, n1))
        n0 = n1
    acc = np.zeros((3, HW))
    qs = np.zeros(HW)
    for a, b in bounds:
        pa = np.zeros((3, HW), f32)
        pq = np.zeros(HW, f32)
        for n in range(a, b):
            ky, kx = divmod(n, k)
            sy = np.clip(yy - P + ky, 0, H - 1).ravel()
            sx = np.clip(xx - P + kx, 0, W - 1).ravel()
            mx, my, mz = pn[:, sy, sx]
            tu0 = sx * ifu + (0.5 - cu) / fu
            tv0 = sy * ifv + (0.5 - cv) / fv
            m2 = fma(mx, mx, fma(my, my, mz * mz))
            im = fma(f32(-0.5), m2, f32(1.5))
            mpx, mpy, mpz = mx * im, my * im, mz * im
            g = tu0 * mx.astype(f64) + tv0 * my.astype(f64) + mz.astype(f64)
            gf = g.astype(f32)
            gu, gv = (g * ifu).astype(f32), (g * ifv).astype(f32)
            xs = np.asarray(xy[n], f32)
            ys = np.asarray(xy[K2 + n], f32)
            t = np.asarray(angle[n], f32)
            w = np.asarray(prob[n], f32)
            if logits:
                t = sigmoid(t, rng) * K_PI
            q = (xs.astype(f64) * (mx.astype(f64) * ifu)
                 + ys.astype(f64) * (my.astype(f64) * ifv)).astype(f32)
            s = fma(xs, xs, ys * ys)
            dd = fma(q, rsq(s, rng), gf)
            Vx = fma(gu, xs, -(q * tu0.astype(f32)))
            Vy = fma(gv, ys, -(q * tv0.astype(f32)))
            n2 = fma(Vx, Vx, fma(Vy, Vy, q * q))
            st, ct = sincos(t)
            S = st * np.copysign(rsq(n2, rng), dd)
            cx = fma(Vy, mpz, q * mpy)
            cy = -fma(q, mpx, Vx * mpz)
            cz = fma(Vx, mpy, -(Vy * mpx))
            vx = fma(cx, S, mpx * ct)
            vy = fma(cy, S, mpy * ct)
            vz = fma(cz, S, mpz * ct)
            cs = fma(vx, rhx, fma(vy, rhy, vz * rhz))
            dc = np.maximum(EPS - cs, f32(0))
            px, py, pz = fma(rx, dc, vx), fma(ry, dc, vy), fma(rz, dc, vz)
            p2 = fma(px, px, fma(py, py, pz * pz))
            if logits:
                d = one_plus_exp_neg(w, rng)
                with np.errstate(over="ignore"):
                    wi = rsq(p2 * d * d, rng)
            else:
                wi = w * rsq(p2, rng)
            pa = np.stack([fma(px, wi, pa[0]), fma(py, wi, pa[1]), fma(pz, wi, pa[2])])
            pq = fma(wi, wi, pq)
        acc += pa.astype(f64)
        qs += pq.astype(f64)
    a2 = (acc ** 2).sum(axis=0)
    out = acc / np.sqrt(np.maximum(a2, 1e-300))
    return out, a2, qs
