/*
 * CPU parity oracle for the DSINE AngMF propagate and RayReLU ops, and for the
 * convex upsample + channel L2-normalise the refiner applies after each
 * propagate (src/dsine_refine.cpp:276-282).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this file; only the tests, the smoke check and the CPU-baseline leg of
 * the benchmark use it, and only to check results or as the timed CPU
 * reference.
 *
 * It restates brovisionml's CPU twin (src/dsine_ops.cpp, the reference CPU
 * path) operation for operation in double precision:
 *   - same operation order, so that a build with -ffp-contract=off reproduces
 *     the reference's double arithmetic bit for bit (libm sin/cos/sqrt);
 *   - std::max semantics ((a < b) ? b : a, which returns `a` when it is NaN);
 *   - kRayEps is the float 1e-2f widened to double (src/dsine_ops.cpp:27),
 *     not the CUDA twin's double 1e-2 (src/dsine_ops.cu:23).
 * It generalises the reference in three ways that reduce to it exactly at
 * B = 1, k = 5, full row range:
 *   - an odd window size k (pad P = (k-1)/2, slot n = ky*k + kx, xy planes
 *     [xs(k*k), ys(k*k)]) -- the reference hardcodes kPs = 5 (:24-26);
 *   - a batch B of NCHW samples with a ray batch stride (0 = one shared ray);
 *   - a row range [y0, y1) so that tests can check bands of a large image.
 *
 * Parity pins (tests/test_oracle_pins.py, tests/test_oracle_upsample.py):
 * every function here is checked
 * against closed forms, library routines (scipy Rotation, torch F.unfold /
 * F.normalize / F.cosine_similarity in float64) and brute force; the
 * reference source itself cannot be compiled in this image (it needs the
 * absent brotensor/tensor.h), so no compiled-reference vectors exist.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

/* ORACLE_MUTATION (default 0) plants one deliberate mistake for the
 * mutation test (tests/test_oracle_pins.py), which checks that the pins
 * catch it; the oracle used everywhere else is built with 0. */
#ifndef ORACLE_MUTATION
#define ORACLE_MUTATION 0
#endif

/* src/dsine_ops.cpp:27 -- constexpr float kRayEps = 1e-2f, used in double
 * expressions, so the effective constant is (double)1e-2f. */
#if ORACLE_MUTATION == 5
static const double kRayEpsF = 1e-2; /* mutation: the CUDA twin's double eps */
#else
static const float kRayEpsF = 1e-2f;
#endif

/* std::max(a, b) == (a < b) ? b : a */
static inline double smax(double a, double b) { return (a < b) ? b : a; }
static inline int imin(int a, int b) { return (b < a) ? b : a; }
static inline int imax(int a, int b) { return (a < b) ? b : a; }

/* axis_angle_to_matrix -- src/dsine_ops.cpp:31-51 (PyTorch3D quaternion form,
 * Taylor branch below 1e-6).  Row-major R. */
void oracle_axis_angle_to_matrix(double ax, double ay, double az, double R[9])
{
    const double angle = sqrt(ax * ax + ay * ay + az * az);
    const double half = angle * 0.5;
    double s;
    if (angle < 1e-6)
        s = 0.5 - (angle * angle) / 48.0;
    else
        s = sin(half) / angle;
    const double r = cos(half);
    const double i = ax * s, j = ay * s, k = az * s;
    const double two_s = 2.0 / (r * r + i * i + j * j + k * k);
    R[0] = 1.0 - two_s * (j * j + k * k);
#if ORACLE_MUTATION == 1 /* mutation: transposed R */
    R[3] = two_s * (i * j - k * r);
    R[2] = two_s * (i * k + j * r);
    R[1] = two_s * (i * j + k * r);
#else
    R[1] = two_s * (i * j - k * r);
    R[2] = two_s * (i * k + j * r);
    R[3] = two_s * (i * j + k * r);
#endif
    R[4] = 1.0 - two_s * (i * i + k * k);
    R[5] = two_s * (j * k - i * r);
    R[6] = two_s * (i * k - j * r);
    R[7] = two_s * (j * k + i * r);
    R[8] = 1.0 - two_s * (i * i + j * j);
}

/* Per-neighbour rotation axis -- src/dsine_ops.cpp:110-138.  Inputs are the
 * neighbour normal (nx,ny,nz), its pixel centre (pix_x,pix_y) and the raw xy
 * pair.  Writes the unit axis (or 0 for the identity fallback) to ax[3]. */
void oracle_axis(double nx, double ny, double nz, double pix_x, double pix_y,
                 double xs, double ys, double fu, double cu, double fv,
                 double cv, double ax[3])
{
    const double xyinv = 1.0 / smax(sqrt(xs * xs + ys * ys), 1e-12);
    xs *= xyinv;
    ys *= xyinv;
    const double du_over_fu = xs / fu;
    const double dv_over_fv = ys / fv;
    const double term_u = (pix_x + xs - cu) / fu;
    const double term_v = (pix_y + ys - cv) / fv;
#if ORACLE_MUTATION == 2 /* mutation: sign of num */
    const double num = (du_over_fu * nx + dv_over_fv * ny);
#else
    const double num = -(du_over_fu * nx + dv_over_fv * ny);
#endif
    double dd = term_u * nx + term_v * ny + nz;
    if (fabs(dd) < 1e-8) {
#if ORACLE_MUTATION == 6 /* mutation: sgn(0) = +1 */
        const double sgn = (dd >= 0.0) ? 1.0 : -1.0;
#else
        const double sgn = (dd > 0.0) ? 1.0 : (dd < 0.0 ? -1.0 : 0.0);
#endif
        dd = 1e-8 * sgn;
    }
    const double dz = num / dd;
    double axx = du_over_fu + dz * term_u;
    double axy = dv_over_fv + dz * term_v;
    double axz = dz;
    const double an = sqrt(axx * axx + axy * axy + axz * axz);
    const double ainv = 1.0 / smax(an, 1e-12);
    axx *= ainv; axy *= ainv; axz *= ainv;
    if (!isfinite(axx) || !isfinite(axy) || !isfinite(axz))
        axx = axy = axz = 0.0;
    ax[0] = axx; ax[1] = axy; ax[2] = axz;
}

/* RayReLU of one vector against one ray, in double -- the arithmetic of
 * src/dsine_ops.cpp:62-74 (standalone op) and :150-160 (fused copy, where the
 * input is the renormalised rotated neighbour).  Writes normalize(n + diff)
 * and, when pinv != NULL, the normalise's factor 1/max(|n + diff|, 1e-12). */
static void ray_relu_core(double nx, double ny, double nz, double rx, double ry,
                          double rz, double out[3], double *pinv)
{
    const double nn = sqrt(nx * nx + ny * ny + nz * nz);
    const double rr = sqrt(rx * rx + ry * ry + rz * rz);
    const double denom = smax(nn * rr, 1e-8);
    const double cs = (nx * rx + ny * ry + nz * rz) / denom;
    const double relu_cm = smax(cs - kRayEpsF, 0.0) + kRayEpsF;
    const double dcoef = relu_cm - cs;
    const double mx = nx + rx * dcoef;
    const double my = ny + ry * dcoef;
    const double mz = nz + rz * dcoef;
    const double inv = 1.0 / smax(sqrt(mx * mx + my * my + mz * mz), 1e-12);
    out[0] = mx * inv; out[1] = my * inv; out[2] = mz * inv;
    if (pinv) *pinv = inv;
}

void oracle_ray_relu_vec(double nx, double ny, double nz, double rx, double ry,
                         double rz, double out[3])
{
    ray_relu_core(nx, ny, nz, rx, ry, rz, out, (double *)0);
}

/* One neighbour's contribution before the prob weight: rotate the neighbour
 * normal about its axis by theta, renormalise, RayReLU against the output
 * pixel's ray -- src/dsine_ops.cpp:110-160. */
static void neighbour_core(double nx, double ny, double nz, double pix_x,
                           double pix_y, double xs, double ys, double theta,
                           double rx, double ry, double rz, double fu, double cu,
                           double fv, double cv, double out[3], double *pinv)
{
    double ax[3], R[9];
    oracle_axis(nx, ny, nz, pix_x, pix_y, xs, ys, fu, cu, fv, cv, ax);
    oracle_axis_angle_to_matrix(ax[0] * theta, ax[1] * theta, ax[2] * theta, R);
    double rnx = R[0] * nx + R[1] * ny + R[2] * nz;
    double rny = R[3] * nx + R[4] * ny + R[5] * nz;
    double rnz = R[6] * nx + R[7] * ny + R[8] * nz;
#if ORACLE_MUTATION == 7 /* mutation: no renormalise after rotating */
    const double rinv = 1.0;
#else
    const double rinv =
        1.0 / smax(sqrt(rnx * rnx + rny * rny + rnz * rnz), 1e-12);
#endif
    rnx *= rinv; rny *= rinv; rnz *= rinv;
    ray_relu_core(rnx, rny, rnz, rx, ry, rz, out, pinv);
}

void oracle_neighbour(double nx, double ny, double nz, double pix_x,
                      double pix_y, double xs, double ys, double theta,
                      double rx, double ry, double rz, double fu, double cu,
                      double fv, double cv, double out[3])
{
    neighbour_core(nx, ny, nz, pix_x, pix_y, xs, ys, theta, rx, ry, rz, fu, cu,
                   fv, cv, out, (double *)0);
}

/* ray_relu_cpu -- src/dsine_ops.cpp:55-76, batched: sample b uses
 * normal + b*3*HW and ray + b*ray_bstride. */
void oracle_ray_relu_f32(float *normal, const float *ray, int B, int H, int W,
                         long long ray_bstride)
{
    const size_t HW = (size_t)H * (size_t)W;
    for (int b = 0; b < B; ++b) {
        float *n = normal + (size_t)b * 3 * HW;
        const float *r = ray + (size_t)b * (size_t)ray_bstride;
        for (size_t p = 0; p < HW; ++p) {
            double o[3];
            oracle_ray_relu_vec(n[p], n[HW + p], n[2 * HW + p], r[p],
                                r[HW + p], r[2 * HW + p], o);
            n[p] = (float)o[0];
            n[HW + p] = (float)o[1];
            n[2 * HW + p] = (float)o[2];
        }
    }
}

/* One output pixel of angmf_propagate_cpu -- src/dsine_ops.cpp:91-170 for a
 * general odd k.  Also returns the double accumulator when acc != NULL, and
 * when qs != NULL the sum over neighbours of (prob / |p|)^2, p a neighbour's
 * RayReLU'd vector before its normalise (the scale of the sum's rounding
 * error in an fp32 evaluation, for the fast kernel's error budget). */
static void angmf_pixel(const float *pn, const float *pr, const float *xyp,
                        const float *ap, const float *rp, double fu, double cu,
                        double fv, double cv, int H, int W, int k, int y, int x,
                        float *op, double *acc_out, double *qs_out)
{
    const size_t HW = (size_t)H * (size_t)W;
    const int P = (k - 1) / 2, K2 = k * k;
    const size_t p = (size_t)y * W + x;
    const double rx = rp[p], ry = rp[HW + p], rz = rp[2 * HW + p];
    double acc0 = 0.0, acc1 = 0.0, acc2 = 0.0, qs = 0.0;
    for (int n = 0; n < K2; ++n) {
#if ORACLE_MUTATION == 4 /* mutation: column-major slots */
        const int kx = n / k, ky = n % k;
#else
        const int ky = n / k, kx = n % k;
#endif
        const int sy = imin(imax(y - P + ky, 0), H - 1); /* replicate */
        const int sx = imin(imax(x - P + kx, 0), W - 1);
        const size_t sp = (size_t)sy * W + sx;
        const double nx = pn[sp], ny = pn[HW + sp], nz = pn[2 * HW + sp];
#if ORACLE_MUTATION == 3 /* mutation: unclamped pixel centre */
        const double pix_x = (x - P + kx) + 0.5, pix_y = (y - P + ky) + 0.5;
#else
        const double pix_x = sx + 0.5, pix_y = sy + 0.5;
#endif
        const double xs = xyp[(size_t)n * HW + p];
        const double ys = xyp[(size_t)(K2 + n) * HW + p];
        const double theta = ap[(size_t)n * HW + p];
        const double w = pr[(size_t)n * HW + p];
        double m[3], pinv;
        neighbour_core(nx, ny, nz, pix_x, pix_y, xs, ys, theta, rx, ry, rz,
                       fu, cu, fv, cv, m, &pinv);
        acc0 += w * m[0]; acc1 += w * m[1]; acc2 += w * m[2];
        qs += (w * pinv) * (w * pinv);
    }
    const double inv =
        1.0 / smax(sqrt(acc0 * acc0 + acc1 * acc1 + acc2 * acc2), 1e-12);
    op[p] = (float)(acc0 * inv);
    op[HW + p] = (float)(acc1 * inv);
    op[2 * HW + p] = (float)(acc2 * inv);
    if (acc_out) {
        acc_out[p] = acc0;
        acc_out[HW + p] = acc1;
        acc_out[2 * HW + p] = acc2;
    }
    if (qs_out) qs_out[p] = qs;
}

/* angmf_propagate_cpu -- src/dsine_ops.cpp:78-172, batched and restricted to
 * output rows [y0, y1) of every sample (rows outside stay untouched).
 * Sample b reads pred_norm + b*3HW, prob + b*K2*HW, xy + b*2*K2*HW,
 * angle + b*K2*HW, ray + b*ray_bstride and writes out + b*3HW.
 * acc (nullable, 3HW per sample) receives the pre-normalisation sum, qs
 * (nullable, HW per sample) the sum of (prob/|p|)^2 (see angmf_pixel).
 * nthreads > 1 splits rows over OpenMP threads (same per-pixel arithmetic). */
void oracle_angmf_propagate_rows_f32(const float *pred_norm, const float *prob,
                                     const float *xy, const float *angle,
                                     const float *ray, double fu, double cu,
                                     double fv, double cv, int B, int H, int W,
                                     int k, long long ray_bstride, float *out,
                                     double *acc, double *qs, int y0, int y1,
                                     int nthreads)
{
    const size_t HW = (size_t)H * (size_t)W;
    const size_t K2 = (size_t)k * (size_t)k;
    if (y0 < 0) y0 = 0;
    if (y1 > H) y1 = H;
    for (int b = 0; b < B; ++b) {
        const float *pn = pred_norm + (size_t)b * 3 * HW;
        const float *pr = prob + (size_t)b * K2 * HW;
        const float *xyp = xy + (size_t)b * 2 * K2 * HW;
        const float *ap = angle + (size_t)b * K2 * HW;
        const float *rp = ray + (size_t)b * (size_t)ray_bstride;
        float *op = out + (size_t)b * 3 * HW;
        double *ac = acc ? acc + (size_t)b * 3 * HW : (double *)0;
        double *qq = qs ? qs + (size_t)b * HW : (double *)0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads) if (nthreads > 1)
        for (int y = y0; y < y1; ++y)
            for (int x = 0; x < W; ++x)
                angmf_pixel(pn, pr, xyp, ap, rp, fu, cu, fv, cv, H, W, k, y, x,
                            op, ac, qq);
    }
}

/* Whole-image convenience wrapper (all rows, one thread). */
void oracle_angmf_propagate_f32(const float *pred_norm, const float *prob,
                                const float *xy, const float *angle,
                                const float *ray, double fu, double cu,
                                double fv, double cv, int B, int H, int W,
                                int k, long long ray_bstride, float *out)
{
    oracle_angmf_propagate_rows_f32(pred_norm, prob, xy, angle, ray, fu, cu,
                                    fv, cv, B, H, W, k, ray_bstride, out,
                                    (double *)0, (double *)0, 0, H, 1);
}

/* ---------------------------------------------------------------------------
 * Convex upsample by s with a 9-tap softmax mask, then (normalize != 0) the
 * channel L2-normalise -- the two calls the refiner makes after each
 * propagate (src/dsine_refine.cpp:276-282: brotensor convex_upsample_forward
 * and l2_normalize_nchw_forward with eps 1e-12), whose arithmetic the
 * reference specifies in include/brovisionml/dsine_refine.h:91-97 (DSINE's
 * upsample_via_mask with replicate padding, then F.normalize):
 *   mask (B, 9*s*s, H, W) viewed as (9, s, s, H, W): channel n*s*s + ky*s + kx
 *   w_n = softmax over n of mask[n, ky, kx, y, x]   (exp(m - max) / sum)
 *   v_c = sum_n w_n * x[c, clamp(y - 1 + n/3), clamp(x - 1 + n%3)]
 *   out[c, s*y + ky, s*x + kx] = v_c / max(|v|, eps)  (or v_c unnormalised)
 * in double, rounded to float once.  A NaN anywhere in a softmax makes its
 * sub-pixel NaN, as torch.softmax does.
 * -------------------------------------------------------------------------*/
static void upsample_subpixel(const float *x, const float *mask, int C, int H, int W, int s,
                              int y, int xx, int ky, int kx, int normalize, double eps,
                              float *out)
{
    const size_t HW = (size_t)H * (size_t)W;
    const size_t p = (size_t)y * W + xx;
    const int s2 = s * s;
    double m[9];
    int nan = 0;
    for (int n = 0; n < 9; ++n) {
#if ORACLE_MUTATION == 8 /* mutation: ky and kx swapped in the mask channel */
        m[n] = mask[((size_t)n * s2 + (size_t)kx * s + ky) * HW + p];
#else
        m[n] = mask[((size_t)n * s2 + (size_t)ky * s + kx) * HW + p];
#endif
        nan |= isnan(m[n]);
    }
    double mx = m[0];
    for (int n = 1; n < 9; ++n)
        if (m[n] > mx) mx = m[n];
    double e[9], sum = 0.0;
    for (int n = 0; n < 9; ++n) {
        e[n] = nan ? NAN : exp(m[n] - mx);
        sum += e[n];
    }
    double v[16];
    for (int c = 0; c < C; ++c) v[c] = 0.0;
    for (int n = 0; n < 9; ++n) {
#if ORACLE_MUTATION == 10 /* mutation: column-major taps */
        const int dy = n % 3 - 1, dx = n / 3 - 1;
#else
        const int dy = n / 3 - 1, dx = n % 3 - 1;
#endif
        const int sy = y + dy, sx = xx + dx;
#if ORACLE_MUTATION == 9 /* mutation: zero padding instead of replicate */
        const int inside = sy >= 0 && sy < H && sx >= 0 && sx < W;
        const size_t sp = inside ? (size_t)sy * W + sx : 0;
#else
        const int inside = 1;
        const size_t sp = (size_t)imin(imax(sy, 0), H - 1) * W + imin(imax(sx, 0), W - 1);
#endif
        const double w = e[n] / sum;
        for (int c = 0; c < C; ++c) v[c] += inside ? w * x[(size_t)c * HW + sp] : 0.0;
    }
    double inv = 1.0;
    if (normalize) {
        double n2 = 0.0;
        for (int c = 0; c < C; ++c) n2 += v[c] * v[c];
#if ORACLE_MUTATION == 11 /* mutation: eps inside the square root */
        inv = 1.0 / sqrt(n2 + eps);
#else
        inv = 1.0 / smax(sqrt(n2), eps);
#endif
    }
    const size_t Ws = (size_t)W * s, HWs = HW * (size_t)s2;
    const size_t q = ((size_t)y * s + ky) * Ws + (size_t)xx * s + kx;
    for (int c = 0; c < C; ++c) out[(size_t)c * HWs + q] = (float)(v[c] * inv);
}

/* x: B x C x H x W; mask: B x 9s^2 x H x W; out: B x C x sH x sW; C <= 16. */
void oracle_convex_upsample_f32(const float *x, const float *mask, int B, int C, int H, int W,
                                int s, int normalize, double eps, float *out, int nthreads)
{
    const size_t HW = (size_t)H * (size_t)W;
    for (int b = 0; b < B; ++b) {
        const float *xb = x + (size_t)b * C * HW;
        const float *mb = mask + (size_t)b * 9 * s * s * HW;
        float *ob = out + (size_t)b * C * HW * s * s;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads) if (nthreads > 1)
        for (int y = 0; y < H; ++y)
            for (int xx = 0; xx < W; ++xx)
                for (int ky = 0; ky < s; ++ky)
                    for (int kx = 0; kx < s; ++kx)
                        upsample_subpixel(xb, mb, C, H, W, s, y, xx, ky, kx, normalize, eps, ob);
    }
}
