// The CPU branch of the DSINE ops' public dispatch: brovisionml's dispatch
// routes CPU tensors to its CPU twin (src/dsine_ops.cpp:178-215 ->
// ray_relu_cpu :55-76, angmf_propagate_cpu :78-172); this library's C++
// dispatch and Python mirror route them here.  Double precision in the
// reference's operation order (angmf_ref.h, the same bodies the GPU's
// reference-order tier runs), so the results equal the reference CPU
// path's bit for bit; rows are split over host threads, which changes no
// result.  Extended like the device entry points: B samples, odd k, a ray
// batch stride, the ray formed from the intrinsics, logits.

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>
#include <string>
#include <thread>
#include <vector>

#include "angmf_ref.h"
#include "bvml_dsine.h"
#include "status.h"

namespace {

using bvml::fail;

// Runs body(y0, y1) over row bands [y0, y1) of [0, rows) on up to nthreads
// threads (0: the hardware's), at least 16 rows per thread.
template <class F>
void for_rows(int rows, int nthreads, F body) {
    int nt = nthreads > 0 ? nthreads : (int)std::thread::hardware_concurrency();
    nt = std::max(1, std::min(nt, rows / 16));
    if (nt == 1) {
        body(0, rows);
        return;
    }
    std::vector<std::thread> pool;
    pool.reserve(nt);
    for (int t = 0; t < nt; ++t) {
        const int y0 = (int)((long long)rows * t / nt), y1 = (int)((long long)rows * (t + 1) / nt);
        pool.emplace_back(body, y0, y1);
    }
    for (auto& th : pool) th.join();
}

int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

}  // namespace

extern "C" {

int bvml_dsine_ray_relu_cpu_f32(float* normal, const float* ray, int B, int H, int W,
                                long long ray_bstride, int nthreads) {
    if (B < 0 || H < 0 || W < 0) return fail(BVML_DSINE_ESHAPE, "ray_relu: B, H and W must be >= 0");
    if (ray_bstride < 0) return fail(BVML_DSINE_ESHAPE, "ray_relu: ray_bstride must be >= 0");
    const long long HW = (long long)H * W;
    if (B == 0 || HW == 0) return BVML_DSINE_OK;
    if (!normal || !ray) return fail(BVML_DSINE_ENULL, "ray_relu: normal and ray must be non-NULL");
    const size_t nbytes = (size_t)B * 3 * HW * sizeof(float);
    const size_t rbytes = ((size_t)(B - 1) * ray_bstride + 3 * HW) * sizeof(float);
    if (bvml::overlaps(normal, nbytes, ray, rbytes))
        return fail(BVML_DSINE_EALIAS, "ray_relu: normal and ray overlap");
    for (int b = 0; b < B; ++b) {
        float* n = normal + (size_t)b * 3 * HW;
        const float* r = ray + (size_t)b * ray_bstride;
        for_rows(H, nthreads, [&](int y0, int y1) {
            for (long long p = (long long)y0 * W; p < (long long)y1 * W; ++p) {
                double ox, oy, oz, inv;
                bvml::ray_relu_ref(n[p], n[HW + p], n[2 * HW + p], r[p], r[HW + p],
                                   r[2 * HW + p], ox, oy, oz, inv);
                n[p] = (float)ox;
                n[HW + p] = (float)oy;
                n[2 * HW + p] = (float)oz;
            }
        });
    }
    return BVML_DSINE_OK;
}

int bvml_dsine_angmf_propagate_cpu_f32(const float* pred_norm, const float* prob,
                                       const float* xy, const float* angle, const float* ray,
                                       double fu, double cu, double fv, double cv, int B, int H,
                                       int W, int k, long long ray_bstride, float* out,
                                       unsigned flags, int nthreads) {
BVML_NO_CONTRACT
    if (flags & ~(BVML_DSINE_FP64 | BVML_DSINE_RAY_FROM_INTRINSICS | BVML_DSINE_LOGITS))
        return fail(BVML_DSINE_EFLAGS, "angmf_propagate: unknown flag bits");
    const bool synth = (flags & BVML_DSINE_RAY_FROM_INTRINSICS) != 0;
    const bool logits = (flags & BVML_DSINE_LOGITS) != 0;
    if (synth) {
        ray = nullptr;
        ray_bstride = 0;
    }
    if (B < 0 || H < 0 || W < 0)
        return fail(BVML_DSINE_ESHAPE, "angmf_propagate: B, H and W must be >= 0");
    if (ray_bstride < 0) return fail(BVML_DSINE_ESHAPE, "angmf_propagate: ray_bstride must be >= 0");
    if (!(k == 1 || k == 3 || k == 5 || k == 7 || k == 9))
        return fail(BVML_DSINE_EK, "angmf_propagate: k must be one of 1, 3, 5, 7, 9");
    const long long HW = (long long)H * W;
    if (B == 0 || HW == 0) return BVML_DSINE_OK;
    if (!pred_norm || !prob || !xy || !angle || (!ray && !synth) || !out)
        return fail(BVML_DSINE_ENULL, "angmf_propagate: all tensors must be non-NULL");
    const long long K2 = (long long)k * k;
    const size_t f = sizeof(float);
    const size_t out_b = (size_t)B * 3 * HW * f;
    if (bvml::overlaps(out, out_b, pred_norm, (size_t)B * 3 * HW * f) ||
        bvml::overlaps(out, out_b, prob, (size_t)B * K2 * HW * f) ||
        bvml::overlaps(out, out_b, xy, (size_t)B * 2 * K2 * HW * f) ||
        bvml::overlaps(out, out_b, angle, (size_t)B * K2 * HW * f) ||
        (!synth && bvml::overlaps(out, out_b, ray, ((size_t)(B - 1) * ray_bstride + 3 * HW) * f)))
        return fail(BVML_DSINE_EALIAS, "angmf_propagate: out overlaps an input");
    const int P = k / 2;
    for (int b = 0; b < B; ++b) {
        const float* pn = pred_norm + (size_t)b * 3 * HW;
        const float* pr = prob + (size_t)b * K2 * HW;
        const float* xyp = xy + (size_t)b * 2 * K2 * HW;
        const float* ap = angle + (size_t)b * K2 * HW;
        const float* rp = synth ? nullptr : ray + (size_t)b * ray_bstride;
        float* op = out + (size_t)b * 3 * HW;
        for_rows(H, nthreads, [&](int y0, int y1) {
            for (int y = y0; y < y1; ++y)
                for (int x = 0; x < W; ++x) {
                    const size_t p = (size_t)y * W + x;
                    double rx, ry, rz;
                    if (synth) {
                        const bvml::Ray3f r = bvml::synth_ray(x, y, fu, cu, fv, cv);
                        rx = r.x;
                        ry = r.y;
                        rz = r.z;
                    } else {
                        rx = rp[p];
                        ry = rp[HW + p];
                        rz = rp[2 * HW + p];
                    }
                    double acc0 = 0.0, acc1 = 0.0, acc2 = 0.0;
                    for (int n = 0; n < K2; ++n) {
                        const int ky = n / k, kx = n % k;
                        const int sy = clampi(y - P + ky, 0, H - 1);
                        const int sx = clampi(x - P + kx, 0, W - 1);
                        const size_t sp = (size_t)sy * W + sx;
                        const float th = ap[(size_t)n * HW + p], wp = pr[(size_t)n * HW + p];
                        double mx, my, mz, pinv;
                        bvml::nbr_ref_f64(pn[sp], pn[HW + sp], pn[2 * HW + sp], sx + 0.5,
                                          sy + 0.5, xyp[(size_t)n * HW + p],
                                          xyp[(size_t)(K2 + n) * HW + p],
                                          logits ? bvml::angle_ref(th) : th, rx, ry, rz, fu, cu,
                                          fv, cv, mx, my, mz, pinv);
                        const double w = logits ? bvml::sigmoid_ref(wp) : wp;
                        acc0 += w * mx;
                        acc1 += w * my;
                        acc2 += w * mz;
                    }
                    const double inv =
                        1.0 / bvml::smax(std::sqrt(acc0 * acc0 + acc1 * acc1 + acc2 * acc2), 1e-12);
                    op[p] = (float)(acc0 * inv);
                    op[HW + p] = (float)(acc1 * inv);
                    op[2 * HW + p] = (float)(acc2 * inv);
                }
        });
    }
    return BVML_DSINE_OK;
}

}  // extern "C"
