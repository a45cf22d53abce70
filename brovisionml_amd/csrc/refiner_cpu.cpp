// The native refiner's host path (bvml_dsine_refiner_forward_cpu): brovisionml's
// Refiner::forward on brotensor's CPU device (src/dsine_refine.cpp:212-294,
// every step a CPU brotensor op there) on host threads, the same loop as the
// device path in refiner.cpp:
//   * the convolutions in fp32, zero padding, each output a float sum over
//     its taps (input channel outermost, then the kernel rows and columns),
//     then the bias added (src/dsine_refine.cpp:94-101);
//   * sigmoid 1 / (1 + e^-x) and tanh in float, ReLU, and the ConvGRU's
//     (1 - z) h + z q in the reference's rounding (:152-157);
//   * RayReLU and the propagate (on the heads' logits, BVML_DSINE_LOGITS)
//     from the kernel library's CPU branch: double precision in the
//     reference's operation order (src/dsine_ops.cpp:55-172);
//   * the ray and uv maps as build_ray8 / build_uv form them
//     (src/dsine_decoder.cpp:242-293);
//   * the convex upsample + normalise (:276-283; its arithmetic is the one
//     include/brovisionml/dsine_refine.h:91-97 specifies) in double,
//     rounded to float once: the mask plus its bias in float, the 9-tap
//     softmax, the weighted sum, then v / max(|v|, 1e-12).
// As on the device, the up-mask head and the upsample run in the last
// iteration only and the first four iterations' heads run for the three
// heads the propagate reads.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "angmf_ref.h"
#include "bvml_dsine.h"
#include "bvml_dsine_refine.h"
#include "refiner_common.h"

namespace {

using namespace bvml_refine;

// Runs body(i0, i1) over [0, n) split across up to nthreads threads (0: the
// hardware's), at least `grain` items per thread.
template <class F>
void parallel(long long n, int nthreads, long long grain, F body) {
    int nt = nthreads > 0 ? nthreads : (int)std::thread::hardware_concurrency();
    nt = (int)std::max(1LL, std::min<long long>(nt, n / std::max(1LL, grain)));
    if (nt == 1) {
        body(0LL, n);
        return;
    }
    std::vector<std::thread> pool;
    pool.reserve(nt);
    for (int t = 0; t < nt; ++t)
        pool.emplace_back(body, n * t / nt, n * (t + 1) / nt);
    for (auto& th : pool) th.join();
}

// y[co] = sum_{ci of co's group, ky, kx} w[co][ci][ky][kx] x[ci][y+ky-p][x+kx-p]
// (zero outside the map; p = k / 2), without bias.  One task per output row.
void conv2d(const float* x, int cin, int H, int W, const float* w, int cout, int k, int groups,
            float* y, int nthreads) {
    const int p = k / 2, cin_g = cin / groups, cout_g = cout / groups;
    const size_t hw = (size_t)H * W;
    parallel((long long)cout * H, nthreads, 8, [&](long long t0, long long t1) {
        std::vector<float> acc((size_t)W);
        for (long long t = t0; t < t1; ++t) {
            const int co = (int)(t / H), yo = (int)(t % H);
            const int g = co / cout_g;
            std::fill(acc.begin(), acc.end(), 0.0f);
            for (int cl = 0; cl < cin_g; ++cl) {
                const float* xc = x + (size_t)(g * cin_g + cl) * hw;
                const float* wc = w + ((size_t)co * cin_g + cl) * k * k;
                for (int ky = 0; ky < k; ++ky) {
                    const int yy = yo + ky - p;
                    if (yy < 0 || yy >= H) continue;
                    const float* row = xc + (size_t)yy * W;
                    for (int kx = 0; kx < k; ++kx) {
                        const float wv = wc[ky * k + kx];
                        const int lo = std::max(0, p - kx), hi = std::min(W, W + p - kx);
                        const float* src = row + (kx - p);
                        for (int xo = lo; xo < hi; ++xo) acc[xo] += wv * src[xo];
                    }
                }
            }
            std::memcpy(y + (size_t)co * hw + (size_t)yo * W, acc.data(), W * sizeof(float));
        }
    });
}

float sigmoidf(float v) { return 1.0f / (1.0f + std::exp(-v)); }

// x[c] = act(x[c] + b[c]) for C planes.
void bias_act(float* x, const float* b, int C, size_t hw, bool relu, int nthreads) {
    parallel(C, nthreads, 1, [&](long long c0, long long c1) {
        for (long long c = c0; c < c1; ++c) {
            float* xc = x + (size_t)c * hw;
            const float bc = b[c];
            for (size_t i = 0; i < hw; ++i) {
                const float v = xc[i] + bc;
                xc[i] = (relu && v < 0.0f) ? 0.0f : v;
            }
        }
    });
}

// The convex upsample by 8 with the mask's bias, then the L2 normalise.
void upsample8(const float* pred, const float* mask, const float* mbias, int H, int W,
               float* up, int nthreads) {
    const size_t hw = (size_t)H * W;
    const int S = kUp, FW = S * W;
    const size_t fhw = (size_t)S * H * FW;
    parallel(H, nthreads, 1, [&](long long y0, long long y1) {
        for (long long y = y0; y < y1; ++y) {
            for (int x = 0; x < W; ++x) {
                double tap[3][9];
                for (int n = 0; n < 9; ++n) {
                    const int yy = std::min(std::max((int)y + n / 3 - 1, 0), H - 1);
                    const int xx = std::min(std::max(x + n % 3 - 1, 0), W - 1);
                    for (int c = 0; c < 3; ++c) tap[c][n] = pred[c * hw + (size_t)yy * W + xx];
                }
                for (int ky = 0; ky < S; ++ky)
                    for (int kx = 0; kx < S; ++kx) {
                        double m[9], mx = -INFINITY;
                        bool nan = false;
                        for (int n = 0; n < 9; ++n) {
                            const int ch = (n * S + ky) * S + kx;
                            m[n] = (double)(mask[(size_t)ch * hw + (size_t)y * W + x] + mbias[ch]);
                            nan = nan || std::isnan(m[n]);
                            mx = std::max(mx, m[n]);
                        }
                        double e[9], s = 0.0;
                        for (int n = 0; n < 9; ++n) s += (e[n] = std::exp(m[n] - mx));
                        double v[3] = {0.0, 0.0, 0.0};
                        for (int n = 0; n < 9; ++n)
                            for (int c = 0; c < 3; ++c) v[c] += (e[n] / s) * tap[c][n];
                        const double nn = std::sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
                        const double inv = 1.0 / std::max(nn, (double)kUpEps);
                        const size_t o = (size_t)(S * y + ky) * FW + (size_t)S * x + kx;
                        for (int c = 0; c < 3; ++c)
                            up[c * fhw + o] = nan ? NAN : (float)(v[c] * inv);
                    }
            }
        }
    });
}

// The loop, after forward_cpu's checks; throws std::bad_alloc when host
// memory runs out.
int run_cpu(const std::vector<std::vector<float>>& wt, const float* normal, const float* feature,
            const float* hidden, int h8, int w8, float fx, float fy, float cx, float cy,
            int orig_h, int orig_w, int pad_t, int pad_l, int out_h, int out_w, float* out,
            float* coarse, int nthreads) {
    const int H = h8, W = w8;
    const size_t hw = (size_t)H * W;
    const double sw = (double)W / orig_w, sh = (double)H / orig_h;
    const double fu = fx * sw, cu = (cx + 0.5) * sw, fv = fy * sh, cv = (cy + 0.5) * sh;

    // [h | feature | uv], [r*h | feature | uv], [h_new | uv], as on the device
    std::vector<float> hx((size_t)kHx * hw), rhx((size_t)kHx * hw), hin((size_t)kHin * hw);
    std::vector<float> zr((size_t)2 * kHidden * hw), z((size_t)kHidden * hw);
    std::vector<float> qp((size_t)kHidden * hw), ray(3 * hw), pred(3 * hw), next(3 * hw);
    std::vector<float> t0((size_t)kHeads * kMid * hw), t1((size_t)kHeads * kMid * hw);
    std::vector<float> head[kHeads];
    for (int h = 0; h < kHeads; ++h) head[h].resize((size_t)kHeadOut[h] * hw);
    float* uv = hx.data() + (size_t)(kHidden + kFeature) * hw;
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x) {
            const size_t i = (size_t)y * W + x;
            uv[i] = (float)(((x + 0.5) - cu) / fu);
            uv[hw + i] = (float)(((y + 0.5) - cv) / fv);
            const bvml::Ray3f rr = bvml::synth_ray(x, y, fu, cu, fv, cv);
            ray[i] = rr.x;
            ray[hw + i] = rr.y;
            ray[2 * hw + i] = rr.z;
        }
    std::memcpy(hx.data(), hidden, (size_t)kHidden * hw * sizeof(float));
    std::memcpy(hx.data() + (size_t)kHidden * hw, feature, (size_t)kFeature * hw * sizeof(float));
    std::memcpy(rhx.data() + (size_t)kHidden * hw, hx.data() + (size_t)kHidden * hw,
                (size_t)kX * hw * sizeof(float));
    std::memcpy(hin.data() + (size_t)kHidden * hw, uv, 2 * hw * sizeof(float));
    std::memcpy(pred.data(), normal, 3 * hw * sizeof(float));
    if (bvml_dsine_ray_relu_cpu_f32(pred.data(), ray.data(), 1, H, W, 0, nthreads) != BVML_DSINE_OK)
        return fail(BVML_DSINE_EPARAM, std::string("forward_cpu: ray_relu: ") +
                                           bvml_dsine_last_error());

    // the checkpoint's convolutions, concatenated as the device path reads them
    std::vector<float> w_zr(wt[kZw]);
    w_zr.insert(w_zr.end(), wt[kRw].begin(), wt[kRw].end());
    std::vector<float> w_h0, b_h0, w_h2, b_h2;
    for (int h = 0; h < kHeads; ++h) {
        w_h0.insert(w_h0.end(), wt[head_w(h, 0)].begin(), wt[head_w(h, 0)].end());
        b_h0.insert(b_h0.end(), wt[head_b(h, 0)].begin(), wt[head_b(h, 0)].end());
        w_h2.insert(w_h2.end(), wt[head_w(h, 1)].begin(), wt[head_w(h, 1)].end());
        b_h2.insert(b_h2.end(), wt[head_b(h, 1)].begin(), wt[head_b(h, 1)].end());
    }
    const float *bz = wt[kZb].data(), *br = wt[kRb].data(), *bq = wt[kQb].data();

    std::vector<float> up;
    const long long fh = (long long)kUp * H, fw = (long long)kUp * W;
    const bool direct = pad_t == 0 && pad_l == 0 && out_h == fh && out_w == fw;
    for (int it = 0; it < kIter; ++it) {
        const bool last = it == kIter - 1;
        const int nh = last ? kHeads : kHeads - 1;
        // ConvGRU (src/dsine_refine.cpp:138-159)
        conv2d(hx.data(), kHx, H, W, w_zr.data(), 2 * kHidden, 5, 1, zr.data(), nthreads);
        parallel(kHidden, nthreads, 1, [&](long long c0, long long c1) {
            for (long long c = c0; c < c1; ++c)
                for (size_t i = c * hw; i < (size_t)(c + 1) * hw; ++i) {
                    z[i] = sigmoidf(zr[i] + bz[c]);
                    rhx[i] = sigmoidf(zr[(size_t)kHidden * hw + i] + br[c]) * hx[i];
                }
        });
        conv2d(rhx.data(), kHx, H, W, wt[kQw].data(), kHidden, 5, 1, qp.data(), nthreads);
        parallel(kHidden, nthreads, 1, [&](long long c0, long long c1) {
            for (long long c = c0; c < c1; ++c)
                for (size_t i = c * hw; i < (size_t)(c + 1) * hw; ++i) {
                    const float q = std::tanh(qp[i] + bq[c]);
                    const float omz = 1.0f - z[i];
                    const float a = omz * hx[i], b = z[i] * q;
                    hx[i] = hin[i] = a + b;
                }
        });
        // the heads (:119-127)
        conv2d(hin.data(), kHin, H, W, w_h0.data(), nh * kMid, 3, 1, t0.data(), nthreads);
        bias_act(t0.data(), b_h0.data(), nh * kMid, hw, true, nthreads);
        conv2d(t0.data(), nh * kMid, H, W, w_h2.data(), nh * kMid, 1, nh, t1.data(), nthreads);
        bias_act(t1.data(), b_h2.data(), nh * kMid, hw, true, nthreads);
        for (int h = 0; h < kHeads - 1; ++h) {
            conv2d(t1.data() + (size_t)h * kMid * hw, kMid, H, W, wt[head_w(h, 2)].data(),
                   kHeadOut[h], 1, 1, head[h].data(), nthreads);
            bias_act(head[h].data(), wt[head_b(h, 2)].data(), kHeadOut[h], hw, false, nthreads);
        }
        // the propagate on the logits (:262-274)
        if (bvml_dsine_angmf_propagate_cpu_f32(pred.data(), head[0].data(), head[1].data(),
                                               head[2].data(), ray.data(), fu, cu, fv, cv, 1, H,
                                               W, kPs, 0, next.data(), BVML_DSINE_LOGITS,
                                               nthreads) != BVML_DSINE_OK)
            return fail(BVML_DSINE_EPARAM, std::string("forward_cpu: angmf_propagate: ") +
                                               bvml_dsine_last_error());
        pred.swap(next);
        if (coarse) std::memcpy(coarse + (size_t)it * 3 * hw, pred.data(), 3 * hw * sizeof(float));
        if (!last) continue;
        // the up-sampled map (:276-283)
        conv2d(t1.data() + (size_t)3 * kMid * hw, kMid, H, W, wt[head_w(3, 2)].data(),
               kHeadOut[3], 1, 1, head[3].data(), nthreads);
        float* dst = out;
        if (!direct) {
            up.resize((size_t)3 * fh * fw);
            dst = up.data();
        }
        upsample8(pred.data(), head[3].data(), wt[head_b(3, 2)].data(), H, W, dst, nthreads);
    }
    if (!direct) {
        // the crop (:289-293)
        for (int c = 0; c < 3; ++c)
            for (int y = 0; y < out_h; ++y)
                std::memcpy(out + ((size_t)c * out_h + y) * out_w,
                            up.data() + (size_t)c * fh * fw + (size_t)(pad_t + y) * fw + pad_l,
                            (size_t)out_w * sizeof(float));
    }
    return BVML_DSINE_OK;
}

}  // namespace

extern "C" int bvml_dsine_refiner_forward_cpu(bvml_dsine_refiner* r, const float* normal,
                                              const float* feature, const float* hidden, int h8,
                                              int w8, float fx, float fy, float cx, float cy,
                                              int orig_h, int orig_w, int pad_t, int pad_l,
                                              int out_h, int out_w, float* out, float* coarse,
                                              int nthreads) {
    if (!r) return fail(BVML_DSINE_ENULL, "forward_cpu: refiner must be non-NULL");
    const auto& wt = host_weights(r);
    const ForwardArgs args{normal, feature, hidden, h8, w8, fx, fy, cx, cy, orig_h, orig_w,
                           pad_t, pad_l, out_h, out_w, out, coarse};
    if (const int st = check_forward(wt, args, "forward_cpu: ")) return st;
    try {
        return run_cpu(wt, normal, feature, hidden, h8, w8, fx, fy, cx, cy, orig_h, orig_w, pad_t,
                       pad_l, out_h, out_w, out, coarse, nthreads);
    } catch (const std::bad_alloc&) {
        return fail(BVML_DSINE_ESIZE, "forward_cpu: out of host memory");
    }
}
