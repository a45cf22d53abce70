// MI355X (gfx950) convex upsample + channel L2-normalise: the step the DSINE
// refiner runs after each AngMF propagate (src/dsine_refine.cpp:276-282,
// brotensor::convex_upsample_forward then l2_normalize_nchw_forward with eps
// 1e-12f), fused into one pass.  Arithmetic as the reference specifies it
// (include/brovisionml/dsine_refine.h:91-97, DSINE's upsample_via_mask with
// replicate padding, then F.normalize):
//   mask (B, 9*s*s, H, W), channel n*s*s + ky*s + kx, n = 3*dy' + dx'
//   w_n   = softmax over the 9 taps n of that channel set, per (y, x, ky, kx)
//   v_c   = sum_n w_n * x[c, clamp(y - 1 + n/3), clamp(x - 1 + n%3)]
//   out[c, s*y + ky, s*x + kx] = v_c / max(|v|, eps)      (or v_c unnormalised)
//
// The op streams the mask once (9*s*s floats per low-res pixel, 2304 B/px at
// s = 8) and writes s*s*C floats per pixel, so HBM bandwidth bounds it; the
// arithmetic is kept below the memory time by a mixed-precision fast path:
//   * weights e_n = 2^((m_n - max) * log2 e) with the hardware exp2 (v_exp_f32)
//     in fp32; the weighted sum and the softmax denominator accumulate in
//     double (exact products of the fp32 weights and inputs);
//   * each sub-pixel carries a bound on its weights' error,
//       |e^_n - e_n| <= e_n * (kExpRel + kArgRel * |t_n|),   t_n = (m_n - max) log2 e,
//     kExpRel for the exp2 itself and kArgRel for the rounding of t_n (two fp32
//     roundings and the float log2 e), so that |v^ - v| <= bnd = sum_n of that
//     bound times |x_n| (plus 2^-126 |x_n| for weights the exp2 flushes to 0);
//     normalising maps it to at most 2 bnd / |v| per component;
//   * a sub-pixel whose |v| is under bnd * 2 / kDirBudget (the normalise would
//     amplify the weights' error past kDirBudget), whose |v|/S is near eps, whose
//     |v|^2 leaves the fp32 range, or any NaN, is recomputed in double with the
//     reference's formula (library exp, w = e / sum, sum of w * x,
//     1 / max(sqrt(|v|^2), eps)) after the lane's fast sub-pixels, from its 9
//     mask values kept in LDS, so a wave pays once per flag of its busiest
//     lane (about 0.14% of sub-pixels on independent random unit normals, far
//     fewer on smooth normal maps);
//   * the normalise of the rest is v * rsq(|v|^2) with the fp32 hardware rsq.
// Every output is within 7.2e-6 per component of the exact one (a bound; the
// typical difference is about 1e-7).
// BVML_DSINE_FP64 runs every sub-pixel through the double body with the
// library exp.
//
// Work split at s = 8: a wave owns 32 consecutive low-res pixels of one
// sub-pixel row ky, 2 lanes per pixel, each lane 4 sub-pixels kx, so each
// channel's output is one 1 KB run (32 px x 8 sub-pixels) of the upsampled
// row, stored as float4s.  upsample8_lds_kernel (H*W a multiple of 4, the
// mask 16-byte aligned) first stages a block's mask planes in LDS with
// direct-to-LDS loads of 512 contiguous bytes per plane; upsample8_kernel
// (any other s = 8 call) loads each lane's values into registers, 128 B per
// plane per wave-wide load, 52-54 us against 44-45 for the staged kernel at
// 256 x 256, C = 3.  The waves of one pixel group (one per ky) are adjacent
// and share its 3x3 taps: four in one block of the register kernel (in L1),
// eight adjacent blocks of the staged kernel (in L2).
// Other scales take one lane per (pixel, ky) with a loop over kx.

#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdint>
#include <string>

#include "bvml_dsine.h"
#include "status.h"

namespace {

using bvml::fail;
using bvml::overlaps;

typedef float f4v __attribute__((ext_vector_type(4)));

// The float nearest log2(e) (relative error 1.3e-8).
constexpr float kLog2E = 1.44269504088896340736f;

// Relative error of v_exp_f32 on [-126, 0]: at most 8.484e-8 over every float
// there (measured exhaustively on gfx950).  Below -126 it returns 0 (outputs
// are not denormal), so a tap's weight is off by at most 2^-126 of the
// largest: kFlushAbs * |x_n|, summed over the taps once.
constexpr float kExpRel = 8.5e-8f;
constexpr float kFlushAbs = 1.18e-38f;
// Error of t_n = (m_n - max) * log2e: the fp32 subtraction and product
// round once each (2^-24 |t| apiece) and the float log2 e adds 1.34e-8 |t|;
// 2^(t(1+d)) = 2^t (1 + d t ln 2 + ...), so the weight's relative error from
// the argument is at most ln 2 * 1.33e-7 * |t|.
constexpr float kArgRel = 9.3e-8f;
// Largest per-component error the weights may cause in a normalised output:
// 2 bnd / |v| <= kDirBudget.  The fp32 rsq (relative error <= 9.4e-8 over
// every float, measured), the rounding of |v|^2 to fp32 and the final
// rounding add at most 1.9e-7, so the fast path stays within 7.2e-6 of the
// exact result.
constexpr float kDirBudget = 7.0e-6f;
constexpr float kThrScale = 2.0f / kDirBudget;

// Lanes the fast path accepts: |v|^2 in [kMinN2, kMaxN2] keeps the fp32 rsq
// in its normal range.
constexpr float kMinN2 = 1e-30f;
constexpr float kMaxN2 = 1e30f;

// mode bits
constexpr int kNormalize = 1;
constexpr int kExact = 2;

// std::max(a, b) == (a < b) ? b : a -- returns a when a is NaN, as the
// reference's F.normalize restatement does (fmax would not).
__device__ __forceinline__ double smax(double a, double b) { return (a < b) ? b : a; }

// The 3x3 replicate-padded neighbourhood of one low-res pixel: x at the 9
// taps (tap n at row y - 1 + n/3, column x - 1 + n%3, clamped) and each tap's
// channel norm in fp32 (used only by the error bound).
template <int C>
struct Taps {
    float v[C][9];
    float nrm[9];
    float flush;  // kFlushAbs * sum of nrm
};

template <int C>
__device__ __forceinline__ void load_taps(const float* __restrict__ xb, long long HW, int H,
                                          int W, int y, int x, Taps<C>& t) {
    const long long row[3] = {(long long)(y > 0 ? y - 1 : 0) * W, (long long)y * W,
                              (long long)(y + 1 < H ? y + 1 : H - 1) * W};
    const int col[3] = {x > 0 ? x - 1 : 0, x, x + 1 < W ? x + 1 : W - 1};
    float q_sum = 0.0f;
#pragma unroll
    for (int n = 0; n < 9; ++n) {
        const long long q = row[n / 3] + col[n % 3];
        float s2 = 0.0f;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            t.v[c][n] = xb[c * HW + q];
            s2 = fmaf(t.v[c][n], t.v[c][n], s2);
        }
        t.nrm[n] = sqrtf(s2);
        q_sum += t.nrm[n];
    }
    t.flush = kFlushAbs * q_sum;
}

// One sub-pixel in double precision: the reference's formula (exp of m - max,
// w = e / sum, sum of w * x, 1 / max(sqrt(|v|^2), eps)) with the library's
// double exp, accumulated as sum(e * x) / sum(e) in one pass over the taps.
template <int C>
__device__ __forceinline__ void exact_subpixel(const float (&m)[9], const Taps<C>& t,
                                               bool normalize, double eps, float (&o)[C]) {
#pragma clang fp contract(off)
    bool nan = false;
#pragma unroll
    for (int n = 0; n < 9; ++n) nan |= __builtin_isnan(m[n]);
    double mx = m[0];
#pragma unroll
    for (int n = 1; n < 9; ++n)
        if ((double)m[n] > mx) mx = m[n];
    double sum = 0.0, v[C];
#pragma unroll
    for (int c = 0; c < C; ++c) v[c] = 0.0;
#pragma unroll
    for (int n = 0; n < 9; ++n) {
        const double e = nan ? __builtin_nan("") : exp((double)m[n] - mx);
        sum += e;
#pragma unroll
        for (int c = 0; c < C; ++c) v[c] += e * (double)t.v[c][n];
    }
    const double rsum = 1.0 / sum;
    double inv = 1.0;
    if (normalize) {
        double n2 = 0.0;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            v[c] *= rsum;
            n2 += v[c] * v[c];
        }
        inv = 1.0 / smax(sqrt(n2), eps);
    } else {
        inv = rsum;
    }
#pragma unroll
    for (int c = 0; c < C; ++c) o[c] = (float)(v[c] * inv);
}

// One sub-pixel on the fp32-weight fast path.  Returns false (o unset) when
// the error bound, a special value or kExact calls for the double body.
// eps_s = 1.01 * eps in float (0 when eps <= 0 or NaN).
template <int C>
__device__ __forceinline__ bool fast_subpixel(const float (&m)[9], const Taps<C>& t, int mode,
                                              float eps_s, float (&o)[C]) {
    float mx = m[0];
#pragma unroll
    for (int n = 1; n < 9; ++n) mx = fmaxf(mx, m[n]);
    double S = 0.0, v[C];
#pragma unroll
    for (int c = 0; c < C; ++c) v[c] = 0.0;
    float bnd = t.flush;
#pragma unroll
    for (int n = 0; n < 9; ++n) {
        const float tn = (m[n] - mx) * kLog2E;
        const float e = __builtin_amdgcn_exp2f(tn);
        const double ed = e;
        S += ed;
#pragma unroll
        for (int c = 0; c < C; ++c) v[c] = fma(ed, (double)t.v[c][n], v[c]);
        bnd = fmaf(e * t.nrm[n], fmaf(-tn, kArgRel, kExpRel), bnd);
    }
    const bool normalize = (mode & kNormalize) != 0;
    bool fast = (mode & kExact) == 0;
    if (normalize) {
        double n2 = 0.0;
#pragma unroll
        for (int c = 0; c < C; ++c) n2 = fma(v[c], v[c], n2);
        const float n2f = (float)n2;
        const float thr = fmaxf(bnd * kThrScale, eps_s * (float)S);
        fast = fast && n2f >= fmaxf(thr * thr, kMinN2) && n2f <= kMaxN2;
        if (fast) {
            const double r = __builtin_amdgcn_rsqf(n2f);
#pragma unroll
            for (int c = 0; c < C; ++c) o[c] = (float)(v[c] * r);
        }
    } else if (fast) {
        const double inv = 1.0 / S;
#pragma unroll
        for (int c = 0; c < C; ++c) o[c] = (float)(v[c] * inv);
    }
    return fast;
}

// s = 8.  Block of 4 waves; wave gw = 8 * group + ky; lane = 2 * i + h owns
// pixel group*32 + i and sub-pixels kx = 4h .. 4h + 3.
constexpr int kLanesPerPx = 2;
constexpr int kSubPerLane = 8 / kLanesPerPx;
constexpr int kPxPerWave = 64 / kLanesPerPx;

template <int C>
__global__ __launch_bounds__(256) void upsample8_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ mask,
                                                        const float* __restrict__ mbias,
                                                        float* __restrict__ out, int H, int W,
                                                        int groups, int mode, float eps_s,
                                                        double eps) {
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int group = gw >> 3, ky = gw & 7;
    if (group >= groups) return;
    const int lane = threadIdx.x & 63;
    const int i = lane / kLanesPerPx, h = lane % kLanesPerPx;
    const long long HW = (long long)H * W;
    const int p = group * kPxPerWave + i;
    if (p >= HW) return;
    const long long b = blockIdx.y;
    const float* xb = x + b * C * HW;
    const float* mb = mask + b * 576 * HW + (long long)(ky * 8 + h * kSubPerLane) * HW + p;
    float* ob = out + b * C * 64 * HW;
    const int y = p / W, xx = p - y * W;

    // every mask load of the lane first, so that all are in flight at once
    float m[kSubPerLane][9];
#pragma unroll
    for (int j = 0; j < kSubPerLane; ++j)
#pragma unroll
        for (int n = 0; n < 9; ++n) m[j][n] = mb[(long long)(n * 64 + j) * HW];
    Taps<C> t;
    load_taps<C>(xb, HW, H, W, y, xx, t);
    // the mask's per-channel bias (the up-mask head's last convolution run
    // without it): one fp32 add per value, as a separate bias pass would do
    if (mbias) {
        const float* bb = mbias + ky * 8 + h * kSubPerLane;
#pragma unroll
        for (int j = 0; j < kSubPerLane; ++j)
#pragma unroll
            for (int n = 0; n < 9; ++n) m[j][n] += bb[n * 64 + j];
    }

    // a flagged sub-pixel's 9 mask values wait in LDS for its recompute
    // (36 KB per workgroup: the 3 workgroups per CU the registers allow use
    // 108 of the 160 KB)
    __shared__ float stash[kSubPerLane][9][256];
    float o[C][kSubPerLane];
    unsigned redo = 0;
#pragma unroll
    for (int j = 0; j < kSubPerLane; ++j) {
        float r[C];
        const bool ok = fast_subpixel<C>(m[j], t, mode, eps_s, r);
#pragma unroll
        for (int c = 0; c < C; ++c) o[c][j] = r[c];
        if (!ok) {
#pragma unroll
            for (int n = 0; n < 9; ++n) stash[j][n][threadIdx.x] = m[j][n];
        }
        redo |= (ok ? 0u : 1u) << j;
    }
    // each lane recomputes its own flagged sub-pixels, one per trip, so a
    // wave makes as many trips as its busiest lane has flags
    const bool normalize = (mode & kNormalize) != 0;
    while (redo) {
        const int j = __builtin_ctz(redo);
        redo &= redo - 1;
        float mj[9];
#pragma unroll
        for (int n = 0; n < 9; ++n) mj[n] = stash[j][n][threadIdx.x];
        float r[C];
        exact_subpixel<C>(mj, t, normalize, eps, r);
#pragma unroll
        for (int jj = 0; jj < kSubPerLane; ++jj)
#pragma unroll
            for (int c = 0; c < C; ++c) o[c][jj] = (j == jj) ? r[c] : o[c][jj];
    }
    // non-temporal stores: the output stream then takes less of the HBM
    // bandwidth the mask stream needs (about 1 us of 51 at 256 x 256, C = 3)
    const long long q = (long long)(8 * y + ky) * (8 * W) + 8 * xx + h * kSubPerLane;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const f4v w = {o[c][0], o[c][1], o[c][2], o[c][3]};
        __builtin_nontemporal_store(w, reinterpret_cast<f4v*>(ob + c * 64 * HW + q));
    }
}

// s = 8, staged through LDS.  A block of 4 waves owns 128 consecutive
// pixels of one sample (P0 .. P0 + 127) at one sub-pixel row ky, and first
// copies the 72 mask planes of that row (9 taps x 8 kx) for its pixels into
// LDS with direct-to-LDS loads: each 16-byte lane load carries 4 pixels, so
// one wave-wide load reads 512 contiguous bytes of each of two planes (the
// register-file loads of upsample8_kernel read 128 bytes of each of two).
// LDS block k = 4n + j (1 KB) holds plane (n, kx = j) in dwords 0..127
// (pixel order) and plane (n, kx = 4 + j) in dwords 128..255, rotated by 32
// pixels, so that a read of both halves' pixel pl hits banks 32 dwords apart.
// Then wave w, lane i + 32h, computes pixel P0 + 32w + i, sub-pixels
// kx = 4h .. 4h + 3, from LDS, as upsample8_kernel does.  Needs HW % 4 == 0
// and a 16-byte-aligned mask; lanes past the sample's last pixel load its
// last 4 pixels instead (in bounds) and store nothing.
constexpr int kLdsPx = 128;
constexpr int kLdsBlocks = 36;
// The mask loads' cache policy: non-temporal (each value is read once).
// 256 x 256, C = 3, cold: 43.8-44.7 us against 46.7-47.0 with the default
// policy; warm (the mask in the Infinity Cache) 39.9-40.4 against 35.9-37.6.
// Blocks of 256 pixels (8 waves, one 1 KB plane segment per load, 72 KB of
// LDS, two blocks per CU) measured 50.9-51.3 us.
constexpr int kLoadNt = 2;

template <int C>
__global__ __launch_bounds__(256) void upsample8_lds_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ mask,
                                                            const float* __restrict__ mbias,
                                                            float* __restrict__ out, int H, int W,
                                                            int mode, float eps_s, double eps) {
    __shared__ __attribute__((aligned(16))) float seg[kLdsBlocks * 256];
    const int g = blockIdx.x >> 3, ky = blockIdx.x & 7;
    // (the wave index read as a scalar: the plane offsets and LDS blocks of
    // the loads below are then scalar too)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int h = lane >> 5, i = lane & 31;
    const long long HW = (long long)H * W;
    const long long b = blockIdx.y;
    const long long P0 = (long long)g * kLdsPx;

    // the wave's 9 blocks: 8 planes x 2 halves ... lane q of half h loads
    // pixels 4 * ((q + 8h) mod 32) .. + 3 of plane (n, 4h + j)
    {
        const float* mb = mask + b * 576 * HW + (long long)(ky * 8 + 4 * h) * HW;
        long long px = P0 + 4 * ((i + 8 * h) & 31);
        px = px < HW - 4 ? px : HW - 4;
#pragma unroll
        for (int t = 0; t < 9; ++t) {
            const int k = wave * 9 + t, n = k >> 2, j = k & 3;
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(mb + (long long)(n * 64 + j) * HW + px),
                reinterpret_cast<__attribute__((address_space(3))) void*>(
                    reinterpret_cast<uintptr_t>(&seg[k * 256])),
                16, 0, kLoadNt);
        }
    }
    const int pl = wave * 32 + i;
    const long long p = P0 + pl;
    const bool live = p < HW;
    const long long pc = live ? p : HW - 1;
    const int y = (int)(pc / W), xx = (int)(pc - (long long)y * W);
    Taps<C> t;
    load_taps<C>(x + b * C * HW, HW, H, W, y, xx, t);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (!live) return;

    const int off = h ? 128 + ((pl - 32) & 127) : pl;
    const float* bb = mbias ? mbias + ky * 8 + h * kSubPerLane : nullptr;
    float o[C][kSubPerLane];
    unsigned redo = 0;
#pragma unroll
    for (int j = 0; j < kSubPerLane; ++j) {
        float m[9];
#pragma unroll
        for (int n = 0; n < 9; ++n) m[n] = seg[(n * 4 + j) * 256 + off];
        if (bb) {
#pragma unroll
            for (int n = 0; n < 9; ++n) m[n] += bb[n * 64 + j];
        }
        float r[C];
        const bool ok = fast_subpixel<C>(m, t, mode, eps_s, r);
#pragma unroll
        for (int c = 0; c < C; ++c) o[c][j] = r[c];
        redo |= (ok ? 0u : 1u) << j;
    }
    // each lane recomputes its own flagged sub-pixels from the staged mask
    const bool normalize = (mode & kNormalize) != 0;
    while (redo) {
        const int j = __builtin_ctz(redo);
        redo &= redo - 1;
        float m[9];
#pragma unroll
        for (int n = 0; n < 9; ++n) m[n] = seg[(n * 4 + j) * 256 + off];
        if (bb) {
#pragma unroll
            for (int n = 0; n < 9; ++n) m[n] += bb[n * 64 + j];
        }
        float r[C];
        exact_subpixel<C>(m, t, normalize, eps, r);
#pragma unroll
        for (int jj = 0; jj < kSubPerLane; ++jj)
#pragma unroll
            for (int c = 0; c < C; ++c) o[c][jj] = (j == jj) ? r[c] : o[c][jj];
    }
    float* ob = out + b * C * 64 * HW;
    const long long q = (long long)(8 * y + ky) * (8 * W) + 8 * xx + h * kSubPerLane;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const f4v w = {o[c][0], o[c][1], o[c][2], o[c][3]};
        __builtin_nontemporal_store(w, reinterpret_cast<f4v*>(ob + c * 64 * HW + q));
    }
}

// Any scale: one lane per (pixel, ky), looping over kx.  Block of 4 waves;
// wave gw = s * group + ky owns pixels group*64 .. group*64 + 63.
template <int C>
__global__ __launch_bounds__(256) void upsample_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ mask,
                                                       const float* __restrict__ mbias,
                                                       float* __restrict__ out, int H, int W,
                                                       int s, int groups, int mode,
                                                       float eps_s, double eps) {
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int group = gw / s, ky = gw - group * s;
    if (group >= groups) return;
    const long long HW = (long long)H * W;
    const int p = group * 64 + (threadIdx.x & 63);
    if (p >= HW) return;
    const long long b = blockIdx.y, s2 = (long long)s * s;
    const float* xb = x + b * C * HW;
    const float* mb = mask + b * 9 * s2 * HW + (long long)ky * s * HW + p;
    float* ob = out + b * C * s2 * HW;
    const int y = p / W, xx = p - y * W;

    Taps<C> t;
    load_taps<C>(xb, HW, H, W, y, xx, t);

    const long long q0 = ((long long)s * y + ky) * ((long long)s * W) + (long long)s * xx;
    for (int kx = 0; kx < s; ++kx) {
        float m[9];
#pragma unroll
        for (int n = 0; n < 9; ++n) m[n] = mb[(n * s2 + kx) * HW];
        if (mbias) {
#pragma unroll
            for (int n = 0; n < 9; ++n) m[n] += mbias[n * s2 + (long long)ky * s + kx];
        }
        float r[C];
        if (!fast_subpixel<C>(m, t, mode, eps_s, r))
            exact_subpixel<C>(m, t, (mode & kNormalize) != 0, eps, r);
#pragma unroll
        for (int c = 0; c < C; ++c) __builtin_nontemporal_store(r[c], ob + c * s2 * HW + q0 + kx);
    }
}

// Samples per launch (grid y).
constexpr int kMaxGridY = 65535;

template <int C>
hipError_t launch_upsample(const float* x, const float* mask, const float* mbias, float* out,
                           int B, int H, int W, int s, int mode, float eps_s, double eps,
                           bool fast8, bool lds8, hipStream_t stream) {
    const long long HW = (long long)H * W;
    const long long s2 = (long long)s * s;
    for (int b0 = 0; b0 < B; b0 += kMaxGridY) {
        const int nb = (B - b0 < kMaxGridY) ? B - b0 : kMaxGridY;
        const float* xc = x + (size_t)b0 * C * HW;
        const float* mc = mask + (size_t)b0 * 9 * s2 * HW;
        float* oc = out + (size_t)b0 * C * s2 * HW;
        if (lds8) {
            const dim3 grid((unsigned)((HW + kLdsPx - 1) / kLdsPx * 8), (unsigned)nb);
            hipLaunchKernelGGL(upsample8_lds_kernel<C>, grid, dim3(256), 0, stream, xc, mc, mbias,
                               oc, H, W, mode, eps_s, eps);
        } else if (fast8) {
            const int groups = (int)((HW + kPxPerWave - 1) / kPxPerWave);
            const long long waves = (long long)groups * 8;
            const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)nb);
            hipLaunchKernelGGL(upsample8_kernel<C>, grid, dim3(256), 0, stream, xc, mc, mbias, oc,
                               H, W, groups, mode, eps_s, eps);
        } else {
            const int groups = (int)((HW + 63) / 64);
            const long long waves = (long long)groups * s;
            const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)nb);
            hipLaunchKernelGGL(upsample_kernel<C>, grid, dim3(256), 0, stream, xc, mc, mbias, oc,
                               H, W, s, groups, mode, eps_s, eps);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

extern "C" {

int bvml_dsine_convex_upsample_bias_f32(const float* x, const float* mask,
                                        const float* mask_bias, int B, int C, int H, int W,
                                        int scale, int normalize, float eps, float* out,
                                        unsigned flags, void* stream) {
    if (flags & ~BVML_DSINE_FP64)
        return fail(BVML_DSINE_EFLAGS, "convex_upsample: unknown flag bits");
    if (B < 0 || H < 0 || W < 0 || C < 1 || scale < 1)
        return fail(BVML_DSINE_ESHAPE,
                    "convex_upsample: B, H and W must be >= 0, C and scale >= 1");
    if (C > 4 || scale > 16)
        return fail(BVML_DSINE_EUNSUP, "convex_upsample: C must be <= 4 and scale <= 16");
    const long long HW = (long long)H * W;
    if (B == 0 || HW == 0) return BVML_DSINE_OK;
    if (!x || !mask || !out)
        return fail(BVML_DSINE_ENULL, "convex_upsample: x, mask and out must be non-NULL");
    // one sample's pixels in an int, and its wave count (groups * 8, or
    // groups * scale) in the grid's x extent (4 waves per block)
    if (HW >= (1LL << 30))
        return fail(BVML_DSINE_ESIZE, "convex_upsample: H*W too large for one launch");
    const long long s2 = (long long)scale * scale;
    const size_t f = sizeof(float);
    const size_t x_b = (size_t)B * C * HW * f;
    const size_t m_b = (size_t)B * 9 * s2 * HW * f;
    const size_t o_b = (size_t)B * C * s2 * HW * f;
    if (overlaps(out, o_b, x, x_b) || overlaps(out, o_b, mask, m_b) ||
        (mask_bias && overlaps(out, o_b, mask_bias, (size_t)9 * s2 * f)))
        return fail(BVML_DSINE_EALIAS, "convex_upsample: out overlaps an input");

    const int mode = (normalize ? kNormalize : 0) | ((flags & BVML_DSINE_FP64) ? kExact : 0);
    const double epsd = eps;
    const float eps_s = (eps > 0.0f) ? (float)(1.01 * epsd) : 0.0f;
    // the s = 8 kernel stores float4s: out must be 16-byte aligned
    const bool fast8 = scale == 8 && (reinterpret_cast<uintptr_t>(out) % 16) == 0;
    // the staged kernel's 16-byte mask loads: planes 16-byte aligned
    const bool lds8 = fast8 && HW % 4 == 0 && (reinterpret_cast<uintptr_t>(mask) % 16) == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    switch (C) {
        case 1: e = launch_upsample<1>(x, mask, mask_bias, out, B, H, W, scale, mode, eps_s, epsd,
                                       fast8, lds8, s); break;
        case 2: e = launch_upsample<2>(x, mask, mask_bias, out, B, H, W, scale, mode, eps_s, epsd,
                                       fast8, lds8, s); break;
        case 3: e = launch_upsample<3>(x, mask, mask_bias, out, B, H, W, scale, mode, eps_s, epsd,
                                       fast8, lds8, s); break;
        default: e = launch_upsample<4>(x, mask, mask_bias, out, B, H, W, scale, mode, eps_s, epsd,
                                       fast8, lds8, s); break;
    }
    if (e != hipSuccess)
        return fail((int)e, std::string("convex_upsample launch: ") + hipGetErrorString(e));
    return BVML_DSINE_OK;
}

int bvml_dsine_convex_upsample_f32(const float* x, const float* mask, int B, int C, int H,
                                   int W, int scale, int normalize, float eps, float* out,
                                   unsigned flags, void* stream) {
    return bvml_dsine_convex_upsample_bias_f32(x, mask, nullptr, B, C, H, W, scale, normalize,
                                               eps, out, flags, stream);
}

}  // extern "C"
