// MI355X (gfx950) kernels for brovisionml's DSINE surface-normal ops and the
// C ABI that launches them (include/bvml_dsine.h).
//
// Two ops, both per-pixel geometry on the /8 NRN grid, fp32 NCHW planes:
//   ray_relu         in-place camera-facing clamp (src/dsine_ops.cpp:55-76)
//   angmf_propagate  fused k x k neighbour rotate + RayReLU + prob-weighted
//                    sum + renormalise (src/dsine_ops.cpp:78-172)
//
// angmf_propagate moves 436 B/px at k=5 but also does about 25 neighbour
// rotations per pixel; at the parity bar (1e-5 per component) the reference's
// all-double formulation costs far more VALU time than the HBM traffic takes,
// so the fast kernel evaluates every neighbour in fp32 where the error
// analysis allows and recomputes the few pixels where it does not:
//   * the rotation axis is algebraically reduced: the reference's
//     normalize(du + dz*tu, dv + dz*tv, dz) with dz = num/dd equals
//     sign(dd) * V/|V| with V = (g*xs/fu - q*tu0, g*ys/fv - q*tv0, -q),
//     g = P0.m (P0 = the source pixel's ray at depth 1) and
//     q = xs*mx/fu + ys*my/fv on the RAW xy pair -- the xy normalisation and
//     the quadratic terms cancel exactly, and V.m == 0, so Rodrigues reduces
//     to m'*cos(t) + (V x m')*sin(t)/|V|, and V x m' = xs e1 + ys e2 - q f
//     with three per-source vectors;
//   * the tile's replicate-padded pred_norm halo is staged in LDS once, one
//     record per source pixel: m' = m/|m|, g (NaN unless m is a unit
//     normal), the double products mx/fu, my/fv, and e1, e2, f;
//   * tier 1 forms q in double (it cancels where the xy pair is nearly
//     perpendicular to m) and everything else -- dd, V x m', sin/cos (the
//     hardware's, with an argument correction), the rotation, RayReLU, the
//     weight prob/|p|, the partial sums -- in fp32;
//   * a pixel goes to tier 2, the same reduced form in double, when a
//     neighbour is outside the fp32 form's domain (|dd| near the
//     reference's 1e-8 clamp, an xy pair out of range, a non-unit source
//     normal, |t| > 3.2, a non-finite value) or when |acc|^2 < kAccRatio2[k] *
//     sum(wi^2), where the final normalise would amplify tier 1's error
//     past the parity bar; and from there to tier 3, the reference-order
//     double body, when a neighbour is outside the double form's domain or
//     the sum still nearly cancels.  The wave that reduces a pixel group
//     recomputes its flagged pixels by itself, one neighbour per lane.
// Workgroups are 8 waves: G waves per 64-pixel group, each evaluating one run
// of the window's neighbours (G = 2, 4 or 8, chosen per launch), so the SPI
// places 2 waves per SIMD and every SIMD carries the same work; two
// workgroups per CU run a 256x256 image in one round.  Launches that fill the
// chip take G = 1 at k = 5 and 7: each wave evaluates the whole window for its
// pixels, with no cross-wave reduction.
// The double-precision body is also available as its own kernel
// (BVML_DSINE_FP64), which reproduces the CPU reference to a few ulps.

#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>

#include "angmf_ref.h"
#include "bvml_dsine.h"
#include "status.h"


namespace {

using bvml::angle_ref;
using bvml::kPiF;
using bvml::kRayEpsF;
using bvml::nbr_ref_f64;
using bvml::ray_relu_ref;
using bvml::sigmoid_ref;
using bvml::smax;
using bvml::synth_ray;

// The fast path takes source normals with | |m|^2 - 1 | <= kUnitM2 (every
// normal this op or RayReLU writes is one) and raw xy pairs with
// kMinXY2 <= |xy|^2 <= kMaxXY2 in fp32 (below, the reference's 1e-12 clamp
// stops normalising; above, the fp32 |xy|^2 could overflow); a neighbour
// outside sends its pixel to the recompute.  Both bounds are one unsigned
// comparison on the float's bits (NaN and negatives fall outside).
constexpr float kUnitM2 = 1e-5f;
constexpr float kMinXY2 = 1e-20f;
constexpr float kMaxXY2 = 1e30f;
constexpr uint32_t kXY2Lo = __builtin_bit_cast(uint32_t, kMinXY2);
constexpr uint32_t kXY2Span = __builtin_bit_cast(uint32_t, kMaxXY2) - kXY2Lo;
// |V|^2 below this (fp32 underflow territory) also sends the pixel there.
constexpr float kMinV2 = 1e-30f;

// Tier 1 error budget.  A pixel's summed error behaves like delta *
// sqrt(sum(wi^2)) (wi = prob/|p|, a term's weight before its final
// normalise, p the RayReLU'd rotation: near the ray's antipode |p| -> eps and
// the rotation's rounding is amplified by 1/|p|, which wi carries).  Measured
// on this kernel over input families built to stress each mechanism (random
// and camera-facing normals, normals facing away, grazing normals, q and g
// cancelling, checkerboards of nearly opposite normals, wide angles and
// fields of view, saturated logits, with and without the activations formed
// in the kernel), 0.5M-3.5M pixels per family and window size in both work
// layouts, and over inputs a hill-climbing search pushed toward the largest
// error of a kept pixel from each family, pixels whose sum nearly cancels
// show delta <= 3.42e-7 at k = 3, 3.54e-7 at k = 5 (saturated logits, the
// whole-window layout, found by the search), 4.41e-7 at k = 7 (grazing
// normals, the whole-window layout) and 3.99e-7 at k = 9.  Summation order does not explain the
// spread (a model of this arithmetic gives the same delta with every
// neighbour summed in double): per-term errors are about 1 ulp of wi in
// every family, and they add coherently where the terms share the pixel's
// ray and look alike.  The final normalise divides the sum by |acc|, so a
// pixel with |acc|^2 < kAccRatio2[k] * sum(wi^2) is recomputed, and with
// delta(k) the measured value plus 10%, the rest stay within
// delta(k) / sqrt(kAccRatio2[k]) <= 7.5e-6 per component, 25% inside the bar
// (the largest kept error measured is 5.8e-6, and the search's 5.2e-6).  At
// k = 1 the sum is one term and cannot cancel.
//
// About 2.3 pixels of a 256x256 image of independent random unit normals with
// angles up to pi/4 fall below the k = 5 threshold; the refiner's
// camera-facing normals practically never do.  A flagged pixel costs its
// group's reducing wave about 2.5 us after the reduce: one round trip to
// reload its inputs (about 1 us under load), the double evaluation (about
// 0.9 us of dependent double arithmetic for one wave) and the lane
// reduction.  A 256x256 call runs all its workgroups at once, so a flagged
// pixel in a late group lengthens the call by up to that much.
constexpr double kAccRatio2[10] = {2.6e-3, 2.6e-3, 0.0, 2.6e-3, 0.0,
                                   2.75e-3, 0.0, 4.2e-3, 0.0, 3.5e-3};

// Tier 2 (the double-precision reduced form of flagged pixels) hands a pixel
// to the reference-order body when its sum nearly cancels: below
// kAccRatio2Ref * sum(wi^2), or |acc| near the reference's 1e-12 clamp.
// Its per-term error is a few 1e-16, so the rest stay within about 1e-7.
constexpr double kAccRatio2Ref = 1e-16;
constexpr double kAcc2Floor = 1e-22;

// The reference clamps |dd| < 1e-8 (src/dsine_ops.cpp:120-123), where the
// reduced axis no longer holds.  Tier 1 forms dd = g + q/|xy| as
// fma(q, rsq(|xy|^2), g) in fp32 with g and q rounded from double: it is
// within 6e-8 |g| + 1.9e-7 |m| / min(|fu|, |fv|) (+ 6e-8 |dd|) of the exact
// value.  A neighbour with |dd| below
//   dd_min = 1.02e-8 + 1e-7 * gmax + 3e-7 / min(|fu|, |fv|),
// gmax the largest |P0| (source ray at depth 1) over the image, sends its
// pixel to the recompute, so the sign of every other dd is the reference's
// and so is the axis -- including where m is nearly parallel to N = D x P0
// (g and q both small), since dd = g + q/|xy| is small then too.  Tier 2's
// double dd is within 1e-15 of the exact value; it sends a neighbour with
// |dd| < kDdClampRef to the reference-order body.
constexpr double kDdClamp = 1.02e-8;
constexpr double kDdClampRef = 1.0001e-8;
// The fp32 path assumes |P0| <= kMaxP0 over the image (a diagonal field of
// view up to about 150 degrees): its |V| stays within fp32 range and its
// error bound above holds.  Wider views run the double-precision kernel.
constexpr double kMaxP0 = 4.0;

__device__ __forceinline__ int clampi(int v, int lo, int hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

// n / d for 0 <= n < 2^21 and 1 <= d given rd = 1/d in fp32 (within 1 ulp):
// n + 0.5 keeps every quotient at least 0.5/d from an integer, more than the
// estimate's error (below n/d * 2^-22).  Callers divide thread and halo
// indices (n < 2^12) by tile widths.
__device__ __forceinline__ int small_div(int n, float rd) {
    return (int)(((float)n + 0.5f) * rd);
}

// Per-launch constants of angmf_propagate.
struct AngmfArgs {
    const float* pn;   // pred_norm
    const float* pr;   // prob
    const float* xy;   // raw xy
    const float* ang;  // angle
    const float* ray;
    float* out;
    double fu, cu, fv, cv;
    long long ray_bstride;
    long long HW;
    int B, H, W;
    // fp32 kernel: TW x TH output tile per workgroup, M groups of 64 pixels,
    // G waves per group (one run of the window's neighbours each) -> 64*M*G
    // threads.
    int G, TW, TH, M, tiles_x, tiles_per_img;
    int range;            // range tiles: 64 M consecutive pixels (TW = W; TH the rows they span)
    double ifu64, ifv64;  // 1/fu, 1/fv
    double tu_c, tv_c;    // (0.5 - cu)/fu, (0.5 - cv)/fv: source ray tu0 = sx/fu + tu_c
    double dd_min;        // tier 1: |dd| below this sends a pixel to the recompute
    int synth_ray;        // form rays from the intrinsics (synth_ray), not from `ray`
    int logits;           // prob and angle are logits (BVML_DSINE_LOGITS)
    int stream_planes;    // whole-window launch past the Infinity Cache: nt plane loads
};

// ---------------------------------------------------------------------------
// Double-precision kernel: one pixel per thread, reference order throughout.
// ---------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(256) void angmf_f64_kernel(AngmfArgs a) {
#pragma clang fp contract(off)
    constexpr int P = K / 2, K2 = K * K;
    const long long HW = a.HW;
    const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long long)a.B * HW) return;
    const int b = (int)(gid / HW);
    const long long p = gid - (long long)b * HW;
    const int y = (int)(p / a.W), x = (int)(p - (long long)y * a.W);
    const float* pn = a.pn + (size_t)b * 3 * HW;
    const float* pr = a.pr + (size_t)b * K2 * HW;
    const float* xyp = a.xy + (size_t)b * 2 * K2 * HW;
    const float* ap = a.ang + (size_t)b * K2 * HW;
    const float* rp = a.synth_ray ? nullptr : a.ray + (size_t)b * a.ray_bstride;
    float* op = a.out + (size_t)b * 3 * HW;

    double rx, ry, rz;
    if (a.synth_ray) {
        const bvml::Ray3f r = synth_ray(x, y, a.fu, a.cu, a.fv, a.cv);
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
        const int ky = n / K, kx = n - ky * K;
        const int sy = clampi(y - P + ky, 0, a.H - 1);
        const int sx = clampi(x - P + kx, 0, a.W - 1);
        const long long sp = (long long)sy * a.W + sx;
        double mx, my, mz, pinv;
        const float th = ap[(size_t)n * HW + p], wp = pr[(size_t)n * HW + p];
        nbr_ref_f64(pn[sp], pn[HW + sp], pn[2 * HW + sp], sx + 0.5, sy + 0.5,
                    xyp[(size_t)n * HW + p], xyp[(size_t)(K2 + n) * HW + p],
                    a.logits ? angle_ref(th) : th, rx, ry, rz, a.fu, a.cu, a.fv, a.cv,
                    mx, my, mz, pinv);
        const double w = a.logits ? sigmoid_ref(wp) : wp;
        acc0 += w * mx;
        acc1 += w * my;
        acc2 += w * mz;
    }
    const double inv = 1.0 / smax(sqrt(acc0 * acc0 + acc1 * acc1 + acc2 * acc2), 1e-12);
    op[p] = (float)(acc0 * inv);
    op[HW + p] = (float)(acc1 * inv);
    op[2 * HW + p] = (float)(acc2 * inv);
}

// ---------------------------------------------------------------------------
// fp32 fast kernel
// ---------------------------------------------------------------------------

// Workgroups go to the 8 XCDs round-robin by their linear index (x fastest).
// Give each XCD a contiguous run of an image's logical tiles so tiles that
// share halo rows and columns share that XCD's L2.  (A launch of several
// samples is remapped per image, along x only.  Remapping its linear index
// instead, so that each XCD takes whole images, cut 32 x 60 x 80's traffic
// from 1.067x to 1.047x the algorithmic bytes but ran slower, cold and warm:
// 18.2-19.1 against 17.5-18.3 us, 15.3-15.8 against 14.1-14.2 warm, and
// 4 x 512 x 512 at k = 7 161 against 156-157 us.)
__device__ __forceinline__ int xcd_remap(int bid, int nb) {
    const int q = nb >> 3, r = nb & 7;
    const int xcd = bid & 7, i = bid >> 3;
    return xcd * q + (xcd < r ? xcd : r) + i;
}

// Load base[byte_off / 4] with a uniform base pointer and a 32-bit per-lane
// byte offset, which maps onto the scalar-base + vector-offset load form.
__device__ __forceinline__ float ldf(const float* base, uint32_t byte_off) {
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + byte_off);
}

// Raw buffer load of one fp32 plane: the descriptor (base, HW*4 bytes) is
// wave-uniform and lives in scalar registers, the lane supplies a 32-bit byte
// offset; an offset past the plane reads 0 instead of faulting.
constexpr int kBufferWord3 = 0x00020000;  // gfx9 raw-buffer descriptor word 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t plane_rsrc(const float* plane, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(plane), (short)0, (int)bytes,
                                             kBufferWord3);
}

__device__ __forceinline__ float ldb(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, 0, 0));
}

// Raw buffer load at a per-lane byte offset plus a wave-uniform one (held in
// an SGPR): one descriptor then serves several planes of a tensor.
__device__ __forceinline__ float ldbs(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, uint32_t soff) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, (int)soff, 0));
}

// The same load with the non-temporal cache policy (nt): the line is not
// kept for reuse.  A whole-window launch whose data exceed the 256 MB
// Infinity Cache reads its neighbour planes this way (kStreamBytes).
__device__ __forceinline__ float ldbs_nt(__amdgpu_buffer_rsrc_t r, uint32_t byte_off,
                                         uint32_t soff) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, (int)soff, 2));
}

// base advanced by plane * plane_bytes bytes (64-bit product of 32-bit factors).
__device__ __forceinline__ const float* at_plane(const float* base, uint32_t plane,
                                                 uint32_t plane_bytes) {
    return reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) +
                                          (uint64_t)plane * plane_bytes);
}

// n / d for 0 <= n < 2^31 and 1 <= d < 2^31 from d's magic number
// mag = floor(2^32 (2^L - d) / d) + 1, L = ceil(log2 d) (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994):
// (umulhi(n, mag) + n) >> L, whose sum cannot wrap for n < 2^31.
__device__ __forceinline__ int magic_div(int n, unsigned mag, int L) {
    return (int)((__umulhi((unsigned)n, mag) + (unsigned)n) >> L);
}

// Store of one output float, non-temporal: the stores of a large launch then
// take less of the HBM bandwidth the input stream is using (measured: 3 us of
// 155 on 4 x 512 x 512 at k = 7, 0.2 us of 8.8 at 256 x 256, k = 5).
__device__ __forceinline__ void stf(float* base, uint32_t byte_off, float v) {
    __builtin_nontemporal_store(v, reinterpret_cast<float*>(reinterpret_cast<char*>(base) +
                                                            byte_off));
}

__device__ __forceinline__ unsigned long long uniform64(unsigned long long v) {
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}

// 1/sqrt(x) in double: the hardware estimate refined by two Newton steps.
__device__ __forceinline__ double rsq64(double x) {
    double y = __builtin_amdgcn_rsq(x);
    double e = fma(-x * y, y, 1.0);
    y = fma(0.5 * y, e, y);
    e = fma(-x * y, y, 1.0);
    return fma(0.5 * y, e, y);
}

// 1/sqrt(x) in double with one Newton step (about 1e-14 relative).
__device__ __forceinline__ double rsq64_1(double x) {
    const double y = __builtin_amdgcn_rsq(x);
    return fma(0.5 * y, fma(-x * y, y, 1.0), y);
}

// 1 + exp(-x) in fp32 from the hardware exp2: the rounding of t = -x log2(e)
// changes exp(-x) by 6e-8 |x| relatively, and sigmoid = 1/(1 + exp(-x)) by
// sigmoid (1 - sigmoid) 6e-8 |x| <= 1.3e-8 absolutely, below its own
// rounding.  +inf below x = -88.7, NaN for NaN.
__device__ __forceinline__ float one_plus_exp_neg(float x) {
    constexpr float kL2E = 1.44269502f;  // log2(e) rounded to float
    return 1.0f + __builtin_amdgcn_exp2f(-x * kL2E);
}

// sigmoid(x) in fp32, within 4 ulps or 3e-8: 1/(1 + exp(-x)) from the hardware
// rcp and one Newton step.  Below x = -87 (sigmoid under 2e-38, a denormal
// or 0 as a float) it returns 0, so -inf gives exactly 0 as the reference's
// sigmoid does; NaN stays NaN.
__device__ __forceinline__ float sigmoid_f32(float x) {
    const bool tiny = x < -87.0f;
    const float d = one_plus_exp_neg(tiny ? 0.0f : x);
    const float r = __builtin_amdgcn_rcpf(d);
    return tiny ? 0.0f : fmaf(r, fmaf(-d, r, 1.0f), r);
}

// sin and cos of t for |t| <= 3.2 in double (callers send larger |t| to the
// reference-order path).  Half-angle polynomials in u = h^2, h = t/2 in
// [0, 1.6]: degree-17/16 Chebyshev fits (computed for this kernel) with
// sin h to 2e-18 and cos h to 2e-17; then sin t = 2 sin h cos h and
// cos t = cos^2 h - sin^2 h.
__device__ __forceinline__ void sincos_small64(double t, double& st, double& ct) {
    const double h = 0.5 * t, u = h * h;
    double p = 2.7284852642995796443e-15;
    p = fma(u, p, -7.6437284923156877094e-13);
    p = fma(u, p, 1.6058969595887581407e-10);
    p = fma(u, p, -2.5052107495717588328e-8);
    p = fma(u, p, 2.7557319218192719186e-6);
    p = fma(u, p, -0.00019841269841251311898);
    p = fma(u, p, 0.0083333333333333107506);
    p = fma(u, p, -0.16666666666666666622);
    const double s = fma(h * u, p, h);
    double q = 4.6220697732871493978e-14;
    q = fma(u, q, -1.1464231827944265041e-11);
    q = fma(u, q, 2.087661624946805833e-9);
    q = fma(u, q, -2.7557317537571715429e-7);
    q = fma(u, q, 0.000024801587290607644376);
    q = fma(u, q, -0.0013888888888853772382);
    q = fma(u, q, 0.041666666666666238695);
    q = fma(u, q, -0.49999999999999999144);
    const double c = fma(u, q, 1.0);
    const double sc = s * c;
    st = sc + sc;
    ct = fma(c, c, -(s * s));
}

// One neighbour in the double-precision reduced form (tier 2, the recompute
// of pixels the fp32 tier flags): the axis as sign(dd) V/|V| and Rodrigues as
// m' cos t + (V x m') sin t/|V| -- the identities the fp32 tier uses -- then
// RayReLU and the normalise as src/dsine_ops.cpp:150-160 (|v| = 1).  Returns
// false, leaving the outputs unset, for a neighbour outside the form's
// domain: a non-unit or non-finite source normal, an xy pair outside
// [kMinXY2, kMaxXY2], |t| > 3.2, |dd| < kDdClampRef, a degenerate V, or a
// non-finite prob or ray; the caller then runs the reference-order body.
// ir = 1/max(|r|, 1e-8); pinv as nbr_ref_f64's.
__device__ __forceinline__ bool nbr_red_f64(float mxf, float myf, float mzf, int sx, int sy,
                                            float xsf, float ysf, float tf, float wf, double rx,
                                            double ry, double rz, double ir, const AngmfArgs& a,
                                            double& ox, double& oy, double& oz, double& pinv) {
    const double mx = mxf, my = myf, mz = mzf, xs = xsf, ys = ysf, t = tf;
    const double m2 = fma(mx, mx, fma(my, my, mz * mz));
    const double s = fma(xs, xs, ys * ys);
    if (!(fabs(m2 - 1.0) <= (double)kUnitM2) || !(s >= (double)kMinXY2) ||
        !(s <= (double)kMaxXY2) || !(fabs(t) <= 3.2) || !isfinite(wf) || !isfinite(rx) ||
        !isfinite(ry) || !isfinite(rz))
        return false;
    const double tu0 = fma((double)sx, a.ifu64, a.tu_c);
    const double tv0 = fma((double)sy, a.ifv64, a.tv_c);
    const double g = fma(tu0, mx, fma(tv0, my, mz));
    const double q = fma(xs * a.ifu64, mx, ys * a.ifv64 * my);
    const double dd = fma(q, rsq64(s), g);
    if (!(fabs(dd) >= kDdClampRef)) return false;
    const double Vx = fma(g * a.ifu64, xs, -q * tu0);
    const double Vy = fma(g * a.ifv64, ys, -q * tv0);
    const double Vz = -q;
    const double n2 = fma(Vx, Vx, fma(Vy, Vy, Vz * Vz));
    if (!(n2 >= 1e-280)) return false;
    double st, ct;
    sincos_small64(t, st, ct);
    const double im = rsq64(m2);
    const double S = st * copysign(rsq64(n2), dd) * im, C = ct * im;
    const double vx = fma(fma(Vy, mz, -Vz * my), S, mx * C);
    const double vy = fma(fma(Vz, mx, -Vx * mz), S, my * C);
    const double vz = fma(fma(Vx, my, -Vy * mx), S, mz * C);
    const double cs = fma(vx, rx, fma(vy, ry, vz * rz)) * ir;
    const double dcoef = (smax(cs - (double)kRayEpsF, 0.0) + (double)kRayEpsF) - cs;
    const double px = fma(rx, dcoef, vx), py = fma(ry, dcoef, vy), pz = fma(rz, dcoef, vz);
    const double p2 = fma(px, px, fma(py, py, pz * pz));
    pinv = (p2 < 1e-24) ? 1e12 : rsq64(p2);
    ox = px * pinv;
    oy = py * pinv;
    oz = pz * pinv;
    return true;
}

// One DPP move of a double (two 32-bit halves); rows outside row_mask keep
// 0.  The data-parallel primitives move within the VALU, with no LDS round
// trip (ds_bpermute, which __shfl_xor uses, costs one per step).
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ double dpp_f64(double v) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)u, CTRL, ROWS, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), CTRL, ROWS, 0xf, false);
    return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

// Sum of v over each LP-lane slot of the wave (LP = 32: lanes 0-31 and 32-63;
// LP = 64: the wave), left in the slot's last lane (31, 63; 63); the other
// lanes hold partial sums.  Each 16-lane row is summed in place by two quad
// permutations and the half-row and row mirrors; then row_bcast15 adds row 0's
// sum into row 1 and row 2's into row 3 (rows 0 and 2 unchanged), and, with
// LP = 64, row_bcast31 adds lane 31's (rows 0 + 1) into row 3.
template <int LP>
__device__ __forceinline__ double slot_sum(double v) {
    v += dpp_f64<0xb1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_f64<0x4e>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_f64<0x141>(v);  // row_half_mirror: lane i of 8 from lane 7 - i
    v += dpp_f64<0x140>(v);  // row_mirror: lane i of 16 from lane 15 - i
    v += dpp_f64<0x142, 0xa>(v);  // row_bcast15 into rows 1 and 3
    if constexpr (LP == 64) v += dpp_f64<0x143, 0x8>(v);  // row_bcast31 into row 3
    return v;
}

// LDS-space (address space 3) views of the halo records: 32-bit addresses
typedef __attribute__((address_space(3))) const char lds_byte;
typedef float lds_f4 __attribute__((ext_vector_type(4)));
typedef double lds_d2 __attribute__((ext_vector_type(2)));

// The source-normal halo of a tile in LDS: one 80-byte record per source
// pixel of the tile's replicate-padded window, read with one address per
// neighbour and immediate offsets (the 80-byte stride leaves consecutive
// lanes' ds_read_b128 free of bank conflicts, where 64 bytes would not).
// With m the raw normal, m' = m/|m|, P0 = (tu0, tv0, 1) the source pixel's
// ray at depth 1 and g = P0.m, the rotation's cross product
// for a neighbour with raw xy pair (xs, ys) and q = xs mx/fu + ys my/fv is
//   c = V x m' = g (D x m') - q (P0 x m'),   D = (xs/fu, ys/fv, 0),
// i.e. c = xs e1 + ys e2 - q f with the per-source vectors
//   e1 = g/fu (ex x m') = (0, -g m'z/fu, g m'y/fu),
//   e2 = g/fv (ey x m') = (g m'z/fv, 0, -g m'x/fv),   f = P0 x m'.
struct alignas(16) HaloRec {
    float4 m;    // m'x, m'y, m'z, g (g NaN unless m is a unit normal)
    double2 ab;  // mx/fu, my/fv: q is formed in double, since it cancels where the
                 // xy pair is nearly perpendicular to m
    float4 e;    // e1.y, e1.z, e2.x, e2.z
    float4 f;    // f = P0 x m', 0
    float4 pad;
};

// The record of source pixel (sy, sx) for its halo slot `rec`.
__device__ __forceinline__ void stage_halo(float mx, float my, float mz, int sx, int sy,
                                           const AngmfArgs& a, HaloRec& rec) {
    const double tu0 = fma((double)sx, a.ifu64, a.tu_c);
    const double tv0 = fma((double)sy, a.ifv64, a.tv_c);
    // 1/|m| as 1.5 - |m|^2/2: exact to 1e-10 for the accepted | |m|^2 - 1 | <= 1e-5
    const float m2 = fmaf(mx, mx, fmaf(my, my, mz * mz));
    const float im = fmaf(-0.5f, m2, 1.5f);
    const float px = mx * im, py = my * im, pz = mz * im;
    const double g0 = fma(tu0, (double)mx, fma(tv0, (double)my, (double)mz));
    const double g = (fabsf(m2 - 1.0f) <= kUnitM2) ? g0 : __builtin_nan("");
    const float gu = (float)(g * a.ifu64), gv = (float)(g * a.ifv64);
    const float tu = (float)tu0, tv = (float)tv0;
    rec.m = make_float4(px, py, pz, (float)g);
    rec.ab = make_double2((double)mx * a.ifu64, (double)my * a.ifv64);
    rec.e = make_float4(-gu * pz, gu * py, gv * pz, -gv * px);
    rec.f = make_float4(fmaf(tv, pz, -py), fmaf(-tu, pz, px), fmaf(tu, py, -(tv * px)), 0.0f);
}

// Waves per 64-pixel group (G, chosen per launch): the group's K*K
// neighbours are split into G near-equal runs of consecutive neighbours
// (row-major over the window), one run per wave.  Workgroups hold kWgWaves = 8
// waves (8/G groups): the SPI places a workgroup of n waves only where every
// SIMD has ceil(n/4) free slots and spreads 8 waves exactly 2 per SIMD, so
// every SIMD carries the same work.  A wave keeps at most lookahead(K, G)
// neighbours' planes in flight, issuing the next neighbour's loads as it
// finishes one.
constexpr int kWgWaves = 8;
// Measured best: at k <= 5, 2 with G = 4 (a 256 x 256 call in one round of
// waves wants each wave's first neighbours' data first: 8.41 against 8.46-8.50
// us with 3, 9.8 with 1) and 3 with G = 2 or 8 (32 x 60 x 80: 17.7-18.4 us
// against 19.7 with 2); 7 at k >= 7 (many rounds); 5 with G = 1 (large
// launches, every wave runs the whole window; 2 to 6 measured on 4 x 512 x 512
// at k = 7).
__host__ __device__ constexpr int lookahead(int K, int G) {
    return G == 1 ? 5 : (K <= 5 ? (G == 4 ? 2 : 3) : 7);
}

// Neighbours whose planes a wave loads before the halo staging and its
// barrier; the rest are loaded after it.
// Measured best: at k <= 5, 1 with G = 2 or 4 and 2 with G = 8 (the small
// launches, latency-bound: 60 x 80 4.03 against 4.14 us cold, 128 x 128
// 4.04-4.06 against 4.08-4.09; 3 or 4 slower); at k >= 7 all of the
// lookahead (7), which overlaps the halo's staging with the first
// neighbours' loads; 3 with G = 1.
__host__ __device__ constexpr int preloads(int K, int G) {
    return G == 1 ? 3 : (K <= 5 ? (G == 8 ? 2 : 1) : 7);
}

// Source-normal halo records of a TW x TH tile.
__host__ __device__ inline int halo_count(int K, int TW, int TH) {
    return (TW + 2 * (K / 2)) * (TH + 2 * (K / 2));
}

// LDS records reserved for the halo: one spare.
__host__ __device__ inline int halo_slots(int K, int TW, int TH) { return halo_count(K, TW, TH) + 1; }

// LDS of the fp32 kernel, in 16-byte units:
//   part[G][64*M]      per-wave fp32 partial (acc.xyz, sum wi^2 or NaN); none
//                      when G = 1
//   halo[nhalo + 1]    source-pixel records (HaloRec, 5 units) + a spare
//   rayl[64*M]         each tile pixel's ray, when formed from the intrinsics
__host__ __device__ inline int lds_units(int K, int G, int M, int TW, int TH, bool synth_ray) {
    return (G > 1 ? G * 64 * M : 0) + 5 * halo_slots(K, TW, TH) + (synth_ray ? 64 * M : 0);
}

// TW (< 2^11), TH (< 2^11) and M (< 2^5) of the fp32 kernel's tile and the
// shift L (< 2^5) of the tiles_x magic number, packed into one kernel argument.
__host__ __device__ inline unsigned pack_tile(int TW, int TH, int M, int L) {
    return (unsigned)TW | ((unsigned)TH << 11) | ((unsigned)M << 22) | ((unsigned)L << 27);
}

// sin t and cos t for |t| <= 3.2 from the hardware sine and cosine (their
// argument in revolutions; within 1.26e-7 of sin(2 pi a), cos(2 pi a) for
// |a| <= 0.51, measured over every float argument): a = t/(2 pi) rounded to
// fp32, e = t - 2 pi a (exactly enough, from a two-word 2 pi), then the
// first-order correction sin(2 pi a + e) = s + e c, cos(2 pi a + e) = c - e s.
constexpr float kInv2Pi = 0.159154943091895335768883763f;
constexpr float k2PiHi = 6.28318548202514648438f;    // 2 pi rounded to float
constexpr float k2PiLo = -1.74845553146951715e-07f;  // 2 pi - k2PiHi
__device__ __forceinline__ void sincos_hw(float t, float& st, float& ct) {
    const float a = t * kInv2Pi;
    const float s = __builtin_amdgcn_sinf(a), c = __builtin_amdgcn_cosf(a);
    const float e = fmaf(-a, k2PiLo, fmaf(-a, k2PiHi, t));
    st = fmaf(e, c, s);
    ct = fmaf(-e, s, c);
}

// One workgroup = M groups of 64 output pixels (a TW x TH tile of sample
// blockIdx.y) x G waves; wave gi * G + r evaluates one run of the window's
// neighbours for the 64 pixels of group gi, one pixel per lane.  The runs'
// roles rotate with gi so the longer run falls on a different SIMD in each
// group.  Each lane loads its run's 4 planes per neighbour in the order it
// consumes them; the source-pixel records come from the tile's halo in LDS;
// the G partials of a pixel meet in LDS, where wave r = 0 of the group sums
// them, writes the pixel, and recomputes the pixels it flags on its own.
//
// Three tiers of arithmetic:
//   1. every pixel (this wave's run, one neighbour per iteration):
//      q = xs mx/fu + ys my/fv in double, rounded once; dd, c, |c|, sin/cos,
//      the rotation, RayReLU, the weight prob/|p| and the partial sums in
//      fp32.  A pixel is flagged when a neighbour leaves the domain (xy
//      range, |t| > 3.2, |dd| < dd_min, a non-unit source normal,
//      |c|^2 < kMinV2, anything non-finite) or when |acc|^2 < kAccRatio2[K] *
//      sum(wi^2);
//   2. flagged pixels, the same reduced form in double (nbr_red_f64), one
//      neighbour per lane of the flagging wave; a pixel with a neighbour
//      outside the double form's domain, or whose double sum still nearly
//      cancels, goes on to
//   3. the reference-order body (nbr_ref_f64) for all its neighbours.
//
// Everything the first loads' addresses depend on comes first in the
// argument list, as scalars: gfx950 preloads up to 14 dwords of kernel
// arguments into SGPRs at wave launch (built with
// -amdgpu-kernarg-preload-count), so a workgroup issues its loads without
// first waiting for a scalar load of its arguments.  The prologue keeps
// scalar work short: no runtime integer division (the tile row comes from a
// host-computed magic number, the wave's group from a constant divisor) and
// one buffer descriptor per input tensor, its planes reached through the
// scalar offset.
template <int K, int G, bool SR, bool LG, bool NT>
__global__ __launch_bounds__(64 * kWgWaves) __attribute__((amdgpu_waves_per_eu(4)))
void angmf_f32_kernel(const float* __restrict__ pred_norm, const float* __restrict__ xy,
                      const float* __restrict__ angle, const float* __restrict__ prob, int W,
                      int H, unsigned tile, int tiles_per_img, int tiles_x, unsigned tx_magic,
                      AngmfArgs a) {
    constexpr int P = K / 2, K2 = K * K;
    constexpr int RUN = K2 / G, REM = K2 % G;  // run lengths RUN + 1 (REM runs) and RUN
    constexpr int NR = RUN + (REM ? 1 : 0);    // longest run
    constexpr int LA = lookahead(K, G) < NR ? lookahead(K, G) : NR;  // neighbours in flight
    // planes held in registers: one slot per neighbour of the run (G > 1,
    // loop fully unrolled), or a ring of LA slots (G = 1, rolled loop)
    constexpr int SL = (G == 1) ? LA : NR;
    extern __shared__ float4 smem[];
    // a tile width of 0 marks a range tile: 64 M consecutive pixels of the
    // row-major image, its halo the full-width rows they span (TH of them at
    // most) and P more on each side
    const bool range = (tile & 0x7ffu) == 0u;
    const int TW = range ? W : (int)(tile & 0x7ffu), TH = (int)((tile >> 11) & 0x7ffu);
    const int M = (int)((tile >> 22) & 0x1fu), LX = (int)(tile >> 27);
    const int npx = 64 * M;
    const int nrow = TH + 2 * P;
    float4* part = smem;
    const int hw = TW + 2 * P, nhalo = hw * nrow;
    const int nslot = nhalo + 1;
    HaloRec* hl = reinterpret_cast<HaloRec*>(part + (G > 1 ? G * npx : 0));
    // (SR) the tile pixels' rays, after the halo
    float4* rayl = reinterpret_cast<float4*>(hl + nslot);

    const int b = blockIdx.y;
    const int lb = xcd_remap(blockIdx.x, tiles_per_img);
    // the tile's first row and column, and (range tiles) its first pixel;
    // tx_magic and LX divide by tiles_x (rectangular tiles) or W (ranges)
    int ty0, tx0, p0 = 0;
    if (range) {
        p0 = lb * npx;
        ty0 = magic_div(p0, tx_magic, LX);
        tx0 = 0;
    } else {
        const int tyi = magic_div(lb, tx_magic, LX);
        ty0 = tyi * TH;
        tx0 = (lb - tyi * tiles_x) * TW;
    }
    const float rtw = __builtin_amdgcn_rcpf((float)TW);
    // image row and column of the tile's pixel jj (0 <= jj < 64 M)
    auto tile_px = [&](int jj, int& yy, int& xx) {
        if (range) {
            const int pp = p0 + jj;
            yy = magic_div(pp, tx_magic, LX);
            xx = pp - yy * W;
        } else {
            const int t = small_div(jj, rtw);
            yy = ty0 + t;
            xx = tx0 + (jj - t * TW);
        }
    };
    const long long HW = (long long)H * W;
    const uint32_t HW4 = (uint32_t)HW * 4u;  // plane bytes; max(NR, 3) * HW4 < 2^32

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int gi = wave / G;
    const int r = wave - gi * G;
    const int role = (r + gi) % G;
    const int n0 = role * RUN + (role < REM ? role : REM);  // first neighbour of the run
    const int nrun = RUN + (role < REM ? 1 : 0);
    const int j = gi * 64 + lane;
    int y, x;
    tile_px(j, y, x);
    const int ty = y - ty0, tx = x - tx0;
    const bool valid = (ty < TH) && (y < H) && (x < W);
    const uint32_t pb = valid ? (uint32_t)(y * W + x) * 4u : 0u;

    // ---- staging: the tile's source normals, with what depends on them only
    // The (TH + 2P) x (TW + 2P) replicate-padded halo of pred_norm, one LDS
    // record pair per source pixel, at most two per thread.  Their loads are
    // each lane's first, so waiting for them waits for nothing else.
    const int nthr = 64 * M * G;
    const float rhw = __builtin_amdgcn_rcpf((float)hw);
    const __amdgpu_buffer_rsrc_t rpn =
        plane_rsrc(at_plane(pred_norm, (uint32_t)b * 3u, HW4), 3u * HW4);
    float hm[3];
    // threads past the halo write the spare record, from clamped coordinates
    const int h0 = min((int)threadIdx.x, nhalo);
    const int hr0 = small_div(h0, rhw), hc0 = h0 - hr0 * hw;
    const int hsy0 = clampi(ty0 - P + hr0, 0, H - 1), hsx0 = clampi(tx0 - P + hc0, 0, W - 1);
    {
        const uint32_t hb = (uint32_t)(hsy0 * W + hsx0) * 4u;
        hm[0] = ldbs(rpn, hb, 0u);
        hm[1] = ldbs(rpn, hb, HW4);
        hm[2] = ldbs(rpn, hb, 2u * HW4);
    }
    // keep the halo loads ahead of the plane loads in the instruction stream
    __builtin_amdgcn_sched_barrier(0);

    // ---- phase A: this wave's run of neighbours for this lane's pixel ------
    // Every lane runs it (lanes past the tile use clamped, in-bounds
    // addresses and discard the result).
    // Loads in consumption order: ray, then per neighbour its 4 planes, at
    // most LA neighbours ahead of the one being evaluated; the planes of the
    // first PRE neighbours go out before the staging.  Vector loads
    // complete in issue order, so the loop consumes them one neighbour at a
    // time: a scheduling barrier after each neighbour's loads keeps them in
    // that order, and the loop's register fences keep the compiler from
    // hoisting one neighbour's arithmetic ahead of the previous one's.
    float rxf, ryf, rzf;
    if constexpr (!SR) {
        const __amdgpu_buffer_rsrc_t rry =
            plane_rsrc(a.ray + (size_t)b * a.ray_bstride, 3u * HW4);
        rxf = ldbs(rry, pb, 0u);
        ryf = ldbs(rry, pb, HW4);
        rzf = ldbs(rry, pb, 2u * HW4);
    }
    float xs[SL], ys[SL], th[SL], wt[SL];
    // planes (sample b, neighbour n0 + i) of each input: one descriptor per
    // tensor at i = 0, plane i at scalar offset i * HW4, into register slot s.
    // A run one shorter than NR re-reads its first planes in the last slot,
    // unused.
    const uint32_t pxy = (uint32_t)b * (2u * K2) + (uint32_t)n0;
    const uint32_t pk = (uint32_t)b * K2 + (uint32_t)n0;
    const uint32_t span = (uint32_t)nrun * HW4;
    const __amdgpu_buffer_rsrc_t rxs = plane_rsrc(at_plane(xy, pxy, HW4), span);
    const __amdgpu_buffer_rsrc_t rys = plane_rsrc(at_plane(xy, pxy + K2, HW4), span);
    const __amdgpu_buffer_rsrc_t rth = plane_rsrc(at_plane(angle, pk, HW4), span);
    const __amdgpu_buffer_rsrc_t rwt = plane_rsrc(at_plane(prob, pk, HW4), span);
    auto load_planes = [&](int i, int sl) {
        const uint32_t so = (i < NR - 1 || nrun == NR) ? (uint32_t)i * HW4 : 0u;
        if constexpr (NT) {
            xs[sl] = ldbs_nt(rxs, pb, so);
            ys[sl] = ldbs_nt(rys, pb, so);
            th[sl] = ldbs_nt(rth, pb, so);
            wt[sl] = ldbs_nt(rwt, pb, so);
        } else {
            xs[sl] = ldbs(rxs, pb, so);
            ys[sl] = ldbs(rys, pb, so);
            th[sl] = ldbs(rth, pb, so);
            wt[sl] = ldbs(rwt, pb, so);
        }
    };
    constexpr int PRE = preloads(K, G) < LA ? preloads(K, G) : LA;
#pragma unroll
    for (int i = 0; i < PRE; ++i) {
        load_planes(i, i);
        __builtin_amdgcn_sched_barrier(0);
    }
    // Threads past the halo write a spare record: an unconditional use keeps
    // the compiler from sinking the halo loads behind the plane loads.
    stage_halo(hm[0], hm[1], hm[2], hsx0, hsy0, a, hl[h0]);
    // A second record per thread (k >= 7, and narrow tiles): loaded here,
    // behind the plane loads, which it then waits for.
    if (nhalo > nthr) {
        const int h = threadIdx.x + nthr;
        if (h < nhalo) {
            const int hr = small_div(h, rhw), hc = h - hr * hw;
            const int sy = clampi(ty0 - P + hr, 0, H - 1), sx = clampi(tx0 - P + hc, 0, W - 1);
            const uint32_t hb = (uint32_t)(sy * W + sx) * 4u;
            stage_halo(ldbs(rpn, hb, 0u), ldbs(rpn, hb, HW4), ldbs(rpn, hb, 2u * HW4), sx, sy, a,
                       hl[h]);
        }
    }
    if constexpr (SR) {
        // each tile pixel's ray, once (pixels past the image: clamped ones)
        if ((int)threadIdx.x < npx) {
            const int t = threadIdx.x;
            int ry, rx;
            tile_px(t, ry, rx);
            const bvml::Ray3f r3 = synth_ray(min(rx, W - 1), min(ry, H - 1), a.fu, a.cu, a.fv,
                                             a.cv);
            rayl[t] = make_float4(r3.x, r3.y, r3.z, 0.0f);
        }
    }
    __syncthreads();
    if constexpr (SR) {
        const float4 r4 = rayl[j];
        rxf = r4.x;
        ryf = r4.y;
        rzf = r4.z;
    }
#pragma unroll
    for (int i = PRE; i < LA; ++i) {
        load_planes(i, i);
        __builtin_amdgcn_sched_barrier(0);
    }
    float4 mine;  // this wave's partial of its pixel
    {
        // cos(v', r) = v'.r / max(|v'||r|, 1e-8) with |v'| = 1.  1/|r| from the
        // hardware rsq and one Newton step: r-hat is shared by all the
        // pixel's neighbours, so its error would not average out over them.
        const float r2 = fmaf(rxf, rxf, fmaf(ryf, ryf, rzf * rzf));
        const float ir0 = __builtin_amdgcn_rsqf(r2);
        const float ir1 = fmaf(0.5f * ir0, fmaf(-r2 * ir0, ir0, 1.0f), ir0);
        const float ir = (r2 < 1e-16f) ? 1e8f : ir1;
        // -r-hat/2 and 2r: the RayReLU shift dc = max(eps - cos, 0) is formed as
        // 2 clamp(eps/2 - v'.r-hat/2) in the dot product's last fma (the
        // clamp's upper bound, 1, is above (eps + 1)/2)
        const float nhx = -0.5f * (rxf * ir), nhy = -0.5f * (ryf * ir), nhz = -0.5f * (rzf * ir);
        const float r2x = 2.0f * rxf, r2y = 2.0f * ryf, r2z = 2.0f * rzf;
        const float dd_min = (float)a.dd_min;
        // this lane's window in the halo (lanes past the tile use its last row)
        const int hrow = (ty < TH) ? ty : TH - 1;
        // (LDS-space pointers: 32-bit record addresses)
        const lds_byte* hbase = (const lds_byte*)reinterpret_cast<const char*>(hl + hrow * hw + tx);
        float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f;
        float qs = 0.0f;  // sum of wi^2, for the cancellation test only
        // the fp32 form's domain over the run, as running extremes: bits of
        // |xy|^2 above kMinXY2, |t|, |dd| and |c|^2.  A NaN drops out of a
        // min or max but not out of the sums: every NaN these would see
        // reaches acc (through q, c, sin/cos or the weight), which phase B
        // flags.
        uint32_t smx = 0u;
        float tmax = 0.0f, ddmin = __builtin_inff(), n2min = __builtin_inff();
        // one neighbour n of the window, its planes' values given: the
        // record offsets come from n in scalar registers, added once each
        // (the compiler would otherwise fold them into a 64-bit
        // multiply-add per neighbour)
        auto eval = [&](int n, float xv, float yv, float thv, float wtv) {
            const int ky = n / K, kx = n - ky * K;
            int roff = (ky * hw + kx) * (int)sizeof(HaloRec);
            asm("" : "+s"(roff));
            const lds_byte* rb = hbase + roff;
            const lds_f4 hm4 = *(const __attribute__((address_space(3))) lds_f4*)rb;
            const lds_d2 ab2 = *(const __attribute__((address_space(3))) lds_d2*)(rb + 16);
            const lds_f4 e4 = *(const __attribute__((address_space(3))) lds_f4*)(rb + 32);
            const lds_f4 f4 = *(const __attribute__((address_space(3))) lds_f4*)(rb + 48);
            const float t = LG ? sigmoid_f32(thv) * kPiF : thv;
            // q in double (exact products, one rounding), the rest fp32;
            // dd = g + q/|xy| is formed from the raw normal as the reference
            // forms it, with 1/|xy| from the fp32 |xy|^2 and rsq (dd_min
            // covers their error)
            const float q = (float)fma((double)xv, ab2.x, (double)yv * ab2.y);
            const float s = fmaf(xv, xv, yv * yv);
            const float dd = fmaf(q, __builtin_amdgcn_rsqf(s), hm4.w);
            // c = V x m' = xs e1 + ys e2 - q f;  v' = m' cos t + c sign(dd) sin t/|c|
            const float cx = fmaf(yv, e4.z, -q * f4.x);
            const float cy = fmaf(xv, e4.x, -q * f4.y);
            const float cz = fmaf(xv, e4.y, fmaf(yv, e4.w, -q * f4.z));
            const float n2 = fmaf(cx, cx, fmaf(cy, cy, cz * cz));
            smx = max(smx, __builtin_bit_cast(uint32_t, s) - kXY2Lo);
            tmax = fmaxf(tmax, fabsf(t));
            ddmin = fminf(ddmin, fabsf(dd));
            n2min = fminf(n2min, n2);
            float st, ct;
            sincos_hw(t, st, ct);
            const float S = st * copysignf(__builtin_amdgcn_rsqf(n2), dd);
            const float vx = fmaf(cx, S, hm4.x * ct);
            const float vy = fmaf(cy, S, hm4.y * ct);
            const float vz = fmaf(cz, S, hm4.z * ct);
            // RayReLU: p = v' + r max(eps - cos, 0) = v' + 2r h, h = clamp(eps/2 - cos/2),
            // then the weight prob/|p|
            const float h = __builtin_amdgcn_fmed3f(
                fmaf(vz, nhz, fmaf(vy, nhy, fmaf(vx, nhx, 0.5f * kRayEpsF))), 0.0f, 1.0f);
            const float px = fmaf(r2x, h, vx), py = fmaf(r2y, h, vy), pz = fmaf(r2z, h, vz);
            // wi = prob / |p|; with logits prob = 1/d, d = 1 + exp(-L), and
            // wi = rsq(|p|^2 d^2) (d = inf: exactly 0)
            const float p2 = fmaf(px, px, fmaf(py, py, pz * pz));
            float wi;
            if constexpr (LG) {
                const float d = one_plus_exp_neg(wtv);
                wi = __builtin_amdgcn_rsqf(p2 * d * d);
            } else {
                wi = wtv * __builtin_amdgcn_rsqf(p2);
            }
            acc0 = fmaf(px, wi, acc0);
            acc1 = fmaf(py, wi, acc1);
            acc2 = fmaf(pz, wi, acc2);
            qs = fmaf(wi, wi, qs);
            // this neighbour done before the next one's data are waited for
            asm volatile("" : "+v"(acc0), "+v"(acc1), "+v"(acc2), "+v"(qs));
        };
        if constexpr (G > 1) {
            // this wave's run, fully unrolled: slot i holds neighbour n0 + i
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                // this neighbour's planes: the fence makes the wait for them
                // the first use (and keeps the last slot's loads out of its
                // branch)
                asm volatile("" : "+v"(xs[i]), "+v"(ys[i]), "+v"(th[i]), "+v"(wt[i]));
                if (i == NR - 1 && nrun != NR) break;
                eval(n0 + i, xs[i], ys[i], th[i], wt[i]);
                if (i + LA < NR) {
                    load_planes(i + LA, i + LA);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        } else {
            // the whole window, LA neighbours at a time: neighbour n lives in
            // slot n % LA, and its slot is refilled with neighbour n + LA
            // once it has been evaluated
            for (int nb = 0; nb < K2; nb += LA) {
#pragma unroll
                for (int sl = 0; sl < LA; ++sl) {
                    const int n = nb + sl;
                    if (n >= K2) break;
                    asm volatile("" : "+v"(xs[sl]), "+v"(ys[sl]), "+v"(th[sl]), "+v"(wt[sl]));
                    eval(n, xs[sl], ys[sl], th[sl], wt[sl]);
                    if (n + LA < K2) {
                        load_planes(n + LA, sl);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
        }
        const bool bad = (smx > kXY2Span) | !(tmax <= 3.2f) | !(ddmin >= dd_min) |
                         !(n2min >= kMinV2);
        mine = make_float4(acc0, acc1, acc2, bad ? __builtin_nanf("") : qs);
        if constexpr (G > 1) part[r * npx + j] = mine;
    }
    if constexpr (G > 1) __syncthreads();

    // ---- phase B: wave r = 0 of each group reduces the G runs, writes the
    // unflagged pixels and recomputes the flagged ones by itself; the other
    // waves are done (no barrier follows).
    if (r != 0) return;
    bool flag = false;
    if (valid) {
        const float4 t0 = (G > 1) ? part[j] : mine;
        double s0 = t0.x, s1 = t0.y, s2 = t0.z, sw = t0.w;
#pragma unroll
        for (int rr = 1; rr < G; ++rr) {
            const float4 t = part[rr * npx + j];
            s0 += t.x;
            s1 += t.y;
            s2 += t.z;
            sw += t.w;
        }
        const double a2 = fma(s0, s0, fma(s1, s1, s2 * s2));
        // 1 / max(|acc|, 1e-12) as the reference; a non-finite or
        // cancelled sum goes to the recompute
        flag = !(a2 >= kAccRatio2[K] * sw) || !(a2 <= 1e300);
        if (!flag) {
            const double inv = (a2 < 1e-24) ? 1e12 : rsq64_1(a2);
            float* op = a.out + (size_t)b * 3 * HW;
            stf(op, pb, (float)(s0 * inv));
            stf(op + HW, pb, (float)(s1 * inv));
            stf(op + 2 * HW, pb, (float)(s2 * inv));
        }
    }
    unsigned long long fm = __ballot(flag);
    if (fm == 0) return;

    // ---- phase C: the group's flagged pixels, tier 2 then tier 3 ----------
    // LP lanes per pixel, one neighbour per lane at a time; inputs are
    // re-read (the workgroup has just read them, so mostly from L2).
    constexpr int LP = (K2 > 32) ? 64 : 32;
    constexpr int PPP = 64 / LP;
    const int slot = lane / LP, il = lane - slot * LP;
    const bool lead = il == LP - 1;  // the lane slot_sum leaves a slot's sums in
    const float* pn = pred_norm + (size_t)b * 3 * HW;
    const float* pr = prob + (size_t)b * K2 * HW;
    const float* xyp = xy + (size_t)b * 2 * K2 * HW;
    const float* ap = angle + (size_t)b * K2 * HW;
    const float* rp = SR ? nullptr : a.ray + (size_t)b * a.ray_bstride;
    float* op = a.out + (size_t)b * 3 * HW;
    while (fm) {
        int src = -1;
#pragma unroll
        for (int sidx = 0; sidx < PPP; ++sidx) {
            const int bitpos = fm ? __ffsll((long long)fm) - 1 : -1;
            if (fm) fm &= fm - 1;
            if (sidx == slot) src = bitpos;
        }
        const bool act = src >= 0;
        const int jj = gi * 64 + (act ? src : 0);
        int fy, fx;
        tile_px(jj, fy, fx);
        const uint32_t fb = (uint32_t)(fy * W + fx) * 4u;
        // one tier over this lane's neighbours of its pixel; returns false
        // (tier 2) when a neighbour is outside the reduced form's domain
        auto tier = [&](auto tier_tag, double& p0, double& p1, double& p2, double& q2) {
            constexpr int TIER = decltype(tier_tag)::value;
            p0 = p1 = p2 = q2 = 0.0;
            if (!act) return;
#pragma unroll 1
            for (int n = il; n < K2; n += LP) {
                const int ky = n / K, kx = n - ky * K;
                const int fsy = clampi(fy - P + ky, 0, H - 1);
                const int fsx = clampi(fx - P + kx, 0, W - 1);
                const uint32_t sb = (uint32_t)(fsy * W + fsx) * 4u;
                // the pixel's ray with the neighbour's inputs: every load of
                // the neighbour in one round trip (loaded before the loop,
                // the ray would be waited for on its own)
                float frx, fry, frz;
                if constexpr (SR) {
                    const bvml::Ray3f rr3 = synth_ray(fx, fy, a.fu, a.cu, a.fv, a.cv);
                    frx = rr3.x;
                    fry = rr3.y;
                    frz = rr3.z;
                } else {
                    frx = ldf(rp, fb);
                    fry = ldf(rp + HW, fb);
                    frz = ldf(rp + 2 * HW, fb);
                }
                const float mx = ldf(pn, sb), my = ldf(pn + HW, sb), mz = ldf(pn + 2 * HW, sb);
                const float xsv = ldf(xyp + (size_t)n * HW, fb);
                const float ysv = ldf(xyp + (size_t)(K2 + n) * HW, fb);
                float thv = ldf(ap + (size_t)n * HW, fb), wv = ldf(pr + (size_t)n * HW, fb);
                // (no use of a loaded value moves above the last load)
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (LG) {
                    thv = angle_ref(thv);
                    wv = sigmoid_ref(wv);
                }
                double ox, oy, oz, pinv;
                if constexpr (TIER == 2) {
                    const double rxd = frx, ryd = fry, rzd = frz;
                    // 1 / max(|r|, 1e-8) from the reciprocal square root
                    // (two Newton steps) rather than a square root and a
                    // division, whose long sequences sit on the flagged
                    // group's path (256 x 256 at k = 5: 8.34 against 8.47 us
                    // per call, same bits); |r|^2 of float components stays
                    // finite in double, and NaN rays go to tier 3 below
                    const double r2d = fma(rxd, rxd, fma(ryd, ryd, rzd * rzd));
                    const double ird = (r2d < 1e-16) ? 1e8 : rsq64(r2d);
                    if (!nbr_red_f64(mx, my, mz, fsx, fsy, xsv, ysv, thv, wv, rxd, ryd, rzd, ird,
                                     a, ox, oy, oz, pinv)) {
                        q2 = __builtin_nan("");
                        continue;
                    }
                } else {
                    nbr_ref_f64(mx, my, mz, fsx + 0.5, fsy + 0.5, xsv, ysv, thv, frx, fry, frz,
                                a.fu, a.cu, a.fv, a.cv, ox, oy, oz, pinv);
                }
                const double w = wv;
                p0 += w * ox;
                p1 += w * oy;
                p2 += w * oz;
                const double wi = w * pinv;
                q2 = fma(wi, wi, q2);
            }
            p0 = slot_sum<LP>(p0);
            p1 = slot_sum<LP>(p1);
            p2 = slot_sum<LP>(p2);
            q2 = slot_sum<LP>(q2);
        };
        // 1 / max(|acc|, 1e-12), with the reference's NaN and Inf results
        auto write = [&](double a0, double a1, double a2) {
            const double n2 = a0 * a0 + a1 * a1 + a2 * a2;
            const double inv = (n2 < 1e-24) ? 1e12 : (n2 == INFINITY ? 0.0 : rsq64(n2));
            stf(op, fb, (float)(a0 * inv));
            stf(op + HW, fb, (float)(a1 * inv));
            stf(op + 2 * HW, fb, (float)(a2 * inv));
        };
        bool need3;
        {
            double a0, a1, a2, aq;
            tier(std::integral_constant<int, 2>{}, a0, a1, a2, aq);
            const double n2 = a0 * a0 + a1 * a1 + a2 * a2;
            // tier 2 hands on a pixel with a neighbour outside its domain
            // (aq NaN) or a sum that nearly cancels
            need3 = act && lead &&
                    (!(n2 >= kAccRatio2Ref * aq) || !(n2 >= kAcc2Floor) || !(n2 <= 1e300));
            if (act && lead && !need3) write(a0, a1, a2);
        }
        if (__ballot(need3)) {
            double a0, a1, a2, aq;
            tier(std::integral_constant<int, 3>{}, a0, a1, a2, aq);
            if (need3) write(a0, a1, a2);
        }
    }
}

// ---------------------------------------------------------------------------
// RayReLU: double precision, reference order; memory-bound (36 B/px).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ray_relu_kernel(float* normal, const float* ray,
                                                       long long HW, long long total,
                                                       long long ray_bstride) {
#pragma clang fp contract(off)
    const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    const long long b = gid / HW;
    const long long p = gid - b * HW;
    float* n = normal + b * 3 * HW;
    const float* r = ray + b * ray_bstride;
    double ox, oy, oz, inv;
    ray_relu_ref(n[p], n[HW + p], n[2 * HW + p], r[p], r[HW + p], r[2 * HW + p], ox, oy, oz, inv);
    n[p] = (float)ox;
    n[HW + p] = (float)oy;
    n[2 * HW + p] = (float)oz;
}

// Four consecutive pixels per lane, as float4 loads and stores of each plane
// (H*W and ray_bstride multiples of 4, 16-byte aligned planes): the same
// reference-order arithmetic per pixel, a quarter of the lanes and memory
// instructions.
__global__ __launch_bounds__(256) void ray_relu4_kernel(float* normal, const float* ray,
                                                        long long HW4, long long total4,
                                                        long long ray_bstride4) {
#pragma clang fp contract(off)
    const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total4) return;
    const long long b = gid / HW4;
    const long long p = gid - b * HW4;
    float4* n = reinterpret_cast<float4*>(normal) + b * 3 * HW4;
    const float4* r = reinterpret_cast<const float4*>(ray) + b * ray_bstride4;
    const float4 nx = n[p], ny = n[HW4 + p], nz = n[2 * HW4 + p];
    const float4 rx = r[p], ry = r[HW4 + p], rz = r[2 * HW4 + p];
    float4 ox, oy, oz;
    double x, y, z, inv;
    ray_relu_ref(nx.x, ny.x, nz.x, rx.x, ry.x, rz.x, x, y, z, inv);
    ox.x = (float)x; oy.x = (float)y; oz.x = (float)z;
    ray_relu_ref(nx.y, ny.y, nz.y, rx.y, ry.y, rz.y, x, y, z, inv);
    ox.y = (float)x; oy.y = (float)y; oz.y = (float)z;
    ray_relu_ref(nx.z, ny.z, nz.z, rx.z, ry.z, rz.z, x, y, z, inv);
    ox.z = (float)x; oy.z = (float)y; oz.z = (float)z;
    ray_relu_ref(nx.w, ny.w, nz.w, rx.w, ry.w, rz.w, x, y, z, inv);
    ox.w = (float)x; oy.w = (float)y; oz.w = (float)z;
    n[p] = ox;
    n[HW4 + p] = oy;
    n[2 * HW4 + p] = oz;
}

// ---------------------------------------------------------------------------
// build_ray8: the ray map from the intrinsics, one pixel per thread.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void build_ray8_kernel(float* ray, double fu, double cu,
                                                         double fv, double cv, int H, int W) {
    const long long HW = (long long)H * W;
    const long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= HW) return;
    const int y = (int)(p / W), x = (int)(p - (long long)y * W);
    const bvml::Ray3f r = synth_ray(x, y, fu, cu, fv, cv);
    ray[p] = r.x;
    ray[HW + p] = r.y;
    ray[2 * HW + p] = r.z;
}

// build_uv: the ray map's first two channels before the normalise
// (src/dsine_decoder.cpp:253-256), one pixel per thread.
__global__ __launch_bounds__(256) void build_uv8_kernel(float* uv, double fu, double cu,
                                                        double fv, double cv, int H, int W) {
    const long long HW = (long long)H * W;
    const long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= HW) return;
    const int y = (int)(p / W), x = (int)(p - (long long)y * W);
    uv[p] = (float)(((x + 0.5) - cu) / fu);
    uv[HW + p] = (float)(((y + 0.5) - cv) / fv);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
using bvml::fail;
using bvml::overlaps;

// Samples per launch of the fp32 kernel (its grid's y extent).
constexpr int kMaxGridY = 65535;

// Magic number of d (1 <= d < 2^31) for magic_div: L = ceil(log2 d),
// mag = floor(2^32 (2^L - d) / d) + 1 < 2^32.
void div_magic(int d, unsigned& mag, int& L) {
    L = 0;
    while ((1LL << L) < d) ++L;
    mag = (unsigned)(((1ULL << 32) * ((1ULL << L) - (unsigned long long)d)) /
                         (unsigned long long)d + 1);
}

// The fp32 kernel's instantiation for window K, G waves per group, and the
// ray and logits modes.
template <int K, int G, bool NT = false>
auto angmf_f32_for(bool synth_ray, bool logits) {
    return synth_ray ? (logits ? angmf_f32_kernel<K, G, true, true, NT>
                               : angmf_f32_kernel<K, G, true, false, NT>)
                     : (logits ? angmf_f32_kernel<K, G, false, true, NT>
                               : angmf_f32_kernel<K, G, false, false, NT>);
}

// Candidate G values per window size, in order of preference (the first
// wins ties in lane utilisation, except between range tiles).  Runs longer
// than lookahead(K, G) neighbours keep only that many of them in flight.
//   K = 5: 4 (runs of 6-7) on wide images; 2 (runs of 12-13) on large narrow
//          launches (range tiles of 256 pixels)
//   K = 7: 4 (runs of 12-13; 64 x 2 tiles halve the halo per pixel against 8
//          waves of runs of 6-7 on 64 x 1 tiles)
//   K = 9: 8 (a 64 x 2 tile's halo does not fit 4 waves' LDS share, and
//          narrow images take range tiles, where 8 wins)
constexpr int kGChoices[10][2] = {{0, 0}, {1, 1}, {0, 0}, {2, 2}, {0, 0},
                                  {4, 2}, {0, 0}, {4, 8}, {0, 0}, {8, 8}};

// A G with more waves per group for launches that leave CUs idle (fewer
// workgroups than CUs with the first choice): the shorter runs shorten each
// wave's dependent chain, which is what such a launch waits on.  k = 5 at
// 60 x 80: 4.47 against 5.19 us; 96 x 96: 4.53 against 5.30; 128 x 128: 4.06
// against 4.96; k = 3 at 60 x 80: 5.11 against 5.72; 128 x 128: 5.44 against
// 6.37 (at 256 x 256, 256 workgroups with G = 2, G = 4 is slower).
constexpr int kGSmall[10] = {0, 0, 0, 4, 0, 8, 0, 0, 0, 0};
constexpr long long kIdleGrid = 256;

// Window sizes with a whole-window variant (G = 1: each wave evaluates all
// k*k neighbours of its 64 pixels in a rolled loop, LA at a time, and writes
// them itself; 64 x 8 tiles, no cross-wave reduction).  A launch that fills
// the chip's kWholeWindowSlots resident workgroups (two per CU) at least
// once, and its last round at least kRoundFill of the way, takes it: its HBM
// stream runs faster (fewer halo records per pixel, one barrier per
// workgroup, fewer loads in flight per lane).  Measured against the
// run-split kernel: 512 x 512 at k = 5, 23.4 against 27.7 us; at k = 7, 39.3
// against 46.4; 4 x 256 x 256, 23.7 against 26.8; 600 x 800 (1.46 rounds),
// 42.8 against 48.9; 1030 x 512 (2.02 rounds), 51.9 against 52.9; but
// 2 x 384 x 384 (1.13 rounds), 31.5 against 30.1.  k = 9's 64 x 8 halo
// exceeds two records per thread.
constexpr bool kWholeWindowOk[10] = {false, false, false, false, false,
                                     true,  false, true,  false, false};
constexpr long long kWholeWindowSlots = 512;
constexpr double kRoundFill = 0.6;
// A whole-window launch that moves more than this (the Infinity Cache) reads
// its neighbour planes with the non-temporal policy: nothing it reads is
// found again in the cache anyway, and keeping it out of the way measured
// 4.8% faster on 4 x 512 x 512 at k = 7 (145.5 against 152.8 us).  Smaller
// launches keep the default policy: a call whose inputs the previous kernel
// has just written finds them in the cache (with nt, 512 x 512 at k = 5 read
// from the cache took 40.0 against 35.9 us).
constexpr double kStreamBytes = 256.0 * (1 << 20);

// LDS one workgroup may use: 64 KB for the run-split kernels (G > 1), so
// that two to three of them share a CU; the whole-window kernel's 64 x 8
// tiles and the range tiles of narrow images take up to 80 KB, two per CU
// (gfx950 has 160 KB per CU and allows it all to one workgroup).
constexpr int kMaxLdsBytes = 65536;
constexpr int kMaxLdsBytesG1 = 81920;

// A kernel whose workgroups take more than 64 KB of LDS must be granted it
// (hipFuncSetAttribute) on each device before its launch.  The grant is made
// once per kernel and device (kMaxLdsBytesG1, every whole-window tile's
// ceiling) and remembered here, so that launches after the first make no
// runtime call for it.
struct LdsGrant {
    std::atomic<const void*> fn{nullptr};
    std::atomic<unsigned long long> devices{0};  // bit d: granted on device d (< 64)
};
LdsGrant g_lds_grants[32];

hipError_t grant_lds(const void* fn) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const unsigned long long bit = (dev >= 0 && dev < 64) ? (1ull << dev) : 0ull;
    for (LdsGrant& g : g_lds_grants) {
        const void* cur = g.fn.load(std::memory_order_acquire);
        if (cur == nullptr) {
            const void* none = nullptr;
            cur = g.fn.compare_exchange_strong(none, fn, std::memory_order_acq_rel) ? fn : none;
        }
        if (cur != fn) continue;
        if (bit != 0 && (g.devices.load(std::memory_order_acquire) & bit) != 0) return hipSuccess;
        e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLdsBytesG1);
        if (e == hipSuccess) g.devices.fetch_or(bit, std::memory_order_acq_rel);
        return e;
    }
    // (more kernels than slots: grant on every launch)
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLdsBytesG1);
}

template <int K>
hipError_t launch_angmf(AngmfArgs a, bool fp64, hipStream_t s) {
    if (fp64) {
        const long long total = (long long)a.B * a.HW;
        const long long grid = (total + 255) / 256;
        hipLaunchKernelGGL(angmf_f64_kernel<K>, dim3((unsigned)grid), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    const size_t lds = (size_t)lds_units(K, a.G, a.M, a.TW, a.TH, a.synth_ray != 0) * 16;
    unsigned mag;
    int L;
    div_magic(a.tiles_x, mag, L);
    const unsigned tile = pack_tile(a.range ? 0 : a.TW, a.TH, a.M, L);
    constexpr int G0 = kGChoices[K][0], G1 = kGChoices[K][1];
    auto kern = (a.G == G0) ? angmf_f32_for<K, G0>(a.synth_ray != 0, a.logits != 0)
                            : angmf_f32_for<K, G1>(a.synth_ray != 0, a.logits != 0);
    if constexpr (kGSmall[K] != 0) {
        if (a.G == kGSmall[K]) kern = angmf_f32_for<K, kGSmall[K]>(a.synth_ray != 0, a.logits != 0);
    }
    if constexpr (kWholeWindowOk[K]) {
        if (a.G == 1)
            kern = a.stream_planes ? angmf_f32_for<K, 1, true>(a.synth_ray != 0, a.logits != 0)
                                   : angmf_f32_for<K, 1, false>(a.synth_ray != 0, a.logits != 0);
    }
    // workgroups past 64 KB of LDS (the whole-window tiles) ask for it
    if (lds > 65536) {
        const hipError_t e = grant_lds(reinterpret_cast<const void*>(kern));
        if (e != hipSuccess) return e;
    }
    // one launch per kMaxGridY samples (grid y = sample)
    for (int b0 = 0; b0 < a.B; b0 += kMaxGridY) {
        const int nb = (a.B - b0 < kMaxGridY) ? a.B - b0 : kMaxGridY;
        AngmfArgs c = a;
        c.pn += (size_t)b0 * 3 * a.HW;
        c.pr += (size_t)b0 * K * K * a.HW;
        c.xy += (size_t)b0 * 2 * K * K * a.HW;
        c.ang += (size_t)b0 * K * K * a.HW;
        if (!a.synth_ray) c.ray += (size_t)b0 * a.ray_bstride;
        c.out += (size_t)b0 * 3 * a.HW;
        c.B = nb;
        const dim3 grid((unsigned)a.tiles_per_img, (unsigned)nb), block(64 * a.M * a.G);
        hipLaunchKernelGGL(kern, grid, block, lds, s, c.pn, c.xy, c.ang, c.pr, a.W, a.H, tile,
                           a.tiles_per_img, a.tiles_x, mag, c);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Whether a TW x TH tile of M groups of G waves fits the kernel: its LDS, and
// at most two halo records per thread.  Range tiles (narrow images) may take
// the whole-window tiles' LDS: their halo is full rows.
bool tile_fits(int K, int G, int M, int TW, int TH, bool synth_ray, bool range = false) {
    const int lim = (G == 1 || range) ? kMaxLdsBytesG1 : kMaxLdsBytes;
    return lds_units(K, G, M, TW, TH, synth_ray) * 16 <= lim &&
           halo_count(K, TW, TH) <= 2 * 64 * M * G;
}

int gcd_int(int a, int b) {
    while (b != 0) {
        const int t = a % b;
        a = b;
        b = t;
    }
    return a;
}

// Rows spanned by a range tile of npx pixels of a W-wide image, at most: its
// first pixel is a multiple of npx, so it starts at a column that is a
// multiple of gcd(npx, W).
int range_rows(int npx, int W) {
    const int g = gcd_int(npx, W);
    return (W - g + npx - 1) / W + 1;
}

// Tiles per image of a launch plan.
long long tiles_per_image(const AngmfArgs& c) {
    if (c.range) return (c.HW + 64LL * c.M - 1) / (64LL * c.M);
    return (long long)((c.W + c.TW - 1) / c.TW) * ((c.H + c.TH - 1) / c.TH);
}

// Tile of the fp32 kernel for G waves per group: wide images (and rows longer
// than a workgroup's 64 * M pixels) take 64 x M tiles (each wave one 256 B row
// segment per plane).  Narrow images (W <= 128) whose rows are not a whole
// number of 64-pixel groups take range tiles: 64 M consecutive pixels of the
// row-major image, so that every group reads exactly two whole 128 B lines
// per plane and no line is split between tiles (full-width tiles of whole
// rows split every other line at W = 80: 1.11x the algorithmic traffic), the
// largest M that fits.  Other narrow images take full-width tiles of TH rows
// with the fewest idle lanes among those that fit.  Returns the fraction of
// lanes that hold a pixel (0 if nothing fits).
double tile_for(AngmfArgs& a, int K, int G) {
    const int mmax = kWgWaves / G;
    a.G = G;
    a.range = 0;
    a.TW = 64;
    a.M = mmax;
    while (a.M > 1 && !tile_fits(K, G, a.M, 64, a.M, a.synth_ray != 0)) --a.M;
    a.TH = a.M;
    double best = tile_fits(K, G, a.M, 64, a.M, a.synth_ray != 0) ? 1.0 : 0.0;
    if (a.W <= 128 && a.W % 64 != 0) {
        for (int m = mmax; m >= 1; --m) {
            const int th = range_rows(64 * m, a.W);
            if (!tile_fits(K, G, m, a.W, th, a.synth_ray != 0, true)) continue;
            a.range = 1;
            a.TW = a.W;
            a.TH = th;
            a.M = m;
            const long long tiles = (a.HW + 64LL * m - 1) / (64LL * m);
            return (double)a.HW / (double)(tiles * 64LL * m);
        }
    }
    if (a.W > 128 || a.W > 64 * mmax) return best;
    best = -1.0;
    for (int th = 1; th <= a.H && th <= 64 * mmax; ++th) {
        const int npx = a.W * th;
        const int m = (npx + 63) / 64;
        if (m > mmax) break;
        const double util = (double)npx / (64.0 * m);
        if (util >= best && tile_fits(K, G, m, a.W, th, a.synth_ray != 0)) {
            best = util;
            a.TW = a.W;
            a.TH = th;
            a.M = m;
        }
    }
    return best < 0.0 ? 0.0 : best;
}

// Workgroups below which a launch is latency-bound: two per CU.
constexpr long long kSmallGrid = 512;

// G and the tile.  A launch that fills the resident whole-window workgroups
// as kWholeWindowOk's note says, with at least 90% of their lanes holding a
// pixel, takes G = 1.  Otherwise, of the two run-split candidates, a launch of
// fewer than kSmallGrid workgroups takes the one with more of them (its runs are
// shorter, so its waves finish sooner); a larger one the one with the most
// lanes holding a pixel, the preferred G on ties, except between range tiles,
// where the second (fewer, larger workgroups) wins ties: 32 x 60 x 80 at
// k = 5 ran 18.0-18.3 us with G = 2 (608 workgroups) against 19.2-19.4 with
// G = 4 (1,216).
void choose_tile(AngmfArgs& a, int K) {
    auto wgs = [](const AngmfArgs& c) { return tiles_per_image(c) * c.B; };
    if (kWholeWindowOk[K] && (long long)K * K * a.HW * 4 < (1LL << 32)) {
        AngmfArgs one = a;
        const double util = tile_for(one, K, 1);
        const long long n = util > 0.0 ? wgs(one) : 0;
        const long long rounds = (n + kWholeWindowSlots - 1) / kWholeWindowSlots;
        if (util >= 0.9 && n >= kWholeWindowSlots &&
            (double)n >= kRoundFill * (double)(rounds * kWholeWindowSlots)) {
            a = one;
            return;
        }
    }
    AngmfArgs alt = a;
    const double u0 = tile_for(a, K, kGChoices[K][0]);
    const long long w0 = wgs(a);
    if (kGChoices[K][1] != kGChoices[K][0]) {
        const double u1 = tile_for(alt, K, kGChoices[K][1]);
        if (u1 > 0.0) {
            const long long w1 = wgs(alt);
            if (u0 <= 0.0)
                a = alt;
            else if (w0 < kSmallGrid || w1 < kSmallGrid)
                a = (w1 > w0) ? alt : a;
            else if (u1 > u0 + 1e-9 || (alt.range && u1 >= u0 - 1e-9))
                a = alt;
        }
    }
    // a launch the first choice leaves with idle CUs takes kGSmall's G when
    // that gives it more workgroups
    if (kGSmall[K] != 0 && u0 > 0.0 && w0 < kIdleGrid) {
        AngmfArgs sm = a;
        if (tile_for(sm, K, kGSmall[K]) > 0.0 && wgs(sm) > wgs(a)) a = sm;
    }
}

// The launch plan of one call: the kernel arguments that depend on the
// shapes, intrinsics and flags (a.G, the tile, dd_min, ...), and whether it
// runs the double-precision kernel (fp64).
int plan_angmf(AngmfArgs& a, int B, int H, int W, int k, double fu, double cu, double fv,
               double cv, unsigned flags, bool& fp64) {
    const long long HW = (long long)H * W;
    const bool synth = (flags & BVML_DSINE_RAY_FROM_INTRINSICS) != 0;
    a.fu = fu; a.cu = cu; a.fv = fv; a.cv = cv;
    a.HW = HW; a.B = B; a.H = H; a.W = W;
    a.ifu64 = 1.0 / fu;
    a.ifv64 = 1.0 / fv;
    a.tu_c = (0.5 - cu) / fu;
    a.tv_c = (0.5 - cv) / fv;
    // gmax: the largest |P0| over the image's pixel centres (at a corner),
    // times the largest |m| the fast path accepts
    double gmax = 0.0;
    for (const int cy : {0, H - 1})
        for (const int cx : {0, W - 1}) {
            const double tu = (cx + 0.5 - cu) / fu, tv = (cy + 0.5 - cv) / fv;
            gmax = std::fmax(gmax, std::sqrt(1.0 + tu * tu + tv * tv));
        }
    gmax *= std::sqrt(1.0 + (double)kUnitM2);
    a.dd_min = kDdClamp + 1e-7 * gmax + 3e-7 / std::fmin(std::fabs(fu), std::fabs(fv));
    a.synth_ray = synth ? 1 : 0;
    a.logits = (flags & BVML_DSINE_LOGITS) ? 1 : 0;
    choose_tile(a, k);
    {
        const double K2 = (double)k * k;
        const double bytes = (double)B * HW * 4.0 * (3.0 + 4.0 * K2 + 3.0) +
                             (synth ? 0.0 : (double)HW * 4.0 * 3.0);
        a.stream_planes = (a.G == 1 && bytes > kStreamBytes) ? 1 : 0;
    }
    if (!tile_fits(k, a.G, a.M, a.TW, a.TH, synth, a.range != 0))
        return fail(BVML_DSINE_ESIZE, "angmf_propagate: no tile fits the kernel's LDS");
    // (range tiles: the kernel divides pixel indices by W with tiles_x's magic)
    a.tiles_x = a.range ? W : (W + a.TW - 1) / a.TW;
    const long long tpi = tiles_per_image(a);
    a.tiles_per_img = (int)(tpi < INT_MAX ? tpi : INT_MAX);

    // The fp32 path assumes intrinsics in the range real cameras produce;
    // anything else runs the double-precision kernel (same results as the
    // reference, which accepts any value).
    const bool sane = std::isfinite(fu) && std::isfinite(fv) && std::isfinite(cu) &&
                      std::isfinite(cv) && std::fabs(fu) >= 1e-3 && std::fabs(fu) <= 1e7 &&
                      std::fabs(fv) >= 1e-3 && std::fabs(fv) <= 1e7 &&
                      std::fabs(cu) <= 1e7 && std::fabs(cv) <= 1e7 && gmax <= kMaxP0;
    // The fp32 kernel addresses a wave's run of neighbour planes (and the 3
    // planes of pred_norm and ray) from one 32-bit buffer offset, and its grid
    // holds one image's tiles in x; larger images also run the
    // double-precision kernel.
    const long long gw = a.G, nrun = (k * k + gw - 1) / gw;
    const long long nplanes = nrun > 3 ? nrun : 3;
    const bool fits32 = nplanes * HW * 4 < (1LL << 32) && tpi < (1LL << 31) &&
                        tpi * 64 * a.M * gw < (1LL << 32);
    fp64 = (flags & BVML_DSINE_FP64) || !sane || !fits32;
    return BVML_DSINE_OK;
}

}  // namespace

extern "C" {

const char* bvml_dsine_version(void) { return "0.2.0"; }

double bvml_dsine_angmf_recompute_ratio(int k, unsigned flags) {
    if (flags & BVML_DSINE_FP64) return 0.0;
    if (!(k == 1 || k == 3 || k == 5 || k == 7 || k == 9)) return -1.0;
    return kAccRatio2[k];
}

int bvml_dsine_build_ray8_f32(float* ray, double fu, double cu, double fv, double cv, int H,
                              int W, void* stream) {
    if (H < 0 || W < 0) return fail(BVML_DSINE_ESHAPE, "build_ray8: H and W must be >= 0");
    const long long HW = (long long)H * W;
    if (HW == 0) return BVML_DSINE_OK;
    if (!ray) return fail(BVML_DSINE_ENULL, "build_ray8: ray must be non-NULL");
    if (HW > (long long)INT_MAX * 64)
        return fail(BVML_DSINE_ESIZE, "build_ray8: H*W too large for one launch");
    const long long grid = (HW + 255) / 256;
    hipLaunchKernelGGL(build_ray8_kernel, dim3((unsigned)grid), dim3(256), 0,
                       static_cast<hipStream_t>(stream), ray, fu, cu, fv, cv, H, W);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail((int)e, std::string("build_ray8 launch: ") + hipGetErrorString(e));
    return BVML_DSINE_OK;
}

int bvml_dsine_build_uv8_f32(float* uv, double fu, double cu, double fv, double cv, int H,
                             int W, void* stream) {
    if (H < 0 || W < 0) return fail(BVML_DSINE_ESHAPE, "build_uv8: H and W must be >= 0");
    const long long HW = (long long)H * W;
    if (HW == 0) return BVML_DSINE_OK;
    if (!uv) return fail(BVML_DSINE_ENULL, "build_uv8: uv must be non-NULL");
    if (HW > (long long)INT_MAX * 64)
        return fail(BVML_DSINE_ESIZE, "build_uv8: H*W too large for one launch");
    const long long grid = (HW + 255) / 256;
    hipLaunchKernelGGL(build_uv8_kernel, dim3((unsigned)grid), dim3(256), 0,
                       static_cast<hipStream_t>(stream), uv, fu, cu, fv, cv, H, W);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail((int)e, std::string("build_uv8 launch: ") + hipGetErrorString(e));
    return BVML_DSINE_OK;
}

int bvml_dsine_ray_relu_f32(float* normal, const float* ray, int B, int H, int W,
                            long long ray_bstride, void* stream) {
    if (B < 0 || H < 0 || W < 0)
        return fail(BVML_DSINE_ESHAPE, "ray_relu: B, H and W must be >= 0");
    if (ray_bstride < 0)
        return fail(BVML_DSINE_ESHAPE, "ray_relu: ray_bstride must be >= 0");
    const long long HW = (long long)H * W;
    if (B == 0 || HW == 0) return BVML_DSINE_OK;
    if (!normal || !ray) return fail(BVML_DSINE_ENULL, "ray_relu: normal and ray must be non-NULL");
    const long long total = (long long)B * HW;
    if (total > (long long)INT_MAX * 256)
        return fail(BVML_DSINE_ESIZE, "ray_relu: B*H*W too large for one launch");
    const size_t nbytes = (size_t)B * 3 * HW * sizeof(float);
    const size_t rbytes = ((size_t)(B - 1) * ray_bstride + 3 * HW) * sizeof(float);
    if (overlaps(normal, nbytes, ray, rbytes))
        return fail(BVML_DSINE_EALIAS, "ray_relu: normal and ray overlap");
    const bool vec4 = HW % 4 == 0 && ray_bstride % 4 == 0 &&
                      (reinterpret_cast<uintptr_t>(normal) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(ray) & 15u) == 0;
    if (vec4) {
        const long long total4 = total / 4;
        hipLaunchKernelGGL(ray_relu4_kernel, dim3((unsigned)((total4 + 255) / 256)), dim3(256), 0,
                           static_cast<hipStream_t>(stream), normal, ray, HW / 4, total4,
                           ray_bstride / 4);
    } else {
        const long long grid = (total + 255) / 256;
        hipLaunchKernelGGL(ray_relu_kernel, dim3((unsigned)grid), dim3(256), 0,
                           static_cast<hipStream_t>(stream), normal, ray, HW, total, ray_bstride);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail((int)e, std::string("ray_relu launch: ") + hipGetErrorString(e));
    return BVML_DSINE_OK;
}

int bvml_dsine_angmf_plan(int B, int H, int W, int k, double fu, double cu, double fv, double cv,
                          unsigned flags, int* waves_per_group, int* tile_w, int* tile_h,
                          int* stream_planes) {
    if (flags & ~(BVML_DSINE_FP64 | BVML_DSINE_RAY_FROM_INTRINSICS | BVML_DSINE_LOGITS))
        return fail(BVML_DSINE_EFLAGS, "angmf_plan: unknown flag bits");
    if (B < 1 || H < 1 || W < 1)
        return fail(BVML_DSINE_ESHAPE, "angmf_plan: B, H and W must be >= 1");
    if (!(k == 1 || k == 3 || k == 5 || k == 7 || k == 9))
        return fail(BVML_DSINE_EK, "angmf_plan: k must be one of 1, 3, 5, 7, 9");
    const long long HW = (long long)H * W;
    if ((long long)B * HW > (long long)INT_MAX * 64 || HW >= (1LL << 30))
        return fail(BVML_DSINE_ESIZE, "angmf_plan: B*H*W too large for one launch");
    AngmfArgs a{};
    bool fp64 = false;
    const int st = plan_angmf(a, B, H, W, k, fu, cu, fv, cv, flags, fp64);
    if (st != BVML_DSINE_OK) return st;
    if (waves_per_group) *waves_per_group = a.G;
    if (tile_w) *tile_w = a.range ? 64 * a.M : a.TW;
    if (tile_h) *tile_h = a.range ? 0 : a.TH;
    if (stream_planes) *stream_planes = a.stream_planes;
    return fp64 ? 0 : 1;
}

int bvml_dsine_angmf_propagate_f32(const float* pred_norm, const float* prob,
                                   const float* xy, const float* angle,
                                   const float* ray, double fu, double cu,
                                   double fv, double cv, int B, int H, int W,
                                   int k, long long ray_bstride, float* out,
                                   unsigned flags, void* stream) {
    if (flags & ~(BVML_DSINE_FP64 | BVML_DSINE_RAY_FROM_INTRINSICS | BVML_DSINE_LOGITS))
        return fail(BVML_DSINE_EFLAGS, "angmf_propagate: unknown flag bits");
    const bool synth = (flags & BVML_DSINE_RAY_FROM_INTRINSICS) != 0;
    if (synth) {
        ray = nullptr;
        ray_bstride = 0;
    }
    if (B < 0 || H < 0 || W < 0)
        return fail(BVML_DSINE_ESHAPE, "angmf_propagate: B, H and W must be >= 0");
    if (ray_bstride < 0)
        return fail(BVML_DSINE_ESHAPE, "angmf_propagate: ray_bstride must be >= 0");
    if (!(k == 1 || k == 3 || k == 5 || k == 7 || k == 9))
        return fail(BVML_DSINE_EK, "angmf_propagate: k must be one of 1, 3, 5, 7, 9");
    const long long HW = (long long)H * W;
    if (B == 0 || HW == 0) return BVML_DSINE_OK;
    if (!pred_norm || !prob || !xy || !angle || (!ray && !synth) || !out)
        return fail(BVML_DSINE_ENULL, "angmf_propagate: all tensors must be non-NULL");
    const long long K2 = (long long)k * k;
    const long long total = (long long)B * HW;
    if (total > (long long)INT_MAX * 64 || HW >= (1LL << 30))
        return fail(BVML_DSINE_ESIZE, "angmf_propagate: B*H*W too large for one launch");
    const size_t f = sizeof(float);
    const size_t out_b = (size_t)B * 3 * HW * f;
    const size_t pn_b = (size_t)B * 3 * HW * f;
    const size_t pr_b = (size_t)B * K2 * HW * f;
    const size_t xy_b = (size_t)B * 2 * K2 * HW * f;
    const size_t an_b = (size_t)B * K2 * HW * f;
    const size_t ry_b = ((size_t)(B - 1) * ray_bstride + 3 * HW) * f;
    if (overlaps(out, out_b, pred_norm, pn_b) || overlaps(out, out_b, prob, pr_b) ||
        overlaps(out, out_b, xy, xy_b) || overlaps(out, out_b, angle, an_b) ||
        (!synth && overlaps(out, out_b, ray, ry_b)))
        return fail(BVML_DSINE_EALIAS, "angmf_propagate: out overlaps an input");

    AngmfArgs a{};
    a.pn = pred_norm; a.pr = prob; a.xy = xy; a.ang = angle; a.ray = ray; a.out = out;
    a.ray_bstride = ray_bstride;
    bool fp64 = false;
    const int st = plan_angmf(a, B, H, W, k, fu, cu, fv, cv, flags, fp64);
    if (st != BVML_DSINE_OK) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    switch (k) {
        case 1: e = launch_angmf<1>(a, fp64, s); break;
        case 3: e = launch_angmf<3>(a, fp64, s); break;
        case 5: e = launch_angmf<5>(a, fp64, s); break;
        case 7: e = launch_angmf<7>(a, fp64, s); break;
        default: e = launch_angmf<9>(a, fp64, s); break;
    }
    if (e != hipSuccess)
        return fail((int)e, std::string("angmf_propagate launch: ") + hipGetErrorString(e));
    return BVML_DSINE_OK;
}

}  // extern "C"
