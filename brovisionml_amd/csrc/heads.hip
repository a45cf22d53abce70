// The refiner's prediction heads after their first (3x3) layer, fused into one
// per-pixel pass on the fp32 matrix cores (the C ABI's
// bvml_dsine_heads_mlp_f32).  Each head of src/dsine_refine.cpp:119-127 is
// conv3x3 -> ReLU -> conv1x1 -> ReLU -> conv1x1; the 3x3 layer runs as a
// convolution without its bias, and for every pixel p and head h this pass
// computes
//   a = relu(t0[64h + c][p] + b0[64h + c])         c < 64   (the 3x3 layer's bias + ReLU)
//   t = relu(W2_h a + b2_h)                                   (the middle 1x1 layer)
//   out_h[o][p] = (W4_h t)[o] + b4_h[o]             o < n_h   (the last 1x1 layer)
// in place of a grouped convolution, the logit convolutions and four
// elementwise passes.  Each sum is fp32 (the products' order is the
// matrix instruction's), then its bias is added once, as a convolution
// followed by a bias add rounds it.
//
// Work layout: a workgroup of 8 waves stages the packed middle layers and the
// small last layers in LDS (96 KB at most), then each wave owns 32 pixels
// (two 16-pixel column blocks), loading the next head's inputs while it
// multiplies the current head's.  The middle
// layer is a 64 x 64 x 32 product of v_mfma_f32_16x16x4_f32 steps: A = W2
// (16 output rows x 4 inputs per step, from the packed weights), B = a (4
// input channels x 16 pixels, loaded with the bias and ReLU applied).  Its
// accumulator lane l holds rows 16 mb + 4 (l / 16) + r (r = 0..3) of pixel
// l % 16, which is exactly the B operand of a step whose 4 inputs are
// {16 mb + 4 g + r : g = 0..3}: the last layer consumes the middle layer's
// registers directly, with W4's inputs packed in that order
// (bvml_dsine_heads_pack_f32).

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <string>

#include "bvml_dsine.h"
#include "pack_layout.h"
#include "status.h"

namespace {

using bvml::fail;
using bvml::overlaps;

constexpr int kHid = bvml::pack::kHeadsHidden;  // the heads' hidden width
constexpr int kMaxHeads = 4;
constexpr int kWaves = 8;      // waves per workgroup
constexpr int kPx = 32;        // pixels per wave
constexpr int kOb = 4;         // last-layer output blocks per pass
constexpr int kW2Floats = bvml::pack::kHeadsW2Floats;  // one head's packed middle layer
// Last layers of at most this many output blocks in all are staged in LDS
// with the middle layers (the prob, xy and angle heads: 2 + 4 + 2 blocks);
// the others (the up-mask head, 36 blocks) pass through an LDS chunk buffer.
constexpr int kLdsOb = 8;
constexpr int kChunkOb = 8;    // a large last layer passes through LDS this many blocks at a time
constexpr int kLdsFloats = kMaxHeads * kW2Floats + (kLdsOb + kChunkOb) * 16 * 64;
// The biases in LDS too: b0 and b2 of every head, and the last layers'
// biases up to kB4Lds floats in all (the others are read from global memory).
// A bias read from global memory inside the products would wait for the next
// head's inputs, whose loads were issued before it (vector loads complete in
// order): 3 heads of 25, 50 and 25 outputs at 256 x 256 took 48.7 us so.
constexpr int kB4Lds = 1024;
constexpr int kBiasFloats = 2 * kMaxHeads * kHid + kB4Lds;

typedef float v4f __attribute__((ext_vector_type(4)));

struct HeadsArgs {
    const float* t0;
    const float* b0;
    const float* b2;
    const float* w2p;                 // [head][j 16][mb 4][64 lanes]
    const float* w4p[kMaxHeads];      // [ob][mb 4][r 4][64 lanes]
    const float* b4[kMaxHeads];       // NULL: no bias
    float* out[kMaxHeads];
    int outs[kMaxHeads];
    int lds_off[kMaxHeads];           // W4p's offset in LDS, -1: read from global
    int b4_off[kMaxHeads];            // b4's offset in the LDS bias region, -1: global or none
    int lds_floats;                   // floats staged in LDS
    int nheads;
    long long HW;
};

__device__ __forceinline__ float relu(float v) { return v < 0.0f ? 0.0f : v; }

// B operands of head h's middle layer for the wave's two 16-pixel blocks:
// relu(t0 + b0) of input channel 64h + 4j + g at this lane's pixels.
__device__ __forceinline__ void load_head_inputs(const HeadsArgs& a, int h, int g,
                                                 const long long* p, const bool* in,
                                                 float (&bf)[16][2]) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int c = kHid * h + 4 * j + g;
        const float* tc = a.t0 + (size_t)c * a.HW;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            // every lane loads (a pixel past the map reads pixel 0; its
            // value is masked where it is used): with the loads under
            // branches, or zeroed here, the compiler waited for all of them,
            // the next head's included, before the current head's products
            bf[j][nb] = tc[in[nb] ? p[nb] : 0];
        }
    }
}

// The last layer on the middle layer's registers t (see above): kOb output
// blocks of 16 at a time, W4 packed at w4, plus the bias b4 (when has_b4),
// into out.
__device__ __forceinline__ void last_layer(const float* __restrict__ w4, const v4f (&t)[4][2],
                                           int n, const float* __restrict__ b4, bool has_b4,
                                           float* __restrict__ out, long long HW, int lane, int g,
                                           const long long* p, const bool* in) {
    const int nob = (n + 15) / 16;
    for (int ob0 = 0; ob0 < nob; ob0 += kOb) {
        const int cnt = nob - ob0 < kOb ? nob - ob0 : kOb;
        v4f oacc[kOb][2];
#pragma unroll
        for (int i = 0; i < kOb; ++i)
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) oacc[i][nb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int i = 0; i < kOb; ++i) {
                    if (i >= cnt) break;
                    const float af = w4[(((ob0 + i) * 4 + mb) * 4 + r) * 64 + lane];
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb)
                        oacc[i][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(af, t[mb][nb][r],
                                                                            oacc[i][nb], 0, 0, 0);
                }
#pragma unroll
        for (int i = 0; i < kOb; ++i) {
            if (i >= cnt) break;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int o = 16 * (ob0 + i) + 4 * g + r;
                if (o >= n) continue;
                float* oc = out + (size_t)o * HW;
                const float bias = has_b4 ? b4[o] : 0.0f;
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
                    if (in[nb]) oc[p[nb]] = has_b4 ? oacc[i][nb][r] + bias : oacc[i][nb][r];
            }
        }
    }
}

__global__ __launch_bounds__(kWaves * 64) void heads_mlp_kernel(HeadsArgs a) {
    __shared__ float lds[kLdsFloats];
    // [b0 of every head | b2 of every head | the staged last-layer biases]
    __shared__ float bl[kBiasFloats];
    {
        const int nb2 = a.nheads * kHid;
        for (int i = threadIdx.x; i < nb2; i += kWaves * 64) {
            bl[i] = a.b0[i];
            bl[kMaxHeads * kHid + i] = a.b2[i];
        }
#pragma unroll
        for (int h = 0; h < kMaxHeads; ++h) {
            if (h >= a.nheads || a.b4_off[h] < 0) continue;
            for (int i = threadIdx.x; i < a.outs[h]; i += kWaves * 64)
                bl[2 * kMaxHeads * kHid + a.b4_off[h] + i] = a.b4[h][i];
        }
    }
    // stage the packed middle layers and the small last layers
    {
        const int n = a.lds_floats;
        const int w2n = a.nheads * kW2Floats;
        for (int i = threadIdx.x * 4; i < n; i += kWaves * 64 * 4) {
            float4 v;
            if (i < w2n) {
                v = *reinterpret_cast<const float4*>(a.w2p + i);
            } else {
                // the staged head whose region holds i: the last one starting
                // at or before it (the regions follow the middle layers in
                // head order)
                int h = 0;
#pragma unroll
                for (int e = 1; e < kMaxHeads; ++e)
                    if (e < a.nheads && a.lds_off[e] >= 0 && i >= a.lds_off[e]) h = e;
                v = *reinterpret_cast<const float4*>(a.w4p[h] + (i - a.lds_off[h]));
            }
            *reinterpret_cast<float4*>(lds + i) = v;
        }
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, col = lane & 15;
    const long long p0 = ((long long)blockIdx.x * kWaves + wave) * kPx;
    // no early exit: a wave past the map's end still takes part in the
    // workgroup's barriers (its loads and stores are masked off)
    long long p[2];
    bool in[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        p[nb] = p0 + 16 * nb + col;
        in[nb] = p[nb] < a.HW;
    }
    float cur[16][2];
    load_head_inputs(a, 0, g, p, in, cur);
#pragma unroll
    for (int h = 0; h < kMaxHeads; ++h) {
        if (h >= a.nheads) break;
        float next[16][2];
        // the next head's inputs (the last head re-reads its own, unused:
        // loads under a branch would leave the compiler unable to count them,
        // and it would wait for all of them before this head's products)
        load_head_inputs(a, h + 1 < a.nheads ? h + 1 : h, g, p, in, next);
        __builtin_amdgcn_sched_barrier(0);
        // middle layer: acc[mb][nb] = W2 (rows 16 mb..) x relu(t0 + b0) (pixels of nb)
        v4f acc[4][2];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        const float* w2 = lds + h * kW2Floats;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float bias = bl[kHid * h + 4 * j + g];
            float bf[2];
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) bf[nb] = in[nb] ? relu(cur[j][nb] + bias) : 0.0f;
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                const float af = w2[(j * 4 + mb) * 64 + lane];
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(af, bf[nb], acc[mb][nb], 0,
                                                                        0, 0);
            }
        }
        // t = relu(acc + b2), in place
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float bias = bl[kMaxHeads * kHid + kHid * h + 16 * mb + 4 * g + r];
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) acc[mb][nb][r] = relu(acc[mb][nb][r] + bias);
            }
        // last layer, from LDS or (a large layer) from global memory: separate
        // calls, so each reads its weights and bias through its own address
        // space
        if (a.lds_off[h] >= 0 && a.b4_off[h] >= 0)
            last_layer(lds + a.lds_off[h], acc, a.outs[h], bl + 2 * kMaxHeads * kHid + a.b4_off[h],
                       true, a.out[h], a.HW, lane, g, p, in);
        else if (a.lds_off[h] >= 0)
            last_layer(lds + a.lds_off[h], acc, a.outs[h], a.b4[h], a.b4[h] != nullptr, a.out[h],
                       a.HW, lane, g, p, in);
        else {
            // a large last layer: kChunkOb blocks at a time through the chunk
            // buffer after the staged weights (uniform across the workgroup)
            float* chunk = lds + a.lds_floats;
            const int nob = (a.outs[h] + 15) / 16;
            for (int c0 = 0; c0 < nob; c0 += kChunkOb) {
                const int cb = nob - c0 < kChunkOb ? nob - c0 : kChunkOb;
                const float* src = a.w4p[h] + (size_t)c0 * 16 * 64;
                __syncthreads();
                // direct-to-LDS loads, 1 KB per wave-wide load (lane l's 16 bytes
                // at the wave's base + 16 l), all in flight at once; a chunk is a
                // whole number of 256-float runs, so each wave's loads are
                // all-lane (a copy through registers waited one round trip per
                // 8 KB, every wave at once)
                for (int i = threadIdx.x * 4; i < cb * 16 * 64; i += kWaves * 64 * 4)
                    __builtin_amdgcn_global_load_lds(
                        static_cast<const void*>(src + i),
                        reinterpret_cast<__attribute__((address_space(3))) void*>(
                            reinterpret_cast<uintptr_t>(chunk + (i - 4 * lane))),
                        16, 0, 0);
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
                const int n = a.outs[h] - 16 * c0 < 16 * cb ? a.outs[h] - 16 * c0 : 16 * cb;
                const float* b4 = a.b4[h] ? a.b4[h] + 16 * c0 : nullptr;
                last_layer(chunk, acc, n, b4, b4 != nullptr, a.out[h] + (size_t)16 * c0 * a.HW,
                           a.HW, lane, g, p, in);
            }
        }
        if (h + 1 < a.nheads) {
#pragma unroll
            for (int j = 0; j < 16; ++j)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) cur[j][nb] = next[j][nb];
        }
    }
}

}  // namespace

extern "C" {

int bvml_dsine_heads_mlp_f32(const float* t0, const float* b0, const float* w2p, const float* b2,
                             const float* const* w4p, const float* const* b4, const int* outs,
                             int nheads, int H, int W, float* const* out, void* stream) {
    if (nheads < 1 || nheads > kMaxHeads)
        return fail(BVML_DSINE_EPARAM, "heads_mlp: nheads must be 1..4");
    if (H < 0 || W < 0) return fail(BVML_DSINE_ESHAPE, "heads_mlp: H and W must be >= 0");
    if (!w4p || !b4 || !outs || !out)
        return fail(BVML_DSINE_ENULL, "heads_mlp: the per-head arrays must be non-NULL");
    const long long HW = (long long)H * W;
    if (HW == 0) return BVML_DSINE_OK;
    if (!t0 || !b0 || !w2p || !b2)
        return fail(BVML_DSINE_ENULL, "heads_mlp: t0, b0, w2p and b2 must be non-NULL");
    if (HW > (long long)INT_MAX * kPx)
        return fail(BVML_DSINE_ESIZE, "heads_mlp: H*W too large for one launch");
    HeadsArgs a{};
    a.t0 = t0;
    a.b0 = b0;
    a.b2 = b2;
    a.w2p = w2p;
    a.nheads = nheads;
    a.HW = HW;
    const size_t t0b = (size_t)nheads * kHid * HW * sizeof(float);
    for (int h = 0; h < nheads; ++h) {
        if (outs[h] < 1 || outs[h] > 4096)
            return fail(BVML_DSINE_EPARAM, "heads_mlp: outs must be 1..4096");
        if (!w4p[h] || !out[h]) return fail(BVML_DSINE_ENULL, "heads_mlp: w4p and out must be non-NULL");
        const size_t ob = (size_t)outs[h] * HW * sizeof(float);
        if (overlaps(out[h], ob, t0, t0b))
            return fail(BVML_DSINE_EALIAS, "heads_mlp: an output overlaps t0");
        for (int e = 0; e < h; ++e)
            if (overlaps(out[h], ob, out[e], (size_t)outs[e] * HW * sizeof(float)))
                return fail(BVML_DSINE_EALIAS, "heads_mlp: outputs overlap");
        a.w4p[h] = w4p[h];
        a.b4[h] = b4[h];
        a.out[h] = out[h];
        a.outs[h] = outs[h];
    }
    // LDS: the middle layers, then each last layer that fits in kLdsOb blocks
    int at = nheads * kW2Floats, staged_ob = 0;
    for (int h = 0; h < kMaxHeads; ++h) a.lds_off[h] = -1;
    for (int h = 0; h < nheads; ++h) {
        const int nob = (outs[h] + 15) / 16;
        if (staged_ob + nob <= kLdsOb) {
            a.lds_off[h] = at;
            at += nob * 16 * 64;
            staged_ob += nob;
        }
    }
    a.lds_floats = at;
    // the last layers' biases in LDS while they fit
    int b4_at = 0;
    for (int h = 0; h < kMaxHeads; ++h) a.b4_off[h] = -1;
    for (int h = 0; h < nheads; ++h)
        if (b4[h] && b4_at + outs[h] <= kB4Lds) {
            a.b4_off[h] = b4_at;
            b4_at += outs[h];
        }
    for (int h = 0; h < nheads; ++h)
        if ((reinterpret_cast<uintptr_t>(w4p[h]) & 15u) != 0)
            return fail(BVML_DSINE_EPARAM, "heads_mlp: w4p must be 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(w2p) & 15u) != 0)
        return fail(BVML_DSINE_EPARAM, "heads_mlp: w2p must be 16-byte aligned");
    const long long per_block = (long long)kWaves * kPx;
    const long long grid = (HW + per_block - 1) / per_block;
    hipLaunchKernelGGL(heads_mlp_kernel, dim3((unsigned)grid), dim3(kWaves * 64), 0,
                       static_cast<hipStream_t>(stream), a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail((int)e, std::string("heads_mlp launch: ") + hipGetErrorString(e));
    return BVML_DSINE_OK;
}

}  // extern "C"
