// The refiner's k x k convolutions (k = 3, 5; stride 1, zero "same" padding)
// as implicit GEMMs on the fp32 matrix cores (the C ABI's bvml_dsine_conv_*):
// rows = output channels, columns = pixels, the reduction over (input
// channel, tap).  No im2col buffer: a workgroup of 4 waves owns a 16 x 16
// pixel tile and 64 or 128 output channels (each wave 64 channels x 4 or 8
// tile rows: 16 or 32 accumulator blocks, so each weight load feeds 4 or 8
// products); for every chunk of 4 input channels it stages the
// tile's halo (TH + k - 1) x (16 + k - 1) in LDS (double-buffered, the next
// chunk's loads in flight during the current chunk's products), then for each
// tap runs v_mfma_f32_16x16x4_f32 steps with
//   A = the packed weights of 16 output channels x the chunk's 4 channels at
//       that tap (bvml_dsine_conv_pack_f32's layout): the chunk's weights
//       read from L2 (one coalesced 256-byte load per step) or, in the 3x3
//       launches of 4 M-blocks, staged in LDS (double-buffered, copied by
//       direct-to-LDS loads; stage_weights),
//   B = the halo at the tap's shift: 4 channels x 16 pixels of one tile row.
// Each sum is fp32 in the matrix instruction's order.  The epilogues fuse
// what the refiner does next (src/dsine_refine.cpp:138-159):
//   kPlain   out = the sum (the bias is added by the consumer)
//   kGates   convz and convr as one convolution whose 16-channel blocks
//            alternate z, r: z = sigmoid(s_z + b_z), rh = sigmoid(s_r + b_r) h
//   kUpdate  convq: h_new = (1 - z) h + z tanh(s + b_q), to h_new and h_copy
// in the rounding of bvml_dsine_gru_gates_f32 / bvml_dsine_gru_update_f32;
//   kHeads   the heads' 3x3 first layers with the rest of each head
//            (src/dsine_refine.cpp:119-127): relu(s + b0), a 64 x 64 1x1
//            layer, relu, the last 1x1 layer, on the matrix cores from the
//            accumulators' registers (bvml_dsine_conv_heads_f32).

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

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kTW = 16;      // tile width: one MFMA column block per tile row
constexpr int kCC = bvml::pack::kConvChunk;  // input channels per chunk (one k-step per tap)
constexpr int kThreads = 256;

enum Epi : int { kPlain = 0, kGates = 1, kUpdate = 2, kHeads = 3 };

struct ConvArgs {
    const float* x;     // cin planes of H x W
    const float* wp;    // packed: [chunk][tap][mblock][64]
    float* out;         // kPlain: cout planes
    const float* b0;    // kGates: b_z, kUpdate: b_q
    const float* b1;    // kGates: b_r
    const float* h;     // kGates, kUpdate: the hidden state (64 planes)
    const float* z;     // kUpdate: the update gate
    float* o0;          // kGates: z, kUpdate: h_new
    float* o1;          // kGates: rh, kUpdate: h_copy (may be NULL)
    const float* s0;    // kGates, kUpdate: sums to add (packed order, the accumulators' start), or NULL
    // kHeads (b0: the 3x3 layer's bias, b1: the middle layers' bias)
    const float* w2q;   // the middle layers, 4096 floats per head in the last-layer layout
    const float* w4p[4];
    const float* b4[4];  // NULL: no bias
    float* hout[4];
    int outs[4];
    int cin, cout, H, W, mblocks, tiles_x;
    long long HW;
};

__device__ __forceinline__ float relu(float v) { return v < 0.0f ? 0.0f : v; }

// base[byte_off / 4] with a uniform base pointer and a 32-bit per-lane byte
// offset: the scalar-base + vector-offset load form, no 64-bit address per load
__device__ __forceinline__ float ldo(const float* base, uint32_t byte_off) {
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + byte_off);
}

// Raw buffer loads of packed weights: the descriptor (base, bytes) in scalar
// registers, a per-lane byte offset and a wave-uniform one (a scalar
// register), so a run of weight loads keeps no address registers of its own.
constexpr int kBufferWord3 = 0x00020000;  // gfx9 raw-buffer descriptor word 3
__device__ __forceinline__ __amdgpu_buffer_rsrc_t weights_rsrc(const float* w, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(w), (short)0, (int)bytes,
                                             kBufferWord3);
}
__device__ __forceinline__ float ldw(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, uint32_t soff) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, (int)soff, 0));
}

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float gru_mix(float z, float h, float q) {
#pragma clang fp contract(off)
    const float omz = 1.0f - z;
    return omz * h + z * q;
}

// K: kernel size; TH: tile rows; WM x WN waves (WM along the channels, WN
// along the tile rows); each wave 4 M-blocks (64 output channels) x NB tile rows.
// KS: groups of those 4 waves that split the input channels (group g takes
// chunks g, g + KS, ...; with KS = 2 the two groups' sums meet in LDS and
// each group finishes half of the tile rows).  A grid with one workgroup per
// CU leaves each SIMD one wave of 4-wave workgroups; with KS = 2 it has two,
// and one wave's MFMAs run while the other waits for its operands.
// Whether a launch stages each chunk's weights in LDS with direct-to-LDS
// loads (the products then wait on LDS reads only) or has every wave read
// its A operands from L2 two taps ahead.  Same-box A/B at 256 x 256, both
// with the operands two taps ahead of the products, bit-identical results:
// only the 3x3 launches of 4 M-blocks per workgroup (the heads' first layer
// at 192 channels) gain by staging, 131 against 156-157 us; staged, the
// others lose: convz + convr 524-531 against 466-472 us, convq 263-266
// against 246-250, the 3x3 layer at 256 channels 167 against 163.
constexpr bool stage_weights(int K, int WM) { return K == 3 && WM == 1; }

template <int K, int TH, int WM, int WN, int EPI, int KS>
// (the fused heads launch holds three 4-wave workgroups per CU, one wave
// per SIMD each, so its registers stay within a third of a SIMD's; convq
// with one wave group, on maps of two or more workgroups per CU, within
// half, where its epilogue's loads, all issued before its stores, would
// otherwise take more)
__global__ __launch_bounds__(kThreads * KS)
__attribute__((amdgpu_waves_per_eu(EPI == kHeads && KS == 1 ? 3 : (EPI == kUpdate && KS == 1 ? 2 : 1)))) void conv_kernel(ConvArgs a) {
    constexpr int P = K / 2;
    constexpr int HR = TH + K - 1, HC = kTW + K - 1, HS = HR * HC;  // halo rows, cols, size
    constexpr int HALO = kCC * HS;                                   // floats per chunk
    constexpr int PER_T = (HALO + kThreads - 1) / kThreads;
    // a channel's halo in LDS starts 16 banks (mod 64) after the previous
    // one's, so the 4 channels a B read takes (16 lanes each) hit disjoint
    // banks: 400 floats at k = 5 already; 324 padded to 336 at k = 3 (1,224
    // and 2,448 bank conflicts per wave unpadded)
    constexpr int HSP = HS + ((16 - HS % 64) + 64) % 64;
    constexpr int NB = TH / WN;                                      // tile rows per wave
    constexpr int TAPS = K * K;
    static_assert(WM * WN == kThreads / 64, "4 waves");
    static_assert(KS == 1 || NB % 2 == 0, "each group of the split finishes NB / 2 rows");
    // the workgroup's weights of one chunk, [tap][its 4 WM M-blocks][64 lanes],
    // staged in LDS (SW) or read by each wave from L2
    constexpr bool SW = stage_weights(K, WM);
    constexpr int WCH = SW ? TAPS * 4 * WM * 64 : 1;
    __shared__ float halo[KS][2][kCC * HSP];
    __shared__ float wts[KS][2][WCH];

    const int ks = (KS > 1) ? (int)threadIdx.x / kThreads : 0;  // the wave group's split
    const int tid = (int)threadIdx.x - ks * kThreads, lane = tid & 63, wave = tid >> 6;
    // the wave's index as a scalar (the weight copies' LDS addresses are per wave)
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    const int g = lane >> 4, col = lane & 15;
    const int wm = wave % WM, wn = wave / WM;
    // (k = 5) each XCD takes a contiguous run of tiles, so neighbouring tiles
    // share their halo lines and output lines in that XCD's L2 (workgroups go
    // to the XCDs in turn): convz + convr over h at 256 x 256 237 against
    // 242-246 us, convq 135-136 against 137-138; the 3x3 layers lose by it
    const int nbx = (int)gridDim.x, bx = (int)blockIdx.x, xcd = bx & 7;
    const int tile = K != 5 ? bx
                            : xcd * (nbx >> 3) + (xcd < (nbx & 7) ? xcd : (nbx & 7)) + (bx >> 3);
    const int tx0 = (tile % a.tiles_x) * kTW, ty0 = (tile / a.tiles_x) * TH;
    const int mb0 = blockIdx.y * (4 * WM) + 4 * wm;  // the wave's first M-block
    const int nchunks = (a.cin + kCC - 1) / kCC;
    // every group makes the same number of trips (the barriers are the
    // workgroup's); a trip past the last chunk stages zeros and multiplies
    // nothing
    const int trips = (nchunks + KS - 1) / KS;

    // halo element e of a chunk: (channel, halo row, halo col), its source
    auto halo_load = [&](int chunk, float (&v)[PER_T]) {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int e = tid + i * kThreads;
            float val = 0.0f;
            if (e < HALO) {
                const int c = chunk * kCC + e / HS, rem = e % HS;
                const int y = ty0 + rem / HC - P, x = tx0 + rem % HC - P;
                if (c < a.cin && y >= 0 && y < a.H && x >= 0 && x < a.W)
                    val = a.x[(size_t)c * a.HW + (size_t)y * a.W + x];
            }
            v[i] = val;
        }
    };
    auto halo_store = [&](int buf, const float (&v)[PER_T]) {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int e = tid + i * kThreads;
            if (e < HALO) halo[ks][buf][(e / HS) * HSP + e % HS] = v[i];
        }
    };
    // a chunk's weights for the workgroup's M-blocks, copied to LDS with
    // direct-to-LDS loads (one M-block of one tap, 256 bytes, per wave-wide
    // load; the group's 4 waves take every 4th): they use no registers, and
    // the products then wait on LDS reads only
    const float* wsrc = a.wp + (size_t)blockIdx.y * (4 * WM) * 64 + lane;
    auto w_load = [&](int chunk, int buf) {
        const float* wc = wsrc + (size_t)chunk * TAPS * a.mblocks * 64;
        for (int i = wave_s; i < TAPS * 4 * WM; i += 4) {
            const int tap = i / (4 * WM), j = i - tap * (4 * WM);
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(wc + ((size_t)tap * a.mblocks + j) * 64),
                reinterpret_cast<__attribute__((address_space(3))) void*>(
                    reinterpret_cast<uintptr_t>(&wts[ks][buf][i * 64])),
                4, 0, 0);
        }
    };

    v4f acc[4][NB];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < NB; ++n) acc[m][n] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // sums to add (the fused launches' sum0) start group 0's accumulators:
    // their loads overlap the first halo's, where a read in the epilogue
    // would stall every workgroup at once (convq over r*h at 256 x 256: 145
    // against 157 us; convz + convr over h 260 against 265)
    if ((EPI == kGates || EPI == kUpdate) && a.s0 && ks == 0) {
        const int x = tx0 + col;
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const int y = ty0 + wn * NB + n;
            if (x >= a.W || y >= a.H) continue;
            const size_t px = (size_t)y * a.W + x;
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[m][n][r] = a.s0[(size_t)(16 * (mb0 + m) + 4 * g + r) * a.HW + px];
        }
    }

    // The A operands from L2 (!SW): a ring of AR register slots, AR - 1 taps
    // ahead of the products.  At k = 5 the ring runs across chunk boundaries
    // (AR = 5 divides the 25 taps, so tap t of every chunk takes slot t % AR):
    // a chunk's first taps are loaded during the previous chunk, ahead of
    // that chunk's halo loads, which the products would otherwise wait for
    // (vector loads complete in issue order), and the barrier between chunks
    // waits for the LDS writes only, leaving those loads in flight across it
    // (convz + convr over h at 256 x 256, with the tile order above: 233-234
    // against 237 us; the [feature, uv] part 232 against 235).  At k = 3,
    // two taps ahead within each chunk (the 256-channel 3x3 layer: 169
    // against 173-175 us with the ring).
    constexpr bool XC = !SW && K == 5;
    constexpr int AR = XC ? 5 : 3;
    static_assert(TAPS % AR == 0, "ring slots divide the taps");
    const size_t tap_stride = (size_t)a.mblocks * 64;
    const float* wbase = a.wp + (size_t)mb0 * 64 + lane;
    float aw[SW ? 1 : AR][4];
    auto a_load = [&](int chunk, int tap, int slot) {
        const float* wc = wbase + ((size_t)chunk * TAPS + tap) * tap_stride;
#pragma unroll
        for (int m = 0; m < 4; ++m) aw[slot][m] = wc[m * 64];
    };
    auto chunk_barrier = [&]() {
        if constexpr (SW) {
            __builtin_amdgcn_s_waitcnt(0);  // the weight copies (counted with the loads)
            __syncthreads();
        } else if constexpr (!XC) {
            __syncthreads();
        } else {
            // this wave's halo writes done (lgkmcnt(0)), then the barrier;
            // the compiler keeps every LDS access on its side of it (the
            // barrier builtin alone is no memory fence to it)
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
    };

    float pre[PER_T];
    halo_load(ks, pre);
    if (SW && ks < nchunks) w_load(ks, 0);
    if constexpr (XC) {
        if (ks < nchunks) {
#pragma unroll
            for (int q = 0; q < AR - 1; ++q) a_load(ks, q, q);
        }
    }
    halo_store(0, pre);
    chunk_barrier();
    for (int trip = 0; trip < trips; ++trip) {
        const int chunk = trip * KS + ks;
        const int buf = trip & 1;
        const bool more = trip + 1 < trips;
        // the next chunk's halo (to registers) and weights (to the other LDS
        // buffer, which every wave finished reading before the last barrier)
        if (more) {
            halo_load(chunk + KS, pre);
            if (SW && chunk + KS < nchunks) w_load(chunk + KS, buf ^ 1);
        }
        if (chunk < nchunks) {
        const float* hb = halo[ks][buf] + g * HSP + (wn * NB) * HC + col;
        if constexpr (!SW) {
        // (the ring's taps past this chunk's last: the next chunk's first;
        // after the last chunk, the last chunk's again, unused)
        const int next_chunk = chunk + KS < nchunks ? chunk + KS : nchunks - 1;
        // the B operands (LDS) two taps ahead, the A operands AR - 1, the
        // loads of each tap issued before the previous tap's products (a
        // scheduling barrier keeps them there: convz + convr at 256 x 256
        // 466-468 us against 504-509 with the compiler's own order and the B
        // operands one tap ahead)
        if constexpr (!XC) {
#pragma unroll
            for (int q = 0; q < AR - 1; ++q) a_load(chunk, q, q);
        }
        float bf[3][NB];
#pragma unroll
        for (int n = 0; n < NB; ++n) bf[0][n] = hb[n * HC];
#pragma unroll
        for (int n = 0; n < NB; ++n) bf[1][n] = hb[n * HC + 1];
#pragma unroll
        for (int t = 0; t < TAPS; ++t) {
            if (t + 2 < TAPS) {
                const int ky = (t + 2) / K, kx = (t + 2) % K;
#pragma unroll
                for (int n = 0; n < NB; ++n) bf[(t + 2) % 3][n] = hb[(n + ky) * HC + kx];
            }
            if (t + AR - 1 < TAPS)
                a_load(chunk, t + AR - 1, (t + AR - 1) % AR);
            else if (XC)
                a_load(next_chunk, t + AR - 1 - TAPS, (t + AR - 1) % AR);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int n = 0; n < NB; ++n)
                    acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(aw[t % AR][m], bf[t % 3][n],
                                                                    acc[m][n], 0, 0, 0);
        }
        } else {
        const float* wl = wts[ks][buf] + (4 * wm) * 64 + lane;
        // the A and B operands (LDS) one tap ahead
        float af[2][4];
#pragma unroll
        for (int m = 0; m < 4; ++m) af[0][m] = wl[m * 64];
        float bf[2][NB];
#pragma unroll
        for (int n = 0; n < NB; ++n) bf[0][n] = hb[n * HC];
#pragma unroll
        for (int t = 0; t < TAPS; ++t) {
            if (t + 1 < TAPS) {
                const int ky = (t + 1) / K, kx = (t + 1) % K;
#pragma unroll
                for (int n = 0; n < NB; ++n) bf[(t + 1) & 1][n] = hb[(n + ky) * HC + kx];
#pragma unroll
                for (int m = 0; m < 4; ++m) af[(t + 1) & 1][m] = wl[((t + 1) * 4 * WM + m) * 64];
            }
            // the next tap's reads stay ahead of this tap's products (a
            // single wave per SIMD would otherwise wait on each read)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int n = 0; n < NB; ++n)
                    acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[t & 1][m], bf[t & 1][n],
                                                                    acc[m][n], 0, 0, 0);
        }
        }
        }
        if (more) halo_store(buf ^ 1, pre);
        chunk_barrier();
    }
    // (KS = 2) the groups' sums meet in LDS and each group finishes half of
    // the tile rows, group 0 the first NB/2 and group 1 the rest: each hands
    // the other its partial of the other's rows (the sums are the same either
    // way round, a + b = b + a), so the epilogue's loads and stores run on
    // all 8 waves (convq over r*h at 256 x 256: 127 against 136-137 us when
    // group 0 finished every row)
    int n_lo = 0, n_hi = NB;
    if constexpr (KS > 1) {
        static_assert(KS == 2, "two wave groups");
        constexpr int HN = NB / 2;
        __shared__ v4f xch[2][4][HN][kThreads];
        if (ks == 0) {
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int j = 0; j < HN; ++j) xch[0][m][j][tid] = acc[m][HN + j];
        } else {
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int j = 0; j < HN; ++j) xch[1][m][j][tid] = acc[m][j];
        }
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int j = 0; j < HN; ++j) acc[m][j] += xch[1][m][j][tid];
        } else {
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int j = 0; j < HN; ++j) acc[m][HN + j] += xch[0][m][j][tid];
        }
        n_lo = ks == 0 ? 0 : HN;
        n_hi = n_lo + HN;
    }

    // epilogue: lane (g, col), register r of acc[m][n] is output channel
    // 16 (mb0 + m) + 4 g + r (in the packed order) at pixel
    // (ty0 + wn NB + n, tx0 + col)
    const int x = tx0 + col;
    if constexpr (EPI == kHeads) {
        // The rest of head h = blockIdx.y (the wave's 64 channels, WM = 1) on
        // the matrix cores, every lane taking part (lanes past the map
        // compute on the zero padding and store nothing):
        //   a = relu(acc + b0);  t = relu(W2 a + b2);  out = W4 t + b4.
        // acc[m][n] holds channels {16 m + 4 g + r} at lane (g, col), which
        // is the B operand of a step whose 4 inputs are those channels, so
        // both 1x1 layers read the previous layer's registers directly, their
        // weights packed in that input order (the last-layer layout).
        static_assert(WM == 1, "one head per wave");
        const int h = blockIdx.y;
        const __amdgpu_buffer_rsrc_t w2 =
            weights_rsrc(a.w2q + (size_t)h * (16 * 4 * 64), 16 * 4 * 64 * 4);
        const float* b0 = a.b0 + 64 * h;
        const float* b2 = a.b1 + 64 * h;
        const int nout = a.outs[h];
        const int nob = (nout + 15) / 16;
        const __amdgpu_buffer_rsrc_t w4 = weights_rsrc(a.w4p[h], 4096u * nob);
        const uint32_t lb = 4u * lane, gb = 16u * g;  // this lane's byte offsets
        const float* b4 = a.b4[h];
        // (the biases' loads are unconditional, from the weights when there is
        // no bias, at a clamped index, and masked where used: under a branch
        // the compiler could not count them, and the products waited for the
        // next block's weights with them)
        const float* b4s = b4 ? b4 : a.w4p[h];
        float* out = a.hout[h];
        // Each step's 4 weights are loaded one step ahead of its products
        // from buffer descriptors (a scheduling barrier keeps them there and
        // keeps the compiler from hoisting every weight load at once, and
        // the descriptors keep 64-bit addresses out of the registers): 162
        // VGPRs, three workgroups per CU.  (256 x 256, 3 heads: 172 us
        // against 182 for the 3x3 layer and bvml_dsine_heads_mlp_f32, 166
        // with the loads below issued ahead; two tile rows per pass,
        // 173-174.)
        {
            // the loads the epilogue's first steps wait on go out together:
            // b0, then the middle layer's first weights
            float b0v[4][4];
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r) b0v[m][r] = ldo(b0, gb + 4u * (16 * m + r));
            float cw[2][4];
#pragma unroll
            for (int r = 0; r < 4; ++r) cw[0][r] = ldw(w2, lb, 256u * r);
            __builtin_amdgcn_sched_barrier(0);
            // a = relu(acc + b0), in place
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
#pragma unroll
                    for (int j = 0; j < NB; ++j)
                        acc[m][j][r] = relu(acc[m][j][r] + b0v[m][r]);
                }
            // t = W2 a: output block mo, step (m, r) takes channels {16 m + 4 g + r}
            v4f t[4][NB];
#pragma unroll
            for (int mo = 0; mo < 4; ++mo)
#pragma unroll
                for (int j = 0; j < NB; ++j) t[mo][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            // b2 and the last layer's first weights and biases, loaded during
            // the middle layer's products (at steps 8 and 12), so that no
            // step waits on a load of its own: with each of them loaded where
            // it is used, every workgroup of the launch stalled on the same
            // round trips at once (256 x 256, 3 heads: 171 against 166 us,
            // same bits)
            float b2v[4][4], cw4[2][4], b4cur[4], b4nxt[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < 16; ++st) {  // st = 4 mo + m
                if (st + 1 < 16) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        cw[(st + 1) & 1][r] = ldw(w2, lb, 256u * ((st + 1) * 4 + r));
                }
                if (st == 8) {
#pragma unroll
                    for (int mo = 0; mo < 4; ++mo)
#pragma unroll
                        for (int r = 0; r < 4; ++r) b2v[mo][r] = ldo(b2, gb + 4u * (16 * mo + r));
                }
                if (st == 12) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) cw4[0][r] = ldw(w4, lb, 256u * r);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int oc = 4 * g + r;
                        b4cur[r] = ldo(b4s, 4u * (uint32_t)(oc < nout ? oc : nout - 1));
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                const int mo = st / 4, m = st % 4;
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int j = 0; j < NB; ++j)
                        t[mo][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            cw[st & 1][r], acc[m][j][r], t[mo][j], 0, 0, 0);
            }
            // t = relu(t + b2)
#pragma unroll
            for (int mo = 0; mo < 4; ++mo)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
#pragma unroll
                    for (int j = 0; j < NB; ++j) t[mo][j][r] = relu(t[mo][j][r] + b2v[mo][r]);
                }
            // out = W4 t + b4, 16 outputs at a time; the next block's first
            // weights and biases load during this block's last step
            for (int ob = 0; ob < nob; ++ob) {
                const uint32_t wb = 4096u * ob;
                v4f o[NB];
#pragma unroll
                for (int j = 0; j < NB; ++j) o[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int mo = 0; mo < 4; ++mo) {
                    if (mo + 1 < 4) {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            cw4[(mo + 1) & 1][r] = ldw(w4, lb, wb + 256u * ((mo + 1) * 4 + r));
                    } else {
                        // (the last block loads its own again, unused: under a
                        // branch these loads would leave the compiler waiting
                        // for them before this step's products)
                        const int nx = ob + 1 < nob ? ob + 1 : ob;
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            cw4[0][r] = ldw(w4, lb, 4096u * (uint32_t)nx + 256u * r);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int oc = 16 * nx + 4 * g + r;
                            b4nxt[r] = ldo(b4s, 4u * (uint32_t)(oc < nout ? oc : nout - 1));
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int j = 0; j < NB; ++j)
                            o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(cw4[mo & 1][r], t[mo][j][r],
                                                                        o[j], 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int oc = 16 * ob + 4 * g + r;
                    if (x >= a.W || oc >= nout) continue;
                    const float bias = b4cur[r];
                    // plane 16 ob + r from a uniform base, plus this lane's
                    // 4 g planes and pixel as a 32-bit byte offset (the map is
                    // at most 2^26 pixels)
                    float* ob_base = out + (size_t)(16 * ob + r) * a.HW;
#pragma unroll
                    for (int j = 0; j < NB; ++j) {
                        const int n = j, y = ty0 + wn * NB + n;
                        if (n < n_lo || n >= n_hi || y >= a.H) continue;
                        const uint32_t off = 4u * (uint32_t)(4 * g * a.HW + y * a.W + x);
                        *reinterpret_cast<float*>(reinterpret_cast<char*>(ob_base) + off) =
                            b4 ? o[j][r] + bias : o[j][r];
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) b4cur[r] = b4nxt[r];
            }
        }
        return;
    }
    if (x >= a.W) return;
    if constexpr (EPI == kPlain) {
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const int y = ty0 + wn * NB + n;
            if (n < n_lo || n >= n_hi || y >= a.H) continue;
            const size_t px = (size_t)y * a.W + x;
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int o = 16 * (mb0 + m) + 4 * g + r;
                    if (o < a.cout) a.out[(size_t)o * a.HW + px] = acc[m][n][r];
                }
        }
        return;
    }
    // The ConvGRU epilogues read the biases and the maps h (and z) and store
    // the gates (the new state).  Every load goes out before the first
    // store: the outputs may not overlap the inputs (the entry points refuse
    // that), but the compiler cannot know it, and with each element's loads
    // after the previous element's stores a wave waited one round trip per
    // element, every workgroup at once (convz + convr over h at 256 x 256:
    // a 30 us epilogue of 64 such elements per lane).
    if constexpr (EPI == kGates) {
        // M-blocks alternate z, r: block 2i holds z channels 16i.., 2i + 1
        // the r channels 16i.. (mb0 is a multiple of 4, so m = 0, 2 are z)
        float bz[2][4], br[2][4], hv[NB][2][4];
#pragma unroll
        for (int mm = 0; mm < 2; ++mm)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // (a clamped index, no branch: a load under a per-lane
                // condition made the next one wait for everything before it)
                const int c = 16 * ((mb0 + 2 * mm) / 2) + 4 * g + r;
                const int cc = c < a.cout / 2 ? c : a.cout / 2 - 1;
                bz[mm][r] = a.b0[cc];
                br[mm][r] = a.b1[cc];
            }
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const int y = ty0 + wn * NB + n;
            const bool row = n >= n_lo && n < n_hi && y < a.H;
            const size_t px = row ? (size_t)y * a.W + x : 0;
#pragma unroll
            for (int mm = 0; mm < 2; ++mm)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int c = 16 * ((mb0 + 2 * mm) / 2) + 4 * g + r;
                    hv[n][mm][r] = (row && c < a.cout / 2) ? a.h[(size_t)c * a.HW + px] : 0.0f;
                }
        }
        // (all of them here: a use after some of the stores below would wait
        // for those stores too, the loads being conditional)
        __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const int y = ty0 + wn * NB + n;
            if (n < n_lo || n >= n_hi || y >= a.H) continue;
            const size_t px = (size_t)y * a.W + x;
#pragma unroll
            for (int mm = 0; mm < 2; ++mm)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = 2 * mm;
                    const int c = 16 * ((mb0 + m) / 2) + 4 * g + r;
                    if (c >= a.cout / 2) continue;
                    const size_t i = (size_t)c * a.HW + px;
                    const float zz = sigmoid(acc[m][n][r] + bz[mm][r]);
                    const float rr = sigmoid(acc[m + 1][n][r] + br[mm][r]);
                    a.o0[i] = zz;
                    a.o1[i] = rr * hv[n][mm][r];
                }
        }
    } else {
        float bq[4][4], zv[NB][4][4], hv[NB][4][4];
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int c = 16 * (mb0 + m) + 4 * g + r;
                bq[m][r] = a.b0[c < a.cout ? c : a.cout - 1];
            }
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const int y = ty0 + wn * NB + n;
            const bool row = n >= n_lo && n < n_hi && y < a.H;
            const size_t px = row ? (size_t)y * a.W + x : 0;
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int c = 16 * (mb0 + m) + 4 * g + r;
                    const bool ok = row && c < a.cout;
                    const size_t i = (size_t)c * a.HW + px;
                    zv[n][m][r] = ok ? a.z[i] : 0.0f;
                    hv[n][m][r] = ok ? a.h[i] : 0.0f;
                }
        }
        __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const int y = ty0 + wn * NB + n;
            if (n < n_lo || n >= n_hi || y >= a.H) continue;
            const size_t px = (size_t)y * a.W + x;
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int c = 16 * (mb0 + m) + 4 * g + r;
                    if (c >= a.cout) continue;
                    const size_t i = (size_t)c * a.HW + px;
                    const float v = gru_mix(zv[n][m][r], hv[n][m][r], tanhf(acc[m][n][r] + bq[m][r]));
                    a.o0[i] = v;
                    if (a.o1) a.o1[i] = v;
                }
        }
    }
}

// Workgroups below which a launch splits the input channels over two wave
// groups (fewer than two 4-wave workgroups per CU).
constexpr long long kSplitGrid = 512;

template <int K, int TH, int WM, int WN, int EPI>
int launch(const ConvArgs& a0, hipStream_t stream, const char* op) {
    ConvArgs a = a0;
    a.tiles_x = (a.W + kTW - 1) / kTW;
    const int tiles_y = (a.H + TH - 1) / TH;
    const int mtiles = a.mblocks / (4 * WM);
    const long long tiles = (long long)a.tiles_x * tiles_y;
    if (tiles > INT_MAX) return fail(BVML_DSINE_ESIZE, std::string(op) + ": too many tiles");
    const dim3 grid((unsigned)tiles, (unsigned)mtiles);
    // (waves of 8 tile rows hold 128 accumulators: two of them per SIMD
    // would spill, so those tiles never split)
    bool split = false;
    if constexpr (TH / WN <= 4) split = tiles * mtiles < kSplitGrid;
    if constexpr (TH / WN <= 4) {
        if (split)
            hipLaunchKernelGGL((conv_kernel<K, TH, WM, WN, EPI, 2>), grid, dim3(2 * kThreads), 0,
                               stream, a);
    }
    if (!split)
        hipLaunchKernelGGL((conv_kernel<K, TH, WM, WN, EPI, 1>), grid, dim3(kThreads), 0, stream,
                           a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail((int)e, std::string(op) + " launch: " + hipGetErrorString(e));
    return BVML_DSINE_OK;
}

using bvml::pack::conv_mblocks;

int check_common(const char* op, const float* x, int cin, int H, int W, const float* wp, int k) {
    if (H < 0 || W < 0 || cin < 1) return fail(BVML_DSINE_ESHAPE, std::string(op) + ": bad shape");
    if (k != 3 && k != 5) return fail(BVML_DSINE_EK, std::string(op) + ": k must be 3 or 5");
    if (!x || !wp) return fail(BVML_DSINE_ENULL, std::string(op) + ": x and wp must be non-NULL");
    if ((long long)H * W * (cin > 256 ? cin : 256) > (1LL << 40))
        return fail(BVML_DSINE_ESIZE, std::string(op) + ": map too large");
    return BVML_DSINE_OK;
}

}  // namespace

extern "C" {

int bvml_dsine_conv_f32(const float* x, int cin, int H, int W, const float* wp, int cout, int k,
                        float* out, void* stream) {
    if (int st = check_common("conv", x, cin, H, W, wp, k)) return st;
    if (cout < 1) return fail(BVML_DSINE_ESHAPE, "conv: bad shape");
    if (!out) return fail(BVML_DSINE_ENULL, "conv: out must be non-NULL");
    const long long HW = (long long)H * W;
    if (HW == 0) return BVML_DSINE_OK;
    if (overlaps(out, (size_t)cout * HW * 4, x, (size_t)cin * HW * 4))
        return fail(BVML_DSINE_EALIAS, "conv: out overlaps x");
    ConvArgs a{};
    a.x = x; a.wp = wp; a.out = out; a.cin = cin; a.cout = cout; a.H = H; a.W = W; a.HW = HW;
    a.mblocks = conv_mblocks(cout);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (a.mblocks % 8 == 0)
        return k == 5 ? launch<5, 16, 2, 2, kPlain>(a, s, "conv")
                      : launch<3, 16, 2, 2, kPlain>(a, s, "conv");
    return k == 5 ? launch<5, 16, 1, 4, kPlain>(a, s, "conv")
                  : launch<3, 16, 1, 4, kPlain>(a, s, "conv");
}

int bvml_dsine_conv_heads_f32(const float* x, int cin, int H, int W, const float* wp, int nheads,
                              const float* b0, const float* w2q, const float* b2,
                              const float* const* w4p, const float* const* b4, const int* outs,
                              float* const* out, void* stream) {
    if (int st = check_common("conv_heads", x, cin, H, W, wp, 3)) return st;
    if (nheads < 1 || nheads > 4)
        return fail(BVML_DSINE_EPARAM, "conv_heads: nheads must be 1..4");
    if (!b0 || !w2q || !b2 || !w4p || !b4 || !outs || !out)
        return fail(BVML_DSINE_ENULL, "conv_heads: pointers must be non-NULL");
    const long long HW = (long long)H * W;
    if (HW > (1LL << 26)) return fail(BVML_DSINE_ESIZE, "conv_heads: more than 2^26 pixels");
    ConvArgs a{};
    const size_t xb = (size_t)cin * HW * 4;
    for (int h = 0; h < nheads; ++h) {
        if (outs[h] < 1 || outs[h] > 4096)
            return fail(BVML_DSINE_EPARAM, "conv_heads: outs must be 1..4096");
        if (!w4p[h] || !out[h])
            return fail(BVML_DSINE_ENULL, "conv_heads: w4p and out must be non-NULL");
        const size_t ob = (size_t)outs[h] * HW * 4;
        if (overlaps(out[h], ob, x, xb))
            return fail(BVML_DSINE_EALIAS, "conv_heads: an output overlaps x");
        for (int e = 0; e < h; ++e)
            if (overlaps(out[h], ob, out[e], (size_t)outs[e] * HW * 4))
                return fail(BVML_DSINE_EALIAS, "conv_heads: outputs overlap");
        a.w4p[h] = w4p[h];
        a.b4[h] = b4[h];
        a.hout[h] = out[h];
        a.outs[h] = outs[h];
    }
    if (HW == 0) return BVML_DSINE_OK;
    a.x = x; a.wp = wp; a.cin = cin; a.cout = 64 * nheads; a.H = H; a.W = W; a.HW = HW;
    a.b0 = b0; a.b1 = b2; a.w2q = w2q;
    a.mblocks = conv_mblocks(64 * nheads);
    return launch<3, 16, 1, 4, kHeads>(a, static_cast<hipStream_t>(stream), "conv_heads");
}

int bvml_dsine_conv_gru_gates_sum_f32(const float* x, int cin, int H, int W, const float* wp,
                                      int C, const float* sum0, const float* bias_z,
                                      const float* bias_r, const float* h, float* z, float* rh,
                                      void* stream) {
    if (int st = check_common("conv_gru_gates", x, cin, H, W, wp, 5)) return st;
    if (C < 1 || C % 32 != 0)
        return fail(BVML_DSINE_ESHAPE, "conv_gru_gates: C must be a multiple of 32");
    if (!bias_z || !bias_r || !h || !z || !rh)
        return fail(BVML_DSINE_ENULL, "conv_gru_gates: pointers must be non-NULL");
    const long long HW = (long long)H * W;
    if (HW == 0) return BVML_DSINE_OK;
    const size_t xb = (size_t)cin * HW * 4, cb = (size_t)C * HW * 4;
    if (overlaps(z, cb, x, xb) || overlaps(rh, cb, x, xb) || overlaps(z, cb, rh, cb) ||
        overlaps(z, cb, h, cb) || overlaps(rh, cb, h, cb) ||
        (sum0 && (overlaps(z, cb, sum0, 2 * cb) || overlaps(rh, cb, sum0, 2 * cb))))
        return fail(BVML_DSINE_EALIAS,
                    "conv_gru_gates: z and rh must not overlap x, h, sum0 or each other");
    ConvArgs a{};
    a.x = x; a.wp = wp; a.cin = cin; a.cout = 2 * C; a.H = H; a.W = W; a.HW = HW;
    a.b0 = bias_z; a.b1 = bias_r; a.h = h; a.o0 = z; a.o1 = rh; a.s0 = sum0;
    a.mblocks = conv_mblocks(2 * C);
    if (a.mblocks % 8 == 0)
        return launch<5, 16, 2, 2, kGates>(a, static_cast<hipStream_t>(stream), "conv_gru_gates");
    return launch<5, 16, 1, 4, kGates>(a, static_cast<hipStream_t>(stream), "conv_gru_gates");
}

int bvml_dsine_conv_gru_gates_f32(const float* x, int cin, int H, int W, const float* wp,
                                  int C, const float* bias_z, const float* bias_r,
                                  const float* h, float* z, float* rh, void* stream) {
    return bvml_dsine_conv_gru_gates_sum_f32(x, cin, H, W, wp, C, nullptr, bias_z, bias_r, h, z,
                                             rh, stream);
}

int bvml_dsine_conv_gru_update_sum_f32(const float* x, int cin, int H, int W, const float* wp,
                                       int C, const float* sum0, const float* bias_q,
                                       const float* z, const float* h, float* h_new,
                                       float* h_copy, void* stream) {
    if (int st = check_common("conv_gru_update", x, cin, H, W, wp, 5)) return st;
    if (C < 1 || C % 64 != 0)
        return fail(BVML_DSINE_ESHAPE, "conv_gru_update: C must be a multiple of 64");
    if (!bias_q || !z || !h || !h_new)
        return fail(BVML_DSINE_ENULL, "conv_gru_update: pointers must be non-NULL");
    const long long HW = (long long)H * W;
    if (HW == 0) return BVML_DSINE_OK;
    const size_t xb = (size_t)cin * HW * 4, cb = (size_t)C * HW * 4;
    // h_new may be h itself (each element is read, then written, by the same
    // lane), but not a partial overlap of it: another lane's write would race
    // this lane's read
    if (overlaps(h_new, cb, x, xb) || (h_copy && overlaps(h_copy, cb, x, xb)) ||
        overlaps(h_new, cb, z, cb) || (h_new != h && overlaps(h_new, cb, h, cb)) ||
        (h_copy && (overlaps(h_copy, cb, z, cb) || overlaps(h_copy, cb, h, cb) ||
                    overlaps(h_copy, cb, h_new, cb))) ||
        (sum0 && (overlaps(h_new, cb, sum0, cb) || (h_copy && overlaps(h_copy, cb, sum0, cb)))))
        return fail(BVML_DSINE_EALIAS, "conv_gru_update: outputs overlap an input");
    ConvArgs a{};
    a.x = x; a.wp = wp; a.cin = cin; a.cout = C; a.H = H; a.W = W; a.HW = HW;
    a.b0 = bias_q; a.z = z; a.h = h; a.o0 = h_new; a.o1 = h_copy; a.s0 = sum0;
    a.mblocks = conv_mblocks(C);
    // 64 channels: one M tile of 4 blocks per wave, all four waves along the rows
    return launch<5, 16, 1, 4, kUpdate>(a, static_cast<hipStream_t>(stream), "conv_gru_update");
}

int bvml_dsine_conv_gru_update_f32(const float* x, int cin, int H, int W, const float* wp, int C,
                                   const float* bias_q, const float* z, const float* h,
                                   float* h_new, float* h_copy, void* stream) {
    return bvml_dsine_conv_gru_update_sum_f32(x, cin, H, W, wp, C, nullptr, bias_q, z, h, h_new,
                                              h_copy, stream);
}

}  // extern "C"
