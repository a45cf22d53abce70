// Test infrastructure for gfx950 (nothing in the product links it):
//   * accuracy sweeps of the hardware transcendentals the fast kernels use
//     (v_sin_f32, v_cos_f32, v_rsq_f32, v_rcp_f32, v_exp_f32, v_sqrt_f32)
//     against double-precision references, over every float argument of a
//     range: the error bounds the kernels' budgets assume
//     (tests/test_gpu_hw_bounds.py);
//   * a streaming read of a buffer, the same-box read ceiling bench.py
//     reports beside the kernels' bandwidth;
//   * a launch loop: K calls of a C-ABI entry point (bvml_dsine_angmf_propagate_f32,
//     reached through the function pointer the caller passes) enqueued back
//     to back from C++ between two events (device-scope release, the HIP
//     flag for timing commands between events), behind a short bounded spin
//     kernel that holds the stream while the host enqueues them, so the
//     events time the K launches on the GPU, not the host's enqueueing.
// Every kernel writes one result per workgroup (the read: per wave), into
// arrays the host sizes to the grid, with vector stores (the spin kernel
// writes nothing).

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

enum Op { kSin = 0, kCos = 1, kRsq = 2, kRcp = 3, kExp2 = 4, kSqrt = 5 };

constexpr int kBlock = 256;
constexpr uint32_t kPerThread = 256;

// Largest absolute and relative error of op over the float bit patterns
// [lo, hi] (the range's magnitudes; `sign` the sign bit to give them), and
// the argument of the largest relative error, per workgroup.
__global__ __launch_bounds__(kBlock) void sweep(int op, uint32_t lo, uint32_t hi, uint32_t sign,
                                                double* out_abs, double* out_rel,
                                                uint32_t* out_arg) {
    __shared__ double sa[kBlock], sr[kBlock];
    __shared__ uint32_t sg[kBlock];
    const uint64_t t = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    double ma = 0.0, mr = 0.0;
    uint32_t marg = 0;
    for (uint32_t i = 0; i < kPerThread; ++i) {
        const uint64_t bits = (uint64_t)lo + t * kPerThread + i;
        if (bits > hi) break;
        const float x = __builtin_bit_cast(float, (uint32_t)bits | sign);
        double ref, got;
        switch (op) {
            case kSin: got = __builtin_amdgcn_sinf(x); ref = sin(2.0 * M_PI * (double)x); break;
            case kCos: got = __builtin_amdgcn_cosf(x); ref = cos(2.0 * M_PI * (double)x); break;
            case kRsq: got = __builtin_amdgcn_rsqf(x); ref = 1.0 / sqrt((double)x); break;
            case kRcp: got = __builtin_amdgcn_rcpf(x); ref = 1.0 / (double)x; break;
            case kExp2: got = __builtin_amdgcn_exp2f(x); ref = exp2((double)x); break;
            default: got = __builtin_amdgcn_sqrtf(x); ref = sqrt((double)x); break;
        }
        const double ea = fabs(got - ref);
        const double er = (ref != 0.0) ? ea / fabs(ref) : ea;
        if (ea > ma) ma = ea;
        if (er > mr) {
            mr = er;
            marg = (uint32_t)bits | sign;
        }
    }
    sa[threadIdx.x] = ma;
    sr[threadIdx.x] = mr;
    sg[threadIdx.x] = marg;
    __syncthreads();
    for (int s = kBlock / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            sa[threadIdx.x] = fmax(sa[threadIdx.x], sa[threadIdx.x + s]);
            if (sr[threadIdx.x + s] > sr[threadIdx.x]) {
                sr[threadIdx.x] = sr[threadIdx.x + s];
                sg[threadIdx.x] = sg[threadIdx.x + s];
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        out_abs[blockIdx.x] = sa[0];
        out_rel[blockIdx.x] = sr[0];
        out_arg[blockIdx.x] = sg[0];
    }
}

typedef float f4v __attribute__((ext_vector_type(4)));

// Sum of n floats (n4 float4s, then the tail): each lane issues U
// independent non-temporal float4 loads (coalesced, kBlock float4s apart)
// before using any, each wave reduces across its lanes and writes one
// partial; one launch covers the buffer once.  Reads 16 B per lane per load,
// writes 4 B per 64 * 16 * U bytes read.
template <int U>
__global__ __launch_bounds__(kBlock) void stream_read(const f4v* p, size_t n4, const float* tail,
                                                      int ntail, float* out) {
    const size_t base = (size_t)blockIdx.x * kBlock * U + threadIdx.x;
    f4v v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t i = base + (size_t)u * kBlock;
        v[u] = (i < n4) ? __builtin_nontemporal_load(p + i) : f4v{0.0f, 0.0f, 0.0f, 0.0f};
    }
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    if (blockIdx.x == 0 && (int)threadIdx.x < ntail) acc += tail[threadIdx.x];
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) out[(size_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6)] = acc;
}

// One wave that waits until `ticks` of the 100 MHz real-time counter have
// passed since it started (bounded: the host caps ticks), then exits.
__global__ __launch_bounds__(64) void spin(uint64_t ticks) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

typedef int (*angmf_fn)(const float*, const float*, const float*, const float*, const float*,
                        double, double, double, double, int, int, int, int, long long, float*,
                        unsigned, void*);

size_t read_grid(size_t n4, int u) { return (n4 + (size_t)kBlock * u - 1) / ((size_t)kBlock * u); }

uint32_t bits_of(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

}  // namespace

extern "C" {

// Largest errors of `op` over every float whose magnitude lies in [lo, hi]
// (0 <= lo <= hi), with the sign of `negative`.  Returns 0 or a hipError_t.
int bvml_probe_hw_error(int op, float lo, float hi, int negative, double* max_abs,
                        double* max_rel, float* argmax) {
    if (!(lo >= 0.0f) || !(hi >= lo)) return -1;
    const uint32_t blo = bits_of(lo), bhi = bits_of(hi);
    const uint64_t n = (uint64_t)bhi - blo + 1;
    const uint64_t threads = (n + kPerThread - 1) / kPerThread;
    const uint32_t blocks = (uint32_t)((threads + kBlock - 1) / kBlock);
    double *da = nullptr, *dr = nullptr;
    uint32_t* dg = nullptr;
    hipError_t e = hipMalloc(&da, blocks * sizeof(double));
    if (e == hipSuccess) e = hipMalloc(&dr, blocks * sizeof(double));
    if (e == hipSuccess) e = hipMalloc(&dg, blocks * sizeof(uint32_t));
    if (e == hipSuccess) {
        hipLaunchKernelGGL(sweep, dim3(blocks), dim3(kBlock), 0, 0, op, blo, bhi,
                           negative ? 0x80000000u : 0u, da, dr, dg);
        e = hipGetLastError();
    }
    std::vector<double> ha(blocks), hr(blocks);
    std::vector<uint32_t> hg(blocks);
    if (e == hipSuccess) e = hipMemcpy(ha.data(), da, blocks * sizeof(double), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(hr.data(), dr, blocks * sizeof(double), hipMemcpyDeviceToHost);
    if (e == hipSuccess)
        e = hipMemcpy(hg.data(), dg, blocks * sizeof(uint32_t), hipMemcpyDeviceToHost);
    if (e == hipSuccess) {
        double a = 0.0, r = 0.0;
        uint32_t g = 0;
        for (uint32_t i = 0; i < blocks; ++i) {
            a = std::fmax(a, ha[i]);
            if (hr[i] > r) {
                r = hr[i];
                g = hg[i];
            }
        }
        *max_abs = a;
        *max_rel = r;
        std::memcpy(argmax, &g, 4);
    }
    (void)hipFree(da);
    (void)hipFree(dr);
    (void)hipFree(dg);
    return (int)e;
}

// Partials of a streaming read of n floats at p into out (out_len floats,
// at least bvml_probe_read_partials(n, u)), U = u float4 loads per lane
// (1, 2, 4 or 8), on `stream`.
int bvml_probe_stream_read(const float* p, size_t n, int u, float* out, size_t out_len,
                           void* stream) {
    const size_t n4 = n / 4;
    const int ntail = (int)(n - 4 * n4);
    const size_t grid = read_grid(n4, u);
    if (grid == 0 || grid > 0x7fffffffu || out_len < grid * (kBlock / 64)) return -1;
    const dim3 g((unsigned)grid), b(kBlock);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const f4v* p4 = reinterpret_cast<const f4v*>(p);
    switch (u) {
        case 1: hipLaunchKernelGGL(stream_read<1>, g, b, 0, st, p4, n4, p + 4 * n4, ntail, out); break;
        case 2: hipLaunchKernelGGL(stream_read<2>, g, b, 0, st, p4, n4, p + 4 * n4, ntail, out); break;
        case 4: hipLaunchKernelGGL(stream_read<4>, g, b, 0, st, p4, n4, p + 4 * n4, ntail, out); break;
        case 8: hipLaunchKernelGGL(stream_read<8>, g, b, 0, st, p4, n4, p + 4 * n4, ntail, out); break;
        default: return -1;
    }
    return (int)hipGetLastError();
}

// K calls of `fn` (an angmf_propagate_f32 entry point), call i on the six
// device pointers ptrs[6 i .. 6 i + 5] (pred_norm, prob, xy, angle, ray, out),
// enqueued back to back on `stream` after a spin of spin_us microseconds
// (at most 100 ms), with events right after the spin and after the last
// call: *ms = the events' elapsed time.  Returns 0, the first non-zero
// status of fn, or a hipError_t.
int bvml_probe_angmf_loop(void* fn, const unsigned long long* ptrs, int K, double fu, double cu,
                          double fv, double cv, int B, int H, int W, int k, unsigned flags,
                          double spin_us, void* stream, float* ms) {
    if (!fn || !ptrs || K < 1 || !ms || !(spin_us >= 0.0) || spin_us > 1e5) return -1;
    const angmf_fn call = reinterpret_cast<angmf_fn>(fn);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    // device-scope release: the events time the launches without a system-scope
    // cache writeback of their own inside the timed region
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipEventCreateWithFlags(&e0, hipEventReleaseToDevice);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&e1, hipEventReleaseToDevice);
    int status = (int)e;
    if (e == hipSuccess) {
        hipLaunchKernelGGL(spin, dim3(1), dim3(64), 0, st, (uint64_t)(spin_us * 100.0));
        e = hipGetLastError();
        if (e == hipSuccess) e = hipEventRecord(e0, st);
        status = (int)e;
        for (int i = 0; i < K && status == 0; ++i) {
            const unsigned long long* p = ptrs + 6 * (size_t)i;
            status = call(reinterpret_cast<const float*>(p[0]), reinterpret_cast<const float*>(p[1]),
                          reinterpret_cast<const float*>(p[2]), reinterpret_cast<const float*>(p[3]),
                          reinterpret_cast<const float*>(p[4]), fu, cu, fv, cv, B, H, W, k, 0,
                          reinterpret_cast<float*>(p[5]), flags, stream);
        }
        if (status == 0 && (e = hipEventRecord(e1, st)) != hipSuccess) status = (int)e;
        if (status == 0 && (e = hipEventSynchronize(e1)) != hipSuccess) status = (int)e;
        if (status == 0 && (e = hipEventElapsedTime(ms, e0, e1)) != hipSuccess) status = (int)e;
        if (status != 0) (void)hipStreamSynchronize(st);
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    return status;
}

// The number of partials bvml_probe_stream_read writes for n floats.
size_t bvml_probe_read_partials(size_t n, int u) {
    return u > 0 ? (read_grid(n / 4, u) == 0 ? 1 : read_grid(n / 4, u)) * (kBlock / 64) : 0;
}

}  // extern "C"
