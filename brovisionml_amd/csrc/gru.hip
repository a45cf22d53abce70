// The refiner's elementwise work around its convolutions, fused (the C ABI's
// bvml_dsine_gru_gates_f32, bvml_dsine_gru_update_f32 and
// bvml_dsine_bias_act_f32).  The reference runs each step as its own
// brotensor op with a full pass over the maps (src/dsine_refine.cpp:104-159:
// conv2d_forward with its bias, sigmoid_forward twice, mul_inplace, two
// concat_nchw_channels, tanh_forward, clone, scale, add_scalar, two muls and
// an add for the ConvGRU; relu_forward after each head convolution).  Here the
// convolutions run without bias and these kernels apply the bias, the
// activation and the gate arithmetic in one pass each, writing straight into
// the channel slices the next convolution reads, so no concatenation is
// materialised.
//
// All maps are fp32 NCHW planes of HW floats; per-channel biases.  Every
// kernel is a grid-stride pass, four floats per lane where the planes and
// pointers allow it.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "bvml_dsine.h"
#include "status.h"

namespace {

using bvml::fail;

constexpr int kBlock = 256;

// The activations in the reference's form: sigmoid 1 / (1 + e^-x) and tanh,
// from the device math library's expf and tanhf (a few ulp each).
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// h_new = (1 - z) h + z q, products and sum rounded as the reference's chain
// of brotensor ops rounds them (src/dsine_refine.cpp:152-157): 1 - z exact
// (scale by -1, add 1), then two products and their sum.
__device__ __forceinline__ float gru_mix(float z, float h, float q) {
#pragma clang fp contract(off)
    const float omz = 1.0f - z;
    return omz * h + z * q;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// z = sigmoid(zr[c] + bz[c]), r = sigmoid(zr[C + c] + br[c]), rh = r * h for
// channel c of C; zr holds the 2C pre-activations (convz's channels, then
// convr's).
__global__ __launch_bounds__(kBlock) void gru_gates_kernel(const float* __restrict__ zr,
                                                           const float* __restrict__ bz,
                                                           const float* __restrict__ br,
                                                           const float* __restrict__ h, int C,
                                                           long long HW, float* __restrict__ z,
                                                           float* __restrict__ rh) {
    const long long n = (long long)C * HW;
    for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (long long)gridDim.x * kBlock) {
        const int c = (int)(i / HW);
        const float zz = sigmoid(zr[i] + bz[c]);
        const float rr = sigmoid(zr[n + i] + br[c]);
        z[i] = zz;
        rh[i] = rr * h[i];
    }
}

__global__ __launch_bounds__(kBlock) void gru_gates4_kernel(const float4* __restrict__ zr,
                                                            const float* __restrict__ bz,
                                                            const float* __restrict__ br,
                                                            const float4* __restrict__ h, int C,
                                                            long long HW4, float4* __restrict__ z,
                                                            float4* __restrict__ rh) {
    const long long n = (long long)C * HW4;
    for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (long long)gridDim.x * kBlock) {
        const int c = (int)(i / HW4);
        const float b0 = bz[c], b1 = br[c];
        const float4 a = zr[i], q = zr[n + i], hv = h[i];
        z[i] = make_float4(sigmoid(a.x + b0), sigmoid(a.y + b0), sigmoid(a.z + b0),
                           sigmoid(a.w + b0));
        rh[i] = make_float4(sigmoid(q.x + b1) * hv.x, sigmoid(q.y + b1) * hv.y,
                            sigmoid(q.z + b1) * hv.z, sigmoid(q.w + b1) * hv.w);
    }
}

// q = tanh(qp[c] + bq[c]); h_new = (1 - z) h + z q, into h_new and (if
// non-NULL) h_copy.  h_new may be h itself (each element is read before it
// is written).
__global__ __launch_bounds__(kBlock) void gru_update_kernel(const float* qp,
                                                            const float* __restrict__ bq,
                                                            const float* z, const float* h,
                                                            int C, long long HW, float* h_new,
                                                            float* h_copy) {
    const long long n = (long long)C * HW;
    for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (long long)gridDim.x * kBlock) {
        const int c = (int)(i / HW);
        const float v = gru_mix(z[i], h[i], tanhf(qp[i] + bq[c]));
        h_new[i] = v;
        if (h_copy) h_copy[i] = v;
    }
}

__global__ __launch_bounds__(kBlock) void gru_update4_kernel(const float4* qp,
                                                             const float* __restrict__ bq,
                                                             const float4* z, const float4* h,
                                                             int C, long long HW4, float4* h_new,
                                                             float4* h_copy) {
    const long long n = (long long)C * HW4;
    for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (long long)gridDim.x * kBlock) {
        const int c = (int)(i / HW4);
        const float b = bq[c];
        const float4 q = qp[i], zz = z[i], hh = h[i];
        const float4 v = make_float4(gru_mix(zz.x, hh.x, tanhf(q.x + b)),
                                     gru_mix(zz.y, hh.y, tanhf(q.y + b)),
                                     gru_mix(zz.z, hh.z, tanhf(q.z + b)),
                                     gru_mix(zz.w, hh.w, tanhf(q.w + b)));
        h_new[i] = v;
        if (h_copy) h_copy[i] = v;
    }
}

// x = act(x + bias[c]) in place; act 0: none, 1: ReLU, v < 0 ? 0 : v (a NaN
// passes through, as through torch.relu).
__global__ __launch_bounds__(kBlock) void bias_act_kernel(float* x, const float* __restrict__ b,
                                                          int C, long long HW, int relu) {
    const long long n = (long long)C * HW;
    for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (long long)gridDim.x * kBlock) {
        const int c = (int)(i / HW);
        const float v = x[i] + b[c];
        x[i] = (relu && v < 0.0f) ? 0.0f : v;
    }
}

__global__ __launch_bounds__(kBlock) void bias_act4_kernel(float4* x, const float* __restrict__ b,
                                                           int C, long long HW4, int relu) {
    const long long n = (long long)C * HW4;
    for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (long long)gridDim.x * kBlock) {
        const int c = (int)(i / HW4);
        const float bb = b[c];
        float4 v = x[i];
        v.x += bb;
        v.y += bb;
        v.z += bb;
        v.w += bb;
        if (relu) {
            v.x = (v.x < 0.0f) ? 0.0f : v.x;
            v.y = (v.y < 0.0f) ? 0.0f : v.y;
            v.z = (v.z < 0.0f) ? 0.0f : v.z;
            v.w = (v.w < 0.0f) ? 0.0f : v.w;
        }
        x[i] = v;
    }
}

// Grid for n work items: enough workgroups for every CU several times over,
// at most one item per lane.
unsigned grid_for(long long n) {
    const long long g = (n + kBlock - 1) / kBlock;
    return (unsigned)(g < 8192 ? (g < 1 ? 1 : g) : 8192);
}

int check_maps(const char* op, int C, long long HW) {
    if (C < 0 || HW < 0) return fail(BVML_DSINE_ESHAPE, std::string(op) + ": C and HW must be >= 0");
    if ((long long)C * HW > (1LL << 40))
        return fail(BVML_DSINE_ESIZE, std::string(op) + ": C*HW too large");
    return BVML_DSINE_OK;
}

}  // namespace

extern "C" {

int bvml_dsine_gru_gates_f32(const float* zr, const float* bias_z, const float* bias_r,
                             const float* h, int C, long long HW, float* z, float* rh,
                             void* stream) {
    int st = check_maps("gru_gates", C, HW);
    if (st != BVML_DSINE_OK) return st;
    if ((long long)C * HW == 0) return BVML_DSINE_OK;
    if (!zr || !bias_z || !bias_r || !h || !z || !rh)
        return fail(BVML_DSINE_ENULL, "gru_gates: all pointers must be non-NULL");
    const size_t map = (size_t)C * HW * sizeof(float);
    if (bvml::overlaps(z, map, zr, 2 * map) || bvml::overlaps(rh, map, zr, 2 * map) ||
        bvml::overlaps(z, map, h, map) || bvml::overlaps(rh, map, h, map) ||
        bvml::overlaps(z, map, rh, map))
        return fail(BVML_DSINE_EALIAS, "gru_gates: z and rh must not overlap zr, h or each other");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (HW % 4 == 0 && aligned16(zr) && aligned16(h) && aligned16(z) && aligned16(rh)) {
        const long long n4 = (long long)C * (HW / 4);
        hipLaunchKernelGGL(gru_gates4_kernel, dim3(grid_for(n4)), dim3(kBlock), 0, s,
                           reinterpret_cast<const float4*>(zr), bias_z, bias_r,
                           reinterpret_cast<const float4*>(h), C, HW / 4,
                           reinterpret_cast<float4*>(z), reinterpret_cast<float4*>(rh));
    } else {
        hipLaunchKernelGGL(gru_gates_kernel, dim3(grid_for((long long)C * HW)), dim3(kBlock), 0, s,
                           zr, bias_z, bias_r, h, C, HW, z, rh);
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? BVML_DSINE_OK
                           : fail((int)e, std::string("gru_gates launch: ") + hipGetErrorString(e));
}

int bvml_dsine_gru_update_f32(const float* q_pre, const float* bias_q, const float* z,
                              const float* h, int C, long long HW, float* h_new, float* h_copy,
                              void* stream) {
    int st = check_maps("gru_update", C, HW);
    if (st != BVML_DSINE_OK) return st;
    if ((long long)C * HW == 0) return BVML_DSINE_OK;
    if (!q_pre || !bias_q || !z || !h || !h_new)
        return fail(BVML_DSINE_ENULL, "gru_update: q_pre, bias_q, z, h and h_new must be non-NULL");
    const size_t map = (size_t)C * HW * sizeof(float);
    // h_new may be h (elementwise in place); nothing else may overlap
    if ((h_new != h && bvml::overlaps(h_new, map, h, map)) ||
        bvml::overlaps(h_new, map, q_pre, map) || bvml::overlaps(h_new, map, z, map) ||
        (h_copy && (bvml::overlaps(h_copy, map, h, map) || bvml::overlaps(h_copy, map, q_pre, map) ||
                    bvml::overlaps(h_copy, map, z, map) || bvml::overlaps(h_copy, map, h_new, map))))
        return fail(BVML_DSINE_EALIAS,
                    "gru_update: h_new (unless it is h) and h_copy must not overlap the inputs");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (HW % 4 == 0 && aligned16(q_pre) && aligned16(z) && aligned16(h) && aligned16(h_new) &&
        (!h_copy || aligned16(h_copy))) {
        const long long n4 = (long long)C * (HW / 4);
        hipLaunchKernelGGL(gru_update4_kernel, dim3(grid_for(n4)), dim3(kBlock), 0, s,
                           reinterpret_cast<const float4*>(q_pre), bias_q,
                           reinterpret_cast<const float4*>(z), reinterpret_cast<const float4*>(h),
                           C, HW / 4, reinterpret_cast<float4*>(h_new),
                           reinterpret_cast<float4*>(h_copy));
    } else {
        hipLaunchKernelGGL(gru_update_kernel, dim3(grid_for((long long)C * HW)), dim3(kBlock), 0,
                           s, q_pre, bias_q, z, h, C, HW, h_new, h_copy);
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? BVML_DSINE_OK
                           : fail((int)e, std::string("gru_update launch: ") + hipGetErrorString(e));
}

int bvml_dsine_bias_act_f32(float* x, const float* bias, int C, long long HW, int relu,
                            void* stream) {
    int st = check_maps("bias_act", C, HW);
    if (st != BVML_DSINE_OK) return st;
    if (relu != 0 && relu != 1) return fail(BVML_DSINE_EPARAM, "bias_act: relu must be 0 or 1");
    if ((long long)C * HW == 0) return BVML_DSINE_OK;
    if (!x || !bias) return fail(BVML_DSINE_ENULL, "bias_act: x and bias must be non-NULL");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (HW % 4 == 0 && aligned16(x)) {
        const long long n4 = (long long)C * (HW / 4);
        hipLaunchKernelGGL(bias_act4_kernel, dim3(grid_for(n4)), dim3(kBlock), 0, s,
                           reinterpret_cast<float4*>(x), bias, C, HW / 4, relu);
    } else {
        hipLaunchKernelGGL(bias_act_kernel, dim3(grid_for((long long)C * HW)), dim3(kBlock), 0, s,
                           x, bias, C, HW, relu);
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? BVML_DSINE_OK
                           : fail((int)e, std::string("bias_act launch: ") + hipGetErrorString(e));
}

}  // extern "C"
