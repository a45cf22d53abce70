// The native refiner's allocation-free forward
// (bvml_dsine_refiner_forward_noalloc): the loop of bvml_dsine_refiner_forward
// on maps placed in `scratch`, a fixed device array of this library, for
// callers that cannot allocate device memory.  It makes no hipMalloc, hipFree
// or MIOpen call: the heads' 3x3 layer runs on this library's convolution
// kernel (bvml_dsine_conv_f32) instead of MIOpen, and the weights must
// already be on the device (a bvml_dsine_refiner_forward since the last
// weight change uploads them).  Every call on one GPU uses that GPU's copy of
// `scratch`: calls that overlap on one GPU race.  Nothing in `scratch` needs
// to start at zero: each forward writes every map before it reads it.

#include <hip/hip_runtime.h>

#include <cstddef>
#include <mutex>
#include <string>

#include "bvml_dsine_refine.h"
#include "refiner_common.h"

namespace {

using namespace bvml_refine;

// 32 MiB: the maps of a grid of up to about 5,500 pixels (1,523 planes per
// pixel; a 60 x 80 grid, the refiner's size for a 480 x 640 image, needs
// 7,310,400 floats).
constexpr size_t kScratchFloats = size_t(8) << 20;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
hipError_t g_status[kMaxDevices];
void* g_scratch[kMaxDevices];  // each device's address of its copy of `scratch`

// Set-up, once per device, with that device current: the address of this
// device's copy of `scratch` (host code uses it, never the array's name).
int scratch_on(int dev, float** out) {
    if (dev < 0 || dev >= kMaxDevices)
        return fail(BVML_DSINE_EUNSUP, "forward_noalloc: device index beyond " +
                                           std::to_string(kMaxDevices - 1));
    std::call_once(g_once[dev], [dev] {
        g_status[dev] = hipGetSymbolAddress(&g_scratch[dev], HIP_SYMBOL(scratch));
    });
    if (g_status[dev] != hipSuccess)
        return fail((int)g_status[dev], std::string("forward_noalloc: hipGetSymbolAddress: ") +
                                            hipGetErrorString(g_status[dev]));
    *out = static_cast<float*>(g_scratch[dev]);
    return BVML_DSINE_OK;
}

}  // namespace

extern "C" int bvml_dsine_refiner_forward_noalloc(bvml_dsine_refiner* r, const float* normal,
                                                  const float* feature, const float* hidden,
                                                  int h8, int w8, float fx, float fy, float cx,
                                                  float cy, int orig_h, int orig_w, int pad_t,
                                                  int pad_l, int out_h, int out_w, float* out,
                                                  float* coarse, void* stream) {
    if (!r) return fail(BVML_DSINE_ENULL, "forward_noalloc: refiner must be non-NULL");
    const ForwardArgs args{normal, feature, hidden, h8, w8, fx, fy, cx, cy, orig_h, orig_w,
                           pad_t, pad_l, out_h, out_w, out, coarse};
    if (const int st = check_forward(host_weights(r), args, "forward_noalloc: ")) return st;
    const size_t hw = (size_t)h8 * w8, need = maps_floats(hw);
    if (need > kScratchFloats)
        return fail(BVML_DSINE_ESIZE,
                    "forward_noalloc: a " + std::to_string(h8) + " x " + std::to_string(w8) +
                        " grid needs " + std::to_string(need) + " floats of scratch; the maximum is " +
                        std::to_string(kScratchFloats) + " (about 5,500 pixels)");
    const int dev = refiner_device(r);
    if (dev < 0 || !refiner_uploaded(r))
        return fail(BVML_DSINE_EWEIGHTS,
                    "forward_noalloc: the weights are not on the device; run "
                    "bvml_dsine_refiner_forward once after setting them");
    int prev = -1;
    hipError_t e = hipGetDevice(&prev);
    if (e != hipSuccess) return fail((int)e, "forward_noalloc: hipGetDevice failed");
    if (prev != dev && (e = hipSetDevice(dev)) != hipSuccess)
        return fail((int)e, "forward_noalloc: hipSetDevice failed");
    float* base = nullptr;
    int st = scratch_on(dev, &base);
    if (st == BVML_DSINE_OK) st = forward_maps(r, maps_at(base, hw), args, stream, true);
    if (prev != dev) (void)hipSetDevice(prev);
    return st;
}
