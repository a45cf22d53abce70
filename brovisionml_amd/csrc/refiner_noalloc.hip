// The native refiner's allocation-free forward
// (bvml_dsine_refiner_forward_noalloc): the loop of bvml_dsine_refiner_forward
// on maps placed in `scratch`, a fixed device array of this library, for
// callers that cannot allocate device memory.  It makes no hipMalloc or hipFree
// call (the same kernels as bvml_dsine_refiner_forward, so the same result,
// bit for bit), and the weights must already be on the device (a bvml_dsine_refiner_forward since the last
// weight change uploads them).  Every call on one GPU uses that GPU's copy of
// `scratch`, so calls on one GPU are put in order: each call's stream waits
// for an event recorded after the previous call's work, whatever stream that
// ran on (inside a stream capture the caller orders the replays).  Nothing in
// `scratch` needs to start at zero: each forward writes every map before it
// reads it.

#include <hip/hip_runtime.h>

#include <cstddef>
#include <mutex>
#include <string>

#include "bvml_dsine_refine.h"
#include "refiner_common.h"

namespace {

using namespace bvml_refine;

// 32 MiB: the maps of a grid of up to 5,086 pixels (1,649 planes per
// pixel; a 60 x 80 grid, the refiner's size for a 480 x 640 image, needs
// 7,915,200 floats).
constexpr size_t kScratchFloats = size_t(8) << 20;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;

// Per device: the address of its copy of `scratch` (host code uses it, never
// the array's name), an event recorded after the last call's work, and a
// lock held while a call waits for that event, enqueues its work and records
// the event again.
struct DeviceSlot {
    std::once_flag once;
    hipError_t status = hipSuccess;
    void* scratch = nullptr;
    hipEvent_t done = nullptr;
    bool recorded = false;
    std::mutex mu;
};
DeviceSlot g_slot[kMaxDevices];

// Set-up, once per device, with that device current.
int slot_on(int dev, DeviceSlot** out) {
    if (dev < 0 || dev >= kMaxDevices)
        return fail(BVML_DSINE_EUNSUP, "forward_noalloc: device index beyond " +
                                           std::to_string(kMaxDevices - 1));
    DeviceSlot& s = g_slot[dev];
    std::call_once(s.once, [&s] {
        s.status = hipGetSymbolAddress(&s.scratch, HIP_SYMBOL(scratch));
        if (s.status == hipSuccess)
            s.status = hipEventCreateWithFlags(&s.done, hipEventDisableTiming);
    });
    if (s.status != hipSuccess)
        return fail((int)s.status, std::string("forward_noalloc: set-up: ") +
                                       hipGetErrorString(s.status));
    *out = &s;
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
                        std::to_string(kScratchFloats) + " (about 5,000 pixels)");
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
    DeviceSlot* slot = nullptr;
    int st = slot_on(dev, &slot);
    if (st == BVML_DSINE_OK) {
        std::lock_guard<std::mutex> lock(slot->mu);
        const hipStream_t strm = static_cast<hipStream_t>(stream);
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(strm, &cap);
        const bool chain = e == hipSuccess && cap == hipStreamCaptureStatusNone;
        if (e != hipSuccess)
            st = fail((int)e, "forward_noalloc: hipStreamIsCapturing failed");
        else if (chain && slot->recorded &&
                 (e = hipStreamWaitEvent(strm, slot->done, 0)) != hipSuccess)
            st = fail((int)e, "forward_noalloc: hipStreamWaitEvent failed");
        if (st == BVML_DSINE_OK) {
            st = forward_maps(r, maps_at(static_cast<float*>(slot->scratch), hw), args, stream);
            // (recorded after a failed call too: the next call waits for
            // whatever this one enqueued)
            if (chain) {
                e = hipEventRecord(slot->done, strm);
                if (e == hipSuccess)
                    slot->recorded = true;
                else if (st == BVML_DSINE_OK)
                    st = fail((int)e, "forward_noalloc: hipEventRecord failed");
            }
        }
    }
    if (prev != dev) (void)hipSetDevice(prev);
    return st;
}
