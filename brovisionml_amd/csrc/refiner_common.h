// What the native refiner's device path (refiner.cpp) and host path
// (refiner_cpu.cpp) share: the loop's sizes, the checkpoint tensors it reads,
// the error state of bvml_dsine_refiner_last_error and forward's argument
// checks.  Private to libbvml_dsine_refine.so.
#pragma once

#include <cstddef>
#include <string>
#include <vector>

#include "bvml_dsine_refine.h"

namespace bvml_refine {

constexpr int kHidden = 64;           // hidden_dim (src/dsine_refine.cpp:172)
constexpr int kFeature = 64;          // the decoder's feature channels
constexpr int kX = kFeature + 2;      // feat_map = cat(feature, uv_8)
constexpr int kHx = kHidden + kX;     // cat(h, feat_map): 130
constexpr int kHin = kHidden + 2;     // cat(h_new, uv_8): 66
constexpr int kUp = 8;                // downsample_ratio (:24)
constexpr int kIter = 5;              // num_iter_test (:25)
constexpr int kPs = 5;                // the propagate's window
constexpr int kHeads = 4;
constexpr int kMid = 64;              // the heads' hidden width (:119-127)
constexpr float kUpEps = 1e-12f;      // l2_normalize_nchw_forward's eps (:281)
constexpr const char* kHeadName[kHeads] = {"prob_head", "xy_head", "angle_head",
                                           "up_prob_head"};
constexpr int kHeadOut[kHeads] = {kPs * kPs, 2 * kPs * kPs, kPs * kPs, 9 * kUp * kUp};

// One checkpoint tensor: its name, output channels and element count.
struct TensorSpec {
    std::string name;
    int c_out;
    long long numel;
};

// The tensors in a fixed order: gru.convz, convr, convq (weight, bias), then
// per head .0, .2, .4 (weight, bias).
const std::vector<TensorSpec>& specs();
int spec_index(const char* name);  // -1 for a name not in specs()

enum : int { kZw = 0, kZb, kRw, kRb, kQw, kQb, kHead0 };
// index of head h's layer (0, 1, 2 = .0, .2, .4) weight / bias
inline int head_w(int h, int layer) { return kHead0 + 6 * h + 2 * layer; }
inline int head_b(int h, int layer) { return head_w(h, layer) + 1; }

// Record msg as the calling thread's last error and return code.
int fail(int code, const std::string& msg);
const char* last_error();
bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes);

struct ForwardArgs {
    const float* normal;
    const float* feature;
    const float* hidden;
    int h8, w8;
    float fx, fy, cx, cy;
    int orig_h, orig_w, pad_t, pad_l, out_h, out_w;
    float* out;
    float* coarse;
};

// forward's argument checks (pointers, sizes, the crop, the intrinsics,
// weights present, no overlap), messages prefixed `who`; 0 or a status.
int check_forward(const std::vector<std::vector<float>>& host, const ForwardArgs& a,
                  const std::string& who);

// The host copy of the refiner's weights, one vector per spec.
const std::vector<std::vector<float>>& host_weights(const bvml_dsine_refiner* r);

// The device maps of one forward: [h | feature | uv], r*h, [h_new | uv], the
// update gate, the heads' 3x3 output, the heads' outputs, the two propagate
// buffers, the ray map, the full-resolution result before the crop, and the
// ConvGRU convolutions' parts over [feature | uv] (constant through the
// iterations: convz + convr's 128 channels in their packed order, then
// convq's 64).
struct Maps {
    float *hx, *rh, *hin, *z, *t0, *head[kHeads], *pred[2], *ray, *up, *cf;
};

// The planes of each map in Maps order (up: 3 * kUp^2 planes); each map
// starts on a 64-float boundary.
constexpr int kMapPlanes[] = {kHx, kHidden, kHin, kHidden, kHeads * kMid, kHeadOut[0],
                              kHeadOut[1], kHeadOut[2], kHeadOut[3], 3, 3, 3, 3 * kUp * kUp,
                              3 * kHidden};
inline size_t maps_floats(size_t hw) {
    size_t total = 0;
    for (int c : kMapPlanes) total += ((size_t)c * hw + 63) & ~(size_t)63;
    return total;
}
inline Maps maps_at(float* base, size_t hw) {
    Maps m{};
    float** order[] = {&m.hx,      &m.rh,      &m.hin,     &m.z,       &m.t0,
                       &m.head[0], &m.head[1], &m.head[2], &m.head[3], &m.pred[0],
                       &m.pred[1], &m.ray,     &m.up,      &m.cf};
    static_assert(sizeof(order) / sizeof(order[0]) == sizeof(kMapPlanes) / sizeof(kMapPlanes[0]),
                  "one plane count per map");
    size_t at = 0;
    for (size_t i = 0; i < sizeof(order) / sizeof(order[0]); ++i) {
        *order[i] = base + at;
        at += ((size_t)kMapPlanes[i] * hw + 63) & ~(size_t)63;
    }
    return m;
}

// The loop of the device forward on the maps m (refiner.cpp), after the
// checks, with the refiner's device current and its weights uploaded.
int forward_maps(bvml_dsine_refiner* r, const Maps& m, const ForwardArgs& a, void* stream);
int refiner_device(const bvml_dsine_refiner* r);    // -1 before the first forward
bool refiner_uploaded(const bvml_dsine_refiner* r);  // weights on the device and current

}  // namespace bvml_refine
