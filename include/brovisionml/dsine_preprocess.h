#pragma once

// The part of brovisionml's include/brovisionml/dsine_preprocess.h (:48-66)
// that the refiner's interface uses: the letterbox transform and the
// preprocess intrinsics, with the reference's names, types and defaults.  A
// brovisionml build uses its own header in place of this one (the refiner
// reads no other member).

namespace brovisionml::dsine {

// Pad-to-a-multiple-of-32 transform of the input image
// (include/brovisionml/dsine_preprocess.h:48-57).
struct DsineTransform {
    int orig_w = 0;
    int orig_h = 0;
    int pad_w = 0;  // multiple of 32, what the model sees
    int pad_h = 0;
    int pad_l = 0;  // zero-pad on the left
    int pad_r = 0;
    int pad_t = 0;  // zero-pad on the top
    int pad_b = 0;
};

// Pinhole intrinsics in pixels of the padded image, before the +0.5 on the
// principal point (include/brovisionml/dsine_preprocess.h:61-66).
struct Intrinsics {
    float fx = 0.0f;
    float fy = 0.0f;
    float cx = 0.0f;
    float cy = 0.0f;
};

}  // namespace brovisionml::dsine
