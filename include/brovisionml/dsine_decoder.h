#pragma once

// The part of brovisionml's include/brovisionml/dsine_decoder.h (:96-102)
// that the refiner's interface uses: the decoder's /8-grid output, with the
// reference's names and layout.  A brovisionml build uses its own header in
// place of this one (the refiner reads no other member).

#include "brotensor/tensor.h"

namespace brovisionml::dsine {

// The decoder's maps on the /8 grid, flat NCHW (1, C*h8*w8) fp32.
struct DecoderOutput {
    brotensor::Tensor normal;   // (1, 3*h8*w8), L2-normalised over channels
    brotensor::Tensor feature;  // (1, 64*h8*w8)
    brotensor::Tensor hidden;   // (1, 64*h8*w8)
    int h8 = 0;
    int w8 = 0;
};

}  // namespace brovisionml::dsine
