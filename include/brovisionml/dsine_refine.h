#pragma once

// DSINE NRN refiner -- drop-in for brovisionml's
// include/brovisionml/dsine_refine.h (:113-145): the same class, members and
// behaviour, so callers of Refiner (load / load_file, to, device, forward)
// compile against it unchanged.  forward runs the 5-iteration ConvGRU +
// AngMF loop of src/dsine_refine.cpp:212-294 and returns the last
// iteration's up-sampled normals cropped to the unpadded image.
//
// On the GPU (brotensor's CUDA tag, the HIP device) the loop is the native
// refiner of include/bvml_dsine_refine.h: this library's gfx950 kernels,
// asynchronously on the null stream.  On the CPU it is the library's host
// path: fp32 convolutions and the CPU branch of the ops, on host threads.
//
// Threads: forward is const, as the reference's, and may be called on one
// Refiner from several threads; the calls take a lock of the object's own
// (load, load_file and to take it too), since the device buffers, the
// uploaded weights and the grid-size state are shared by its forwards.
//
// Weights load from a safetensors file (F32, F16 or BF16, widened to fp32)
// under the top-level keys gru.conv{z,r,q}.*, {prob,xy,angle,up_prob}_head.*
// (src/dsine_refine.cpp:51-91).  Errors throw std::runtime_error prefixed
// "dsine::Refiner: " (src/dsine_refine.cpp:22-30).

#include <memory>
#include <string>

#include "brotensor/tensor.h"
#include "brovisionml/dsine_decoder.h"
#include "brovisionml/dsine_preprocess.h"

namespace brovisionml::dsine {

class Refiner {
public:
    Refiner();
    ~Refiner();
    Refiner(Refiner&&) noexcept;
    Refiner& operator=(Refiner&&) noexcept;

    // Loads <dir>/model.safetensors, or the file at `path`.
    void load(const std::string& dir);
    void load_file(const std::string& path);

    // The device forward runs on (CPU until called); the decoder output
    // passed to forward() must live there.
    void to(brotensor::Device dev);
    brotensor::Device device() const;

    // The refined normals as a (1, 3*H*W) tensor on the refiner's device,
    // H = tf.orig_h, W = tf.orig_w, L2-normalised per pixel.  `intrins` are
    // the raw preprocess intrinsics (the +0.5 is applied here); origH, origW
    // the padded dims (the /8 grid is dec.h8 x dec.w8).
    brotensor::Tensor forward(const DecoderOutput& dec, const Intrinsics& intrins, int origH,
                              int origW, const DsineTransform& tf) const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace brovisionml::dsine
