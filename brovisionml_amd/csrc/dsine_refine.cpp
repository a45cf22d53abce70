// brovisionml::dsine::Refiner (include/brovisionml/dsine_refine.h): the class
// of the reference's include/brovisionml/dsine_refine.h:113-145 and
// src/dsine_refine.cpp:161-294 over the native refiner's C ABI
// (include/bvml_dsine_refine.h).  The weights live in the native refiner
// (host copy; the device copy is made at the first GPU forward); to() only
// records the device, as the reference's to() is the point after which
// forward runs there.  forward dispatches on that device: brotensor's CUDA
// tag (the HIP device) runs the device path on the null stream, CPU the host
// path.  Uses only the brotensor::Tensor members of include/brotensor/tensor.h,
// so it compiles against brotensor's own header too.

#include "brovisionml/dsine_refine.h"

#include <cstddef>
#include <mutex>
#include <stdexcept>
#include <string>

#include "bvml_dsine_refine.h"

namespace brovisionml::dsine {

namespace {

using brotensor::Device;
using brotensor::Tensor;

const std::string kWho = "dsine::Refiner: ";

[[noreturn]] void fail(const std::string& msg) { throw std::runtime_error(kWho + msg); }

[[noreturn]] void fail_status(int st) {
    throw std::runtime_error(kWho + bvml_dsine_refiner_last_error() + " (status " +
                             std::to_string(st) + ")");
}

void need_map(const Tensor& t, Device dev, std::size_t n, const char* name) {
    if (t.device != dev) fail(std::string("decoder ") + name + " is not on the refiner's device");
    const std::size_t have = static_cast<std::size_t>(t.rows) * static_cast<std::size_t>(t.cols);
    if (have != n)
        fail(std::string("decoder ") + name + " holds " + std::to_string(have) +
             " elements, expected " + std::to_string(n));
    if (n != 0 && t.data == nullptr) fail(std::string("decoder ") + name + " has no storage");
}

}  // namespace

// The engine's device buffers, uploaded weights and grid-size state are
// shared by every forward of the object, so each call holds `mu` while it
// uses the engine: forward is const (the reference's signature) and may be
// called from several threads.
struct Refiner::Impl {
    bvml_dsine_refiner* engine = nullptr;
    bool loaded = false;
    Device device = Device::CPU;
    mutable std::mutex mu;

    Impl() {
        if (const int st = bvml_dsine_refiner_create(&engine)) fail_status(st);
    }
    ~Impl() { bvml_dsine_refiner_destroy(engine); }
    Impl(const Impl&) = delete;
    Impl& operator=(const Impl&) = delete;
};

Refiner::Refiner() : impl_(std::make_unique<Impl>()) {}
Refiner::~Refiner() = default;
Refiner::Refiner(Refiner&&) noexcept = default;
Refiner& Refiner::operator=(Refiner&&) noexcept = default;

void Refiner::load(const std::string& dir) { load_file(dir + "/model.safetensors"); }

void Refiner::load_file(const std::string& path) {
    std::lock_guard<std::mutex> lock(impl_->mu);
    if (const int st = bvml_dsine_refiner_load_file(impl_->engine, path.c_str())) fail_status(st);
    impl_->loaded = true;
}

void Refiner::to(Device dev) {
    std::lock_guard<std::mutex> lock(impl_->mu);
    if (!impl_->loaded) fail("to() called before load()");
    if (dev != Device::CPU && dev != Device::CUDA)
        fail("to(): a device this library does not run (CPU and the HIP GPU only)");
    impl_->device = dev;
}

Device Refiner::device() const {
    std::lock_guard<std::mutex> lock(impl_->mu);
    return impl_->device;
}

Tensor Refiner::forward(const DecoderOutput& dec, const Intrinsics& intrins, int origH, int origW,
                        const DsineTransform& tf) const {
    const Impl& m = *impl_;
    std::lock_guard<std::mutex> lock(m.mu);
    if (!m.loaded) fail("forward() called before load()");
    if (dec.h8 < 1 || dec.w8 < 1) fail("forward(): the decoder grid is empty");
    const std::size_t hw = static_cast<std::size_t>(dec.h8) * static_cast<std::size_t>(dec.w8);
    need_map(dec.normal, m.device, 3 * hw, "normal");
    need_map(dec.feature, m.device, 64 * hw, "feature");
    need_map(dec.hidden, m.device, 64 * hw, "hidden");
    if (tf.orig_h < 1 || tf.orig_w < 1) fail("forward(): the transform's image is empty");
    Tensor out = Tensor::empty_on(m.device, 1, 3 * tf.orig_h * tf.orig_w);
    const float* n = static_cast<const float*>(dec.normal.data);
    const float* f = static_cast<const float*>(dec.feature.data);
    const float* h = static_cast<const float*>(dec.hidden.data);
    float* o = static_cast<float*>(out.data);
    const int st =
        m.device == Device::CPU
            ? bvml_dsine_refiner_forward_cpu(m.engine, n, f, h, dec.h8, dec.w8, intrins.fx,
                                             intrins.fy, intrins.cx, intrins.cy, origH, origW,
                                             tf.pad_t, tf.pad_l, tf.orig_h, tf.orig_w, o, nullptr,
                                             0)
            : bvml_dsine_refiner_forward(m.engine, n, f, h, dec.h8, dec.w8, intrins.fx,
                                         intrins.fy, intrins.cx, intrins.cy, origH, origW,
                                         tf.pad_t, tf.pad_l, tf.orig_h, tf.orig_w, o, nullptr,
                                         nullptr);
    if (st != 0) fail_status(st);
    return out;
}

}  // namespace brovisionml::dsine
