#pragma once

// The subset of brotensor::Tensor that brovisionml's DSINE ops touch
// (src/dsine_ops.cpp:57-89, src/dsine_ops.cu:178): a device tag, a raw data
// pointer, a (rows, cols) fp32 matrix shape, mat / zeros_on constructors,
// host accessors and to().  brotensor itself is a separate project; when this
// library is built into brovisionml, brotensor's own header takes this one's
// place and nothing else changes.  Storage is reference-counted: copies share
// it, as brotensor's tensors do.

#include <cstddef>
#include <memory>

namespace brotensor {

enum class Device { CPU, HIP };

class Tensor {
public:
    Device device = Device::CPU;
    void* data = nullptr;
    int rows = 0;
    int cols = 0;

    Tensor() = default;

    // Uninitialised fp32 (rows x cols) matrix on the host.
    static Tensor mat(int rows, int cols);
    // Zero-filled fp32 (rows x cols) matrix on `dev`.
    static Tensor zeros_on(Device dev, int rows, int cols);

    std::size_t numel() const { return static_cast<std::size_t>(rows) * static_cast<std::size_t>(cols); }

    // Host views; throw std::runtime_error unless device == CPU.
    const float* host_f32() const;
    float* host_f32_mut();

    // Deep copy onto `dev` (the same tensor when already there).
    Tensor to(Device dev) const;

private:
    std::shared_ptr<void> storage_;
};

}  // namespace brotensor
