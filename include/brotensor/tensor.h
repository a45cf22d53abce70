#pragma once

// The subset of brotensor::Tensor that brovisionml's DSINE ops touch
// (src/dsine_ops.cpp:57-89, src/dsine_ops.cu:178), with brotensor's own names:
// the device tag (brotensor's enumerators CPU, CUDA and Metal; a HIP build of
// brotensor runs its GPU device under the CUDA tag), a raw data pointer, the
// (rows, cols) fp32 matrix shape, the mat / zeros_on / empty_on constructors,
// the host accessors and to().  This library's C++ layer uses nothing else, so
// it compiles unchanged against brotensor's own header
// (tests/cpp/brotensor_api/ checks that).  Storage is reference-counted:
// copies share it, as brotensor's tensors do.

#include <cstddef>
#include <memory>

namespace brotensor {

enum class Device { CPU, CUDA, Metal };

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
    // Uninitialised fp32 (rows x cols) matrix on `dev`.
    static Tensor empty_on(Device dev, int rows, int cols);

    // Host views; throw std::runtime_error unless device == CPU.
    const float* host_f32() const;
    float* host_f32_mut();

    // Deep copy onto `dev` (the same tensor when already there).
    Tensor to(Device dev) const;

private:
    std::shared_ptr<void> storage_;
};

}  // namespace brotensor
