#pragma once

// Compile check only: brotensor::Tensor as brovisionml's sources use it,
// declarations and no definitions.  brotensor is a sibling repository that
// the reference does not vendor, so each member below is one that a
// reference source file touches:
//   Device { CPU, CUDA, Metal }  src/dsine_refine.cpp:166,225 (CPU), the CUDA
//                                launcher src/dsine_ops.cu:178 (CUDA), brotensor's
//                                Metal backend (CMakeLists.txt:21-24)
//   Dtype::FP32, .dtype          src/sam_mask_decoder.cpp:357
//   .device .data .rows .cols    src/dsine_ops.cu:165-186, src/dinov2.cpp:260
//   mat(rows, cols)              src/dsine_ops.cpp:83
//   zeros_on(dev, rows, cols[, dtype])  src/dsine_ops.cu:178, src/sam.cpp:179
//   empty_on(dev, rows, cols[, dtype])  src/sam_mask_decoder.cpp:297
//   host_f32() / host_f32_mut()  src/dsine_ops.cpp:84-89
//   to(dev)                      src/dsine_refine.cpp:201
// The library's C++ layer and launchers header must compile against this
// header (no other enumerator, no other member), which is what makes them a
// drop-in next to brotensor's real header.

namespace brotensor {

enum class Device { CPU, CUDA, Metal };
enum class Dtype { FP32, FP16 };

class Tensor {
public:
    Device device;
    Dtype dtype;
    void* data;
    int rows;
    int cols;

    static Tensor mat(int rows, int cols);
    static Tensor zeros_on(Device dev, int rows, int cols, Dtype dtype = Dtype::FP32);
    static Tensor empty_on(Device dev, int rows, int cols, Dtype dtype = Dtype::FP32);
    const float* host_f32() const;
    float* host_f32_mut();
    Tensor to(Device dev) const;
};

}  // namespace brotensor
