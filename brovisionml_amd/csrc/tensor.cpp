// Minimal brotensor::Tensor storage (include/brotensor/tensor.h): host memory
// from operator new, device memory (the CUDA and Metal tags alike: the one
// HIP device) from hipMalloc, both reference-counted.

#include "brotensor/tensor.h"

#include <hip/hip_runtime.h>

#include <cstring>
#include <new>
#include <stdexcept>
#include <string>

namespace brotensor {

namespace {

[[noreturn]] void fail(const std::string& msg) { throw std::runtime_error("brotensor: " + msg); }

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(e));
}

std::shared_ptr<void> host_alloc(std::size_t bytes) {
    void* p = ::operator new(bytes == 0 ? 1 : bytes);
    return std::shared_ptr<void>(p, [](void* q) { ::operator delete(q); });
}

std::size_t elements(const Tensor& t) {
    return static_cast<std::size_t>(t.rows) * static_cast<std::size_t>(t.cols);
}

std::shared_ptr<void> device_alloc(std::size_t bytes) {
    void* p = nullptr;
    hip_check(hipMalloc(&p, bytes == 0 ? 1 : bytes), "hipMalloc");
    return std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
}

}  // namespace

Tensor Tensor::mat(int rows, int cols) {
    if (rows < 0 || cols < 0) fail("negative shape");
    Tensor t;
    t.rows = rows;
    t.cols = cols;
    t.storage_ = host_alloc(elements(t) * sizeof(float));
    t.data = t.storage_.get();
    return t;
}

Tensor Tensor::empty_on(Device dev, int rows, int cols) {
    if (rows < 0 || cols < 0) fail("negative shape");
    Tensor t;
    t.device = dev;
    t.rows = rows;
    t.cols = cols;
    const std::size_t bytes = elements(t) * sizeof(float);
    t.storage_ = (dev == Device::CPU) ? host_alloc(bytes) : device_alloc(bytes);
    t.data = t.storage_.get();
    return t;
}

Tensor Tensor::zeros_on(Device dev, int rows, int cols) {
    Tensor t = empty_on(dev, rows, cols);
    const std::size_t bytes = elements(t) * sizeof(float);
    if (dev == Device::CPU)
        std::memset(t.data, 0, bytes);
    else
        hip_check(hipMemset(t.data, 0, bytes), "hipMemset");
    return t;
}

const float* Tensor::host_f32() const {
    if (device != Device::CPU) fail("host_f32() on a device tensor");
    return static_cast<const float*>(data);
}

float* Tensor::host_f32_mut() {
    if (device != Device::CPU) fail("host_f32_mut() on a device tensor");
    return static_cast<float*>(data);
}

Tensor Tensor::to(Device dev) const {
    if (dev == device) return *this;
    Tensor t;
    t.device = dev;
    t.rows = rows;
    t.cols = cols;
    const std::size_t bytes = elements(*this) * sizeof(float);
    if (dev == Device::CPU) {
        t.storage_ = host_alloc(bytes);
        hip_check(hipMemcpy(t.storage_.get(), data, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    } else {
        t.storage_ = device_alloc(bytes);
        hip_check(hipMemcpy(t.storage_.get(), data, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    t.data = t.storage_.get();
    return t;
}

}  // namespace brotensor
