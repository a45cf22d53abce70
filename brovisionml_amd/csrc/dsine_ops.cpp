// brovisionml::dsine::{ray_relu, angmf_propagate}: the public dispatch of
// src/dsine_ops.cpp:174-215, device-agnostic as the reference's is.  CPU
// tensors go to this library's CPU branch (bvml_dsine_*_cpu_f32, double
// precision in the reference's operation order); tensors on the GPU go to the
// gfx950 kernels through the inline launchers of brovisionml/dsine_ops_gpu.h.
// `out` is allocated on the inputs' device on every call, as the reference
// allocates it (src/dsine_ops.cpp:83, src/dsine_ops.cu:178).  Device and shape
// checks throw with the reference's "dsine ops: " prefix; a launch error
// throws "dsine hip: ".
//
// This file and the launchers header use only the brotensor::Tensor members
// the reference's own dsine_ops.cpp uses (device, data, rows, cols, mat,
// empty_on, host_f32, host_f32_mut), so the file compiles against brotensor's
// header as well as against include/brotensor/tensor.h.

#include "brovisionml/dsine_ops.h"

#include <climits>
#include <cstddef>
#include <stdexcept>
#include <string>

#include "brovisionml/dsine_ops_gpu.h"
#include "bvml_dsine.h"

namespace brovisionml::dsine {

namespace {

using brotensor::Device;
using brotensor::Tensor;

[[noreturn]] void fail(const std::string& msg) { throw std::runtime_error("dsine ops: " + msg); }

[[noreturn]] void fail_cpu(const std::string& what) {
    throw std::runtime_error("dsine ops: " + what + ": " + bvml_dsine_last_error());
}

std::size_t elements(const Tensor& t) {
    return static_cast<std::size_t>(t.rows) * static_cast<std::size_t>(t.cols);
}

void need_size(const Tensor& t, std::size_t n, const char* op, const char* name) {
    if (elements(t) != n)
        fail(std::string(op) + ": " + name + " holds " + std::to_string(elements(t)) +
             " elements, expected " + std::to_string(n));
    if (n != 0 && t.data == nullptr) fail(std::string(op) + ": " + name + " has no storage");
}

// The GPU this library drives: brotensor's CUDA tag.  Metal tensors have no
// device path here.
void need_known_device(Device dev, const char* op) {
    if (dev != Device::CPU && dev != Device::CUDA)
        fail(std::string(op) + ": tensors on a device this library does not run (CPU and the "
             "HIP GPU only)");
}

void need_hw(int H, int W, const char* op) {
    if (H < 0 || W < 0) fail(std::string(op) + ": H and W must be >= 0");
    if (static_cast<long long>(H) * W * 50 > INT_MAX)
        fail(std::string(op) + ": 50*H*W exceeds a tensor row");
}

void angmf_check(const Tensor& pred_norm, const Tensor& prob, const Tensor& xy,
                 const Tensor& angle, const Tensor& ray, int H, int W, const char* op) {
    const Device dev = pred_norm.device;
    if (prob.device != dev || xy.device != dev || angle.device != dev || ray.device != dev)
        fail(std::string(op) + ": all inputs must share a device");
    need_known_device(dev, op);
    need_hw(H, W, op);
    const std::size_t hw = static_cast<std::size_t>(H) * W;
    need_size(pred_norm, 3 * hw, op, "pred_norm");
    need_size(prob, 25 * hw, op, "prob");
    need_size(xy, 50 * hw, op, "xy");
    need_size(angle, 25 * hw, op, "angle");
    need_size(ray, 3 * hw, op, "ray");
}

void angmf(const Tensor& pred_norm, const Tensor& prob, const Tensor& xy, const Tensor& angle,
           const Tensor& ray, double fu, double cu, double fv, double cv, int H, int W,
           Tensor& out, unsigned flags, const char* op) {
    angmf_check(pred_norm, prob, xy, angle, ray, H, W, op);
    if (pred_norm.device != Device::CPU) {
        detail::angmf_propagate_cuda_flags(pred_norm, prob, xy, angle, ray, fu, cu, fv, cv, H, W,
                                           out, flags);
        return;
    }
    Tensor res = Tensor::mat(1, 3 * H * W);
    if (H > 0 && W > 0 &&
        bvml_dsine_angmf_propagate_cpu_f32(pred_norm.host_f32(), prob.host_f32(), xy.host_f32(),
                                           angle.host_f32(), ray.host_f32(), fu, cu, fv, cv, 1,
                                           H, W, 5, 0, res.host_f32_mut(), flags,
                                           0) != BVML_DSINE_OK)
        fail_cpu(op);
    out = res;
}

}  // namespace

void ray_relu(Tensor& normal, const Tensor& ray, int H, int W) {
    if (normal.device != ray.device) fail("ray_relu: normal and ray must share a device");
    need_known_device(normal.device, "ray_relu");
    need_hw(H, W, "ray_relu");
    const std::size_t n3 = static_cast<std::size_t>(3) * H * W;
    need_size(normal, n3, "ray_relu", "normal");
    need_size(ray, n3, "ray_relu", "ray");
    if (n3 == 0) return;
    if (normal.device != Device::CPU) {
        detail::ray_relu_cuda(normal, ray, H, W);
        return;
    }
    if (bvml_dsine_ray_relu_cpu_f32(normal.host_f32_mut(), ray.host_f32(), 1, H, W, 0, 0) !=
        BVML_DSINE_OK)
        fail_cpu("ray_relu");
}

void angmf_propagate(const Tensor& pred_norm, const Tensor& prob, const Tensor& xy,
                     const Tensor& angle, const Tensor& ray, double fu, double cu,
                     double fv, double cv, int H, int W, Tensor& out) {
    angmf(pred_norm, prob, xy, angle, ray, fu, cu, fv, cv, H, W, out, BVML_DSINE_DEFAULT,
          "angmf_propagate");
}

void angmf_propagate_logits(const Tensor& pred_norm, const Tensor& prob_logits,
                            const Tensor& xy, const Tensor& angle_logits, const Tensor& ray,
                            double fu, double cu, double fv, double cv, int H, int W,
                            Tensor& out) {
    angmf(pred_norm, prob_logits, xy, angle_logits, ray, fu, cu, fv, cv, H, W, out,
          BVML_DSINE_LOGITS, "angmf_propagate_logits");
}

namespace {

void upsample(const Tensor& x, const Tensor& mask, int N, int C, int H, int W, int scale,
              bool normalize, float eps, Tensor& out, const char* op) {
    if (x.device != mask.device) fail(std::string(op) + ": x and mask must share a device");
    if (x.device == Device::CPU)
        fail(std::string(op) + ": tensors are on the CPU; this op replaces brotensor's GPU "
             "kernels only");
    need_known_device(x.device, op);
    if (N < 0 || C < 1 || H < 0 || W < 0 || scale < 1)
        fail(std::string(op) + ": N, H and W must be >= 0, C and scale >= 1");
    const std::size_t hw = static_cast<std::size_t>(H) * W;
    const std::size_t s2 = static_cast<std::size_t>(scale) * scale;
    need_size(x, static_cast<std::size_t>(N) * C * hw, op, "x");
    need_size(mask, static_cast<std::size_t>(N) * 9 * s2 * hw, op, "mask");
    if (C * s2 * hw > static_cast<std::size_t>(INT_MAX))
        fail(std::string(op) + ": C*scale^2*H*W exceeds a tensor row");
    out = Tensor::empty_on(x.device, N, static_cast<int>(C * s2 * hw));
    if (N == 0 || hw == 0) return;
    const int st = bvml_dsine_convex_upsample_f32(
        static_cast<const float*>(x.data), static_cast<const float*>(mask.data), N, C, H, W, scale,
        normalize ? 1 : 0, eps, static_cast<float*>(out.data), BVML_DSINE_DEFAULT, nullptr);
    if (st != BVML_DSINE_OK) detail::hip_launch_failed((std::string(op) + " launch").c_str(), st);
}

}  // namespace

void convex_upsample_normalize(const Tensor& x, const Tensor& mask, int N, int C, int H, int W,
                               int scale, float eps, Tensor& out) {
    upsample(x, mask, N, C, H, W, scale, true, eps, out, "convex_upsample_normalize");
}

void convex_upsample(const Tensor& x, const Tensor& mask, int N, int C, int H, int W, int scale,
                     Tensor& out) {
    upsample(x, mask, N, C, H, W, scale, false, 0.0f, out, "convex_upsample");
}

}  // namespace brovisionml::dsine
