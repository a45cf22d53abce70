// brovisionml::dsine::ray_relu / angmf_propagate on the HIP device: the public
// dispatch of src/dsine_ops.cpp:174-215 with the GPU branch routed to the
// C ABI (include/bvml_dsine.h).  Device and shape checks throw with the
// reference's "dsine ops: " prefix; a launch error throws "dsine hip: ".

#include "brovisionml/dsine_ops.h"

#include <climits>
#include <stdexcept>
#include <string>

#include "bvml_dsine.h"

namespace brovisionml::dsine {

namespace {

using brotensor::Device;
using brotensor::Tensor;

[[noreturn]] void fail(const std::string& msg) { throw std::runtime_error("dsine ops: " + msg); }

[[noreturn]] void fail_hip(const char* what, int status) {
    throw std::runtime_error(std::string("dsine hip: ") + what + ": " + bvml_dsine_last_error() +
                             " (status " + std::to_string(status) + ")");
}

void need_size(const Tensor& t, std::size_t n, const char* op, const char* name) {
    if (t.numel() != n)
        fail(std::string(op) + ": " + name + " holds " + std::to_string(t.numel()) +
             " elements, expected " + std::to_string(n));
    if (n != 0 && t.data == nullptr) fail(std::string(op) + ": " + name + " has no storage");
}

}  // namespace

namespace detail {

void ray_relu_gpu(Tensor& normal, const Tensor& ray, int H, int W) {
    const int st = bvml_dsine_ray_relu_f32(static_cast<float*>(normal.data),
                                           static_cast<const float*>(ray.data), 1, H, W, 0,
                                           nullptr);
    if (st != BVML_DSINE_OK) fail_hip("ray_relu launch", st);
}

namespace {

void angmf_launch(const Tensor& pred_norm, const Tensor& prob, const Tensor& xy,
                  const Tensor& angle, const Tensor& ray, double fu, double cu, double fv,
                  double cv, int H, int W, Tensor& out, unsigned flags) {
    const std::size_t n3 = static_cast<std::size_t>(3) * H * W;
    const bool reuse = out.device == Device::HIP && out.rows == 1 && out.numel() == n3 &&
                       out.data != nullptr && out.data != pred_norm.data &&
                       out.data != prob.data && out.data != xy.data &&
                       out.data != angle.data && out.data != ray.data;
    if (!reuse) out = Tensor::zeros_on(Device::HIP, 1, static_cast<int>(n3));
    const int st = bvml_dsine_angmf_propagate_f32(
        static_cast<const float*>(pred_norm.data), static_cast<const float*>(prob.data),
        static_cast<const float*>(xy.data), static_cast<const float*>(angle.data),
        static_cast<const float*>(ray.data), fu, cu, fv, cv, 1, H, W, 5, 0,
        static_cast<float*>(out.data), flags, nullptr);
    if (st != BVML_DSINE_OK) fail_hip("angmf_propagate launch", st);
}

}  // namespace

void angmf_propagate_gpu(const Tensor& pred_norm, const Tensor& prob, const Tensor& xy,
                         const Tensor& angle, const Tensor& ray, double fu, double cu,
                         double fv, double cv, int H, int W, Tensor& out) {
    angmf_launch(pred_norm, prob, xy, angle, ray, fu, cu, fv, cv, H, W, out,
                 BVML_DSINE_DEFAULT);
}

}  // namespace detail

void ray_relu(Tensor& normal, const Tensor& ray, int H, int W) {
    if (normal.device != ray.device) fail("ray_relu: normal and ray must share a device");
    if (normal.device == Device::CPU)
        fail("ray_relu: tensors are on the CPU; this library implements the HIP device path");
    if (H < 0 || W < 0) fail("ray_relu: H and W must be >= 0");
    const std::size_t n3 = static_cast<std::size_t>(3) * H * W;
    need_size(normal, n3, "ray_relu", "normal");
    need_size(ray, n3, "ray_relu", "ray");
    if (n3 == 0) return;
    detail::ray_relu_gpu(normal, ray, H, W);
}

namespace {

void angmf_check(const Tensor& pred_norm, const Tensor& prob, const Tensor& xy,
                 const Tensor& angle, const Tensor& ray, int H, int W, const char* op) {
    const Device dev = pred_norm.device;
    if (prob.device != dev || xy.device != dev || angle.device != dev || ray.device != dev)
        fail(std::string(op) + ": all inputs must share a device");
    if (dev == Device::CPU)
        fail(std::string(op) + ": tensors are on the CPU; this library implements the HIP "
             "device path");
    if (H < 0 || W < 0) fail(std::string(op) + ": H and W must be >= 0");
    const std::size_t hw = static_cast<std::size_t>(H) * W;
    need_size(pred_norm, 3 * hw, op, "pred_norm");
    need_size(prob, 25 * hw, op, "prob");
    need_size(xy, 50 * hw, op, "xy");
    need_size(angle, 25 * hw, op, "angle");
    need_size(ray, 3 * hw, op, "ray");
}

}  // namespace

void angmf_propagate(const Tensor& pred_norm, const Tensor& prob, const Tensor& xy,
                     const Tensor& angle, const Tensor& ray, double fu, double cu,
                     double fv, double cv, int H, int W, Tensor& out) {
    angmf_check(pred_norm, prob, xy, angle, ray, H, W, "angmf_propagate");
    detail::angmf_propagate_gpu(pred_norm, prob, xy, angle, ray, fu, cu, fv, cv, H, W, out);
}

void angmf_propagate_logits(const Tensor& pred_norm, const Tensor& prob_logits,
                            const Tensor& xy, const Tensor& angle_logits, const Tensor& ray,
                            double fu, double cu, double fv, double cv, int H, int W,
                            Tensor& out) {
    angmf_check(pred_norm, prob_logits, xy, angle_logits, ray, H, W, "angmf_propagate_logits");
    detail::angmf_launch(pred_norm, prob_logits, xy, angle_logits, ray, fu, cu, fv, cv, H, W,
                         out, BVML_DSINE_LOGITS);
}

namespace {

void upsample(const Tensor& x, const Tensor& mask, int N, int C, int H, int W, int scale,
              bool normalize, float eps, Tensor& out, const char* op) {
    if (x.device != mask.device) fail(std::string(op) + ": x and mask must share a device");
    if (x.device == Device::CPU)
        fail(std::string(op) + ": tensors are on the CPU; this library implements the HIP "
             "device path");
    if (N < 0 || C < 1 || H < 0 || W < 0 || scale < 1)
        fail(std::string(op) + ": N, H and W must be >= 0, C and scale >= 1");
    const std::size_t hw = static_cast<std::size_t>(H) * W;
    const std::size_t s2 = static_cast<std::size_t>(scale) * scale;
    need_size(x, static_cast<std::size_t>(N) * C * hw, op, "x");
    need_size(mask, static_cast<std::size_t>(N) * 9 * s2 * hw, op, "mask");
    const std::size_t n_out = static_cast<std::size_t>(N) * C * s2 * hw;
    if (C * s2 * hw > static_cast<std::size_t>(INT_MAX))
        fail(std::string(op) + ": C*scale^2*H*W exceeds a tensor row");
    const bool reuse = out.device == Device::HIP && out.rows == N && out.numel() == n_out &&
                       out.data != nullptr && out.data != x.data && out.data != mask.data;
    if (!reuse) out = Tensor::zeros_on(Device::HIP, N, static_cast<int>(n_out / (N ? N : 1)));
    if (n_out == 0) return;
    const int st = bvml_dsine_convex_upsample_f32(
        static_cast<const float*>(x.data), static_cast<const float*>(mask.data), N, C, H, W, scale,
        normalize ? 1 : 0, eps, static_cast<float*>(out.data), BVML_DSINE_DEFAULT, nullptr);
    if (st != BVML_DSINE_OK) fail_hip((std::string(op) + " launch").c_str(), st);
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
