#pragma once

// The GPU launchers of brovisionml's DSINE ops, header-only, for a
// brovisionml build that keeps its own src/dsine_ops.cpp (public dispatch and
// CPU twin) and swaps only its device launchers: detail::ray_relu_cuda and
// detail::angmf_propagate_cuda keep the names and parameter lists of
// src/dsine_ops_cuda.h:13-23 (the names follow brotensor's CUDA device tag,
// under which a HIP build of brotensor runs its GPU) and replace the bodies
// of src/dsine_ops.cu:159-191 with calls into the C ABI of libbvml_dsine.so
// (include/bvml_dsine.h).  Being inline, they add no symbol that could
// collide with brovisionml's own.  Inputs are fp32 tensors on the GPU; `out`
// becomes a new tensor on their device, as the reference allocates it
// (src/dsine_ops.cu:178; uninitialised here, since the kernel writes every
// element); launches are asynchronous on the null stream.  A launch error
// throws "dsine hip: ..." where the reference throws "dsine cuda: ..."
// (src/dsine_ops.cu:25-29).

#include <stdexcept>
#include <string>

#include "brotensor/tensor.h"
#include "bvml_dsine.h"

namespace brovisionml::dsine::detail {

[[noreturn]] inline void hip_launch_failed(const char* what, int status) {
    throw std::runtime_error(std::string("dsine hip: ") + what + ": " + bvml_dsine_last_error() +
                             " (status " + std::to_string(status) + ")");
}

inline void ray_relu_cuda(brotensor::Tensor& normal, const brotensor::Tensor& ray, int H, int W) {
    const int st = bvml_dsine_ray_relu_f32(static_cast<float*>(normal.data),
                                           static_cast<const float*>(ray.data), 1, H, W, 0,
                                           nullptr);
    if (st != BVML_DSINE_OK) hip_launch_failed("ray_relu launch", st);
}

// angmf_propagate on the GPU with the C ABI's flags (BVML_DSINE_DEFAULT for
// the reference's op).
inline void angmf_propagate_cuda_flags(const brotensor::Tensor& pred_norm,
                                       const brotensor::Tensor& prob,
                                       const brotensor::Tensor& xy,
                                       const brotensor::Tensor& angle,
                                       const brotensor::Tensor& ray, double fu, double cu,
                                       double fv, double cv, int H, int W, brotensor::Tensor& out,
                                       unsigned flags) {
    // The inputs' pointers are taken before `out` is replaced, so an `out`
    // that is one of the inputs still reads the caller's data.
    const float* pn = static_cast<const float*>(pred_norm.data);
    const float* pr = static_cast<const float*>(prob.data);
    const float* xyp = static_cast<const float*>(xy.data);
    const float* an = static_cast<const float*>(angle.data);
    const float* ry = static_cast<const float*>(ray.data);
    brotensor::Tensor res = brotensor::Tensor::empty_on(pred_norm.device, 1, 3 * H * W);
    if (H > 0 && W > 0) {
        const int st = bvml_dsine_angmf_propagate_f32(pn, pr, xyp, an, ry, fu, cu, fv, cv, 1, H,
                                                      W, 5, 0, static_cast<float*>(res.data),
                                                      flags, nullptr);
        if (st != BVML_DSINE_OK) hip_launch_failed("angmf_propagate launch", st);
    }
    out = res;
}

inline void angmf_propagate_cuda(const brotensor::Tensor& pred_norm,
                                const brotensor::Tensor& prob, const brotensor::Tensor& xy,
                                const brotensor::Tensor& angle, const brotensor::Tensor& ray,
                                double fu, double cu, double fv, double cv, int H, int W,
                                brotensor::Tensor& out) {
    angmf_propagate_cuda_flags(pred_norm, prob, xy, angle, ray, fu, cu, fv, cv, H, W, out,
                              BVML_DSINE_DEFAULT);
}

}  // namespace brovisionml::dsine::detail
