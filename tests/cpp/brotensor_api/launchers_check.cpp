// Compile check: a brovisionml build that keeps its own src/dsine_ops.cpp
// includes the launchers header where src/dsine_ops.cpp:8-10 includes
// dsine_ops_cuda.h, and calls detail::ray_relu_cuda / angmf_propagate_cuda as
// src/dsine_ops.cpp:187 and :209-210 do.  Built with -fsyntax-only against
// brotensor_api/brotensor/tensor.h.

#include "brovisionml/dsine_ops_gpu.h"

namespace brovisionml::dsine {

void launchers_check(brotensor::Tensor& n, const brotensor::Tensor& pr, const brotensor::Tensor& xy,
                     const brotensor::Tensor& an, const brotensor::Tensor& ray, int H, int W,
                     brotensor::Tensor& out) {
    detail::ray_relu_cuda(n, ray, H, W);
    detail::angmf_propagate_cuda(n, pr, xy, an, ray, 1.0, 0.5, 1.0, 0.5, H, W, out);
}

}  // namespace brovisionml::dsine
