#pragma once

// DSINE NRN ops -- drop-in for brovisionml's include/brovisionml/dsine_ops.h
// (:17-56): the same namespace, names and signatures, so
// src/dsine_refine.cpp:242 and :271-272 compile against it unchanged.
// Tensors are (1, C*H*W) fp32 NCHW.  Each op dispatches on its inputs' device,
// as the reference's does (src/dsine_ops.cpp:178-215): CPU tensors run this
// library's CPU branch (double precision in the reference's operation order;
// results equal the reference CPU twin's bit for bit); tensors on the GPU
// (brotensor's CUDA tag, which a HIP build of brotensor uses for its device)
// run the gfx950 kernels, asynchronously on the null stream like the
// reference's default-stream launches (src/dsine_ops.cu:2-4).
//
// Errors throw std::runtime_error prefixed "dsine ops: " (argument and device
// checks, src/dsine_ops.cpp:18-22) or "dsine hip: " (a HIP runtime error at
// launch; the reference's "dsine cuda: ", src/dsine_ops.cu:25-29).

#include "brotensor/tensor.h"

namespace brovisionml::dsine {

// RayReLU (eps 1e-2) of a (1, 3*H*W) unit-normal map against the L2-normalised
// 3-channel ray_8, in place -- include/brovisionml/dsine_ops.h:19-26.
void ray_relu(brotensor::Tensor& normal, const brotensor::Tensor& ray,
              int H, int W);

// Fused AngMF propagate over the 5x5 window -- include/brovisionml/dsine_ops.h:28-54.
//   pred_norm (1, 3HW), prob (1, 25HW) sigmoid(prob_head), xy (1, 50HW) raw
//   [xs(25), ys(25)], angle (1, 25HW) sigmoid(angle_head)*pi, ray (1, 3HW);
//   fu, cu, fv, cv the grid-scaled intrinsics (src/dsine_refine.cpp:232-237).
// `out` becomes a new (1, 3HW) tensor on the inputs' device, as the
// reference allocates it (src/dsine_ops.cpp:83, src/dsine_ops.cu:178): a
// tensor the caller held in `out` before keeps its contents.
void angmf_propagate(const brotensor::Tensor& pred_norm,
                     const brotensor::Tensor& prob,
                     const brotensor::Tensor& xy,
                     const brotensor::Tensor& angle,
                     const brotensor::Tensor& ray,
                     double fu, double cu, double fv, double cv,
                     int H, int W,
                     brotensor::Tensor& out);

// angmf_propagate on the prob and angle heads' raw logits: the op applies
// the activations the refiner applies before each propagate
// (src/dsine_refine.cpp:262-267: sigmoid, and sigmoid * kPi), so the two
// elementwise passes over them disappear.  No counterpart in the reference;
// the result matches angmf_propagate given the correctly rounded float
// activations, to the same tolerance (bit for bit on the CPU branch).
void angmf_propagate_logits(const brotensor::Tensor& pred_norm,
                            const brotensor::Tensor& prob_logits,
                            const brotensor::Tensor& xy,
                            const brotensor::Tensor& angle_logits,
                            const brotensor::Tensor& ray,
                            double fu, double cu, double fv, double cv,
                            int H, int W,
                            brotensor::Tensor& out);

// The refiner's post-propagate step (src/dsine_refine.cpp:276-282), whose
// reference is two brotensor calls:
//   convex_upsample_forward(x, mask, N, C, H, W, scale, up)
//   l2_normalize_nchw_forward(up, N, C, scale*H, scale*W, eps, up)
// convex_upsample_normalize runs both in one pass; convex_upsample is the first
// alone.  x (N, C*H*W) with C <= 4, mask (N, 9*scale^2*H*W) with scale <= 16
// (channel n*scale^2 + ky*scale + kx, tap n = 3*(dy+1) + (dx+1), replicate
// padding), both fp32 on the GPU; `out` becomes a new (N, C*scale^2*H*W) fp32
// tensor on their device.  These replace brotensor's GPU kernels only: CPU
// tensors throw (brotensor's CPU versions stay brotensor's).
void convex_upsample_normalize(const brotensor::Tensor& x, const brotensor::Tensor& mask,
                               int N, int C, int H, int W, int scale, float eps,
                               brotensor::Tensor& out);
void convex_upsample(const brotensor::Tensor& x, const brotensor::Tensor& mask, int N, int C,
                     int H, int W, int scale, brotensor::Tensor& out);

}  // namespace brovisionml::dsine
