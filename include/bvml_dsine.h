/*
 * bvml_dsine.h -- C ABI of the MI355X (gfx950) DSINE surface-normal ops.
 *
 * These entry points are the drop-in boundary for brovisionml's two GPU
 * kernels.  They replace the launchers the reference declares in
 * src/dsine_ops_cuda.h:13-23 (detail::ray_relu_cuda, detail::angmf_propagate_cuda)
 * and implemented in src/dsine_ops.cu:159-191; the C++ layer
 * (include/brovisionml/dsine_ops.h) forwards to them with the reference's own
 * signatures.  Plain pointers and scalars only: every pointer is a device
 * pointer (hipMalloc'd, or any HIP-visible device allocation) to contiguous
 * fp32 NCHW planes, every call is asynchronous on `stream` (NULL = the null
 * stream, as the reference launches on the default stream), and nothing
 * throws.
 *
 * The *_cpu_f32 entry points are the CPU branch of the same ops and take host
 * pointers instead.
 *
 * Layout (H, W: the /8 grid; HW = H*W; K2 = k*k; sample b of B):
 *   pred_norm  b*3*HW      + c*HW      + y*W + x     c in [0,3)
 *   prob       b*K2*HW     + n*HW      + ...         n = ky*k + kx
 *   xy         b*2*K2*HW   + n*HW (xs), (K2+n)*HW (ys)
 *   angle      b*K2*HW     + n*HW
 *   ray        b*ray_bstride + c*HW    (ray_bstride 0 = one ray shared by all)
 *   out        b*3*HW      + c*HW
 * With B = 1, k = 5 and ray_bstride = 0 this is exactly the reference's
 * (1, C*H*W) tensor layout (include/brovisionml/dsine_ops.h:35-46).
 *
 * Return value: 0 on success; a negative BVML_DSINE_E* code for a rejected
 * argument (nothing is launched); a positive hipError_t value when the HIP
 * runtime reports an error at launch.  bvml_dsine_last_error() returns the
 * calling thread's message for the last non-zero status.
 */
#ifndef BVML_DSINE_H
#define BVML_DSINE_H

#ifdef __cplusplus
extern "C" {
#endif

#define BVML_DSINE_OK 0
#define BVML_DSINE_ENULL (-1)     /* a required pointer is NULL */
#define BVML_DSINE_ESHAPE (-2)    /* B, H or W negative */
#define BVML_DSINE_EK (-3)        /* k not one of 1, 3, 5, 7, 9 */
#define BVML_DSINE_ESIZE (-4)     /* a plane index or grid would overflow */
#define BVML_DSINE_EALIAS (-5)    /* out overlaps an input */
#define BVML_DSINE_EFLAGS (-6)    /* unknown flag bits */
#define BVML_DSINE_EPARAM (-7)    /* fu/fv zero or non-finite, cu/cv non-finite */
#define BVML_DSINE_EUNSUP (-8)    /* a size outside what the kernels support */

/* Flag bits for bvml_dsine_angmf_propagate_f32. */
#define BVML_DSINE_DEFAULT 0u
/* Run every neighbour in double precision in the reference's operation
 * order (one pixel per lane, no fp32 fast path): the parity anchor. */
#define BVML_DSINE_FP64 1u
/* Form each pixel's ray from fu, cu, fv, cv in the kernel, bit-identical to
 * the reference's build_ray8 (src/dsine_decoder.cpp:242-259, :276-293), which
 * the refiner builds from the same grid-scaled intrinsics
 * (src/dsine_refine.cpp:229-237), instead of reading a ray tensor: `ray` may
 * then be NULL and ray_bstride is ignored.  No counterpart in the reference;
 * saves the 3 ray planes (12 B/px) and the host-side build. */
#define BVML_DSINE_RAY_FROM_INTRINSICS 2u
/* `prob` and `angle` hold the prob and angle heads' raw logits, and the
 * kernel applies the activations the refiner applies to them before each
 * propagate (src/dsine_refine.cpp:262-267: apply_sigmoid(prob);
 * apply_sigmoid(angle); scale_inplace(angle, kPi) with the float kPi of
 * src/dsine_refine.cpp:26): prob = sigmoid(L), angle = sigmoid(L) * kPi.
 * Results match the op given the correctly rounded float activations, to the
 * same bar.  No counterpart in the reference; saves the two elementwise
 * passes over 2 k^2 planes (read and write) per refiner iteration. */
#define BVML_DSINE_LOGITS 4u

/*
 * RayReLU in place (eps = 1e-2), B samples.
 * Replaces detail::ray_relu_cuda (src/dsine_ops_cuda.h:13-14,
 * src/dsine_ops.cu:159-168); arithmetic of src/dsine_ops.cpp:55-76.
 *   normal : B x 3 x HW, read and written
 *   ray    : 3 x HW per sample at ray + b*ray_bstride (0 = shared)
 * HW == 0 or B == 0 returns 0 without launching (src/dsine_ops.cu:162).
 */
int bvml_dsine_ray_relu_f32(float* normal, const float* ray, int B, int H,
                            int W, long long ray_bstride, void* stream);

/*
 * Fused AngMF propagate, B samples, odd window k.
 * Replaces detail::angmf_propagate_cuda (src/dsine_ops_cuda.h:16-23,
 * src/dsine_ops.cu:170-191); arithmetic of src/dsine_ops.cpp:78-172, with
 * k generalising the reference's fixed 5x5 window (src/dsine_ops.cpp:24-26).
 * fu, cu, fv, cv: the grid-scaled intrinsics the caller computes at
 * src/dsine_refine.cpp:232-237, shared by all samples.
 * `out` is caller-allocated (B x 3 x HW) and must not overlap any input
 * (the reference allocates it per call, src/dsine_ops.cu:178).
 */
int bvml_dsine_angmf_propagate_f32(const float* pred_norm, const float* prob,
                                   const float* xy, const float* angle,
                                   const float* ray, double fu, double cu,
                                   double fv, double cv, int B, int H, int W,
                                   int k, long long ray_bstride, float* out,
                                   unsigned flags, void* stream);

/*
 * The launch plan bvml_dsine_angmf_propagate_f32 takes for these arguments,
 * without launching anything: 1 if the call runs the fp32 kernel, 0 if it
 * runs the double-precision kernel, or a negative BVML_DSINE_E* status.
 * *waves_per_group receives the waves that share one 64-pixel group (1: each
 * wave evaluates the whole window; 2, 4, 8: the window's neighbours split
 * into runs), *tile_w and *tile_h the workgroup's tile (*tile_h 0: a range
 * tile, *tile_w consecutive pixels of the row-major image), *stream_planes 1
 * when the launch reads its neighbour planes with the non-temporal cache
 * policy (a whole-window launch larger than the Infinity Cache); any of the
 * four may be NULL.  No counterpart in the reference: for tests and tuning.
 */
int bvml_dsine_angmf_plan(int B, int H, int W, int k, double fu, double cu, double fv,
                          double cv, unsigned flags, int* waves_per_group, int* tile_w,
                          int* tile_h, int* stream_planes);

/*
 * The /8-grid ray map, 3 x H x W fp32 planes, as the reference's build_ray8
 * (src/dsine_decoder.cpp:276-293, through get_ray_core :242-259) forms it on
 * the host: ray_x = float(((x + 0.5) - cu) / fu), ray_y likewise with cv, fv,
 * then [ray_x, ray_y, 1] L2-normalised in double and each channel rounded to
 * float.  fu, cu, fv, cv are the grid-scaled intrinsics with the +0.5 on the
 * principal point already applied (src/dsine_refine.cpp:232-237); the result
 * is bit-identical to the host's.  No counterpart on the reference's device
 * path (it builds the map on the host and copies it over).
 */
int bvml_dsine_build_ray8_f32(float* ray, double fu, double cu, double fv,
                              double cv, int H, int W, void* stream);

/*
 * The /8-grid uv map, 2 x H x W fp32 planes, as the reference's build_uv
 * (src/dsine_decoder.cpp:262-274, through get_ray_core :242-259) forms it on
 * the host: u = float(((x + 0.5) - cu) / fu), v = float(((y + 0.5) - cv) / fv),
 * bit-identical to the host's; the same fu, cu, fv, cv as build_ray8.  No
 * counterpart on the reference's device path (the refiner builds the map on
 * the host and copies it over, src/dsine_refine.cpp:222-228).
 */
int bvml_dsine_build_uv8_f32(float* uv, double fu, double cu, double fv, double cv, int H,
                             int W, void* stream);

/*
 * Convex upsample by `scale` with a 9-tap softmax mask, fused with the channel
 * L2-normalise (normalize != 0), B samples.  Replaces the two brotensor calls
 * the refiner makes after each propagate (src/dsine_refine.cpp:276-282:
 * convex_upsample_forward(pred_norm, up_mask, N, C, H, W, scale, up), then
 * l2_normalize_nchw_forward(up, N, C, scale*H, scale*W, 1e-12f, up)); the
 * arithmetic is the one the reference specifies at
 * include/brovisionml/dsine_refine.h:91-97 (DSINE's upsample_via_mask with
 * replicate padding, then F.normalize):
 *   x    : B x C x H x W
 *   mask : B x 9*scale^2 x H x W, channel n*scale^2 + ky*scale + kx, tap
 *          n = 3*(dy+1) + (dx+1) for the neighbour (y+dy, x+dx), clamped
 *   out  : B x C x (scale*H) x (scale*W); sub-pixel (ky, kx) of (y, x) is
 *          softmax_n(mask)-weighted sum of the taps, then / max(|v|, eps)
 * C in 1..4 and scale in 1..16 (BVML_DSINE_EUNSUP otherwise); the refiner
 * uses C = 3, scale = 8, eps = 1e-12f.  A NaN in a sub-pixel's 9 mask values
 * makes that sub-pixel NaN.  Within 7.2e-6 per component of the
 * double-precision result (a bound; typically 1e-7); flags BVML_DSINE_FP64
 * computes every sub-pixel in double.  `out` is caller-allocated and must not
 * overlap x or mask.  Any alignment works; at scale 8 a 16-byte-aligned `out`
 * and mask with H*W a multiple of 4 take the fastest kernel (the result is
 * the same bit for bit).
 */
int bvml_dsine_convex_upsample_f32(const float* x, const float* mask, int B, int C, int H,
                                   int W, int scale, int normalize, float eps, float* out,
                                   unsigned flags, void* stream);

/*
 * The same with a per-channel bias on the mask (mask_bias: 9*scale^2 floats,
 * or NULL for none): each mask value is mask + mask_bias[channel], one fp32
 * add, as the bias add after the refiner's up-mask head (its last 1x1
 * convolution, src/dsine_refine.cpp:119-127) would round it, so that
 * convolution can run without its bias and the separate pass over the
 * 9*scale^2 planes goes.  No counterpart in the reference.
 */
int bvml_dsine_convex_upsample_bias_f32(const float* x, const float* mask,
                                        const float* mask_bias, int B, int C, int H, int W,
                                        int scale, int normalize, float eps, float* out,
                                        unsigned flags, void* stream);

/*
 * The CPU branch of the same two ops, for host pointers: brovisionml's public
 * dispatch sends CPU tensors to its CPU twin (src/dsine_ops.cpp:178-215 ->
 * ray_relu_cpu :55-76, angmf_propagate_cpu :78-172); these are this
 * library's, in double precision in the reference's operation order (the
 * results equal the reference CPU path's bit for bit), with the device entry
 * points' arguments, flags (BVML_DSINE_FP64 changes nothing here) and
 * checks.  nthreads: host threads over the rows (0 = the hardware's; the
 * result does not depend on it).  They make no HIP call.
 */
int bvml_dsine_ray_relu_cpu_f32(float* normal, const float* ray, int B, int H, int W,
                                long long ray_bstride, int nthreads);
int bvml_dsine_angmf_propagate_cpu_f32(const float* pred_norm, const float* prob,
                                       const float* xy, const float* angle, const float* ray,
                                       double fu, double cu, double fv, double cv, int B, int H,
                                       int W, int k, long long ray_bstride, float* out,
                                       unsigned flags, int nthreads);

/*
 * The fast path's cancellation threshold for a propagate call with window
 * size k and `flags`: a pixel whose fp32 sum satisfies
 * |acc|^2 < ratio * sum_i (prob_i / |p_i|)^2 (p_i a neighbour's RayReLU'd
 * vector before its normalise) is recomputed in double, since the final
 * normalise would amplify the fp32 rounding past the parity bar.  0 for
 * BVML_DSINE_FP64 (nothing is recomputed), -1 for a k the op rejects.  No
 * counterpart in the reference: it lets a caller count, on its own data, how
 * many pixels take the slower path.
 */
double bvml_dsine_angmf_recompute_ratio(int k, unsigned flags);

/*
 * The refiner's elementwise steps around its convolutions, fused (no
 * counterpart in the reference, whose ConvGRU and heads run each step as its
 * own brotensor op, src/dsine_refine.cpp:104-159).  Maps are fp32 NCHW, C
 * planes of HW floats on the device; biases hold C floats.  The convolutions
 * run without their bias; these apply it.
 *
 * bvml_dsine_gru_gates_f32: zr holds 2C planes, convz's then convr's
 *   pre-activations; z = sigmoid(zr[c] + bias_z[c]) and
 *   rh = sigmoid(zr[C + c] + bias_r[c]) * h.  z and rh must not overlap zr,
 *   h or each other.
 * bvml_dsine_gru_update_f32: h_new = (1 - z) h + z tanh(q_pre + bias_q), in
 *   the reference's rounding order (src/dsine_refine.cpp:152-157), written to
 *   h_new and, when h_copy is non-NULL, to h_copy too.  h_new may be h.
 * bvml_dsine_bias_act_f32: x = x + bias[c] in place, then ReLU if relu is 1
 *   (v < 0 ? 0 : v).
 */
int bvml_dsine_gru_gates_f32(const float* zr, const float* bias_z, const float* bias_r,
                             const float* h, int C, long long HW, float* z, float* rh,
                             void* stream);
int bvml_dsine_gru_update_f32(const float* q_pre, const float* bias_q, const float* z,
                              const float* h, int C, long long HW, float* h_new, float* h_copy,
                              void* stream);
int bvml_dsine_bias_act_f32(float* x, const float* bias, int C, long long HW, int relu,
                            void* stream);

/*
 * The refiner's four prediction heads after their first layer, fused into one
 * per-pixel pass on the fp32 matrix cores (no counterpart in the reference,
 * where each head is conv3x3 -> ReLU -> conv1x1 -> ReLU -> conv1x1 of
 * brotensor ops, src/dsine_refine.cpp:119-127).  For heads h < nheads and
 * every pixel p of the H x W map:
 *   a = relu(t0[64h + c][p] + b0[64h + c])       c < 64: the 3x3 layer's
 *                                                output without its bias
 *   t = relu(W2_h a + b2_h)                      W2_h: head h's 64 x 64 1x1
 *   out[h][o][p] = (W4_h t)[o] + b4[h][o]        o < outs[h]; b4[h] NULL: no bias
 * Each sum in fp32, then its bias added once.  W2 and W4 in the layout
 * bvml_dsine_heads_pack_f32 writes: w2p holds nheads * 4096 floats, w4p[h]
 * bvml_dsine_heads_packed_size(outs[h]).  t0: 64 * nheads planes; b0, b2:
 * 64 * nheads floats; out[h]: outs[h] planes, not overlapping t0 or each
 * other.  nheads 1..4, outs 1..4096.  ReLU is v < 0 ? 0 : v.
 * bvml_dsine_heads_pack_f32 runs on the host: w2 holds the nheads 64 x 64
 * middle-layer weights (OIHW, 1x1) back to back, w4[h] head h's outs[h] x 64
 * last-layer weights.
 */
int bvml_dsine_heads_mlp_f32(const float* t0, const float* b0, const float* w2p,
                             const float* b2, const float* const* w4p, const float* const* b4,
                             const int* outs, int nheads, int H, int W, float* const* out,
                             void* stream);
int bvml_dsine_heads_pack_f32(const float* w2, const float* const* w4, const int* outs,
                              int nheads, float* w2p, float* const* w4p);
long long bvml_dsine_heads_packed_size(int out);

/*
 * The refiner's k x k convolutions (k = 3 or 5, stride 1, zero padding k/2:
 * the ConvGRU's 5x5 layers and the heads' 3x3 first layers,
 * src/dsine_refine.cpp:94-101, :119-158), as implicit GEMMs on the fp32
 * matrix cores, with no im2col buffer.  x: cin planes of H x W; the weights
 * in the layout bvml_dsine_conv_pack_f32 writes from OIHW weights (cout, cin,
 * k, k), bvml_dsine_conv_packed_size(cout, cin, k) floats, 16-byte aligned.
 * Each sum in fp32; no bias (the consumer adds it, or the fused epilogue):
 *   bvml_dsine_conv_f32            out = conv(x) (cout planes)
 *   bvml_dsine_conv_gru_gates_f32  convz and convr as one 5x5 convolution of
 *     2C filters (packed with interleave = 1 from [W_z; W_r]); writes
 *     z = sigmoid(s_z + bias_z) and rh = sigmoid(s_r + bias_r) * h, as
 *     bvml_dsine_gru_gates_f32 does from the two sums; C % 32 == 0
 *   bvml_dsine_conv_gru_update_f32 convq (C filters, 5x5); writes
 *     h_new = (1 - z) h + z tanh(s + bias_q) to h_new and, when non-NULL,
 *     h_copy, as bvml_dsine_gru_update_f32 does; h_new may be h; C % 64 == 0
 *   bvml_dsine_conv_gru_gates_sum_f32, bvml_dsine_conv_gru_update_sum_f32
 *     the same with sums to add before the bias: sum0 holds 2C (gates) or C
 *     (update) planes in the packed channel order, i.e. what
 *     bvml_dsine_conv_f32 writes with the same packing (interleave = 1 for
 *     the gates), or NULL.  By linearity, conv(x, W) = conv(x_a, W_a) +
 *     conv(x_b, W_b) over a split of the input channels: the refiner
 *     computes the part over its constant channels (feature, uv) once per
 *     forward and passes it as sum0 to every iteration's convolution over
 *     the hidden state (each sum still fp32, in another order)
 * Outputs must not overlap x (or, for the fused ones, the other inputs and
 * each other).  No counterpart in the reference (brotensor's conv2d_forward
 * followed by its elementwise ops).
 */
long long bvml_dsine_conv_packed_size(int cout, int cin, int k);
int bvml_dsine_conv_pack_f32(const float* w, int cout, int cin, int k, int interleave,
                             float* wp);
int bvml_dsine_conv_f32(const float* x, int cin, int H, int W, const float* wp, int cout, int k,
                        float* out, void* stream);
int bvml_dsine_conv_gru_gates_f32(const float* x, int cin, int H, int W, const float* wp, int C,
                                  const float* bias_z, const float* bias_r, const float* h,
                                  float* z, float* rh, void* stream);
int bvml_dsine_conv_gru_update_f32(const float* x, int cin, int H, int W, const float* wp, int C,
                                   const float* bias_q, const float* z, const float* h,
                                   float* h_new, float* h_copy, void* stream);
int bvml_dsine_conv_gru_gates_sum_f32(const float* x, int cin, int H, int W, const float* wp,
                                      int C, const float* sum0, const float* bias_z,
                                      const float* bias_r, const float* h, float* z, float* rh,
                                      void* stream);
int bvml_dsine_conv_gru_update_sum_f32(const float* x, int cin, int H, int W, const float* wp,
                                       int C, const float* sum0, const float* bias_q,
                                       const float* z, const float* h, float* h_new,
                                       float* h_copy, void* stream);

/*
 * The heads' 3x3 first layers with the rest of the heads in the
 * convolution's epilogue: what bvml_dsine_conv_f32 (k = 3, cout = 64 nheads)
 * followed by bvml_dsine_heads_mlp_f32 computes, without the 64 nheads-plane
 * map between them.  For heads h < nheads and every pixel p:
 *   a = relu(conv3x3(x)[64h + c][p] + b0[64h + c])   c < 64
 *   t = relu(W2_h a + b2_h)
 *   out[h][o][p] = (W4_h t)[o] + b4[h][o]             o < outs[h]; b4[h] NULL: no bias
 * wp: the 3x3 weights of the nheads x 64 filters (bvml_dsine_conv_pack_f32,
 * k = 3); w2q: each head's W2 in the last-layer layout, nheads *
 * bvml_dsine_heads_packed_size(64) floats back to back (bvml_dsine_heads_pack_f32
 * with W2_h as a 64-output last layer); w4p[h], b0, b2, b4, outs as
 * bvml_dsine_heads_mlp_f32 takes them.  Each sum fp32 (the middle layer's
 * products in another order than bvml_dsine_heads_mlp_f32's), then its
 * bias added once.  nheads 1..4, outs 1..4096, at most 2^26 pixels; the
 * outputs must not overlap x or each other.  No counterpart in the
 * reference (src/dsine_refine.cpp:119-127 runs each head as three
 * convolutions and two ReLUs of brotensor ops).
 */
int bvml_dsine_conv_heads_f32(const float* x, int cin, int H, int W, const float* wp, int nheads,
                              const float* b0, const float* w2q, const float* b2,
                              const float* const* w4p, const float* const* b4, const int* outs,
                              float* const* out, void* stream);

/* Message for the calling thread's last non-zero status ("" if none). */
const char* bvml_dsine_last_error(void);

/* Library version string, e.g. "0.1.0". */
const char* bvml_dsine_version(void);

#ifdef __cplusplus
}
#endif

#endif /* BVML_DSINE_H */
