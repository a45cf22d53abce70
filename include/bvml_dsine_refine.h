/*
 * bvml_dsine_refine.h -- C ABI of the native NRN refiner: DSINE's
 * 5-iteration refinement loop on one HIP device (MI355X, gfx950).
 *
 * It replaces brovisionml's Refiner (the reference's
 * include/brovisionml/dsine_refine.h:113-145, src/dsine_refine.cpp:161-294):
 * the same weights, the same loop and the same result, in C++ over this
 * library's kernels (bvml_dsine.h) -- RayReLU, the ConvGRU's 5x5
 * convolutions as fp32 matrix-core implicit GEMMs with the gates and the
 * update fused, the heads after their 3x3 layer in one fused pass, the
 * propagate on the heads' raw logits, the convex upsample with its mask
 * bias -- and the heads' 3x3 layer on the same fp32 matrix-core convolution.
 * Its kernels and their launch shapes depend on the grid size only, so a
 * forward gives the same bits in every process.  The C++ class of
 * include/brovisionml/dsine_refine.h sits on top of it.
 *
 * Lifecycle: create (no HIP call) -> weights (load_file, or set_tensor per
 * tensor) -> forward, any number of times, at any grid size -> destroy.
 * The first forward binds the refiner to the calling thread's current HIP
 * device; later forwards make that device current and restore the caller's.
 * The first forward after a weight change uploads the weights (a
 * synchronous copy, after the device has finished any forward still
 * reading the old weights), and the first forward at a grid size allocates
 * its buffers (after the device has finished any forward still using the
 * previous size's): run one forward eagerly before capturing forwards into
 * a HIP graph.  Calls on one refiner from two host threads at once are not
 * allowed (the C++ Refiner class serializes its own); distinct refiners are
 * independent.
 *
 * Return value: 0 on success, a negative BVML_DSINE_E* code for a rejected
 * argument or missing weights (nothing is launched), a positive hipError_t
 * value for a HIP runtime error.  bvml_dsine_refiner_last_error() returns
 * the calling thread's message for the last non-zero status.
 */
#ifndef BVML_DSINE_REFINE_H
#define BVML_DSINE_REFINE_H

#include "bvml_dsine.h"

#ifdef __cplusplus
extern "C" {
#endif

#define BVML_DSINE_EWEIGHTS (-9)  /* a checkpoint tensor missing, of the wrong size or dtype */
#define BVML_DSINE_EFILE (-10)    /* the checkpoint cannot be read or is not safetensors */
#define BVML_DSINE_ELIB (-11)     /* reserved (no longer returned: the refiner uses no library
                                     convolution) */

typedef struct bvml_dsine_refiner bvml_dsine_refiner;

/* A refiner with no weights; makes no HIP call. */
int bvml_dsine_refiner_create(bvml_dsine_refiner** out);

/* Frees the refiner's device memory (NULL is a no-op). */
void bvml_dsine_refiner_destroy(bvml_dsine_refiner* r);

/*
 * Loads every refiner tensor from a safetensors checkpoint: the top-level
 * gru.conv{z,r,q}.{weight,bias} and {prob,xy,angle,up_prob}_head.{0,2,4}.
 * {weight,bias} (src/dsine_refine.cpp:51-91, :185-195), F32, F16 or BF16,
 * widened to fp32 as the reference's loader widens them (src/weights_util.h:27-63).
 * Other tensors in the file are ignored.  On error nothing changes.
 */
int bvml_dsine_refiner_load_file(bvml_dsine_refiner* r, const char* path);

/*
 * Sets one tensor, by its checkpoint name, from numel host fp32 values
 * (weights in OIHW order).  numel must be what the name holds:
 * bvml_dsine_refiner_tensor_numel(name).
 */
int bvml_dsine_refiner_set_tensor(bvml_dsine_refiner* r, const char* name, const float* data,
                                  long long numel);

/* The element count of the named checkpoint tensor, -1 for a name the
 * refiner does not read. */
long long bvml_dsine_refiner_tensor_numel(const char* name);

/* Copies a tensor the refiner holds back to numel host floats (for tests).
 * BVML_DSINE_EWEIGHTS if it has not been set. */
int bvml_dsine_refiner_get_tensor(const bvml_dsine_refiner* r, const char* name, float* data,
                                  long long numel);

/*
 * Runs Refiner::forward (src/dsine_refine.cpp:212-294) on device pointers:
 *   normal, feature, hidden: the decoder's /8-grid maps, 3, 64 and 64 fp32
 *     planes of h8 x w8 (include/brovisionml/dsine_decoder.h:96-102)
 *   fx, fy, cx, cy: the raw preprocess intrinsics (the +0.5 on the principal
 *     point is applied here, as build_ray8 applies it)
 *   orig_h, orig_w: the padded image size the /8 grid came from
 *   pad_t, pad_l, out_h, out_w: the crop of the 8*h8 x 8*w8 result
 *     (DsineTransform's pad_t, pad_l, orig_h, orig_w, src/dsine_refine.cpp:289-293)
 *   out: 3 x out_h x out_w fp32 planes, the refined unit normals
 *   coarse: NULL, or 5 x 3 x h8 x w8 floats that receive each iteration's
 *     propagated /8-grid normal (the loop's pred_norm)
 * Asynchronous on `stream` (NULL = the null stream).  Only the last
 * iteration's up-sampled map is the result (the reference computes and
 * discards the others), so the up-mask head's work runs in the last
 * iteration only.  out and coarse must not overlap the inputs.
 */
int bvml_dsine_refiner_forward(bvml_dsine_refiner* r, const float* normal, const float* feature,
                               const float* hidden, int h8, int w8, float fx, float fy,
                               float cx, float cy, int orig_h, int orig_w, int pad_t, int pad_l,
                               int out_h, int out_w, float* out, float* coarse, void* stream);

/*
 * The same loop on the CPU, for host pointers (Refiner::forward on
 * brotensor's CPU device, every step a CPU op in the reference): fp32
 * convolutions (a float sum over each output's taps, then the bias), the
 * ConvGRU's and heads' activations in float, RayReLU and the propagate from
 * the CPU branch of bvml_dsine.h (double precision in the reference's
 * operation order), the convex upsample + normalise in double rounded to
 * float once.  nthreads: host threads (0 = the hardware's; the result does
 * not depend on it).  Makes no HIP call.
 */
int bvml_dsine_refiner_forward_cpu(bvml_dsine_refiner* r, const float* normal,
                                   const float* feature, const float* hidden, int h8, int w8,
                                   float fx, float fy, float cx, float cy, int orig_h,
                                   int orig_w, int pad_t, int pad_l, int out_h, int out_w,
                                   float* out, float* coarse, int nthreads);

/*
 * bvml_dsine_refiner_forward on maps in a fixed device array of this library
 * instead of allocated ones: the variant for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  It
 * calls no hipMalloc or hipFree (the same kernels as
 * bvml_dsine_refiner_forward: the same result, bit for bit), and the weights
 * must already be on the device: a bvml_dsine_refiner_forward after the last
 * load_file / set_tensor uploads them (else BVML_DSINE_EWEIGHTS).  The array
 * holds 8,388,608 floats (32 MiB) per GPU, the maps of a grid of up to
 * 5,086 pixels (1,649 planes; a 60 x 80 grid needs 7,915,200 floats); a
 * larger grid returns BVML_DSINE_ESIZE.  Every call on one GPU uses that
 * GPU's array, which keeps the last call's contents (nothing in it needs to
 * start at zero), so calls on one GPU run in the order they were made: each
 * call's stream first waits for an event this library records after the
 * previous call's work, whatever stream that ran on.  Under stream capture
 * the call neither waits nor records (the caller orders the graph's
 * replays).  The first call on a device creates that event (set-up, once).
 * Arguments, checks and results otherwise as bvml_dsine_refiner_forward.
 */
int bvml_dsine_refiner_forward_noalloc(bvml_dsine_refiner* r, const float* normal,
                                       const float* feature, const float* hidden, int h8,
                                       int w8, float fx, float fy, float cx, float cy,
                                       int orig_h, int orig_w, int pad_t, int pad_l, int out_h,
                                       int out_w, float* out, float* coarse, void* stream);

/* Message for the calling thread's last non-zero refiner status ("" if none). */
const char* bvml_dsine_refiner_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* BVML_DSINE_REFINE_H */
