// Stand-ins for the C ABI's device entry points (include/bvml_dsine.h), for
// the sanitizer builds of test_dsine_ops and test_dsine_refine: they compile
// the host code (the C++ layer, the CPU branch, the refiner's host path and
// checkpoint reader, the error state, the oracle) with AddressSanitizer and
// UBSan and link no GPU code.  Their cpu modes call none of these; each
// fails loudly if it ever is.

#include "bvml_dsine.h"

#include <cstdio>
#include <cstdlib>

namespace {
[[noreturn]] void no_device(const char* fn) {
    std::fprintf(stderr, "%s called in a build without device code\n", fn);
    std::abort();
}
}  // namespace

extern "C" {

int bvml_dsine_ray_relu_f32(float*, const float*, int, int, int, long long, void*) {
    no_device("bvml_dsine_ray_relu_f32");
}

int bvml_dsine_angmf_propagate_f32(const float*, const float*, const float*, const float*,
                                   const float*, double, double, double, double, int, int, int,
                                   int, long long, float*, unsigned, void*) {
    no_device("bvml_dsine_angmf_propagate_f32");
}

int bvml_dsine_convex_upsample_f32(const float*, const float*, int, int, int, int, int, int,
                                   float, float*, unsigned, void*) {
    no_device("bvml_dsine_convex_upsample_f32");
}

int bvml_dsine_convex_upsample_bias_f32(const float*, const float*, const float*, int, int, int,
                                        int, int, int, float, float*, unsigned, void*) {
    no_device("bvml_dsine_convex_upsample_bias_f32");
}

int bvml_dsine_build_ray8_f32(float*, double, double, double, double, int, int, void*) {
    no_device("bvml_dsine_build_ray8_f32");
}

int bvml_dsine_build_uv8_f32(float*, double, double, double, double, int, int, void*) {
    no_device("bvml_dsine_build_uv8_f32");
}

int bvml_dsine_gru_gates_f32(const float*, const float*, const float*, const float*, int,
                             long long, float*, float*, void*) {
    no_device("bvml_dsine_gru_gates_f32");
}

int bvml_dsine_gru_update_f32(const float*, const float*, const float*, const float*, int,
                              long long, float*, float*, void*) {
    no_device("bvml_dsine_gru_update_f32");
}

int bvml_dsine_bias_act_f32(float*, const float*, int, long long, int, void*) {
    no_device("bvml_dsine_bias_act_f32");
}

int bvml_dsine_heads_mlp_f32(const float*, const float*, const float*, const float*,
                             const float* const*, const float* const*, const int*, int, int, int,
                             float* const*, void*) {
    no_device("bvml_dsine_heads_mlp_f32");
}

int bvml_dsine_conv_f32(const float*, int, int, int, const float*, int, int, float*, void*) {
    no_device("bvml_dsine_conv_f32");
}

int bvml_dsine_conv_gru_gates_f32(const float*, int, int, int, const float*, int, const float*,
                                  const float*, const float*, float*, float*, void*) {
    no_device("bvml_dsine_conv_gru_gates_f32");
}

int bvml_dsine_conv_gru_update_f32(const float*, int, int, int, const float*, int, const float*,
                                   const float*, const float*, float*, float*, void*) {
    no_device("bvml_dsine_conv_gru_update_f32");
}

int bvml_dsine_conv_gru_gates_sum_f32(const float*, int, int, int, const float*, int,
                                      const float*, const float*, const float*, const float*,
                                      float*, float*, void*) {
    no_device("bvml_dsine_conv_gru_gates_sum_f32");
}

int bvml_dsine_conv_gru_update_sum_f32(const float*, int, int, int, const float*, int,
                                       const float*, const float*, const float*, const float*,
                                       float*, float*, void*) {
    no_device("bvml_dsine_conv_gru_update_sum_f32");
}

int bvml_dsine_conv_heads_f32(const float*, int, int, int, const float*, int, const float*,
                              const float*, const float*, const float* const*,
                              const float* const*, const int*, float* const*, void*) {
    no_device("bvml_dsine_conv_heads_f32");
}

}  // extern "C"
