// Drop-in test of brovisionml::dsine::{ray_relu, angmf_propagate[_logits],
// convex_upsample[_normalize]} (the C++
// surface of include/brovisionml/dsine_ops.h), in the style of the
// reference's tests (tests/test_dsine_refine.cpp:48-53: CHECK + failure count).
//
//   test_dsine_ops cpu   error behaviour and the CPU branch of the dispatch
//                        (bit for bit against the oracle); makes no GPU call
//   test_dsine_ops gpu   the refiner's call pattern (src/dsine_refine.cpp:241-282:
//                        ray_relu once, then chained angmf_propagate calls, then
//                        the convex upsample + normalise)
//                        on a 60x80 grid against the CPU oracle
// The oracle (oracle/_build/liboracle_dsine.so) is linked to check results only.

#include "brovisionml/dsine_ops.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

extern "C" {
void oracle_ray_relu_f32(float* normal, const float* ray, int B, int H, int W,
                         long long ray_bstride);
void oracle_angmf_propagate_f32(const float* pred_norm, const float* prob, const float* xy,
                                const float* angle, const float* ray, double fu, double cu,
                                double fv, double cv, int B, int H, int W, int k,
                                long long ray_bstride, float* out);
void oracle_convex_upsample_f32(const float* x, const float* mask, int B, int C, int H, int W,
                                int s, int normalize, double eps, float* out, int nthreads);
}

using brotensor::Device;
using brotensor::Tensor;
namespace ops = brovisionml::dsine;

static int g_failures = 0;

#define CHECK(cond) do {                                                    \
    if (!(cond)) {                                                          \
        std::printf("  FAIL  %s:%d  %s\n", __FILE__, __LINE__, #cond);      \
        ++g_failures;                                                       \
    }                                                                       \
} while (0)

template <class F>
static bool throws_with(F f, const char* prefix, const char* needle) {
    try {
        f();
    } catch (const std::runtime_error& e) {
        const std::string m = e.what();
        const bool ok = m.rfind(prefix, 0) == 0 && m.find(needle) != std::string::npos;
        if (!ok) std::printf("    message was: %s\n", m.c_str());
        return ok;
    }
    return false;
}

// A tensor that claims to live on a device without touching the GPU: only
// the device tag matters for the dispatch checks exercised in cpu mode.
static Tensor fake_device(int rows, int cols, Device dev = Device::CUDA) {
    Tensor t = Tensor::mat(rows, cols);
    t.device = dev;
    return t;
}

static void test_errors() {
    std::printf("  error behaviour\n");
    const int H = 4, W = 6, HW = H * W;
    Tensor n = Tensor::mat(1, 3 * HW), r = Tensor::mat(1, 3 * HW);
    Tensor pr = Tensor::mat(1, 25 * HW), xy = Tensor::mat(1, 50 * HW), an = Tensor::mat(1, 25 * HW);
    Tensor out;
    // Device mismatch (src/dsine_ops.cpp:180-181, 200-202).
    Tensor dn = fake_device(1, 3 * HW);
    CHECK(throws_with([&] { ops::ray_relu(dn, r, H, W); }, "dsine ops: ",
                      "normal and ray must share a device"));
    CHECK(throws_with([&] { ops::angmf_propagate(dn, pr, xy, an, r, 1, 1, 1, 1, H, W, out); },
                      "dsine ops: ", "all inputs must share a device"));
    // Wrong sizes are rejected before any launch.
    Tensor dr = fake_device(1, 3 * HW), dpr = fake_device(1, 25 * HW), dxy = fake_device(1, 49 * HW);
    Tensor dan = fake_device(1, 25 * HW);
    CHECK(throws_with([&] { ops::angmf_propagate(dn, dpr, dxy, dan, dr, 1, 1, 1, 1, H, W, out); },
                      "dsine ops: ", "xy holds"));
    CHECK(throws_with([&] { ops::ray_relu(dn, dr, H + 1, W); }, "dsine ops: ", "normal holds"));
    CHECK(throws_with([&] { ops::ray_relu(dn, dr, -1, W); }, "dsine ops: ", "H and W"));
    // ... and on the CPU as well
    CHECK(throws_with([&] { ops::ray_relu(n, r, H, W + 1); }, "dsine ops: ", "normal holds"));
    CHECK(throws_with([&] { ops::angmf_propagate(n, pr, Tensor::mat(1, 49 * HW), an, r, 1, 1, 1, 1,
                                                 H, W, out); },
                      "dsine ops: ", "xy holds"));
    // Metal tensors have no path here
    Tensor mn = fake_device(1, 3 * HW, Device::Metal), mr = fake_device(1, 3 * HW, Device::Metal);
    CHECK(throws_with([&] { ops::ray_relu(mn, mr, H, W); }, "dsine ops: ", "does not run"));
    // convex upsample (+ normalise): the same checks
    Tensor mk = Tensor::mat(1, 576 * HW), dmk = fake_device(1, 576 * HW);
    CHECK(throws_with([&] { ops::convex_upsample_normalize(n, mk, 1, 3, H, W, 8, 1e-12f, out); },
                      "dsine ops: ", "CPU"));
    CHECK(throws_with([&] { ops::convex_upsample(dn, mk, 1, 3, H, W, 8, out); }, "dsine ops: ",
                      "x and mask must share a device"));
    CHECK(throws_with([&] { ops::convex_upsample(dn, dmk, 1, 3, H, W, 4, out); }, "dsine ops: ",
                      "mask holds"));
    CHECK(throws_with([&] { ops::convex_upsample_normalize(dn, dmk, 1, 2, H, W, 8, 1e-12f, out); },
                      "dsine ops: ", "x holds"));
    CHECK(throws_with([&] { ops::convex_upsample(dn, dmk, 1, 3, H, W, 0, out); }, "dsine ops: ",
                      "scale >= 1"));
}

static Tensor from_vec(const std::vector<float>& v);
struct Inputs;
static Inputs make_inputs(int H, int W, unsigned seed);
static void test_cpu_branch();

// Unit normals, sigmoid probs, raw xy, angles, ray_8 of a 480x640 image
// (intrins_from_fov + build_ray8, src/dsine_preprocess.cpp:35-46,
// src/dsine_decoder.cpp:242-293).
struct Inputs {
    int H, W;
    double fu, cu, fv, cv;
    std::vector<float> n, prob, xy, angle, ray;
};

static Inputs make_inputs(int H, int W, unsigned seed) {
    Inputs in;
    in.H = H;
    in.W = W;
    const int HW = H * W, origH = 8 * H, origW = 8 * W;
    const double kPi = 3.14159265358979323846;
    const double f = (std::max(origH, origW) / 2.0) / std::tan((60.0 / 2.0) * kPi / 180.0);
    const float fx = static_cast<float>(f), cx = static_cast<float>(origW / 2.0 - 0.5),
                cy = static_cast<float>(origH / 2.0 - 0.5);
    const double sw = static_cast<double>(W) / origW, sh = static_cast<double>(H) / origH;
    in.fu = fx * sw;
    in.cu = (cx + 0.5) * sw;
    in.fv = fx * sh;
    in.cv = (cy + 0.5) * sh;
    std::mt19937 rng(seed);
    std::normal_distribution<double> nd;
    in.n.resize(3 * HW);
    for (int p = 0; p < HW; ++p) {
        const double a = nd(rng), b = nd(rng), c = nd(rng), l = std::sqrt(a * a + b * b + c * c);
        in.n[p] = static_cast<float>(a / l);
        in.n[HW + p] = static_cast<float>(b / l);
        in.n[2 * HW + p] = static_cast<float>(c / l);
    }
    in.prob.resize(25 * HW);
    for (auto& v : in.prob) v = static_cast<float>(1.0 / (1.0 + std::exp(-nd(rng))));
    in.xy.resize(50 * HW);
    for (auto& v : in.xy) v = static_cast<float>(nd(rng));
    in.angle.resize(25 * HW);
    for (auto& v : in.angle) v = static_cast<float>(0.1 * nd(rng));
    in.ray.resize(3 * HW);
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x) {
            const int p = y * W + x;
            const double rx = static_cast<float>(((x + 0.5) - in.cu) / in.fu);
            const double ry = static_cast<float>(((y + 0.5) - in.cv) / in.fv);
            const double inv = 1.0 / std::max(std::sqrt(rx * rx + ry * ry + 1.0), 1e-12);
            in.ray[p] = static_cast<float>(rx * inv);
            in.ray[HW + p] = static_cast<float>(ry * inv);
            in.ray[2 * HW + p] = static_cast<float>(1.0 * inv);
        }
    return in;
}

static Tensor from_vec(const std::vector<float>& v) {
    Tensor t = Tensor::mat(1, static_cast<int>(v.size()));
    std::memcpy(t.host_f32_mut(), v.data(), v.size() * sizeof(float));
    return t;
}

static Tensor upload(const std::vector<float>& v) { return from_vec(v).to(Device::CUDA); }

static bool same_bits(const Tensor& t, const std::vector<float>& want) {
    if (t.device != Device::CPU || static_cast<std::size_t>(t.rows) * t.cols != want.size())
        return false;
    return std::memcmp(t.host_f32(), want.data(), want.size() * sizeof(float)) == 0;
}

// The CPU branch of the dispatch (src/dsine_ops.cpp:183-185, :203-206):
// ray_relu in place, then chained angmf_propagate calls and the logits
// variant, each bit for bit against the oracle, which restates the
// reference CPU twin in its operation order.
static void test_cpu_branch() {
    std::printf("  CPU branch of the dispatch (37x53, bit for bit)\n");
    const int H = 37, W = 53;
    Inputs in = make_inputs(H, W, 3);
    Tensor ray = from_vec(in.ray), prob = from_vec(in.prob), xy = from_vec(in.xy),
           angle = from_vec(in.angle), pred_norm = from_vec(in.n);
    ops::ray_relu(pred_norm, ray, H, W);
    std::vector<float> want_n = in.n;
    oracle_ray_relu_f32(want_n.data(), in.ray.data(), 1, H, W, 0);
    CHECK(same_bits(pred_norm, want_n));
    std::vector<float> want_out(3 * H * W);
    for (int it = 0; it < 2; ++it) {
        Tensor held = Tensor::mat(1, 3 * H * W), out = held;
        ops::angmf_propagate(pred_norm, prob, xy, angle, ray, in.fu, in.cu, in.fv, in.cv, H, W,
                             out);
        CHECK(out.device == Device::CPU && out.rows == 1 && out.cols == 3 * H * W);
        CHECK(out.data != held.data);  // a new tensor, as src/dsine_ops.cpp:83 makes
        oracle_angmf_propagate_f32(want_n.data(), in.prob.data(), in.xy.data(), in.angle.data(),
                                   in.ray.data(), in.fu, in.cu, in.fv, in.cv, 1, H, W, 5, 0,
                                   want_out.data());
        CHECK(same_bits(out, want_out));
        pred_norm = out;
        want_n = want_out;
    }
    // `out` the same object as pred_norm: the result is still the propagate
    // of the caller's pred_norm
    Tensor self = pred_norm;
    ops::angmf_propagate(self, prob, xy, angle, ray, in.fu, in.cu, in.fv, in.cv, H, W, self);
    oracle_angmf_propagate_f32(want_n.data(), in.prob.data(), in.xy.data(), in.angle.data(),
                               in.ray.data(), in.fu, in.cu, in.fv, in.cv, 1, H, W, 5, 0,
                               want_out.data());
    CHECK(same_bits(self, want_out));
    // logits: the CPU branch applies the correctly rounded float activations
    std::mt19937 rng(5);
    std::normal_distribution<double> nd;
    const float kPi = 3.14159265358979323846f;
    std::vector<float> lp(in.prob.size()), la(in.angle.size()), sp(lp.size()), ang(la.size());
    for (std::size_t i = 0; i < lp.size(); ++i) {
        lp[i] = static_cast<float>(3.0 * nd(rng));
        la[i] = static_cast<float>(3.0 * nd(rng));
        sp[i] = static_cast<float>(1.0 / (1.0 + std::exp(-static_cast<double>(lp[i]))));
        ang[i] = static_cast<float>(1.0 / (1.0 + std::exp(-static_cast<double>(la[i])))) * kPi;
    }
    Tensor lout;
    ops::angmf_propagate_logits(pred_norm, from_vec(lp), xy, from_vec(la), ray, in.fu, in.cu,
                                in.fv, in.cv, H, W, lout);
    oracle_angmf_propagate_f32(want_n.data(), sp.data(), in.xy.data(), ang.data(), in.ray.data(),
                               in.fu, in.cu, in.fv, in.cv, 1, H, W, 5, 0, want_out.data());
    CHECK(same_bits(lout, want_out));
    // the oracle's convex upsample on a closed form: equal mask logits give
    // each tap weight 1/9, so a constant map upsamples to itself and
    // normalises to its direction
    {
        const int uh = 3, uw = 4, us = 2, uhw = uh * uw;
        std::vector<float> x(3 * uhw), m(9 * us * us * uhw, 0.25f), up(3 * us * us * uhw);
        for (int p = 0; p < uhw; ++p) {
            x[p] = 3.0f;
            x[uhw + p] = 0.0f;
            x[2 * uhw + p] = 4.0f;
        }
        oracle_convex_upsample_f32(x.data(), m.data(), 1, 3, uh, uw, us, 0, 0.0, up.data(), 1);
        double e = 0.0;
        const int n = us * us * uhw;
        for (int p = 0; p < n; ++p)
            e = std::max({e, std::fabs(up[p] - 3.0), std::fabs(static_cast<double>(up[n + p])),
                          std::fabs(up[2 * n + p] - 4.0)});
        CHECK(e <= 1e-6);
        oracle_convex_upsample_f32(x.data(), m.data(), 1, 3, uh, uw, us, 1, 1e-12, up.data(), 1);
        e = 0.0;
        for (int p = 0; p < n; ++p)
            e = std::max({e, std::fabs(up[p] - 0.6), std::fabs(static_cast<double>(up[n + p])),
                          std::fabs(up[2 * n + p] - 0.8)});
        CHECK(e <= 1e-6);
    }
    // empty maps: out is an empty CPU tensor
    Tensor e = Tensor::mat(1, 0), eout;
    ops::angmf_propagate(e, e, e, e, e, 1, 1, 1, 1, 0, W, eout);
    CHECK(eout.device == Device::CPU && eout.rows == 1 && eout.cols == 0);
}

static double max_abs(const Tensor& dev, const std::vector<float>& want) {
    Tensor h = dev.to(Device::CPU);
    double m = 0.0;
    for (std::size_t i = 0; i < want.size(); ++i)
        m = std::max(m, std::fabs(static_cast<double>(h.host_f32()[i]) - want[i]));
    return m;
}

static void test_refiner_call_pattern() {
    std::printf("  refiner call pattern on the device (60x80)\n");
    const int H = 60, W = 80;
    Inputs in = make_inputs(H, W, 7);
    Tensor ray = upload(in.ray), prob = upload(in.prob), xy = upload(in.xy), angle = upload(in.angle);
    // pred_norm = RayReLU(decoder normal)
    Tensor pred_norm = upload(in.n);
    ops::ray_relu(pred_norm, ray, H, W);
    std::vector<float> want_n = in.n;
    oracle_ray_relu_f32(want_n.data(), in.ray.data(), 1, H, W, 0);
    const double e0 = max_abs(pred_norm, want_n);
    std::printf("    ray_relu max-abs %.3e\n", e0);
    CHECK(e0 <= 2.5e-7);
    // chained angmf_propagate (out feeds the next call, src/dsine_refine.cpp:271-273)
    std::vector<float> want_out(3 * H * W);
    for (int it = 0; it < 3; ++it) {
        Tensor new_pred;
        ops::angmf_propagate(pred_norm, prob, xy, angle, ray, in.fu, in.cu, in.fv, in.cv, H, W,
                             new_pred);
        CHECK(new_pred.device == Device::CUDA && new_pred.rows == 1 &&
              new_pred.cols == 3 * H * W);
        oracle_angmf_propagate_f32(want_n.data(), in.prob.data(), in.xy.data(), in.angle.data(),
                                   in.ray.data(), in.fu, in.cu, in.fv, in.cv, 1, H, W, 5, 0,
                                   want_out.data());
        const double e = max_abs(new_pred, want_out);
        std::printf("    angmf_propagate call %d max-abs %.3e\n", it, e);
        CHECK(e <= 1e-5);
        // the oracle chains its own output; the device chains the device's
        pred_norm = std::move(new_pred);
        want_n = want_out;
    }
    // `out` becomes a new tensor on the inputs' device (src/dsine_ops.cu:178):
    // a tensor the caller held in it keeps its contents.
    std::vector<float> want_next(3 * H * W);
    oracle_angmf_propagate_f32(want_n.data(), in.prob.data(), in.xy.data(), in.angle.data(),
                               in.ray.data(), in.fu, in.cu, in.fv, in.cv, 1, H, W, 5, 0,
                               want_next.data());
    Tensor held = Tensor::zeros_on(Device::CUDA, 1, 3 * H * W), out = held;
    ops::angmf_propagate(pred_norm, prob, xy, angle, ray, in.fu, in.cu, in.fv, in.cv, H, W, out);
    CHECK(out.data != held.data && out.device == Device::CUDA);
    CHECK(max_abs(held, std::vector<float>(3 * H * W, 0.0f)) == 0.0);
    CHECK(max_abs(out, want_next) <= 1e-5);
    // `out` the same object as pred_norm still propagates the caller's data.
    Tensor self = pred_norm;
    ops::angmf_propagate(self, prob, xy, angle, ray, in.fu, in.cu, in.fv, in.cv, H, W, self);
    CHECK(self.data != pred_norm.data);
    CHECK(max_abs(self, want_next) <= 1e-5);
    // the same step on the heads' raw logits: the kernel applies sigmoid and
    // sigmoid * pi (src/dsine_refine.cpp:262-267); the oracle takes the
    // correctly rounded float activations
    std::mt19937 rng(11);
    std::normal_distribution<double> nd;
    {
        const float kPi = 3.14159265358979323846f;
        std::vector<float> lp(in.prob.size()), la(in.angle.size());
        std::vector<float> sp(lp.size()), ang(la.size());
        for (std::size_t i = 0; i < lp.size(); ++i) {
            lp[i] = static_cast<float>(2.0 * nd(rng));
            la[i] = static_cast<float>(2.0 * nd(rng));
            sp[i] = static_cast<float>(1.0 / (1.0 + std::exp(-static_cast<double>(lp[i]))));
            ang[i] = static_cast<float>(1.0 / (1.0 + std::exp(-static_cast<double>(la[i])))) * kPi;
        }
        Tensor dlp = upload(lp), dla = upload(la), lout;
        ops::angmf_propagate_logits(pred_norm, dlp, xy, dla, ray, in.fu, in.cu, in.fv, in.cv, H,
                                    W, lout);
        CHECK(lout.device == Device::CUDA && lout.rows == 1 && lout.cols == 3 * H * W);
        oracle_angmf_propagate_f32(want_n.data(), sp.data(), in.xy.data(), ang.data(),
                                   in.ray.data(), in.fu, in.cu, in.fv, in.cv, 1, H, W, 5, 0,
                                   want_out.data());
        const double el = max_abs(lout, want_out);
        std::printf("    angmf_propagate_logits max-abs %.3e\n", el);
        CHECK(el <= 1e-5);
    }
    // up_pred_norm = normalize(convex_upsample(pred_norm, up_mask)) -- the
    // refiner's step after each propagate (src/dsine_refine.cpp:276-282)
    std::vector<float> mask(576 * H * W);
    for (auto& v : mask) v = static_cast<float>(nd(rng));
    std::vector<float> pn_host(3 * H * W), want_up(3 * 64 * H * W);
    {
        Tensor h = pred_norm.to(Device::CPU);
        std::memcpy(pn_host.data(), h.host_f32(), pn_host.size() * sizeof(float));
    }
    Tensor up_mask = upload(mask), up;
    ops::convex_upsample_normalize(pred_norm, up_mask, 1, 3, H, W, 8, 1e-12f, up);
    CHECK(up.device == Device::CUDA && up.rows == 1 && up.cols == 3 * 64 * H * W);
    oracle_convex_upsample_f32(pn_host.data(), mask.data(), 1, 3, H, W, 8, 1, (double)1e-12f,
                               want_up.data(), 1);
    const double eu = max_abs(up, want_up);
    std::printf("    convex_upsample_normalize max-abs %.3e\n", eu);
    CHECK(eu <= 1e-5);
    ops::convex_upsample(pred_norm, up_mask, 1, 3, H, W, 8, up);
    oracle_convex_upsample_f32(pn_host.data(), mask.data(), 1, 3, H, W, 8, 0, 0.0,
                               want_up.data(), 1);
    const double er = max_abs(up, want_up);
    std::printf("    convex_upsample max-abs %.3e\n", er);
    CHECK(er <= 1e-6);
    CHECK(hipDeviceSynchronize() == hipSuccess);
}

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    std::printf("test_dsine_ops (%s):\n", mode.c_str());
    try {
        if (mode == "cpu") {
            test_errors();
            test_cpu_branch();
        } else if (mode == "gpu") {
            int n = 0;
            if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
                std::printf("  no HIP device\n");
                return 2;
            }
            test_refiner_call_pattern();
        } else {
            std::printf("  unknown mode\n");
            return 2;
        }
    } catch (const std::exception& e) {
        std::printf("  error: %s\n", e.what());
        return 1;
    }
    if (g_failures == 0) {
        std::printf("  OK\n");
        return 0;
    }
    std::printf("  %d failure(s)\n", g_failures);
    return 1;
}
