// Drop-in test of brovisionml::dsine::Refiner (include/brovisionml/dsine_refine.h,
// the class of the reference's include/brovisionml/dsine_refine.h:113-145),
// in the style of the reference's tests (tests/test_dsine_refine.cpp: CHECK +
// failure count).
//
//   test_dsine_refine errors
//       the class's error behaviour (src/dsine_refine.cpp:22-30, :197-208,
//       :215-216); makes no GPU call
//   test_dsine_refine run <cpu|gpu> <weights.safetensors> <case.bin> <out.bin>
//       load_file, to(device), forward on the decoder maps and intrinsics of
//       case.bin; writes the (1, 3*H*W) result to out.bin (the Python tests
//       compare it with the native refiner's own forward)
//   test_dsine_refine parse <file>...
//       load_file on each file, printing "ok" or the error (the sanitizer
//       run feeds it malformed checkpoints)
//
// case.bin: int32 h8, w8, orig_h, orig_w, pad_t, pad_l, out_h, out_w; float32
// fx, fy, cx, cy; then the normal (3), feature (64) and hidden (64) planes.

#include "brovisionml/dsine_refine.h"

#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

using brotensor::Device;
using brotensor::Tensor;
namespace ds = brovisionml::dsine;

static int g_failures = 0;

#define CHECK(cond) do {                                                    \
    if (!(cond)) {                                                          \
        std::printf("  FAIL  %s:%d  %s\n", __FILE__, __LINE__, #cond);      \
        ++g_failures;                                                       \
    }                                                                       \
} while (0)

template <class F>
static bool throws_with(F f, const char* needle) {
    try {
        f();
    } catch (const std::runtime_error& e) {
        const std::string m = e.what();
        const bool ok = m.rfind("dsine::Refiner: ", 0) == 0 && m.find(needle) != std::string::npos;
        if (!ok) std::printf("    message was: %s\n", m.c_str());
        return ok;
    }
    return false;
}

static void test_errors() {
    std::printf("  error behaviour\n");
    ds::Refiner r;
    CHECK(r.device() == Device::CPU);
    CHECK(throws_with([&] { r.to(Device::CUDA); }, "to() called before load()"));
    ds::DecoderOutput dec;
    dec.h8 = 2;
    dec.w8 = 2;
    ds::Intrinsics in;
    ds::DsineTransform tf;
    CHECK(throws_with([&] { r.forward(dec, in, 16, 16, tf); }, "forward() called before load()"));
    CHECK(throws_with([&] { r.load("/nonexistent-dir"); }, "cannot open '/nonexistent-dir/model.safetensors'"));
    CHECK(throws_with([&] { r.load_file(""); }, "cannot open"));
    CHECK(r.device() == Device::CPU);
    // moves keep the refiner usable
    ds::Refiner moved(std::move(r));
    CHECK(moved.device() == Device::CPU);
    ds::Refiner assigned;
    assigned = std::move(moved);
    CHECK(throws_with([&] { assigned.to(Device::CUDA); }, "to() called before load()"));
}

struct Case {
    int h8 = 0, w8 = 0, orig_h = 0, orig_w = 0, pad_t = 0, pad_l = 0, out_h = 0, out_w = 0;
    float fx = 0, fy = 0, cx = 0, cy = 0;
    std::vector<float> normal, feature, hidden;
};

static bool read_case(const char* path, Case& c) {
    std::FILE* f = std::fopen(path, "rb");
    if (!f) return false;
    int hdr[8];
    float intr[4];
    bool ok = std::fread(hdr, sizeof(int), 8, f) == 8 && std::fread(intr, sizeof(float), 4, f) == 4;
    if (ok) {
        c.h8 = hdr[0]; c.w8 = hdr[1]; c.orig_h = hdr[2]; c.orig_w = hdr[3];
        c.pad_t = hdr[4]; c.pad_l = hdr[5]; c.out_h = hdr[6]; c.out_w = hdr[7];
        c.fx = intr[0]; c.fy = intr[1]; c.cx = intr[2]; c.cy = intr[3];
        const size_t hw = (size_t)c.h8 * c.w8;
        c.normal.resize(3 * hw);
        c.feature.resize(64 * hw);
        c.hidden.resize(64 * hw);
        ok = std::fread(c.normal.data(), sizeof(float), 3 * hw, f) == 3 * hw &&
             std::fread(c.feature.data(), sizeof(float), 64 * hw, f) == 64 * hw &&
             std::fread(c.hidden.data(), sizeof(float), 64 * hw, f) == 64 * hw;
    }
    std::fclose(f);
    return ok;
}

static Tensor host_tensor(const std::vector<float>& v) {
    Tensor t = Tensor::mat(1, (int)v.size());
    std::memcpy(t.host_f32_mut(), v.data(), v.size() * sizeof(float));
    return t;
}

static int run(const char* mode, const char* weights, const char* case_path, const char* out_path) {
    const Device dev = std::strcmp(mode, "gpu") == 0 ? Device::CUDA : Device::CPU;
    Case c;
    if (!read_case(case_path, c)) {
        std::printf("cannot read %s\n", case_path);
        return 2;
    }
    ds::Refiner r;
    r.load_file(weights);
    r.to(dev);
    CHECK(r.device() == dev);
    ds::DecoderOutput dec;
    dec.normal = host_tensor(c.normal).to(dev);
    dec.feature = host_tensor(c.feature).to(dev);
    dec.hidden = host_tensor(c.hidden).to(dev);
    dec.h8 = c.h8;
    dec.w8 = c.w8;
    ds::Intrinsics in;
    in.fx = c.fx; in.fy = c.fy; in.cx = c.cx; in.cy = c.cy;
    ds::DsineTransform tf;
    tf.orig_h = c.out_h; tf.orig_w = c.out_w; tf.pad_t = c.pad_t; tf.pad_l = c.pad_l;
    // a decoder map on the other device is refused
    ds::DecoderOutput wrong = dec;
    wrong.normal = host_tensor(c.normal);
    if (dev != Device::CPU)
        CHECK(throws_with([&] { r.forward(wrong, in, c.orig_h, c.orig_w, tf); },
                          "decoder normal is not on the refiner's device"));
    ds::DecoderOutput small = dec;
    small.h8 = c.h8 + 1;
    CHECK(throws_with([&] { r.forward(small, in, c.orig_h, c.orig_w, tf); }, "elements, expected"));
    Tensor out = r.forward(dec, in, c.orig_h, c.orig_w, tf);
    CHECK(out.device == dev);
    CHECK(out.rows == 1 && out.cols == 3 * c.out_h * c.out_w);
    // a second forward gives the same result
    Tensor again = r.forward(dec, in, c.orig_h, c.orig_w, tf).to(Device::CPU);
    Tensor host = out.to(Device::CPU);
    CHECK(std::memcmp(host.host_f32(), again.host_f32(), (size_t)host.cols * sizeof(float)) == 0);
    std::FILE* f = std::fopen(out_path, "wb");
    if (!f) return 2;
    std::fwrite(host.host_f32(), sizeof(float), (size_t)host.cols, f);
    std::fclose(f);
    return 0;
}

int main(int argc, char** argv) {
    if (argc < 2) {
        std::printf("usage: %s errors | run <cpu|gpu> <weights> <case.bin> <out.bin> | parse <file>...\n",
                    argv[0]);
        return 2;
    }
    const std::string mode = argv[1];
    try {
        if (mode == "errors") {
            test_errors();
        } else if (mode == "run" && argc == 6) {
            const int st = run(argv[2], argv[3], argv[4], argv[5]);
            if (st) return st;
        } else if (mode == "parse") {
            for (int i = 2; i < argc; ++i) {
                ds::Refiner r;
                try {
                    r.load_file(argv[i]);
                    std::printf("%s: ok\n", argv[i]);
                } catch (const std::runtime_error& e) {
                    std::printf("%s: %s\n", argv[i], e.what());
                }
            }
        } else {
            std::printf("unknown mode %s\n", mode.c_str());
            return 2;
        }
    } catch (const std::exception& e) {
        std::printf("  FAIL  uncaught: %s\n", e.what());
        ++g_failures;
    }
    if (g_failures) {
        std::printf("%d failure(s)\n", g_failures);
        return 1;
    }
    std::printf("OK\n");
    return 0;
}
