// The native NRN refiner (include/bvml_dsine_refine.h): brovisionml's Refiner
// (src/dsine_refine.cpp:161-294) on one HIP device, over this library's C ABI
// (include/bvml_dsine.h).
//
// Once per forward, the ConvGRU convolutions' parts over [feature | uv], the
// channels no iteration changes (conv(cat(h, x), W) = conv(h, W_h) + conv(x,
// W_x)):
//   cf_zr = conv5x5([feature | uv], [W_z; W_r] over those channels), cf_q likewise
//                                                            bvml_dsine_conv_f32
// Per iteration (src/dsine_refine.cpp:255-287), on persistent per-grid maps:
//   z, r*h = gates of conv5x5(h, [W_z; W_r] over h) + cf_zr  bvml_dsine_conv_gru_gates_sum_f32
//   h    = (1 - z) h + z tanh(conv5x5(r*h, W_q over h) + cf_q + b_q),
//          also into [h | uv]                                bvml_dsine_conv_gru_update_sum_f32
//   prob, xy, angle = the three heads (conv3x3 -> ReLU -> conv1x1 -> ReLU -> conv1x1)
//          on [h | uv], the 1x1 layers in the 3x3 layer's epilogue
//                                                            bvml_dsine_conv_heads_f32, 66 -> 192
//          (last iteration, all four heads: t0 = conv3x3, 66 -> 256, then the 1x1 layers
//          on relu(t0 + b0)                     bvml_dsine_conv_f32, bvml_dsine_heads_mlp_f32)
//   pred = angmf_propagate(pred, prob, xy, angle) on logits  bvml_dsine_angmf_propagate_f32
// and, in the last iteration only, the up-mask head (its 1x1 layers in the
// same heads pass) and the convex upsample + normalise with its bias (the
// reference computes
// an up-sampled map every iteration but returns the last one only,
// src/dsine_refine.cpp:276-283, :289-293, so the others are dead work).  In
// the first four iterations the heads run for the three heads the propagate
// reads (their 3x3 layer at 192 channels); the last iteration runs all four
// (256).  The convolutions run without their bias; the fused kernels add it
// in the reference's rounding (a bias add after the convolution's sum).
//
// Every convolution is this library's implicit GEMM on the fp32 matrix cores
// (conv.hip): the kernels, their launch shapes and so their summation order
// depend on the grid size only, so a forward's result is the same in every
// process and from both forward entry points (a library that picks its
// algorithm by measured or estimated time, as MIOpen's immediate mode does,
// changes its rounding with the process's history).  The maps are allocated
// once per grid size.

#include "bvml_dsine_refine.h"
#include "refiner_common.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace bvml_refine {

namespace {
thread_local std::string g_last_error;
}  // namespace

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

const char* last_error() { return g_last_error.c_str(); }

bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes) {
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a0 < b0 + bbytes && b0 < a0 + abytes;
}

const std::vector<TensorSpec>& specs() {
    static const std::vector<TensorSpec> v = [] {
        std::vector<TensorSpec> s;
        auto conv = [&s](const std::string& p, int co, int ci, int k) {
            s.push_back({p + ".weight", co, (long long)co * ci * k * k});
            s.push_back({p + ".bias", co, co});
        };
        for (const char* g : {"convz", "convr", "convq"})
            conv(std::string("gru.") + g, kHidden, kHx, 5);
        for (int h = 0; h < kHeads; ++h) {
            const std::string p = kHeadName[h];
            conv(p + ".0", kMid, kHin, 3);
            conv(p + ".2", kMid, kMid, 1);
            conv(p + ".4", kHeadOut[h], kMid, 1);
        }
        return s;
    }();
    return v;
}

int spec_index(const char* name) {
    const auto& s = specs();
    for (size_t i = 0; i < s.size(); ++i)
        if (s[i].name == name) return (int)i;
    return -1;
}

int check_forward(const std::vector<std::vector<float>>& host, const ForwardArgs& a,
                  const std::string& who) {
    if (!a.normal || !a.feature || !a.hidden || !a.out)
        return fail(BVML_DSINE_ENULL,
                    who + "refiner, normal, feature, hidden and out must be non-NULL");
    if (a.h8 < 1 || a.w8 < 1 || a.orig_h < 1 || a.orig_w < 1)
        return fail(BVML_DSINE_ESHAPE, who + "h8, w8, orig_h and orig_w must be >= 1");
    const long long fh = (long long)kUp * a.h8, fw = (long long)kUp * a.w8;
    if (a.pad_t < 0 || a.pad_l < 0 || a.out_h < 1 || a.out_w < 1 ||
        a.pad_t + (long long)a.out_h > fh || a.pad_l + (long long)a.out_w > fw)
        return fail(BVML_DSINE_ESHAPE, who + "the crop (pad_t " + std::to_string(a.pad_t) +
                                           ", pad_l " + std::to_string(a.pad_l) + ", " +
                                           std::to_string(a.out_h) + " x " +
                                           std::to_string(a.out_w) + ") must lie inside the " +
                                           std::to_string(fh) + " x " + std::to_string(fw) +
                                           " result");
    if (3 * fh * fw > 0x7FFFFFFFll)
        return fail(BVML_DSINE_ESIZE, who + "3 x 8h8 x 8w8 exceeds a tensor row");
    if (!std::isfinite(a.fx) || !std::isfinite(a.fy) || a.fx == 0.0f || a.fy == 0.0f ||
        !std::isfinite(a.cx) || !std::isfinite(a.cy))
        return fail(BVML_DSINE_EPARAM, who + "fx, fy must be finite and non-zero, cx, cy finite");
    const auto& s = specs();
    for (size_t i = 0; i < s.size(); ++i)
        if (host[i].empty())
            return fail(BVML_DSINE_EWEIGHTS, who + "tensor '" + s[i].name + "' not set");
    const size_t hw = (size_t)a.h8 * a.w8, b = sizeof(float);
    const size_t outb = (size_t)3 * a.out_h * a.out_w * b, cb = (size_t)kIter * 3 * hw * b;
    for (const auto& in : {std::make_pair((const void*)a.normal, 3 * hw * b),
                           std::make_pair((const void*)a.feature, kFeature * hw * b),
                           std::make_pair((const void*)a.hidden, kHidden * hw * b)}) {
        if (overlaps(a.out, outb, in.first, in.second) ||
            (a.coarse && overlaps(a.coarse, cb, in.first, in.second)))
            return fail(BVML_DSINE_EALIAS, who + "out and coarse must not overlap the inputs");
    }
    if (a.coarse && overlaps(a.coarse, cb, a.out, outb))
        return fail(BVML_DSINE_EALIAS, who + "out and coarse must not overlap");
    return BVML_DSINE_OK;
}

}  // namespace bvml_refine

namespace {

using namespace bvml_refine;

// ---------------------------------------------------------------------------
// safetensors: an 8-byte little-endian header length, a JSON header mapping
// each tensor name to {"dtype", "shape", "data_offsets": [begin, end]} (byte
// offsets into the data that follows the header), optional "__metadata__".
// ---------------------------------------------------------------------------
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    double num = 0.0;
    bool integral = false;        // a literal with no fraction or exponent
    unsigned long long uint = 0;  // its value when integral and non-negative
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const std::string& key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonParser {
public:
    JsonParser(const char* p, const char* end) : p_(p), end_(end) {}

    bool document(Json& out) {
        if (!value(out, 0)) return false;
        ws();
        return p_ == end_;
    }

private:
    const char* p_;
    const char* end_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* s) {
        const size_t n = std::strlen(s);
        if ((size_t)(end_ - p_) < n || std::memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void put_utf8(std::string& s, unsigned cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(unsigned& v) {
        if (end_ - p_ < 4) return false;
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string& s) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_) {
            const char c = *p_++;
            if (c == '"') return true;
            if ((unsigned char)c < 0x20) return false;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) return false;
            const char e = *p_++;
            switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    unsigned cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {  // a surrogate pair
                        unsigned lo;
                        if (!lit("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return false;
                    }
                    put_utf8(s, cp);
                    break;
                }
                default: return false;
            }
        }
        return false;
    }
    bool number(Json& v) {
        const char* s = p_;
        if (p_ < end_ && *p_ == '-') ++p_;
        const char* digits = p_;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ == digits) return false;
        bool integral = true;
        if (p_ < end_ && *p_ == '.') {
            integral = false;
            ++p_;
            const char* f = p_;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
            if (p_ == f) return false;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            const char* f = p_;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
            if (p_ == f) return false;
        }
        const std::string text(s, p_);
        v.kind = Json::Num;
        v.num = std::strtod(text.c_str(), nullptr);
        v.integral = integral && *s != '-' && (p_ - digits) <= 19;
        if (v.integral) v.uint = std::strtoull(text.c_str(), nullptr, 10);
        return true;
    }
    bool value(Json& v, int depth) {
        if (depth > 16) return false;
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = Json::Obj;
            ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            for (;;) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                ++p_;
                Json child;
                if (!value(child, depth + 1)) return false;
                v.obj.emplace_back(std::move(key), std::move(child));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = Json::Arr;
            ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            for (;;) {
                Json child;
                if (!value(child, depth + 1)) return false;
                v.arr.push_back(std::move(child));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '"') {
            v.kind = Json::Str;
            return string(v.str);
        }
        if (lit("true") || lit("false")) {
            v.kind = Json::Bool;
            return true;
        }
        if (lit("null")) {
            v.kind = Json::Null;
            return true;
        }
        return number(v);
    }
};

// IEEE binary16 bits to float (exact: every half is a float).
float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        const float mag = std::ldexp((float)m, -24);  // zero or a subnormal
        std::memcpy(&bits, &mag, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

float bf16_to_float(uint16_t b) {
    const uint32_t bits = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

struct FileCloser {
    void operator()(std::FILE* f) const { std::fclose(f); }
};

// Reads the refiner's tensors of a safetensors file into `out` (one vector
// per spec); returns a status and sets the error message.
int read_checkpoint(const char* path, std::vector<std::vector<float>>& out) {
    const std::string who = "load_file: ";
    std::unique_ptr<std::FILE, FileCloser> f(std::fopen(path, "rb"));
    if (!f) return fail(BVML_DSINE_EFILE, who + "cannot open '" + path + "'");
    if (std::fseek(f.get(), 0, SEEK_END) != 0)
        return fail(BVML_DSINE_EFILE, who + "cannot seek '" + path + "'");
    const long long size = std::ftell(f.get());
    std::rewind(f.get());
    unsigned char len8[8];
    if (size < 8 || std::fread(len8, 1, 8, f.get()) != 8)
        return fail(BVML_DSINE_EFILE, who + "'" + path + "' is too short for a safetensors file");
    unsigned long long hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | len8[i];
    if (hlen == 0 || hlen > 100000000ull || (long long)hlen > size - 8)
        return fail(BVML_DSINE_EFILE, who + "'" + path + "' has a bad header length");
    std::string header(hlen, '\0');
    if (std::fread(&header[0], 1, hlen, f.get()) != hlen)
        return fail(BVML_DSINE_EFILE, who + "cannot read the header of '" + path + "'");
    Json root;
    if (!JsonParser(header.data(), header.data() + header.size()).document(root) ||
        root.kind != Json::Obj)
        return fail(BVML_DSINE_EFILE, who + "'" + path + "' has a malformed JSON header");
    const long long data0 = 8 + (long long)hlen, data_bytes = size - data0;

    const auto& s = specs();
    std::vector<std::vector<float>> got(s.size());
    for (size_t i = 0; i < s.size(); ++i) {
        const std::string& name = s[i].name;
        const Json* t = root.get(name);
        if (!t) return fail(BVML_DSINE_EWEIGHTS, who + "missing tensor '" + name + "'");
        const Json* dt = t->get("dtype");
        const Json* shape = t->get("shape");
        const Json* offs = t->get("data_offsets");
        if (t->kind != Json::Obj || !dt || dt->kind != Json::Str || !shape ||
            shape->kind != Json::Arr || !offs || offs->kind != Json::Arr || offs->arr.size() != 2 ||
            !offs->arr[0].integral || !offs->arr[1].integral)
            return fail(BVML_DSINE_EFILE, who + "tensor '" + name + "' has a malformed entry");
        int item;
        if (dt->str == "F32") item = 4;
        else if (dt->str == "F16" || dt->str == "BF16") item = 2;
        else
            return fail(BVML_DSINE_EWEIGHTS,
                        who + "unsupported dtype " + dt->str + " (key '" + name + "')");
        long long numel = 1;
        for (const Json& d : shape->arr) {
            if (!d.integral || d.uint > (1ull << 40))
                return fail(BVML_DSINE_EFILE, who + "tensor '" + name + "' has a bad shape");
            numel *= (long long)d.uint;
            if (numel > (1ll << 40))
                return fail(BVML_DSINE_EFILE, who + "tensor '" + name + "' has a bad shape");
        }
        if (numel != s[i].numel)
            return fail(BVML_DSINE_EWEIGHTS, who + "tensor '" + name + "' has " +
                                                 std::to_string(numel) + " elements, expected " +
                                                 std::to_string(s[i].numel));
        if (shape->arr.empty() || (long long)shape->arr[0].uint != s[i].c_out)
            return fail(BVML_DSINE_EWEIGHTS, who + "tensor '" + name + "' has " +
                                                 std::to_string(shape->arr.empty()
                                                                    ? 0ull
                                                                    : shape->arr[0].uint) +
                                                 " output channels, expected " +
                                                 std::to_string(s[i].c_out));
        const unsigned long long b = offs->arr[0].uint, e = offs->arr[1].uint;
        if (e < b || e > (unsigned long long)data_bytes ||
            e - b != (unsigned long long)numel * item)
            return fail(BVML_DSINE_EFILE, who + "tensor '" + name + "' has bad data offsets");
        std::vector<unsigned char> raw(e - b);
        if (std::fseek(f.get(), (long)(data0 + (long long)b), SEEK_SET) != 0 ||
            std::fread(raw.data(), 1, raw.size(), f.get()) != raw.size())
            return fail(BVML_DSINE_EFILE, who + "cannot read tensor '" + name + "'");
        std::vector<float>& dst = got[i];
        dst.resize((size_t)numel);
        for (long long j = 0; j < numel; ++j) {
            const unsigned char* q = raw.data() + j * item;
            if (item == 4) {
                uint32_t bits = (uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) |
                                ((uint32_t)q[3] << 24);
                std::memcpy(&dst[j], &bits, 4);
            } else {
                const uint16_t h = (uint16_t)(q[0] | (q[1] << 8));
                dst[j] = dt->str == "F16" ? half_to_float(h) : bf16_to_float(h);
            }
        }
    }
    out = std::move(got);
    return BVML_DSINE_OK;
}

// ---------------------------------------------------------------------------
// Device side
// ---------------------------------------------------------------------------
int hip_fail(hipError_t e, const std::string& what) {
    return fail((int)e, "forward: " + what + ": " + hipGetErrorString(e));
}

// Restores the caller's current device on scope exit.
class DeviceScope {
public:
    explicit DeviceScope(int dev) {
        if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
        if (prev_ != dev) status_ = hipSetDevice(dev);
    }
    ~DeviceScope() {
        int cur = -1;
        if (prev_ >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev_)
            (void)hipSetDevice(prev_);
    }
    hipError_t status() const { return status_; }

private:
    int prev_ = -1;
    hipError_t status_ = hipSuccess;
};

size_t round64(size_t n) { return (n + 63) & ~(size_t)63; }

}  // namespace

struct bvml_dsine_refiner {
    std::vector<std::vector<float>> host = std::vector<std::vector<float>>(specs().size());
    bool dirty = true;  // host weights newer than the device copy

    int device = -1;  // bound at the first forward

    // weights on the device, one allocation
    float* warena = nullptr;
    // convz + convr and convq, each split by input channels into the part
    // over h (every iteration) and the part over [feature | uv] (once per
    // forward), packed for the implicit-GEMM kernels
    const float *w_zr_h = nullptr, *w_zr_f = nullptr, *b_z = nullptr, *b_r = nullptr;
    const float *w_q_h = nullptr, *w_q_f = nullptr, *b_q = nullptr;
    const float *b_h0 = nullptr, *w2p = nullptr, *b_h2 = nullptr;
    // the three propagate heads' middle layers in the last-layer layout, for
    // bvml_dsine_conv_heads_f32
    const float* w2q = nullptr;
    const float* w_h0p[2] = {};  // the 3x3 layer packed for bvml_dsine_conv_f32 (192, 256 filters)
    const float* w4p[kHeads] = {};  // the 1x1 layers packed for bvml_dsine_heads_mlp_f32
    const float* b4[kHeads] = {};

    // the maps of one grid size, one allocation
    int H = 0, W = 0;
    float* arena = nullptr;
    Maps maps{};  // the maps' places in `arena` (maps_at)

    void drop_grid() {
        if (arena) (void)hipFree(arena);
        arena = nullptr;
        H = W = 0;
    }

    ~bvml_dsine_refiner() {
        if (device < 0) return;
        DeviceScope scope(device);
        drop_grid();
        if (warena) (void)hipFree(warena);
    }

    int upload();
    int plan(int H, int W);
};

// Copies the host weights into the device arena, in the layout the kernels
// read: [W_z; W_r] as one 128-filter weight, the four heads' first layers as
// one 192- and one 256-filter weight (each head's filters contiguous, prob,
// xy, angle, up_mask: the first three heads are a prefix), all three packed
// for bvml_dsine_conv_*, and the heads' 1x1 layers packed for
// bvml_dsine_heads_mlp_f32 (and the first three heads' middle layers again,
// in the last-layer layout, for bvml_dsine_conv_heads_f32).
int bvml_dsine_refiner::upload() {
    std::vector<float> w2(kHeads * kMid * kMid), w2p_h((size_t)kHeads * 4096);
    std::vector<std::vector<float>> w4p_h(kHeads);
    const float* w4src[kHeads];
    float* w4dst[kHeads];
    for (int h = 0; h < kHeads; ++h) {
        std::memcpy(&w2[(size_t)h * kMid * kMid], host[head_w(h, 1)].data(),
                    (size_t)kMid * kMid * sizeof(float));
        w4p_h[h].resize((size_t)bvml_dsine_heads_packed_size(kHeadOut[h]));
        w4src[h] = host[head_w(h, 2)].data();
        w4dst[h] = w4p_h[h].data();
    }
    if (const int st = bvml_dsine_heads_pack_f32(w2.data(), w4src, kHeadOut, kHeads, w2p_h.data(),
                                                 w4dst))
        return fail(st, std::string("forward: heads_pack: ") + bvml_dsine_last_error());
    // W2 of each of the first three heads packed as a 64-output last layer
    constexpr int kProp = kHeads - 1;
    const long long w2q_n = bvml_dsine_heads_packed_size(kMid);
    std::vector<float> w2q_h((size_t)kProp * w2q_n), w2p_tmp((size_t)kProp * 4096);
    {
        const float* src[kProp];
        float* dst[kProp];
        int outs[kProp];
        for (int h = 0; h < kProp; ++h) {
            src[h] = &w2[(size_t)h * kMid * kMid];
            dst[h] = &w2q_h[(size_t)h * w2q_n];
            outs[h] = kMid;
        }
        if (const int st = bvml_dsine_heads_pack_f32(w2.data(), src, outs, kProp, w2p_tmp.data(),
                                                     dst))
            return fail(st, std::string("forward: heads_pack: ") + bvml_dsine_last_error());
    }
    // [W_z; W_r] with their 16-channel blocks interleaved, and W_q, each as
    // its input channels [0, kHidden) (h) and [kHidden, kHx) (feature, uv):
    // conv(cat(h, x), W) = conv(h, W_h) + conv(x, W_x)
    std::vector<float> wzr(host[kZw]);
    wzr.insert(wzr.end(), host[kRw].begin(), host[kRw].end());
    auto in_slice = [](const std::vector<float>& w, int cout, int c0, int c1) {
        std::vector<float> out;
        out.reserve((size_t)cout * (c1 - c0) * 25);
        for (int o = 0; o < cout; ++o)
            out.insert(out.end(), w.begin() + ((size_t)o * kHx + c0) * 25,
                       w.begin() + ((size_t)o * kHx + c1) * 25);
        return out;
    };
    std::vector<float> wsplit_p[4];
    {
        const std::vector<float>* src[4] = {&wzr, &wzr, &host[kQw], &host[kQw]};
        const int cout[4] = {2 * kHidden, 2 * kHidden, kHidden, kHidden};
        const int c0[4] = {0, kHidden, 0, kHidden}, c1[4] = {kHidden, kHx, kHidden, kHx};
        const int il[4] = {1, 1, 0, 0};
        for (int i = 0; i < 4; ++i) {
            const std::vector<float> w = in_slice(*src[i], cout[i], c0[i], c1[i]);
            wsplit_p[i].resize((size_t)bvml_dsine_conv_packed_size(cout[i], c1[i] - c0[i], 5));
            if (const int st = bvml_dsine_conv_pack_f32(w.data(), cout[i], c1[i] - c0[i], 5, il[i],
                                                        wsplit_p[i].data()))
                return fail(st, std::string("forward: conv_pack: ") + bvml_dsine_last_error());
        }
    }
    std::vector<float> wh0;
    for (int h = 0; h < kHeads; ++h)
        wh0.insert(wh0.end(), host[head_w(h, 0)].begin(), host[head_w(h, 0)].end());
    std::vector<float> wh0_p[2];
    for (int i = 0; i < 2; ++i) {
        const int co = (3 + i) * kMid;
        wh0_p[i].resize((size_t)bvml_dsine_conv_packed_size(co, kHin, 3));
        if (const int st = bvml_dsine_conv_pack_f32(wh0.data(), co, kHin, 3, 0, wh0_p[i].data()))
            return fail(st, std::string("forward: conv_pack: ") + bvml_dsine_last_error());
    }
    using Src = std::vector<const std::vector<float>*>;
    std::vector<std::pair<const float**, Src>> parts;
    parts.push_back({&w_zr_h, {&wsplit_p[0]}});
    parts.push_back({&w_zr_f, {&wsplit_p[1]}});
    parts.push_back({&b_z, {&host[kZb]}});
    parts.push_back({&b_r, {&host[kRb]}});
    parts.push_back({&w_q_h, {&wsplit_p[2]}});
    parts.push_back({&w_q_f, {&wsplit_p[3]}});
    parts.push_back({&b_q, {&host[kQb]}});
    Src h0b, h2b;
    for (int h = 0; h < kHeads; ++h) {
        h0b.push_back(&host[head_b(h, 0)]);
        h2b.push_back(&host[head_b(h, 1)]);
    }
    parts.push_back({&w_h0p[0], {&wh0_p[0]}});
    parts.push_back({&w_h0p[1], {&wh0_p[1]}});
    parts.push_back({&b_h0, h0b});
    parts.push_back({&w2p, {&w2p_h}});
    parts.push_back({&w2q, {&w2q_h}});
    parts.push_back({&b_h2, h2b});
    for (int h = 0; h < kHeads; ++h) {
        parts.push_back({&w4p[h], {&w4p_h[h]}});
        parts.push_back({&b4[h], {&host[head_b(h, 2)]}});
    }
    std::vector<size_t> offset;
    size_t total = 0;
    for (const auto& p : parts) {
        offset.push_back(total);
        size_t n = 0;
        for (const std::vector<float>* v : p.second) n += v->size();
        total += round64(n);
    }
    std::vector<float> staging(total, 0.0f);
    for (size_t k = 0; k < parts.size(); ++k) {
        size_t at = offset[k];
        for (const std::vector<float>* v : parts[k].second) {
            std::memcpy(&staging[at], v->data(), v->size() * sizeof(float));
            at += v->size();
        }
    }
    if (!warena) {
        const hipError_t e = hipMalloc(&warena, total * sizeof(float));
        if (e != hipSuccess) {
            warena = nullptr;
            return hip_fail(e, "hipMalloc of the weights");
        }
    } else {
        // a forward queued earlier, on any stream of the device, may still be
        // reading the weights: wait for it before overwriting them
        const hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
    }
    const hipError_t e = hipMemcpy(warena, staging.data(), total * sizeof(float),
                                   hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "weight upload");
    for (size_t k = 0; k < parts.size(); ++k) *parts[k].first = warena + offset[k];
    dirty = false;
    return BVML_DSINE_OK;
}

// Allocates the maps of an H x W grid.  The maps of the previous size are
// freed first, once every forward queued on any stream of the device (which
// may still be reading them) has finished.
int bvml_dsine_refiner::plan(int h, int w) {
    if (arena && H == h && W == w) return BVML_DSINE_OK;
    if (arena) {
        const hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
    }
    drop_grid();
    const size_t hw = (size_t)h * w;
    const hipError_t e = hipMalloc(&arena, maps_floats(hw) * sizeof(float));
    if (e != hipSuccess) {
        arena = nullptr;
        return hip_fail(e, "hipMalloc of the maps");
    }
    maps = maps_at(arena, hw);
    H = h;
    W = w;
    return BVML_DSINE_OK;
}

const std::vector<std::vector<float>>& bvml_refine::host_weights(const bvml_dsine_refiner* r) {
    return r->host;
}

// The loop of Refiner::forward on the maps `m`, after forward's checks, with
// the refiner's device current and its weights on it.
int bvml_refine::forward_maps(bvml_dsine_refiner* r, const Maps& m, const ForwardArgs& a,
                              void* stream) {
    const int h8 = a.h8, w8 = a.w8, pad_t = a.pad_t, pad_l = a.pad_l;
    const int out_h = a.out_h, out_w = a.out_w;
    float* out = a.out;
    float* coarse = a.coarse;
    const size_t hw = (size_t)h8 * w8, b = sizeof(float);
    const long long fh = (long long)kUp * h8, fw = (long long)kUp * w8;
    const hipStream_t strm = static_cast<hipStream_t>(stream);
    int st;
    // the grid-scaled intrinsics (src/dsine_refine.cpp:232-237)
    const double sw = (double)w8 / a.orig_w, sh = (double)h8 / a.orig_h;
    const double fu = a.fx * sw, cu = (a.cx + 0.5) * sw, fv = a.fy * sh, cv = (a.cy + 0.5) * sh;
    const int C = kHidden;
    auto copy = [&](float* dst, const float* src, size_t planes) {
        return hipMemcpyAsync(dst, src, planes * hw * b, hipMemcpyDeviceToDevice, strm);
    };
    // a kernel library status, with its message
    auto ck = [](int status, const char* what) {
        return status == BVML_DSINE_OK
                   ? BVML_DSINE_OK
                   : fail(status, std::string("forward: ") + what + ": " + bvml_dsine_last_error());
    };
    hipError_t e;
    // hx = [h | feature | uv], rh = r*h, hin = [h_new | uv]
    float* uv = m.hx + (size_t)(kHidden + kFeature) * hw;
    if ((st = ck(bvml_dsine_build_uv8_f32(uv, fu, cu, fv, cv, h8, w8, stream), "build_uv8")) ||
        (st = ck(bvml_dsine_build_ray8_f32(m.ray, fu, cu, fv, cv, h8, w8, stream), "build_ray8")))
        return st;
    // (h itself is not copied: the first iteration reads the decoder's
    // hidden state, and its update writes h_new into hx)
    if ((e = copy(m.hx + (size_t)kHidden * hw, a.feature, kFeature)) != hipSuccess ||
        (e = copy(m.hin + (size_t)kHidden * hw, uv, 2)) != hipSuccess ||
        (e = copy(m.pred[0], a.normal, 3)) != hipSuccess)
        return hip_fail(e, "hipMemcpyAsync");
    // pred_norm = RayReLU(decoder.normal, ray_8)  (:240-242)
    if ((st = ck(bvml_dsine_ray_relu_f32(m.pred[0], m.ray, 1, h8, w8, 0, stream), "ray_relu")))
        return st;
    // the ConvGRU convolutions' parts over [feature | uv], which no
    // iteration changes: once per forward instead of once per iteration
    float* cf_zr = m.cf;
    float* cf_q = m.cf + (size_t)2 * kHidden * hw;
    const float* xf = m.hx + (size_t)kHidden * hw;
    if ((st = ck(bvml_dsine_conv_f32(xf, kX, h8, w8, r->w_zr_f, 2 * kHidden, 5, cf_zr, stream),
                 "conv")) ||
        (st = ck(bvml_dsine_conv_f32(xf, kX, h8, w8, r->w_q_f, kHidden, 5, cf_q, stream), "conv")))
        return st;

    const bool direct = pad_t == 0 && pad_l == 0 && out_h == fh && out_w == fw;
    int cur = 0;
    for (int it = 0; it < kIter; ++it) {
        const bool last = it == kIter - 1;
        const int nh = last ? kHeads : kHeads - 1;
        // ConvGRU (:138-159): the two 5x5 convolutions over h (r*h) plus
        // their parts over [feature | uv], with the gates and the update in
        // their epilogues; h_new goes to hx (over h after the first
        // iteration, which reads the decoder's hidden state) and into hin
        const float* h = it == 0 ? a.hidden : m.hx;
        if ((st = ck(bvml_dsine_conv_gru_gates_sum_f32(h, kHidden, h8, w8, r->w_zr_h, C, cf_zr,
                                                       r->b_z, r->b_r, h, m.z, m.rh, stream),
                     "conv_gru_gates")) ||
            (st = ck(bvml_dsine_conv_gru_update_sum_f32(m.rh, kHidden, h8, w8, r->w_q_h, C, cf_q,
                                                        r->b_q, m.z, h, m.hx, m.hin, stream),
                     "conv_gru_update")))
            return st;
        // the heads (:119-127, :257-267, :276): in the first four iterations
        // the three the propagate reads, as their 3x3 layer with the rest in
        // its epilogue; in the last all four, the 3x3 layers, then the rest
        // in one pass (the up-mask head's last layer, 576 outputs, is too
        // large to fuse); the up-mask head's last bias is the upsample's
        const float* b4[kHeads] = {r->b4[0], r->b4[1], r->b4[2], nullptr};
        if (!last) {
            if ((st = ck(bvml_dsine_conv_heads_f32(m.hin, kHin, h8, w8, r->w_h0p[0], nh, r->b_h0,
                                                   r->w2q, r->b_h2, r->w4p, b4, kHeadOut, m.head,
                                                   stream), "conv_heads")))
                return st;
        } else if ((st = ck(bvml_dsine_conv_f32(m.hin, kHin, h8, w8, r->w_h0p[1], nh * kMid, 3,
                                                m.t0, stream), "conv")) ||
                   (st = ck(bvml_dsine_heads_mlp_f32(m.t0, r->b_h0, r->w2p, r->b_h2, r->w4p, b4,
                                                     kHeadOut, nh, h8, w8, m.head, stream),
                            "heads_mlp"))) {
            return st;
        }
        // the propagate on the logits (:262-274)
        if ((st = ck(bvml_dsine_angmf_propagate_f32(m.pred[cur], m.head[0], m.head[1],
                                                    m.head[2], m.ray, fu, cu, fv, cv, 1, h8, w8,
                                                    kPs, 0, m.pred[cur ^ 1], BVML_DSINE_LOGITS,
                                                    stream), "angmf_propagate")))
            return st;
        cur ^= 1;
        if (coarse && (e = copy(coarse + (size_t)it * 3 * hw, m.pred[cur], 3)) != hipSuccess)
            return hip_fail(e, "hipMemcpyAsync");
        if (!last) continue;
        // up_pred_norm = normalize(convex_upsample(pred_norm, up_mask))  (:276-283)
        float* dst = direct ? out : m.up;
        if ((st = ck(bvml_dsine_convex_upsample_bias_f32(m.pred[cur], m.head[3], r->b4[3], 1, 3,
                                                         h8, w8, kUp, 1, kUpEps, dst, 0, stream),
                     "convex_upsample")))
            return st;
    }
    if (!direct) {
        // the crop to the unpadded image (:289-293)
        for (int c = 0; c < 3; ++c) {
            const float* src = m.up + (size_t)c * fh * fw + (size_t)pad_t * fw + pad_l;
            e = hipMemcpy2DAsync(out + (size_t)c * out_h * out_w, (size_t)out_w * b, src,
                                 (size_t)fw * b, (size_t)out_w * b, (size_t)out_h,
                                 hipMemcpyDeviceToDevice, strm);
            if (e != hipSuccess) return hip_fail(e, "hipMemcpy2DAsync");
        }
    }
    return BVML_DSINE_OK;
}

int bvml_refine::refiner_device(const bvml_dsine_refiner* r) { return r->device; }

bool bvml_refine::refiner_uploaded(const bvml_dsine_refiner* r) {
    return r->warena != nullptr && !r->dirty;
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int bvml_dsine_refiner_create(bvml_dsine_refiner** out) {
    if (!out) return fail(BVML_DSINE_ENULL, "create: out must be non-NULL");
    *out = new (std::nothrow) bvml_dsine_refiner();
    if (!*out) return fail(BVML_DSINE_ESIZE, "create: out of host memory");
    return BVML_DSINE_OK;
}

void bvml_dsine_refiner_destroy(bvml_dsine_refiner* r) { delete r; }

long long bvml_dsine_refiner_tensor_numel(const char* name) {
    if (!name) return -1;
    const int i = spec_index(name);
    return i < 0 ? -1 : specs()[i].numel;
}

int bvml_dsine_refiner_load_file(bvml_dsine_refiner* r, const char* path) {
    if (!r || !path) return fail(BVML_DSINE_ENULL, "load_file: refiner and path must be non-NULL");
    std::vector<std::vector<float>> got;
    const int st = read_checkpoint(path, got);
    if (st != BVML_DSINE_OK) return st;
    r->host = std::move(got);
    r->dirty = true;
    return BVML_DSINE_OK;
}

int bvml_dsine_refiner_set_tensor(bvml_dsine_refiner* r, const char* name, const float* data,
                                  long long numel) {
    if (!r || !name || !data)
        return fail(BVML_DSINE_ENULL, "set_tensor: refiner, name and data must be non-NULL");
    const int i = spec_index(name);
    if (i < 0) return fail(BVML_DSINE_EWEIGHTS, std::string("set_tensor: unknown tensor '") + name +
                                                    "'");
    if (numel != specs()[i].numel)
        return fail(BVML_DSINE_EWEIGHTS, std::string("set_tensor: tensor '") + name + "' has " +
                                             std::to_string(numel) + " elements, expected " +
                                             std::to_string(specs()[i].numel));
    r->host[i].assign(data, data + numel);
    r->dirty = true;
    return BVML_DSINE_OK;
}

int bvml_dsine_refiner_get_tensor(const bvml_dsine_refiner* r, const char* name, float* data,
                                  long long numel) {
    if (!r || !name || !data)
        return fail(BVML_DSINE_ENULL, "get_tensor: refiner, name and data must be non-NULL");
    const int i = spec_index(name);
    if (i < 0) return fail(BVML_DSINE_EWEIGHTS, std::string("get_tensor: unknown tensor '") + name +
                                                    "'");
    if (r->host[i].empty())
        return fail(BVML_DSINE_EWEIGHTS, std::string("get_tensor: tensor '") + name + "' not set");
    if (numel != specs()[i].numel)
        return fail(BVML_DSINE_EWEIGHTS, std::string("get_tensor: tensor '") + name + "' has " +
                                             std::to_string(specs()[i].numel) + " elements, not " +
                                             std::to_string(numel));
    std::memcpy(data, r->host[i].data(), (size_t)numel * sizeof(float));
    return BVML_DSINE_OK;
}

const char* bvml_dsine_refiner_last_error(void) { return bvml_refine::last_error(); }

int bvml_dsine_refiner_forward(bvml_dsine_refiner* r, const float* normal, const float* feature,
                               const float* hidden, int h8, int w8, float fx, float fy,
                               float cx, float cy, int orig_h, int orig_w, int pad_t, int pad_l,
                               int out_h, int out_w, float* out, float* coarse, void* stream) {
    if (!r) return fail(BVML_DSINE_ENULL, "forward: refiner must be non-NULL");
    const ForwardArgs args{normal, feature, hidden, h8, w8, fx, fy, cx, cy, orig_h, orig_w,
                           pad_t, pad_l, out_h, out_w, out, coarse};
    if (const int st = check_forward(r->host, args, "forward: ")) return st;
    if (r->device < 0) {
        int d = 0;
        const hipError_t e = hipGetDevice(&d);
        if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
        r->device = d;
    }
    DeviceScope scope(r->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    int st;
    if (r->dirty && (st = r->upload()) != BVML_DSINE_OK) return st;
    if ((st = r->plan(h8, w8)) != BVML_DSINE_OK) return st;
    return bvml_refine::forward_maps(r, r->maps, args, stream);
}

}  // extern "C"
