// Host-side packing of the refiner's weights for its matrix-core kernels
// (the C ABI's bvml_dsine_heads_pack_f32, bvml_dsine_conv_pack_f32 and their
// sizes): each 64-lane operand fragment of a v_mfma_f32_16x16x4_f32 step laid
// out contiguously, so the kernels load it with one coalesced 256-byte access
// (layouts in pack_layout.h).  Plain host code: no HIP call.

#include <cstddef>

#include "bvml_dsine.h"
#include "pack_layout.h"
#include "status.h"

using bvml::fail;
using namespace bvml::pack;

extern "C" {

int bvml_dsine_heads_pack_f32(const float* w2, const float* const* w4, const int* outs,
                              int nheads, float* w2p, float* const* w4p) {
    if (nheads < 1 || nheads > 4)
        return fail(BVML_DSINE_EPARAM, "heads_pack: nheads must be 1..4");
    if (!w2 || !w4 || !outs || !w2p || !w4p)
        return fail(BVML_DSINE_ENULL, "heads_pack: pointers must be non-NULL");
    for (int h = 0; h < nheads; ++h) {
        if (outs[h] < 1 || outs[h] > 4096)
            return fail(BVML_DSINE_EPARAM, "heads_pack: outs must be 1..4096");
        if (!w4[h] || !w4p[h]) return fail(BVML_DSINE_ENULL, "heads_pack: pointers must be non-NULL");
    }
    for (int h = 0; h < nheads; ++h) {
        for (int j = 0; j < 16; ++j)
            for (int mb = 0; mb < 4; ++mb)
                for (int l = 0; l < 64; ++l)
                    w2p[(((size_t)h * 16 + j) * 4 + mb) * 64 + l] =
                        w2[((size_t)h * kHeadsHidden + 16 * mb + (l & 15)) * kHeadsHidden + 4 * j +
                           (l >> 4)];
        const int nob = (outs[h] + 15) / 16;
        for (int ob = 0; ob < nob; ++ob)
            for (int mb = 0; mb < 4; ++mb)
                for (int r = 0; r < 4; ++r)
                    for (int l = 0; l < 64; ++l) {
                        const int o = 16 * ob + (l & 15), k = 16 * mb + 4 * (l >> 4) + r;
                        w4p[h][(((size_t)ob * 4 + mb) * 4 + r) * 64 + l] =
                            o < outs[h] ? w4[h][(size_t)o * kHeadsHidden + k] : 0.0f;
                    }
    }
    return BVML_DSINE_OK;
}

long long bvml_dsine_heads_packed_size(int out) {
    if (out < 1 || out > 4096) return -1;
    return heads_w4_floats(out);
}

long long bvml_dsine_conv_packed_size(int cout, int cin, int k) {
    if (cout < 1 || cin < 1 || (k != 3 && k != 5)) return -1;
    const long long chunks = (cin + kConvChunk - 1) / kConvChunk;
    return chunks * k * k * conv_mblocks(cout) * 64LL;
}

int bvml_dsine_conv_pack_f32(const float* w, int cout, int cin, int k, int interleave,
                             float* wp) {
    if (!w || !wp) return fail(BVML_DSINE_ENULL, "conv_pack: w and wp must be non-NULL");
    if (cout < 1 || cin < 1) return fail(BVML_DSINE_ESHAPE, "conv_pack: bad shape");
    if (k != 3 && k != 5) return fail(BVML_DSINE_EK, "conv_pack: k must be 3 or 5");
    if (interleave && cout % 32 != 0)
        return fail(BVML_DSINE_EPARAM, "conv_pack: interleaved weights need cout % 32 == 0");
    const int mblocks = conv_mblocks(cout), taps = k * k, chunks = (cin + kConvChunk - 1) / kConvChunk;
    for (int ch = 0; ch < chunks; ++ch)
        for (int t = 0; t < taps; ++t)
            for (int mb = 0; mb < mblocks; ++mb)
                for (int l = 0; l < 64; ++l) {
                    const int c = ch * kConvChunk + (l >> 4);
                    int o = 16 * mb + (l & 15);
                    if (interleave) {
                        // block 2i: channels 16i.. of the first half (z), 2i + 1:
                        // channels 16i.. of the second half (r)
                        const int half = cout / 2;
                        o = (mb & 1 ? half : 0) + 16 * (mb >> 1) + (l & 15);
                        if (16 * (mb >> 1) >= half) o = cout;  // padding block
                    }
                    const size_t dst = (((size_t)ch * taps + t) * mblocks + mb) * 64 + l;
                    wp[dst] = (o < cout && c < cin) ? w[((size_t)o * cin + c) * taps + t] : 0.0f;
                }
    return BVML_DSINE_OK;
}

}  // extern "C"
