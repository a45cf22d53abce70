// The packed weight layouts of the refiner's matrix-core kernels (conv.hip,
// heads.hip), shared by the kernels and the host packing (pack.cpp).
#pragma once

namespace bvml::pack {

// conv.hip: [chunk of 4 input channels][tap][16-channel M-block][64 lanes],
// lane l holding output channel 16 mb + l % 16, input channel 4 chunk + l / 16.
constexpr int kConvChunk = 4;

// 16-channel M-blocks of packed convolution weights: a multiple of 4 (each
// wave takes 4); launches with two waves along the channels need 8.
inline int conv_mblocks(int cout) { return (cout + 63) / 64 * 4; }

// heads.hip: the middle layer [head][j 16][mb 4][64 lanes], lane l holding
// W2[16 mb + l % 16][4 j + l / 16]; the last layer [ob][mb 4][r 4][64 lanes],
// lane l holding W4[16 ob + l % 16][16 mb + 4 (l / 16) + r].
constexpr int kHeadsHidden = 64;
constexpr int kHeadsW2Floats = 16 * 4 * 64;
inline long long heads_w4_floats(int out) { return (long long)((out + 15) / 16) * 4 * 4 * 64; }

}  // namespace bvml::pack
