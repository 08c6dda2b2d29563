// osh_conv_pair.h -- launch arguments of the fused 3x3 pair (osh_conv_pair.hip).
#pragma once

#include "osh_common.h"

namespace osh {

struct PairArgs {
    int h, w, c0;  // map and input channels (a multiple of 16)
    int tiles_w;
    const float *x;   // [c0][h][w]
    const float *wa;  // first conv, packed (conv16_pack, im2col order when it has 16 outputs)
    const float *ba;
    const float *wb;  // second conv, packed (im2col order when it has 16 outputs)
    const float *bb;
    const float *res;  // [c2][h][w] added after the activation, or null
    float *ya;         // [c1][h][w] intermediate, or null
    float *y;          // [c2][h][w]
};

// Launches tile `tile` (0 .. conv_pair_tile_count()-1) for c1 = 16 cb1 and
// c2 = 16 cb2 channels (cb 1, 2 or 4); SiLU on both convs.
osh_status conv_pair_launch(const PairArgs &a, int cb1, int cb2, hipStream_t st, int tile);
int conv_pair_tile_count();

// A bottleneck with an 8-channel intermediate: 16 -> 8 (im2col order) ->
// 16 (the first-layer chain), 3x3 stride 1 pad 1 on one map, SiLU; wa packed
// by conv16_pack in the im2col order, wb raw OIHW [16][8][3][3].
osh_status conv_pair8_launch(const PairArgs &a, hipStream_t st, int tile);

// A network's first conv (3x3 over c0 <= 4 planes, 16 outputs) and the 3x3
// pad-1 conv that reads its output (16 -> 32 or 64 channels).
struct FirstPairArgs {
    int h, w, c0;  // first conv's input map and planes (1 .. 4)
    int pt, pl;    // its top and left pads
    int ah, aw;    // its output map, the second conv's input
    int bh, bw;    // the second conv's output map
    int tiles_w;
    const float *x;   // [c0][h][w]
    const float *wa;  // [16][c0][3][3] (the first-layer kernel's packing: raw)
    const float *ba;
    const float *wb;  // second conv, conv16_pack in the NCHWc order
    const float *bb;
    const float *res;  // [m][bh][bw] added after the activation, or null
    float *ya;         // [16][ah][aw] intermediate, or null
    float *y;          // [m][bh][bw]
};

// Launches tile `tile` (0 .. first_pair_tile_count()-1): first conv stride
// sa, second conv stride sb (1 or 2 each), 16 cb2 outputs (cb2 2 or 4); SiLU.
osh_status first_pair_launch(const FirstPairArgs &a, int sa, int sb, int cb2, hipStream_t st, int tile);
int first_pair_tile_count();

}  // namespace osh
