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

}  // namespace osh
