// osh_conv_grp.hip -- grouped launches of the LDS-patch 3x3 tiles (conv16s_group_kernel): one launch for several independent convolutions.
//
// Tile instantiations live in translation units of their own so that the
// library's sources compile in parallel; the kernels are in the headers.
#include "osh_conv16s.h"

namespace osh {

// Tiles kC16sCount .. 2 kC16sCount - 1 are the same tiles, one workgroup per
// CU; 2 kC16sCount and up the streamed one-block tiles.
osh_status conv16s_group_launch(ConvGroup g, int act, hipStream_t st, int tile, int s) {
    if (tile >= 2 * kC16sCount) {
        switch (tile - 2 * kC16sCount) {
        case 0: return conv16_group_launch_t<1, 1, 1>(g, act, st);
        case 1: return conv16_group_launch_t<1, 1, 4>(g, act, st);
        case 2: return conv16_group_launch_t<1, 2, 1>(g, act, st);
        default: return conv16_group_launch_t<2, 1, 1>(g, act, st);
        }
    }
    const bool ex = tile >= kC16sCount;
    if (ex) tile -= kC16sCount;
#define OSH_GROUP_TILE(TM, BV, TWL)                                                         \
    return s == 1 ? conv16s_group_launch_t<TM, BV, TWL, 1, 3, 1, false>(g, act, st, ex) \
                  : conv16s_group_launch_t<TM, BV, TWL, 2, 3, 1, false>(g, act, st, ex)
    switch (tile) {
    case 0: OSH_GROUP_TILE(1, 1, 16);
    case 1: OSH_GROUP_TILE(1, 2, 16);
    case 2: OSH_GROUP_TILE(1, 4, 16);
    case 3: OSH_GROUP_TILE(2, 2, 16);
    case 4: OSH_GROUP_TILE(1, 1, 8);
    case 5: OSH_GROUP_TILE(1, 2, 8);
    case 6: OSH_GROUP_TILE(2, 2, 8);
    case 7: OSH_GROUP_TILE(1, 2, 4);
    case 8: OSH_GROUP_TILE(1, 4, 4);
    case 9: OSH_GROUP_TILE(1, 4, 8);
    default: OSH_GROUP_TILE(2, 4, 8);
    }
#undef OSH_GROUP_TILE
}

}  // namespace osh
