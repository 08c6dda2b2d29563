// osh_conv_pw.hip -- launches of the pointwise LDS tiles (conv16s_kernel with KS = 1), alone and grouped.
//
// Tile instantiations live in translation units of their own so that the
// library's sources compile in parallel; the kernels are in the headers.
#include "osh_conv16s.h"

namespace osh {

// A 1x1 stride-1 conv reads and writes each pixel's own channels only, so
// any H' x W' with H' W' = H W gives the same outputs from the same chains.
// A map whose width is not a multiple of the tile's TWL columns (40 or 20
// wide for 16-column tiles: the last tile of each row would run 8 or 12
// columns past the map, MFMA work on nothing) is laid out TWL pixels wide
// instead, so every tile is full.
template <int TWL>
inline osh_conv_params pw_layout(const osh_conv_params &p) {
    osh_conv_params q = p;
    const long long hw = (long long)p.h * p.w;
    if (p.w % TWL != 0 && hw % TWL == 0 && hw / TWL <= 0x7fffffffLL) {
        q.w = q.ow = TWL;
        q.h = q.oh = (int)(hw / TWL);
    }
    return q;
}

template <int TM, int BV, int TWL, int CB = 4>
inline osh_status pw16_launch_v(const osh_conv_params *p0, const float *x, const float *w, const float *bias,
                                const float *res, int act, float *y, hipStream_t st) {
    const osh_conv_params q = pw_layout<TWL>(*p0);
    const osh_conv_params *p = &q;
    const bool vec = p->w % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    if (vec) return conv16s_launch_t<TM, BV, TWL, 1, 1, CB, true>(p, x, w, bias, res, act, y, st);
    return conv16s_launch_t<TM, BV, TWL, 1, 1, CB, false>(p, x, w, bias, res, act, y, st);
}

osh_status pw16_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                       const float *res, int act, float *y, hipStream_t st, int v) {
    switch (v) {
    case 0: return pw16_launch_v<1, 1, 16>(p, x, w, bias, res, act, y, st);
    case 1: return pw16_launch_v<1, 2, 16>(p, x, w, bias, res, act, y, st);
    case 2: return pw16_launch_v<1, 4, 16>(p, x, w, bias, res, act, y, st);
    case 3: return pw16_launch_v<2, 2, 16>(p, x, w, bias, res, act, y, st);
    case 4: return pw16_launch_v<2, 4, 16>(p, x, w, bias, res, act, y, st);
    case 5: return pw16_launch_v<1, 2, 4>(p, x, w, bias, res, act, y, st);
    case 6: return pw16_launch_v<1, 4, 4>(p, x, w, bias, res, act, y, st);
    case 7: return pw16_launch_v<2, 4, 4>(p, x, w, bias, res, act, y, st);
    case 8: return pw16_launch_v<1, 1, 16, 8>(p, x, w, bias, res, act, y, st);
    case 9: return pw16_launch_v<1, 1, 16, 16>(p, x, w, bias, res, act, y, st);
    case 10: return pw16_launch_v<1, 2, 16, 8>(p, x, w, bias, res, act, y, st);
    default: return pw16_launch_v<1, 2, 16, 16>(p, x, w, bias, res, act, y, st);
    }
}

template <int TM, int BV, int TWL, int CB = 4>
static osh_status pw16_group_v(ConvGroup g, int act, hipStream_t st, bool vec) {
    for (int i = 0; i < g.count; i++) g.p[i] = pw_layout<TWL>(g.p[i]);
    return vec ? conv16s_group_launch_t<TM, BV, TWL, 1, 1, CB, true>(g, act, st)
               : conv16s_group_launch_t<TM, BV, TWL, 1, 1, CB, false>(g, act, st);
}

osh_status pw16_group_launch(ConvGroup g, int act, hipStream_t st, int tile, bool vec) {
    switch (tile) {
    case 0: return pw16_group_v<1, 1, 16>(g, act, st, vec);
    case 1: return pw16_group_v<1, 2, 16>(g, act, st, vec);
    case 2: return pw16_group_v<1, 4, 16>(g, act, st, vec);
    case 3: return pw16_group_v<2, 2, 16>(g, act, st, vec);
    case 4: return pw16_group_v<2, 4, 16>(g, act, st, vec);
    case 5: return pw16_group_v<1, 2, 4>(g, act, st, vec);
    case 6: return pw16_group_v<1, 4, 4>(g, act, st, vec);
    case 7: return pw16_group_v<2, 4, 4>(g, act, st, vec);
    case 8: return pw16_group_v<1, 1, 16, 8>(g, act, st, vec);
    case 9: return pw16_group_v<1, 1, 16, 16>(g, act, st, vec);
    case 10: return pw16_group_v<1, 2, 16, 8>(g, act, st, vec);
    default: return pw16_group_v<1, 2, 16, 16>(g, act, st, vec);
    }
}

}  // namespace osh
