// osh_conv_i2c.hip -- launches of the 3x3 tiles in the im2col order: the LDS-patch tiles (conv16s_kernel with
// I2C) and the streamed one-block tiles (conv16_kernel with I2C).
//
// Tile instantiations live in translation units of their own so that the
// library's sources compile in parallel; the kernels are in the headers.
#include "osh_conv16s.h"

namespace osh {

osh_status conv16si_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                           const float *res, int act, float *y, hipStream_t st, int v) {
    switch (v) {
    case 0: return conv16s_launch_s<1, 1, 16, false, true>(p, x, w, bias, res, act, y, st);
    case 1: return conv16s_launch_s<1, 2, 16, false, true>(p, x, w, bias, res, act, y, st);
    case 2: return conv16s_launch_s<1, 4, 16, false, true>(p, x, w, bias, res, act, y, st);
    case 3: return conv16s_launch_s<2, 2, 16, false, true>(p, x, w, bias, res, act, y, st);
    case 4: return conv16s_launch_s<1, 1, 8, false, true>(p, x, w, bias, res, act, y, st);
    case 5: return conv16s_launch_s<1, 2, 8, false, true>(p, x, w, bias, res, act, y, st);
    case 6: return conv16s_launch_s<2, 2, 8, false, true>(p, x, w, bias, res, act, y, st);
    case 7: return conv16s_launch_s<1, 2, 4, false, true>(p, x, w, bias, res, act, y, st);
    case 8: return conv16s_launch_s<1, 4, 4, false, true>(p, x, w, bias, res, act, y, st);
    case 9: return conv16s_launch_s<1, 4, 8, false, true>(p, x, w, bias, res, act, y, st);
    default: return conv16s_launch_s<2, 4, 8, false, true>(p, x, w, bias, res, act, y, st);
    }
}

osh_status conv16wi_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                           const float *res, int act, float *y, hipStream_t st, int v) {
    switch (v) {
    case 0: return conv16_launch_t<1, 1, 1, true>(p, x, w, bias, res, act, y, st);
    case 1: return conv16_launch_t<1, 1, 4, true>(p, x, w, bias, res, act, y, st);
    case 2: return conv16_launch_t<1, 2, 1, true>(p, x, w, bias, res, act, y, st);
    default: return conv16_launch_t<2, 1, 1, true>(p, x, w, bias, res, act, y, st);
    }
}

}  // namespace osh
