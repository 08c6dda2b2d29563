// osh_conv_str.hip -- launches of the streamed 3x3 tiles (conv16_kernel, conv16l_kernel; four or one wave per workgroup).
//
// Tile instantiations live in translation units of their own so that the
// library's sources compile in parallel; the kernels are in the headers.
#include "osh_conv16.h"

namespace osh {

osh_status conv16w_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                          const float *res, int act, float *y, hipStream_t st, int v) {
    switch (v) {
    case 0: return conv16_launch_t<1, 1, 1>(p, x, w, bias, res, act, y, st);
    case 1: return conv16_launch_t<1, 2, 1>(p, x, w, bias, res, act, y, st);
    case 2: return conv16_launch_t<2, 1, 1>(p, x, w, bias, res, act, y, st);
    default: return conv16_launch_t<2, 2, 1>(p, x, w, bias, res, act, y, st);
    }
}

osh_status conv16_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                         const float *res, int act, float *y, hipStream_t st, int forced) {
    int best = -1;
    if (forced >= 0 && forced < kC16Count) {
        best = forced;
    } else {
        double bc = 0;
        const int cus = device_cus();
        for (int i = 0; i < kC16Count; i++) {
            if (!conv16_fits(p, kC16[i])) continue;
            const double c = conv16_cost(p, kC16[i], cus);
            if (best < 0 || c < bc) best = i, bc = c;
        }
    }
    if (!conv16_fits(p, kC16[best])) best -= 6;  // forced LDS tile too large: same tile from L2
    switch (best) {
    case 0: return conv16_launch_t<1, 1>(p, x, w, bias, res, act, y, st);
    case 1: return conv16_launch_t<2, 1>(p, x, w, bias, res, act, y, st);
    case 2: return conv16_launch_t<4, 1>(p, x, w, bias, res, act, y, st);
    case 3: return conv16_launch_t<1, 2>(p, x, w, bias, res, act, y, st);
    case 4: return conv16_launch_t<2, 2>(p, x, w, bias, res, act, y, st);
    case 5: return conv16_launch_t<4, 2>(p, x, w, bias, res, act, y, st);
    case 6: return conv16l_launch_t<1, 1>(p, x, w, bias, res, act, y, st);
    case 7: return conv16l_launch_t<2, 1>(p, x, w, bias, res, act, y, st);
    case 8: return conv16l_launch_t<4, 1>(p, x, w, bias, res, act, y, st);
    case 9: return conv16l_launch_t<1, 2>(p, x, w, bias, res, act, y, st);
    case 10: return conv16l_launch_t<2, 2>(p, x, w, bias, res, act, y, st);
    default: return conv16l_launch_t<4, 2>(p, x, w, bias, res, act, y, st);
    }
}

}  // namespace osh
