// osh_conv3x3_ws.h -- weight-stationary 3x3 conv (pad 1, dilation 1, group 1,
// stride 1 or 2) for C = 16, 32, 64 or 128 input channels, gfx950 FP32 MFMA.
//
// A workgroup owns one tile of 32 output channels and KS = C/16 waves.  Wave q
// keeps the MFMA A-operands of its K slice -- 32 oc x input channels
// [16q, 16q+16) x 9 taps = 72 v_mfma_f32_32x32x2f32 steps -- in 72 VGPRs for the
// whole kernel, so weights are read from memory once per workgroup.  The
// workgroup then walks output tiles of 32 pixels (TR rows x TC columns, TC
// dividing the output width) with a grid stride:
//   - each wave stages the halo patch of its 16 channels in its own LDS region
//     ([2][PR][2][PITCH][4]: channel ch sits at [(ch >> 2) & 1][..][ch >> 3][..][ch & 3],
//     columns de-interleaved even/odd for stride 2) -- no workgroup barrier;
//     the next tile's patch is fetched into registers while the current one is
//     multiplied;
//   - 72 MFMAs accumulate the wave's partial sums (B = patch, two ds_read_b128
//     per tap);
//   - the KS partial tiles meet in LDS; the sum bias + p0 + p1 + ... + p(KS-1)
//     (fixed order) goes through the activation and out to NCHW.
// Reference semantics: NchwcConv / Im2Col / PackedConv (src/OnnxSharp/Kernels/
// NchwcConv.cs:533-605, ConvKernels.cs:554-563); the reduction order differs
// from their single FMA chain by rounding only.
#pragma once

#include <cstdlib>

#include "osh_common.h"

namespace osh {

constexpr int WS_CPW = 16;  // input channels per wave
constexpr int WS_STEPS = WS_CPW / 2 * 9;  // MFMA k-steps per wave (72)

inline int conv3x3_ws_tc(const osh_conv_params *p) {
    if (p->ow % 8 == 0) return 8;
    if (p->ow % 4 == 0) return 4;
    return 0;
}

inline bool conv3x3_ws_eligible(const osh_conv_params *p) {
    const int ks = p->c / WS_CPW;
    return p->group == 1 && p->kh == 3 && p->kw == 3 && p->dh == 1 && p->dw == 1 && p->pt == 1 && p->pl == 1 &&
           p->sh == p->sw && (p->sh == 1 || p->sh == 2) && p->c % WS_CPW == 0 &&
           (ks == 1 || ks == 2 || ks == 4 || ks == 8) && conv3x3_ws_tc(p) != 0 &&
           (long long)WS_CPW * p->h * p->w < (1LL << 31);
}

inline size_t conv3x3_ws_packed_bytes(const osh_conv_params *p) {
    size_t mt = (p->m + 31) / 32, ks = p->c / WS_CPW;
    return mt * ks * WS_STEPS * 64 * sizeof(float);
}

// packed[mt][q][f (18)][lane (64)][4]: step s = 4f + i = tap*8 + j holds, for
// lane (l32, lhi), w[mt*32 + l32][16q + 8*lhi + j][tap]  (0 beyond M).
__global__ void conv3x3_ws_pack_kernel(int M, int C, const float *__restrict__ w, float *__restrict__ out,
                                       long long total) {
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    int i4 = (int)(idx % 4);
    long long t = idx / 4;
    int lane = (int)(t % 64);
    t /= 64;
    int f = (int)(t % (WS_STEPS / 4));
    t /= WS_STEPS / 4;
    int ks = C / WS_CPW;
    int q = (int)(t % ks);
    int mt = (int)(t / ks);
    int step = 4 * f + i4;
    int tap = step / 8, j = step % 8;
    int oc = mt * 32 + (lane & 31);
    int ch = q * WS_CPW + 8 * (lane >> 5) + j;
    out[idx] = oc < M ? w[((long long)oc * C + ch) * 9 + tap] : 0.f;
}

inline osh_status conv3x3_ws_pack(const osh_conv_params *p, const float *w, void *packed, hipStream_t st) {
    long long total = (long long)(conv3x3_ws_packed_bytes(p) / sizeof(float));
    hipLaunchKernelGGL(conv3x3_ws_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, p->m, p->c, w,
                       (float *)packed, total);
    OSH_LAUNCH_CHECK("conv3x3_ws_pack_kernel");
    return OSH_OK;
}

template <int S, int TC, int KS, int ACT>
__global__ __launch_bounds__(KS * 64) void conv3x3_ws_kernel(osh_conv_params p, const float *__restrict__ x,
                                                            const float *__restrict__ wpk,
                                                            const float *__restrict__ bias,
                                                            float *__restrict__ y) {
    constexpr int TR = 32 / TC;
    constexpr int PR = (TR - 1) * S + 3;  // patch rows
    constexpr int PC = (TC - 1) * S + 3;  // patch cols
    constexpr int HALFC = (PC + 1) / 2;   // even columns first when S == 2
    constexpr int PITCH = S == 1 ? PC : 2 * HALFC;
    constexpr int PATCH = 2 * PR * 2 * PITCH * 4;  // floats per wave
    constexpr int NPOS = PR * PC;                   // patch positions
    constexpr int PPL = (NPOS + 63) / 64;            // positions per lane
    constexpr int P_PER = PPL * WS_CPW;              // prefetch registers per lane

    __shared__ __align__(16) float Pw[KS][PATCH];
    __shared__ __align__(16) float Red[KS > 1 ? 2 : 1][KS > 1 ? KS : 1][16][64];

    const int lane = threadIdx.x & 63;
    const int q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave index, kept scalar
    const int l32 = lane & 31, lhi = lane >> 5;
    const int mt = blockIdx.y;
    const int H = p.h, W = p.w;
    const int tiles_x = p.ow / TC, tiles_y = (p.oh + TR - 1) / TR;
    const int tiles_img = tiles_x * tiles_y;
    const int total = p.n * tiles_img;
    const long long plane = (long long)H * W;

    // A operands of this wave's K slice, resident for the whole kernel
    float a[WS_STEPS];
    {
        const float4 *wsrc = reinterpret_cast<const float4 *>(wpk) + (long long)(mt * KS + q) * (WS_STEPS / 4) * 64;
#pragma unroll
        for (int f = 0; f < WS_STEPS / 4; f++) {
            float4 v = wsrc[f * 64 + lane];
            a[4 * f + 0] = v.x;
            a[4 * f + 1] = v.y;
            a[4 * f + 2] = v.z;
            a[4 * f + 3] = v.w;
        }
    }

    // bias of the accumulator rows this wave finishes (rows r = q, q + KS, ...)
    float bq[16 / KS];
#pragma unroll
    for (int k = 0; k < 16 / KS; k++) {
        const int r = q + k * KS;
        const int oc = mt * 32 + 8 * (r >> 2) + 4 * lhi + (r & 3);
        bq[k] = bias && oc < p.m ? bias[oc] : 0.f;
    }

    // Lane-owned patch positions: the lane loads position k*64 + lane for all 16
    // channels of its wave, so the per-tile address work is a few adds per
    // position and the LDS writes use immediate channel offsets.
    float *__restrict__ pw = &Pw[q][0];
    float rp[P_PER];
    int pos_pr[PPL], pos_pc[PPL], pos_lds[PPL];
#pragma unroll
    for (int k = 0; k < PPL; k++) {
        const int pos = k * 64 + lane;
        const int pc = pos < NPOS ? pos % PC : 0, pr = pos < NPOS ? pos / PC : 0;
        const int sc = S == 1 ? pc : ((pc & 1) ? HALFC + (pc >> 1) : (pc >> 1));
        pos_pr[k] = pos < NPOS ? pr : -(1 << 20);  // positions past the patch are never in the image
        pos_pc[k] = pc;
        pos_lds[k] = pr * 2 * PITCH * 4 + sc * 4;
    }
    auto chan_lds = [](int ch) { return ((ch >> 2) & 1) * PR * 2 * PITCH * 4 + (ch >> 3) * PITCH * 4 + (ch & 3); };

    // The gather loads from clamped, in-bounds addresses straight into the
    // prefetch registers; the in-image bit of each position zeroes the halo when
    // the patch is written to LDS, so all loads of a tile are in flight together.
    unsigned okmask = 0;
    auto load_tile = [&](int t) {
        const int n = t / tiles_img, rem = t - n * tiles_img;
        const int ty = rem / tiles_x, tx = rem - ty * tiles_x;
        const int iy0 = ty * TR * S - 1, ix0 = tx * TC * S - 1;
        const float *__restrict__ xb = x + ((long long)n * p.c + q * WS_CPW) * plane;
        okmask = 0;
#pragma unroll
        for (int k = 0; k < PPL; k++) {
            const int iy = iy0 + pos_pr[k], ix = ix0 + pos_pc[k];
            const bool ok = (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
            okmask |= (unsigned)ok << k;
            const int iyc = min(max(iy, 0), H - 1), ixc = min(max(ix, 0), W - 1);
            const unsigned off = (unsigned)(iyc * W + ixc);
#pragma unroll
            for (int ch = 0; ch < WS_CPW; ch++) rp[k * WS_CPW + ch] = (xb + ch * plane)[off];
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int k = 0; k < PPL; k++) {
            const bool ok = (okmask >> k) & 1;
            if (k * 64 + lane < NPOS) {
#pragma unroll
                for (int ch = 0; ch < WS_CPW; ch++) pw[pos_lds[k] + chan_lds(ch)] = ok ? rp[k * WS_CPW + ch] : 0.f;
            }
        }
    };

    const int pr0 = (l32 / TC) * S;  // patch row of tap ky = 0 for this lane's pixel
    const int pcl = l32 % TC;        // pixel column inside the tile
    auto scol = [&](int kx) { return S == 1 ? pcl + kx : (kx == 1 ? HALFC + pcl : pcl + (kx >> 1)); };
    auto bptr = [&](int jh, int ky, int kx) {
        return reinterpret_cast<const float4 *>(&pw[((jh * PR + pr0 + ky) * 2 + lhi) * PITCH * 4 + scol(kx) * 4]);
    };

    int t = blockIdx.x;
    if (t < total) {
        load_tile(t);
        store_tile();
    }
    int rb = 0;
    for (; t < total; t += gridDim.x) {
        const int tn = t + gridDim.x;
        if (tn < total) load_tile(tn);

        f32x16 acc = {};
        float4 b0 = *bptr(0, 0, 0), b1 = *bptr(1, 0, 0);
#pragma unroll
        for (int tap = 0; tap < 9; tap++) {
            float4 n0, n1;
            if (tap < 8) {
                n0 = *bptr(0, (tap + 1) / 3, (tap + 1) % 3);
                n1 = *bptr(1, (tap + 1) / 3, (tap + 1) % 3);
            }
            const float *at = &a[tap * 8];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(at[0], b0.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(at[1], b0.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(at[2], b0.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(at[3], b0.w, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(at[4], b1.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(at[5], b1.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(at[6], b1.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(at[7], b1.w, acc, 0, 0, 0);
            if (tap < 8) {
                b0 = n0;
                b1 = n1;
            }
        }

        // output pixel of this lane
        const int n = t / tiles_img, rem = t - n * tiles_img;
        const int ty = rem / tiles_x, tx = rem - ty * tiles_x;
        const int oy = ty * TR + l32 / TC, ox = tx * TC + pcl;
        float *__restrict__ yp = y + ((long long)n * p.m) * p.oh * p.ow + (long long)oy * p.ow + ox;
        const long long ostride = (long long)p.oh * p.ow;
        if constexpr (KS == 1) {
            if (oy < p.oh) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int oc = mt * 32 + 8 * (r >> 2) + 4 * lhi + (r & 3);
                    if (oc < p.m) yp[oc * ostride] = activate<ACT>(bq[r] + acc[r]);
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; r++) Red[rb][q][r][lane] = acc[r];
            __syncthreads();
            if (oy < p.oh) {
#pragma unroll
                for (int k = 0; k < 16 / KS; k++) {
                    const int r = q + k * KS;
                    const int oc = mt * 32 + 8 * (r >> 2) + 4 * lhi + (r & 3);
                    float v = bq[k];
#pragma unroll
                    for (int qq = 0; qq < KS; qq++) v += Red[rb][qq][r][lane];
                    if (oc < p.m) yp[oc * ostride] = activate<ACT>(v);
                }
            }
            rb ^= 1;
        }
        if (tn < total) store_tile();
    }
}

// Workgroups per CU of the persistent grid (ONNXSHARP_HIP_WS_WGS_PER_CU, default 2;
// the knob follows the reference's ONNXSHARP_* environment switches).
inline int ws_wgs_per_cu() {
    static int v = 0;
    if (!v) {
        const char *e = getenv("ONNXSHARP_HIP_WS_WGS_PER_CU");
        v = e ? atoi(e) : 2;
        if (v < 1 || v > 8) v = 2;
    }
    return v;
}

inline osh_status conv3x3_ws_launch(const osh_conv_params *p, const float *x, const float *wpk, const float *bias,
                                    int act, float *y, hipStream_t st) {
    const int tc = conv3x3_ws_tc(p), ks = p->c / WS_CPW;
    const int mtiles = (p->m + 31) / 32;
    const long long tiles = (long long)p->n * (p->ow / tc) * ((p->oh + 32 / tc - 1) / (32 / tc));
    long long per = ((long long)device_cus() * ws_wgs_per_cu() + mtiles - 1) / mtiles;
    if (per > tiles) per = tiles;
    if (per < 1) per = 1;
    if (mtiles > 65535) return fail(OSH_E_UNSUPPORTED, "Conv: too many output channels");
    dim3 grid((unsigned)per, mtiles), block(ks * 64);
#define OSH_WS_LAUNCH(S_, TC_, KS_)                                                                         \
    OSH_DISPATCH_ACT(act, ACT, hipLaunchKernelGGL((conv3x3_ws_kernel<S_, TC_, KS_, ACT>), grid, block, 0, st, \
                                                  *p, x, wpk, bias, y))
#define OSH_WS_KS(S_, TC_)                    \
    switch (ks) {                             \
    case 1: OSH_WS_LAUNCH(S_, TC_, 1); break; \
    case 2: OSH_WS_LAUNCH(S_, TC_, 2); break; \
    case 4: OSH_WS_LAUNCH(S_, TC_, 4); break; \
    default: OSH_WS_LAUNCH(S_, TC_, 8); break; \
    }
    if (p->sh == 1) {
        if (tc == 8) { OSH_WS_KS(1, 8) } else { OSH_WS_KS(1, 4) }
    } else {
        if (tc == 8) { OSH_WS_KS(2, 8) } else { OSH_WS_KS(2, 4) }
    }
#undef OSH_WS_KS
#undef OSH_WS_LAUNCH
    OSH_LAUNCH_CHECK("conv3x3_ws_kernel");
    return OSH_OK;
}

}  // namespace osh
