// osh_conv3x3_wi.h -- wave-independent 3x3 conv (stride 1, pad 1, dilation 1,
// group 1) for C = 16, 32 or 64 input channels, gfx950 FP32 MFMA.
//
// A workgroup owns 32 output channels; their weights (32 oc x C x 9 taps, at
// most 72 KiB) are copied into LDS once, in MFMA-operand order.  Each of the
// four waves then works alone -- no barrier after the weight copy -- on output
// tiles of 4 rows x 8 columns (32 pixels), taking tiles with a grid stride:
//   - the wave gathers the 6 x 10 halo patch of all C channels (one patch
//     position per lane, all channels of that position; buffer loads with the
//     channel offset in an SGPR) into registers while it multiplies the
//     previous tile, then writes it to its own LDS region with ds_write_b128;
//   - v_mfma_f32_32x32x2f32 over the full K = 9 taps x C channels, A = weights
//     (32 oc x channel pair), B = patch (channel pair x 32 pixels), one
//     ds_read_b128 per operand per four k-steps;
//   - bias, activation and the NCHW store straight from the accumulators.
// Accumulation order per output: bias, then 16-channel block -> tap (ky, kx)
// -> channel pairs (2i, 2i + 1) in ascending order.  The MFMA adds the pair's
// two products one after the other with one rounding each, so this is the
// reference's NCHWc chain (src/OnnxSharp/Kernels/NchwcConv.cs:533-605: bias,
// then icb -> ky -> kx -> lane16) bit for bit.  A lane-half's float4 holds
// the even (lower half) or odd (upper half) channels of a group of 8.
#pragma once

#include <type_traits>

#include "osh_common.h"

namespace osh {

inline bool conv3x3_wi_eligible(const osh_conv_params *p) {
    return p->group == 1 && p->kh == 3 && p->kw == 3 && p->dh == 1 && p->dw == 1 && p->pt == 1 && p->pl == 1 &&
           p->sh == 1 && p->sw == 1 && (p->c == 16 || p->c == 32 || p->c == 64) && p->ow % 8 == 0 &&
           (long long)p->c * p->h * p->w * 4 < (1LL << 31) &&  // buffer ranges fit 31 bits
           (long long)p->m * p->oh * p->ow * 4 < (1LL << 31);
}

inline size_t conv3x3_wi_packed_bytes(const osh_conv_params *p) {
    return (size_t)((p->m + 31) / 32) * 9 * p->c * 32 * sizeof(float);
}

// packed[mt][tap][g (C/8)][lhi][oc 32][j 4] = w[mt*32 + oc][8g + 2j + lhi][tap]  (0 beyond M)
__global__ void conv3x3_wi_pack_kernel(int M, int C, const float *__restrict__ w, float *__restrict__ out,
                                       long long total) {
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    int j = (int)(idx % 4);
    long long t = idx / 4;
    int oc = (int)(t % 32);
    t /= 32;
    int lhi = (int)(t % 2);
    t /= 2;
    int g = (int)(t % (C / 8));
    t /= C / 8;
    int tap = (int)(t % 9);
    int mt = (int)(t / 9);
    int m = mt * 32 + oc, ch = 8 * g + 2 * j + lhi;
    out[idx] = m < M ? w[((long long)m * C + ch) * 9 + tap] : 0.f;
}

inline osh_status conv3x3_wi_pack(const osh_conv_params *p, const float *w, void *packed, hipStream_t st) {
    long long total = (long long)(conv3x3_wi_packed_bytes(p) / sizeof(float));
    hipLaunchKernelGGL(conv3x3_wi_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, p->m, p->c, w,
                       (float *)packed, total);
    OSH_LAUNCH_CHECK("conv3x3_wi_pack_kernel");
    return OSH_OK;
}

constexpr unsigned WI_BUF_WORD3 = 0x00020000u;  // raw 32-bit buffer (gfx9 family)

template <int C, int ACT>
__global__ __launch_bounds__(256) void conv3x3_wi_kernel(osh_conv_params p, const float *__restrict__ x,
                                                        const float *__restrict__ wpk,
                                                        const float *__restrict__ bias, float *__restrict__ y) {
    constexpr int TC = 8, TR = 4, PR = 6, PC = 10, NPOS = PR * PC;  // 60 patch positions
    // LDS row pitch of the patch: 12 positions, so the two pixel rows read by a
    // 16-lane group (2 x 128 B) fall on disjoint halves of the 64 banks
    constexpr int PCP = 12;
    constexpr int G = C / 8;                                       // channel groups
    constexpr int WF = 9 * C * 32;                                 // weight floats per oc tile
    constexpr int PATCH = C * PR * PCP;                            // patch floats per wave
    static_assert(NPOS <= 64, "one patch position per lane");

    __shared__ __align__(16) float Wsh[WF];
    __shared__ __align__(16) float Psh[4][PATCH];

    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31, lhi = lane >> 5;
    const int mt = blockIdx.y;
    const int H = p.h, W = p.w;
    const int tiles_x = p.ow / TC, tiles_y = (p.oh + TR - 1) / TR;
    const int tiles_img = tiles_x * tiles_y;
    const int total = p.n * tiles_img;
    const int plane = H * W;

    // this lane's patch position (lanes 60..63 own none)
    const bool has_pos = lane < NPOS;
    const int ppr = has_pos ? lane / PC : 0, ppc = has_pos ? lane % PC : 0;
    float *__restrict__ pw = Psh[wv];
    // LDS float offset of channel ch at this lane's position: [g][pr][lhi'][pc][j]
    const int pos_lds = ppr * 2 * PCP * 4 + ppc * 4;
    auto chan_lds = [](int g, int h) { return (g * PR * 2 + h) * PCP * 4; };

    // A wave may have at most 63 vector-memory instructions outstanding, so the
    // C loads of a tile are issued in batches of at most 32 (the second batch
    // half-way through the previous tile's taps).
    constexpr int LB = C < 32 ? C : 32;
    float rp[C];
    bool rp_ok = false;
    auto load_tile = [&](int t, auto half_tag) {
        constexpr int half = decltype(half_tag)::value;
        const int n = t / tiles_img, rem = t - n * tiles_img;
        const int ty = rem / tiles_x, tx = rem - ty * tiles_x;
        const int iy = ty * TR - 1 + ppr, ix = tx * TC - 1 + ppc;
        if constexpr (half == 0) rp_ok = has_pos && (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
        const int iyc = min(max(iy, 0), H - 1), ixc = min(max(ix, 0), W - 1);
        const float *xb = x + (long long)n * C * plane;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(xb), (short)0, C * plane * 4, WI_BUF_WORD3);
        const int voff = (iyc * W + ixc) * 4;
#pragma unroll
        for (int k = 0; k < LB; k++) {  // the builtin returns the raw 32 bits
            const int ch = half * LB + k;
            if (ch < C) rp[ch] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, voff, ch * plane * 4, 0));
        }
    };
    // Halo positions (outside the image) are written as zeros by a masked second
    // set of stores rather than per-register selects: LDS stores cost no VALU.
    auto store_tile = [&]() {
        if (!has_pos) return;
        if (rp_ok) {
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int h = 0; h < 2; h++) {  // slot h: channels 8g + h, +2, +4, +6
                    const int c0 = 8 * g + h;
                    *reinterpret_cast<float4 *>(&pw[chan_lds(g, h) + pos_lds]) =
                        make_float4(rp[c0], rp[c0 + 2], rp[c0 + 4], rp[c0 + 6]);
                }
        } else {
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int h = 0; h < 2; h++)
                    *reinterpret_cast<float4 *>(&pw[chan_lds(g, h) + pos_lds]) = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };

    // B operand address of this lane's pixel: [g][pr0 + ky][lhi][pc0 + kx][4]
    const int pr0 = l32 / TC, pc0 = l32 % TC;
    auto bptr = [&](int g, int ky, int kx) {
        return reinterpret_cast<const float4 *>(&pw[((g * PR + pr0 + ky) * 2 + lhi) * PCP * 4 + (pc0 + kx) * 4]);
    };
    auto aptr = [&](int tap, int g) {
        return reinterpret_cast<const float4 *>(&Wsh[((tap * G + g) * 2 + lhi) * 32 * 4 + l32 * 4]);
    };

    const int step = gridDim.x * 4;
    int t = blockIdx.x * 4 + wv;
    // the first tile's gather is issued before the weight copy so both latencies overlap
    if (t < total) load_tile(t, std::integral_constant<int, 0>{});
    // weights of this oc tile -> LDS (once), six loads per thread in flight
    {
        const float4 *src = reinterpret_cast<const float4 *>(wpk + (long long)mt * WF);
        float4 *dst = reinterpret_cast<float4 *>(Wsh);
#pragma unroll 6
        for (int e = threadIdx.x; e < WF / 4; e += 256) dst[e] = src[e];
    }
    // bias of this lane's 16 accumulator rows
    float bacc[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int oc = mt * 32 + 8 * (r >> 2) + 4 * lhi + (r & 3);
        bacc[r] = bias && oc < p.m ? bias[oc] : 0.f;
    }

    if constexpr (C > LB) {
        if (t < total) load_tile(t, std::integral_constant<int, 1>{});
    }
    __syncthreads();
    if (t < total) store_tile();
    for (; t < total; t += step) {
        const int tn = t + step;
        if (tn < total) load_tile(tn, std::integral_constant<int, 0>{});

        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = bacc[r];
        // k order: 16-channel block -> tap -> the block's two groups of 8 -> four
        // channel pairs.  The ky loop stays rolled (kx and the groups are
        // unrolled: 24 MFMAs per iteration) so the scheduler cannot hoist all
        // operand loads of the tile at once; the operands of the next k-group
        // are read while the current four MFMAs run, across tap and block
        // boundaries.
        constexpr int ICB = C / 16;
        float4 av = *aptr(0, 0), bv = *bptr(0, 0, 0);
        auto run_blocks = [&](int icb0, int icb1) {
            for (int icb = icb0; icb < icb1; icb++) {
                const int g0 = 2 * icb;
                const int gnext = icb + 1 < ICB ? g0 + 2 : g0;  // after the last block: a harmless re-read
#pragma unroll 1
                for (int ky = 0; ky < 3; ky++) {
#pragma unroll
                    for (int kx = 0; kx < 3; kx++) {
                        const int tap = ky * 3 + kx;
#pragma unroll
                        for (int gg = 0; gg < 2; gg++) {
                            float4 an, bn;
                            if (gg == 0) {
                                an = *aptr(tap, g0 + 1);
                                bn = *bptr(g0 + 1, ky, kx);
                            } else if (kx < 2) {
                                an = *aptr(tap + 1, g0);
                                bn = *bptr(g0, ky, kx + 1);
                            } else if (ky < 2) {
                                an = *aptr(tap + 1, g0);
                                bn = *bptr(g0, ky + 1, 0);
                            } else {
                                an = *aptr(0, gnext);
                                bn = *bptr(gnext, 0, 0);
                            }
                            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, acc, 0, 0, 0);
                            av = an;
                            bv = bn;
                        }
                    }
                }
            }
        };
        if constexpr (C > LB) {
            run_blocks(0, ICB / 2);
            if (tn < total) load_tile(tn, std::integral_constant<int, 1>{});
            run_blocks(ICB / 2, ICB);
        } else {
            run_blocks(0, ICB);
        }

        // Epilogue.  Full 32-channel tiles use buffer stores with each accumulator
        // register's channel offset in an SGPR; every address is inside image n's
        // output, except lanes whose pixel row lies below the image, which get a
        // vector offset past the buffer end so the store is dropped.  A partial last
        // channel tile takes guarded plain stores.
        {
            const int n = t / tiles_img, rem = t - n * tiles_img;
            const int ty = rem / tiles_x, tx = rem - ty * tiles_x;
            const int oy = ty * TR + pr0, ox = tx * TC + pc0;
            const int ostride = p.oh * p.ow;
            if (mt * 32 + 32 <= p.m) {
                const __amdgpu_buffer_rsrc_t ys = __builtin_amdgcn_make_buffer_rsrc(
                    y + (long long)n * p.m * ostride, (short)0, p.m * ostride * 4, WI_BUF_WORD3);
                const int voff = oy < p.oh ? ((mt * 32 + 4 * lhi) * ostride + oy * p.ow + ox) * 4 : 0x7fffffff;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int dr = 8 * (r >> 2) + (r & 3);  // channel row of register r relative to 4*lhi
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(activate<ACT>(acc[r])), ys, voff,
                                                          dr * ostride * 4, 0);
                }
            } else if (oy < p.oh) {
                float *__restrict__ yp = y + ((long long)n * p.m) * ostride + (long long)oy * p.ow + ox;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int oc = mt * 32 + 8 * (r >> 2) + 4 * lhi + (r & 3);
                    if (oc < p.m) yp[(long long)oc * ostride] = activate<ACT>(acc[r]);
                }
            }
        }
        if (tn < total) store_tile();
    }
}

inline osh_status conv3x3_wi_launch(const osh_conv_params *p, const float *x, const float *wpk, const float *bias,
                                    int act, float *y, hipStream_t st, int cus) {
    const int mtiles = (p->m + 31) / 32;
    const long long tiles = (long long)p->n * (p->ow / 8) * ((p->oh + 3) / 4);
    // one workgroup (4 waves) per CU, spread over the oc tiles; every wave gets
    // ceil(tiles / waves) tiles at most
    long long per = (cus + mtiles - 1) / mtiles;
    long long need = (tiles + 3) / 4;
    if (per > need) per = need;
    if (per < 1) per = 1;
    if (mtiles > 65535) return fail(OSH_E_UNSUPPORTED, "Conv: too many output channels");
    dim3 grid((unsigned)per, mtiles), block(256);
#define OSH_WI_LAUNCH(C_) \
    OSH_DISPATCH_ACT(act, ACT, hipLaunchKernelGGL((conv3x3_wi_kernel<C_, ACT>), grid, block, 0, st, *p, x, wpk, bias, y))
    switch (p->c) {
    case 16: OSH_WI_LAUNCH(16); break;
    case 32: OSH_WI_LAUNCH(32); break;
    default: OSH_WI_LAUNCH(64); break;
    }
#undef OSH_WI_LAUNCH
    OSH_LAUNCH_CHECK("conv3x3_wi_kernel");
    return OSH_OK;
}

}  // namespace osh
