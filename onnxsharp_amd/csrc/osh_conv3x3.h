// osh_conv3x3.h -- 3x3 / pad 1 / dilation 1 / group 1 conv, stride 1 or 2,
// as an FP32 MFMA implicit GEMM over an LDS halo tile (gfx950).
//
// The reference runs these layers through NchwcConv on AVX-512 hosts
// (src/OnnxSharp/Kernels/NchwcConv.cs:109-142,533-605: blocked layout, 16
// accumulators per row group) and through PackedConv / Im2Col elsewhere.  Here
// a workgroup owns 64 output channels x TH output rows x 32 output columns.
// Per chunk of CI input channels it stages
//   - the input halo patch  [(TH-1)*S+3 rows][2][31*S+3 cols][4]  (zero outside
//     the image; channel ci lives at [ci / 4][..][ci % 4]; for S = 2 each row is
//     stored even columns first, then odd columns, so the stride-2 taps of 32
//     neighbouring pixels are consecutive), and
//   - the packed weights    [9 taps][2][64 oc][4]                 (one contiguous
//     block, same channel split),
// so a lane fetches the operands of four k-steps with one ds_read_b128 each.
// Every wave issues v_mfma_f32_32x32x2f32 with A = weights (32 oc x channel
// pair) and B = patch (channel pair x 32 pixels of one output row); the next
// tap's operands are loaded while the current tap's four MFMAs run.  The
// accumulation order per output is: bias, then chunk of 8 channels -> tap
// (ky, kx) -> channel pairs (s, s + 4), an NchwcConv-like order
// (icb -> ky -> kx -> lane) with 8-channel blocks.
#pragma once

#include "osh_common.h"

namespace osh {

constexpr int C3_CI = 8;   // input channels per K chunk
constexpr int C3_BM = 64;  // output channels per workgroup

inline bool conv3x3_eligible(const osh_conv_params *p) {
    return p->group == 1 && p->kh == 3 && p->kw == 3 && p->dh == 1 && p->dw == 1 && p->pt == 1 && p->pl == 1 &&
           p->sh == p->sw && (p->sh == 1 || p->sh == 2) && p->ow >= 24;
}

inline size_t conv3x3_packed_bytes(const osh_conv_params *p) {
    size_t mt = (p->m + C3_BM - 1) / C3_BM, chunks = (p->c + C3_CI - 1) / C3_CI;
    return mt * chunks * 9 * C3_CI * C3_BM * sizeof(float);
}

// packed[mt][chunk][tap][ci / 4][oc 64][ci % 4] = w[mt*64 + oc][chunk*CI + ci][tap] (0 beyond M or C).
__global__ void conv3x3_pack_kernel(int M, int C, const float *__restrict__ w, float *__restrict__ out,
                                    long long total) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    int c4 = (int)(i % 4);
    long long t = i / 4;
    int oc = (int)(t % C3_BM);
    t /= C3_BM;
    int chi = (int)(t % 2);
    t /= 2;
    int ci = chi * 4 + c4;
    int tap = (int)(t % 9);
    t /= 9;
    int chunks = (C + C3_CI - 1) / C3_CI;
    int chunk = (int)(t % chunks);
    int mt = (int)(t / chunks);
    int m = mt * C3_BM + oc, c = chunk * C3_CI + ci;
    out[i] = (m < M && c < C) ? w[((long long)m * C + c) * 9 + tap] : 0.f;
}

inline osh_status conv3x3_pack(const osh_conv_params *p, const float *w, void *packed, hipStream_t st) {
    long long total = (long long)(conv3x3_packed_bytes(p) / sizeof(float));
    hipLaunchKernelGGL(conv3x3_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, p->m, p->c, w,
                       (float *)packed, total);
    OSH_LAUNCH_CHECK("conv3x3_pack_kernel");
    return OSH_OK;
}

template <int S, int TH, int ACT>
__global__ __launch_bounds__(TH * 2 * 64) void conv3x3_kernel(osh_conv_params p, const float *__restrict__ x,
                                                             const float *__restrict__ wpk,
                                                             const float *__restrict__ bias,
                                                             const float *__restrict__ res,
                                                             float *__restrict__ y) {
    constexpr int CI = C3_CI;
    static_assert(CI == 8, "the operand layout splits a chunk into two groups of four channels");
    constexpr int NW = TH * 2;             // waves: (row, oc half)
    constexpr int THREADS = NW * 64;
    constexpr int PR = (TH - 1) * S + 3;   // patch rows
    constexpr int PC = 31 * S + 3;         // patch cols
    constexpr int HALF = (PC + 1) / 2;     // even columns stored first when S == 2
    constexpr int PITCH = S == 1 ? PC : 2 * HALF;
    constexpr int PE = CI * PR * PC;       // patch elements per chunk
    constexpr int P_PER = (PE + THREADS - 1) / THREADS;
    constexpr int WE4 = 9 * CI * C3_BM / 4;  // weight float4 per chunk
    constexpr int W_PER = (WE4 + THREADS - 1) / THREADS;

    __shared__ __align__(16) float Xs[2][PR][2][PITCH][4];
    __shared__ __align__(16) float Ws[2][9][2][C3_BM][4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wrow = wave >> 1, whalf = wave & 1;
    const int ox0 = blockIdx.x * 32;
    const int oy0 = blockIdx.y * TH;
    const int mtiles = (p.m + C3_BM - 1) / C3_BM;
    const int mt = blockIdx.z % mtiles;
    const int n = blockIdx.z / mtiles;
    const int chunks = (p.c + CI - 1) / CI;
    const int H = p.h, W = p.w;
    const float *__restrict__ xn = x + (long long)n * p.c * H * W;
    const float *__restrict__ wm = wpk + (long long)mt * chunks * 9 * CI * C3_BM;
    const int iy0 = oy0 * S - 1, ix0 = ox0 * S - 1;

    float rp[P_PER];
    float4 rw[W_PER];

    auto load_chunk = [&](int ch) {
        const int c0 = ch * CI;
#pragma unroll
        for (int i = 0; i < P_PER; i++) {
            int e = tid + i * THREADS;
            float v = 0.f;
            if (e < PE) {
                int ci = e / (PR * PC);
                int r = (e / PC) % PR;
                int col = e % PC;
                int c = c0 + ci, iy = iy0 + r, ix = ix0 + col;
                if (c < p.c && (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W)
                    v = xn[((long long)c * H + iy) * W + ix];
            }
            rp[i] = v;
        }
        const float4 *wsrc = reinterpret_cast<const float4 *>(wm + (long long)ch * 9 * CI * C3_BM);
#pragma unroll
        for (int i = 0; i < W_PER; i++) {
            int e = tid + i * THREADS;
            rw[i] = e < WE4 ? wsrc[e] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };

    auto store_chunk = [&](int buf) {
#pragma unroll
        for (int i = 0; i < P_PER; i++) {
            int e = tid + i * THREADS;
            if (e < PE) {
                int ci = e / (PR * PC);
                int r = (e / PC) % PR;
                int col = e % PC;
                int sc = S == 1 ? col : ((col & 1) ? HALF + (col >> 1) : (col >> 1));
                Xs[buf][r][ci >> 2][sc][ci & 3] = rp[i];
            }
        }
        float4 *wdst = reinterpret_cast<float4 *>(&Ws[buf][0][0][0][0]);
#pragma unroll
        for (int i = 0; i < W_PER; i++) {
            int e = tid + i * THREADS;
            if (e < WE4) wdst[e] = rw[i];
        }
    };

    // accumulators start at the bias (NchwcConv.Row initialises its 16 accumulators with it)
    f32x16 acc;
    const int l32 = lane & 31, lhi = lane >> 5;
    const int oc_base = mt * C3_BM + whalf * 32;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        int oc = oc_base + 8 * (r >> 2) + 4 * lhi + (r & 3);
        acc[r] = (bias && oc < p.m) ? bias[oc] : 0.f;
    }

    // stored column of pixel l32 for tap kx
    auto scol = [&](int kx) { return S == 1 ? l32 + kx : (kx == 1 ? HALF + l32 : l32 + (kx >> 1)); };

    load_chunk(0);
    store_chunk(0);
    __syncthreads();
    for (int ch = 0; ch < chunks; ch++) {
        const int buf = ch & 1;
        if (ch + 1 < chunks) load_chunk(ch + 1);
        const float4 *wa = reinterpret_cast<const float4 *>(&Ws[buf][0][lhi][whalf * 32 + l32][0]);
        constexpr int WTAP4 = 2 * C3_BM;  // float4 stride between taps
        float4 a = wa[0];
        float4 b = *reinterpret_cast<const float4 *>(&Xs[buf][wrow * S][lhi][scol(0)][0]);
#pragma unroll
        for (int tap = 0; tap < 9; tap++) {
            float4 an, bn;
            if (tap < 8) {
                const int ky = (tap + 1) / 3, kx = (tap + 1) % 3;
                an = wa[(tap + 1) * WTAP4];
                bn = *reinterpret_cast<const float4 *>(&Xs[buf][wrow * S + ky][lhi][scol(kx)][0]);
            }
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, acc, 0, 0, 0);
            if (tap < 8) {
                a = an;
                b = bn;
            }
        }
        if (ch + 1 < chunks) store_chunk(buf ^ 1);
        __syncthreads();
    }

    const int oy = oy0 + wrow, ox = ox0 + l32;
    if (oy < p.oh && ox < p.ow) {
        const long long base = ((long long)n * p.m) * p.oh * p.ow + (long long)oy * p.ow + ox;
        float *yrow = y + base;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            int oc = oc_base + 8 * (r >> 2) + 4 * lhi + (r & 3);
            if (oc < p.m) {
                float v = activate<ACT>(acc[r]);
                if (res) v += res[base + (long long)oc * p.oh * p.ow];
                yrow[(long long)oc * p.oh * p.ow] = v;
            }
        }
    }
}

inline osh_status conv3x3_launch(const osh_conv_params *p, const float *x, const float *wpk, const float *bias,
                                 const float *res, int act, float *y, hipStream_t st) {
    constexpr int TH = 2;
    const int mtiles = (p->m + C3_BM - 1) / C3_BM;
    dim3 grid((p->ow + 31) / 32, (p->oh + TH - 1) / TH, p->n * mtiles);
    dim3 block(TH * 2 * 64);
    if (p->sh == 1) {
        OSH_DISPATCH_ACT(act, ACT, hipLaunchKernelGGL((conv3x3_kernel<1, TH, ACT>), grid, block, 0, st, *p, x, wpk, bias, res, y));
    } else {
        OSH_DISPATCH_ACT(act, ACT, hipLaunchKernelGGL((conv3x3_kernel<2, TH, ACT>), grid, block, 0, st, *p, x, wpk, bias, res, y));
    }
    OSH_LAUNCH_CHECK("conv3x3_kernel");
    return OSH_OK;
}

}  // namespace osh
