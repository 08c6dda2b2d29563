// osh_winograd.h -- Winograd F(2x2, 3x3) convolution (stride 1, pad 1) on
// v_mfma_f32_16x16x4f32, in the arithmetic of the reference's Winograd.cs:
//
//   weights  u = G g G^T with the 1/2 factors          (Winograd.cs:125-166)
//   input    v = B^T d B of each 4x4 patch (pad = 0)   (Winograd.cs:260-357)
//   product  M[comp][oc][tile] = sum over ic, ascending, of U[comp][oc][ic] * V[comp][ic][tile],
//            one fmaf chain from 0                       (Winograd.cs:234-258 -> GemmKernel.Multiply)
//   output   y = A^T M A, bias added last               (Winograd.cs:444-536)
//
// then the fused activation and an optional residual, as the other conv
// kernels apply them.  Every transform is the reference's sequence of single
// IEEE additions (this file is built with -ffp-contract=off), and the MFMA
// adds its four lane-group products one after another like fmaf, with ic in
// ascending order, so the result is the reference's Winograd path bit for
// bit (the GEMM's scalar tail columns aside: GemmKernel.MultiplyRow sums
// columns past the last full 8-column vector of a partial 16-column panel
// with separate multiply and add).
//
// One workgroup (4 waves) owns 16 output channels x 16 tiles (a tile is a
// 2x2 output block; tiles run over batch, tile row, tile column) for all 16
// components.  Per chunk of 16 input channels its 256 threads each transform
// one (ic, tile) patch into LDS as [comp][ic 16][tile 16]; wave w runs the
// MFMA chains of components 4w .. 4w+3 (the B operand of a k4 step is 64
// consecutive floats of one component).  The input patches are loaded two
// chunks ahead, the weight fragments likewise, and the component planes are
// double-buffered.  At the end the accumulators go through LDS as
// [comp][oc 16][tile 16] and each thread transforms one (oc, tile) to its 2x2
// outputs.
#pragma once

#include "osh_common.h"

namespace osh {

// Winograd.TryConv3x3's gate (Winograd.cs:58-122) on a resolved conv.
inline bool winograd_eligible(const osh_conv_params *p, long long max_pixels) {
    return p->group == 1 && p->kh == 3 && p->kw == 3 && p->sh == 1 && p->sw == 1 && p->dh == 1 && p->dw == 1 &&
           p->pt == 1 && p->pl == 1 && p->c >= 8 && p->m >= 8 && p->oh == p->h && p->ow == p->w && p->h >= 6 &&
           p->w >= 6 && (long long)p->h * p->w <= max_pixels && (long long)p->m * p->c * 16 <= (1LL << 24) &&
           (long long)p->n * p->c * p->h * p->w < (1LL << 31) && (long long)p->n * p->m * p->h * p->w < (1LL << 31) &&
           (long long)p->n * ((p->h + 1) / 2) * ((p->w + 1) / 2) <= 16LL * 65535;  // grid y
}

// Packed U: [16 comps][ceil(M/16)][ceil(C/16)][64 lanes][4]; lane (j, g) =
// (lane & 15, lane >> 4) holds U[comp][16*ob + j][16*cb + 4*s + g] in slot s,
// zero for padding channels.
inline size_t winograd_packed_bytes(const osh_conv_params *p) {
    return (size_t)16 * ((p->m + 15) / 16) * ((p->c + 15) / 16) * 256 * sizeof(float);
}

__global__ void wino_pack_kernel(int M, int C, const float *__restrict__ w, float *__restrict__ out) {
    const int ocbs = (M + 15) / 16, cbs = (C + 15) / 16;
    const long long total = (long long)ocbs * 16 * cbs * 16;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int oc = (int)(idx / (cbs * 16)), ic = (int)(idx % (cbs * 16));
    float u[16];
    if (oc < M && ic < C) {
        const float *g = w + ((long long)oc * C + ic) * 9;
        float s[12];
        for (int j = 0; j < 3; j++) {  // s = G g (4x3)
            const float g0 = g[j], g1 = g[3 + j], g2 = g[6 + j];
            s[j] = g0;
            s[3 + j] = (g0 + g1 + g2) * 0.5f;
            s[6 + j] = (g0 - g1 + g2) * 0.5f;
            s[9 + j] = g2;
        }
        for (int i = 0; i < 4; i++) {  // u = s G^T (4x4)
            const float a = s[i * 3], b = s[i * 3 + 1], c = s[i * 3 + 2];
            u[i * 4] = a;
            u[i * 4 + 1] = (a + b + c) * 0.5f;
            u[i * 4 + 2] = (a - b + c) * 0.5f;
            u[i * 4 + 3] = c;
        }
    } else {
        for (int i = 0; i < 16; i++) u[i] = 0.0f;
    }
    const int ob = oc >> 4, j = oc & 15, cb = ic >> 4, icl = ic & 15;
    const int lane = (icl & 3) * 16 + j, slot = icl >> 2;
    for (int comp = 0; comp < 16; comp++)
        out[((((long long)comp * ocbs + ob) * cbs + cb) * 64 + lane) * 4 + slot] = u[comp];
}

struct WinoPatch {
    float d[16];
};

template <int ACT>
__global__ __launch_bounds__(256) void wino_f23_kernel(osh_conv_params p, const float *__restrict__ x,
                                                       const float4 *__restrict__ up,
                                                       const float *__restrict__ bias,
                                                       const float *__restrict__ res, float *__restrict__ y) {
    __shared__ __attribute__((aligned(16))) float vs[2][16 * 256];  // [buf][comp][ic 16][tile 16]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int C = p.c, H = p.h, W = p.w, M = p.m;
    const int tilesX = (W + 1) >> 1, tilesY = (H + 1) >> 1, T = tilesX * tilesY;
    const int ocbs = (M + 15) >> 4, cbs = (C + 15) >> 4;
    const int ob = blockIdx.x;
    // thread role for the transforms: (channel row tid >> 4, tile tid & 15)
    const int row = tid >> 4, tl = tid & 15;
    const long long tg = (long long)blockIdx.y * 16 + tl;
    const bool tile_ok = tg < (long long)p.n * T;
    int img = 0, ty = 0, tx = 0;
    if (tile_ok) {
        img = (int)(tg / T);
        const int t = (int)(tg % T);
        ty = t / tilesX;
        tx = t - ty * tilesX;
    }
    const int y0 = 2 * ty - 1, x0 = 2 * tx - 1;
    const float *xin = x + (long long)img * C * H * W;

    auto load_patch = [&](int cb) {
        WinoPatch q;
        const int ic = cb * 16 + row;
        const bool ok = tile_ok && ic < C;
        const float *xc = xin + (long long)(ok ? ic : 0) * H * W;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int yy = y0 + i;
            const bool rok = ok && yy >= 0 && yy < H;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int xx = x0 + j;
                q.d[i * 4 + j] = (rok && xx >= 0 && xx < W) ? xc[(long long)yy * W + xx] : 0.0f;
            }
        }
        return q;
    };
    // V = B^T d B, stored at [comp][row][tl]
    auto transform_store = [&](const WinoPatch &q, float *vb) {
        float t[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float d0 = q.d[j], d1 = q.d[4 + j], d2 = q.d[8 + j], d3 = q.d[12 + j];
            t[j] = d0 - d2;
            t[4 + j] = d1 + d2;
            t[8 + j] = d2 - d1;
            t[12 + j] = d1 - d3;
        }
        float *dst = vb + row * 16 + tl;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float a = t[i * 4], b = t[i * 4 + 1], c2 = t[i * 4 + 2], d3 = t[i * 4 + 3];
            dst[(i * 4) * 256] = a - c2;
            dst[(i * 4 + 1) * 256] = b + c2;
            dst[(i * 4 + 2) * 256] = c2 - b;
            dst[(i * 4 + 3) * 256] = b - d3;
        }
    };
    // weight fragments of this wave's four components for chunk cb
    const float4 *ub = up + (long long)ob * cbs * 64 + lane;
    const long long ucomp = (long long)ocbs * cbs * 64;
    auto load_u = [&](int cb, float4 u[4]) {
#pragma unroll
        for (int q = 0; q < 4; q++) u[q] = ub[(4 * wave + q) * ucomp + (long long)cb * 64];
    };

    f32x4 acc[4];
#pragma unroll
    for (int q = 0; q < 4; q++) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};

    WinoPatch p0 = load_patch(0), p1;
    float4 u0[4], u1[4], u2[4];
    load_u(0, u0);
    if (cbs > 1) {
        p1 = load_patch(1);
        load_u(1, u1);
    }
    transform_store(p0, vs[0]);
    __syncthreads();
    const int boff = (lane >> 4) * 16 + (lane & 15);  // B operand: V[k = lane >> 4][tile = lane & 15]
    for (int cb = 0; cb < cbs; cb++) {
        const int buf = cb & 1;
        const bool pre = cb + 2 < cbs;
        if (pre) {
            p0 = load_patch(cb + 2);
            load_u(cb + 2, u2);
        }
        const float *vb = vs[buf] + 4 * wave * 256 + boff;
#pragma unroll
        for (int s = 0; s < 4; s++) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float a = s == 0 ? u0[q].x : s == 1 ? u0[q].y : s == 2 ? u0[q].z : u0[q].w;
                acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vb[q * 256 + s * 64], acc[q], 0, 0, 0);
            }
        }
        if (cb + 1 < cbs) transform_store(p1, vs[buf ^ 1]);
        __syncthreads();
        p1 = p0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            u0[q] = u1[q];
            u1[q] = u2[q];
        }
    }
    // accumulators -> [comp][oc 16][tile 16]; D[row 4g + r][col j]
    {
        float *ms = vs[0] + 4 * wave * 256 + (lane >> 4) * 64 + (lane & 15);
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int r = 0; r < 4; r++) ms[q * 256 + r * 16] = acc[q][r];
    }
    __syncthreads();
    const int oc = ob * 16 + row;
    if (!tile_ok || oc >= M) return;
    float m[16];
#pragma unroll
    for (int comp = 0; comp < 16; comp++) m[comp] = vs[0][comp * 256 + row * 16 + tl];
    float t[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {  // A^T M
        const float m0 = m[j], m1 = m[4 + j], m2 = m[8 + j], m3 = m[12 + j];
        t[j] = m0 + m1 + m2;
        t[4 + j] = m1 - m2 - m3;
    }
    const float b = bias ? bias[oc] : 0.0f;
    float o[4];
    o[0] = t[0] + t[1] + t[2] + b;  // (A^T M) A, bias last
    o[1] = t[1] - t[2] - t[3] + b;
    o[2] = t[4] + t[5] + t[6] + b;
    o[3] = t[5] - t[6] - t[7] + b;
    const int oy = 2 * ty, ox = 2 * tx;
    const long long base = ((long long)img * M + oc) * H * W;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int yy = oy + (e >> 1), xx = ox + (e & 1);
        if (yy < H && xx < W) {
            const long long at = base + (long long)yy * W + xx;
            float v = activate<ACT>(o[e]);
            if (res) v = v + res[at];
            y[at] = v;
        }
    }
}

inline osh_status winograd_pack(const osh_conv_params *p, const float *w, void *out, hipStream_t st) {
    const long long total = (long long)((p->m + 15) / 16) * 16 * ((p->c + 15) / 16) * 16;
    OSH_LAUNCH(wino_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, p->m, p->c, w,
                       static_cast<float *>(out));
    OSH_LAUNCH_CHECK("wino_pack_kernel");
    return OSH_OK;
}

}  // namespace osh
