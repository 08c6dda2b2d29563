// osh_igemm.h -- FP32 MFMA (v_mfma_f32_32x32x2f32) implicit-GEMM tile for gfx950.
//
//   C[m, n] = act( init(m, n) + sum_k A[m, k] * B[k, n] )    (k ascending)
//
// A is a row-major [M, K] matrix (MatMul's A, or Conv weights OIHW seen as
// [M, C/group*KH*KW]).  B is either a dense row-major [K, N] matrix (MatMul's
// B, or an NCHW activation seen as [C, H*W] for a 1x1 conv) or the implicit
// im2col matrix of a conv input, gathered on the fly (k = ic*KH*KW + ky*KW + kx,
// n = oy*OW + ox -- the reference's im2col order, ConvKernels.cs:554-563).
//
// The accumulator starts at the bias and runs over k in ascending pairs, the
// order of the reference's FMA chain (GemmKernel.cs:1130-1207) up to the MFMA
// pairing.  Tiles are staged through LDS with a register prefetch of the next
// K chunk (two LDS buffers, one barrier per chunk).
#pragma once

#include "osh_common.h"

namespace osh {

enum { B_DENSE = 0, B_IM2COL = 1 };

struct IgemmArgs {
    int M, N, K;
    const float *A;
    int lda;
    long long strideA;  // per z-slice (batch * group)
    const float *B;
    int ldb;
    long long strideB;
    float *C;
    int ldc;
    long long strideC;
    const float *row_bias;   // indexed by m (+ z-slice offset bias_stride)
    const float *col_bias;   // indexed by n
    const float *col_scale;  // indexed by n
    const float *res;        // optional residual, laid out as C: C = act(...) + res
    int bias_stride;         // row_bias offset per z-slice (conv groups)
    int zdiv;                // z = outer * zdiv + inner; strides apply as below
    long long strideA_in, strideB_in, strideC_in;  // per inner index (conv group)
    // im2col geometry (B_IM2COL)
    int H, W, KH, KW, sh, sw, dh, dw, pt, pl, OW;
};

template <int BM, int BN, int WM, int WN, int BMODE, bool VEC_A, bool VEC_B, int ACT>
__global__ __launch_bounds__(WM *WN * 64) void igemm_f32_kernel(IgemmArgs p) {
    constexpr int BK = 16;
    constexpr int THREADS = WM * WN * 64;
    constexpr int WTM = BM / WM;  // wave tile rows
    constexpr int WTN = BN / WN;  // wave tile cols
    constexpr int TM = WTM / 32;
    constexpr int TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be 32-multiples");
    constexpr int PADA = 4, PADB = 4;
    constexpr int A_VEC = BM * BK / 4;  // float4 slots per A chunk
    constexpr int A_PER = (A_VEC + THREADS - 1) / THREADS;
    constexpr int B_VEC = BK * BN / 4;
    constexpr int B_PER_V = (B_VEC + THREADS - 1) / THREADS;
    constexpr int B_PER_S = BK * BN / THREADS;  // scalar gather slots (im2col)
    static_assert(BMODE != B_IM2COL || (THREADS % BN == 0 && (BK * BN) % THREADS == 0), "im2col mapping");

    __shared__ __align__(16) float As[2][BK][BM + PADA];
    __shared__ __align__(16) float Bs[2][BK][BN + PADB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int z = blockIdx.z;
    const int zo = z / p.zdiv, zi = z % p.zdiv;

    const float *__restrict__ A = p.A + zo * p.strideA + zi * p.strideA_in;
    const float *__restrict__ B = p.B + zo * p.strideB + zi * p.strideB_in;
    float *__restrict__ Cp = p.C + zo * p.strideC + zi * p.strideC_in;
    const float *__restrict__ Rp = p.res ? p.res + zo * p.strideC + zi * p.strideC_in : nullptr;
    const float *__restrict__ row_bias = p.row_bias ? p.row_bias + zi * p.bias_stride : nullptr;
    const int M = p.M, N = p.N, K = p.K;

    // ---- per-thread im2col column (fixed across chunks)
    int my_n = 0, iy0 = 0, ix0 = 0;
    bool n_ok = false;
    if constexpr (BMODE == B_IM2COL) {
        my_n = tid % BN;
        int n = n0 + my_n;
        n_ok = n < N;
        int oy = n_ok ? n / p.OW : 0;
        int ox = n_ok ? n - oy * p.OW : 0;
        iy0 = oy * p.sh - p.pt;
        ix0 = ox * p.sw - p.pl;
    }
    const int KHW = p.KH * p.KW;

    float4 ra[A_PER];
    float4 rbv[B_PER_V];
    float rbs[B_PER_S > 0 ? B_PER_S : 1];

    auto load_chunk = [&](int k0) {
        // A: [BM][BK] slice, float4 along k
#pragma unroll
        for (int i = 0; i < A_PER; i++) {
            int e = tid + i * THREADS;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (e < A_VEC) {
                int m = e / (BK / 4), kq = (e % (BK / 4)) * 4;
                int gm = m0 + m, gk = k0 + kq;
                if (gm < M) {
                    const float *src = A + (long long)gm * p.lda + gk;
                    if (VEC_A && gk + 3 < K) {
                        v = *reinterpret_cast<const float4 *>(src);
                    } else {
                        v.x = gk + 0 < K ? src[0] : 0.f;
                        v.y = gk + 1 < K ? src[1] : 0.f;
                        v.z = gk + 2 < K ? src[2] : 0.f;
                        v.w = gk + 3 < K ? src[3] : 0.f;
                    }
                }
            }
            ra[i] = v;
        }
        if constexpr (BMODE == B_DENSE) {
#pragma unroll
            for (int i = 0; i < B_PER_V; i++) {
                int e = tid + i * THREADS;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (e < B_VEC) {
                    int k = e / (BN / 4), nq = (e % (BN / 4)) * 4;
                    int gk = k0 + k, gn = n0 + nq;
                    if (gk < K) {
                        const float *src = B + (long long)gk * p.ldb + gn;
                        if (VEC_B && gn + 3 < N) {
                            v = *reinterpret_cast<const float4 *>(src);
                        } else {
                            v.x = gn + 0 < N ? src[0] : 0.f;
                            v.y = gn + 1 < N ? src[1] : 0.f;
                            v.z = gn + 2 < N ? src[2] : 0.f;
                            v.w = gn + 3 < N ? src[3] : 0.f;
                        }
                    }
                }
                rbv[i] = v;
            }
        } else {
#pragma unroll
            for (int i = 0; i < B_PER_S; i++) {
                int k = tid / BN + i * (THREADS / BN);
                int gk = k0 + k;
                float v = 0.f;
                if (n_ok && gk < K) {
                    int ic = gk / KHW;
                    int r = gk - ic * KHW;
                    int ky = r / p.KW;
                    int kx = r - ky * p.KW;
                    int iy = iy0 + ky * p.dh, ix = ix0 + kx * p.dw;
                    if ((unsigned)iy < (unsigned)p.H && (unsigned)ix < (unsigned)p.W)
                        v = B[((long long)ic * p.H + iy) * p.W + ix];
                }
                rbs[i] = v;
            }
        }
    };

    auto store_chunk = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_PER; i++) {
            int e = tid + i * THREADS;
            if (e < A_VEC) {
                int m = e / (BK / 4), kq = (e % (BK / 4)) * 4;
                As[buf][kq + 0][m] = ra[i].x;
                As[buf][kq + 1][m] = ra[i].y;
                As[buf][kq + 2][m] = ra[i].z;
                As[buf][kq + 3][m] = ra[i].w;
            }
        }
        if constexpr (BMODE == B_DENSE) {
#pragma unroll
            for (int i = 0; i < B_PER_V; i++) {
                int e = tid + i * THREADS;
                if (e < B_VEC) {
                    int k = e / (BN / 4), nq = (e % (BN / 4)) * 4;
                    *reinterpret_cast<float4 *>(&Bs[buf][k][nq]) = rbv[i];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < B_PER_S; i++) {
                int k = tid / BN + i * (THREADS / BN);
                Bs[buf][k][my_n] = rbs[i];
            }
        }
    };

    // ---- accumulator init = bias (reference order: bias first, GemmKernel.cs:1128-1152)
    f32x16 acc[TM][TN];
    const int lrow = 4 * (lane >> 5);  // row offset of this lane inside a 32x32 tile
    const int lcol = lane & 31;
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            int gn = n0 + wn * WTN + tn * 32 + lcol;
            float cb = 0.f;
            if (!p.col_scale && p.col_bias && gn < N) cb = p.col_bias[gn];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float v = cb;
                if (!p.col_scale && !p.col_bias && row_bias) {
                    int gm = m0 + wm * WTM + tm * 32 + 8 * (r >> 2) + lrow + (r & 3);
                    v = gm < M ? row_bias[gm] : 0.f;
                }
                acc[tm][tn][r] = v;
            }
        }

    const int nchunks = (K + BK - 1) / BK;
    load_chunk(0);
    store_chunk(0);
    __syncthreads();

    for (int c = 0; c < nchunks; c++) {
        const int buf = c & 1;
        if (c + 1 < nchunks) load_chunk((c + 1) * BK);
#pragma unroll
        for (int s = 0; s < BK / 2; s++) {
            const int kk = 2 * s + (lane >> 5);
            float a[TM], b[TN];
#pragma unroll
            for (int tm = 0; tm < TM; tm++) a[tm] = As[buf][kk][wm * WTM + tm * 32 + lcol];
#pragma unroll
            for (int tn = 0; tn < TN; tn++) b[tn] = Bs[buf][kk][wn * WTN + tn * 32 + lcol];
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int tn = 0; tn < TN; tn++)
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[tm], b[tn], acc[tm][tn], 0, 0, 0);
        }
        if (c + 1 < nchunks) store_chunk(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: column scale (fmaf), activation, store
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            int gn = n0 + wn * WTN + tn * 32 + lcol;
            if (gn >= N) continue;
            float cs = 0.f, cb = 0.f;
            if (p.col_scale) {
                cs = p.col_scale[gn];
                cb = p.col_bias ? p.col_bias[gn] : 0.f;
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                int gm = m0 + wm * WTM + tm * 32 + 8 * (r >> 2) + lrow + (r & 3);
                if (gm < M) {
                    float v = acc[tm][tn][r];
                    if (p.col_scale) v = __builtin_fmaf(v, cs, cb);
                    v = activate<ACT>(v);
                    if (Rp) v += Rp[(long long)gm * p.ldc + gn];
                    Cp[(long long)gm * p.ldc + gn] = v;
                }
            }
        }
}

}  // namespace osh
