// osh_gemm16.h -- FP32 GEMM on v_mfma_f32_16x16x4f32 with k in order, for
// dense row-major A[M,K] x B[K,N] (MatMul, 1x1 conv).
//
//   C[m, n] = act( init(m, n) + sum_k A[m, k] * B[k, n] )
//
// init is the column bias, else the row bias (GemmKernel.cs:1128-1152); with
// a column scale the result is fmaf(sum, scale[n], col_bias[n])
// (GemmKernel.cs:1210-1241).
//
// Summation order.  v_mfma_f32_16x16x4f32 adds its four products to the
// accumulator one after another in lane-group order (k = k0 + g for lane group
// g = lane / 16), each step rounded like an fmaf; so with k0 stepping by 4 from
// 0 every output element is the reference's k-ascending fmaf chain started at
// the bias, bit for bit.  No split of K across waves is made for that reason.
//
// Decomposition.  The unit of work is a 16 x 16 output block; a wave owns a
// (16*TM) x (16*BV*TN) tile and runs its whole K.  Waves are independent (no
// barriers): the four waves of a workgroup take four consecutive row tiles of
// one column tile, so their B reads meet in the CU's L1.  The host picks the
// tile so that the number of waves fits the 1024 SIMDs in as few rounds as
// possible (e.g. 1024 x 768 -> 3072 blocks -> 1024 waves of 16 x 48).
//
// Operands (lane (j, g) = (lane & 15, lane >> 4)), per chunk of KC k:
//   * A is staged through the wave's own LDS slice (no barriers: a wave's LDS
//     accesses complete in order): 16-byte global loads along k are stored as
//     [row][g][s] per 16-k group (k = 4s + g), so one ds_read_b128 gives a lane
//     its operands A[row j][k0 + 4s + g] for four k4 steps;
//   * B comes straight from global memory: per k4 step one BV-wide buffer load
//     of B[k0 + 4s + g][col .. col + BV - 1], col = 16*BV*tn + BV*j; component
//     q feeds output block q of the tile, whose column j stands for col + q, so
//     a lane stores BV adjacent columns at once.
// k offsets live in scalar registers.  Rows past M and columns past N are
// clamped for loads and never stored; the K tail (K % KC) is loaded with
// guarded loads and zero-filled, and a zero product leaves the chain unchanged.
#pragma once

#include "osh_common.h"
#include "osh_igemm.h"

namespace osh {

template <int BV>
struct G16Vec {
    float v[BV];
};

template <int BV>
__device__ __forceinline__ G16Vec<BV> g16_load_b(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    G16Vec<BV> o;
    if constexpr (BV == 4) {
        auto u = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
#pragma unroll
        for (int q = 0; q < 4; q++) o.v[q] = __uint_as_float(u[q]);
    } else if constexpr (BV == 3) {
        auto u = __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, 0);
#pragma unroll
        for (int q = 0; q < 3; q++) o.v[q] = __uint_as_float(u[q]);
    } else if constexpr (BV == 2) {
        auto u = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
#pragma unroll
        for (int q = 0; q < 2; q++) o.v[q] = __uint_as_float(u[q]);
    } else {
        o.v[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
    }
    return o;
}

// Per-wave LDS slice for A: [buf 2][tm][kgroup KC/16][row 16][g 4][s 4] floats.
template <int TM, int KC>
struct G16Lds {
    static constexpr int CHUNK = TM * (KC / 16) * 16 * 16;  // floats per buffer
    static constexpr int WAVE = 2 * CHUNK;
};

template <int TM, int KC>
struct G16A {
    float4 v[TM][KC / 16];  // a lane's 16-byte slots of an A chunk (global -> LDS)
};
template <int TM, int KC>
struct G16AV {
    float4 v[TM][KC / 16];  // a lane's MFMA operands of an A chunk (LDS -> MFMA)
};
template <int TN, int BV, int KC>
struct G16B {
    G16Vec<BV> v[KC / 4][TN];  // one BV-wide load per k4 step and column block
};

template <int TM, int TN, int BV, int KC, int ACT>
__global__ __launch_bounds__(256) void gemm16_kernel(IgemmArgs p, int tiles_m) {
    constexpr int STEPS = KC / 4;
    constexpr int AU = KC / 16;  // A float4 slots per lane per 16-row block
    constexpr int KQ = KC / 4;   // float4 slots per row of a chunk
    constexpr int CH = G16Lds<TM, KC>::CHUNK;
    static_assert(KC % 32 == 0, "a chunk is whole 16-k groups and 64 lanes x 16 rows of slots");
    __shared__ __align__(16) float lds[4 * G16Lds<TM, KC>::WAVE];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int groups_m = (tiles_m + 3) / 4;
    const int mt = (blockIdx.x % groups_m) * 4 + wave;
    const int nt = blockIdx.x / groups_m;
    if (mt >= tiles_m) return;  // whole wave; the kernel has no barriers
    const int m0 = mt * 16 * TM, n0 = nt * 16 * BV * TN;

    const int z = blockIdx.y;
    const int zo = z / p.zdiv, zi = z % p.zdiv;
    const float *__restrict__ A = p.A + zo * p.strideA + zi * p.strideA_in;
    const float *__restrict__ B = p.B + zo * p.strideB + zi * p.strideB_in;
    float *__restrict__ C = p.C + zo * p.strideC + zi * p.strideC_in;
    const float *__restrict__ R = p.res ? p.res + zo * p.strideC + zi * p.strideC_in : nullptr;
    const float *__restrict__ row_bias = p.row_bias ? p.row_bias + zi * p.bias_stride : nullptr;
    const int M = p.M, N = p.N, K = p.K, lda = p.lda, ldb = p.ldb;
    const int bytes_a = (int)(((long long)(M - 1) * lda + K) * 4);
    const int bytes_b = (int)(((long long)(K - 1) * ldb + N) * 4);
    float *wl = lds + wave * G16Lds<TM, KC>::WAVE;

    // A slot e = lane + 64u of a 16-row block: row e / KQ, k = 4 * (e % KQ);
    // element c of the slot is k = 4kq + c -> LDS [kg = kq/4][row][g = c][s = kq%4]
    int voa[TM][AU], lw[TM][AU];
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int u = 0; u < AU; u++) {
            const int e = lane + 64 * u, r = e / KQ, kq = e % KQ;
            voa[tm][u] = (min(m0 + 16 * tm + r, M - 1) * lda + 4 * kq) * 4;
            lw[tm][u] = ((tm * (KC / 16) + (kq >> 2)) * 16 + r) * 16 + (kq & 3);
        }
    const int lr = j * 16 + g * 4;  // lane (j, g) reads [tm][kg][j][g][0..3]
    int vob[TN];
#pragma unroll
    for (int tn = 0; tn < TN; tn++) vob[tn] = (g * ldb + min(n0 + 16 * BV * tn + BV * j, N - BV)) * 4;

    f32x4 acc[TM][TN * BV];
#pragma unroll
    for (int tn = 0; tn < TN; tn++)
#pragma unroll
        for (int q = 0; q < BV; q++) {
            const int col = min(n0 + 16 * BV * tn + BV * j + q, N - 1);
            const float cb = (!p.col_scale && p.col_bias) ? p.col_bias[col] : 0.f;
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float v = cb;
                    if (!p.col_scale && !p.col_bias && row_bias)
                        v = row_bias[min(m0 + 16 * tm + 4 * g + r, M - 1)];
                    acc[tm][tn * BV + q][r] = v;
                }
        }

    const int nfull = K / KC;

    // Full chunks only (k0 + KC <= K): unguarded loads, scalar k offsets.
    auto load_a = [&](G16A<TM, KC> &R, int c) {
        __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void *)A, (short)0, bytes_a, 0x00020000);
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int u = 0; u < AU; u++) {
                auto v = __builtin_amdgcn_raw_buffer_load_b128(ra, voa[tm][u], c * KC * 4, 0);
                R.v[tm][u] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                                         __uint_as_float(v[3]));
            }
    };
    auto load_b = [&](G16B<TN, BV, KC> &R, int c) {
        __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void *)B, (short)0, bytes_b, 0x00020000);
#pragma unroll
        for (int s = 0; s < STEPS; s++)
#pragma unroll
            for (int tn = 0; tn < TN; tn++) R.v[s][tn] = g16_load_b<BV>(rb, vob[tn], (c * KC + 4 * s) * ldb * 4);
    };
    auto stage_a = [&](const G16A<TM, KC> &R, int buf) {
        float *dst = wl + buf * CH;
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int u = 0; u < AU; u++) {
                dst[lw[tm][u] + 0] = R.v[tm][u].x;
                dst[lw[tm][u] + 4] = R.v[tm][u].y;
                dst[lw[tm][u] + 8] = R.v[tm][u].z;
                dst[lw[tm][u] + 12] = R.v[tm][u].w;
            }
    };
    auto read_a = [&](G16AV<TM, KC> &V, int buf) {
        const float *src = wl + buf * CH;
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int kg = 0; kg < KC / 16; kg++)
                V.v[tm][kg] = *reinterpret_cast<const float4 *>(src + (tm * (KC / 16) + kg) * 256 + lr);
    };
    auto compute = [&](const G16AV<TM, KC> &V, const G16B<TN, BV, KC> &R) {
#pragma unroll
        for (int s = 0; s < STEPS; s++) {
            const int kg = s >> 2, s4 = s & 3;
#pragma unroll
            for (int tm = 0; tm < TM; tm++) {
                const float4 &a4 = V.v[tm][kg];
                const float a = s4 == 0 ? a4.x : s4 == 1 ? a4.y : s4 == 2 ? a4.z : a4.w;
#pragma unroll
                for (int tn = 0; tn < TN; tn++)
#pragma unroll
                    for (int q = 0; q < BV; q++)
                        acc[tm][tn * BV + q] =
                            __builtin_amdgcn_mfma_f32_16x16x4f32(a, R.v[s][tn].v[q], acc[tm][tn * BV + q], 0, 0, 0);
            }
        }
    };

    if (nfull > 0) {
        // Pipeline: while chunk c computes, A(c+1) sits in LDS, A(c+2) and
        // B(c+1) are in flight.  Prefetch indices are clamped to the last full
        // chunk (redundant reloads, in bounds) so the loop body has no branches.
        const int last = nfull - 1;
        G16A<TM, KC> ra;
        G16B<TN, BV, KC> rb0, rb1;
        G16AV<TM, KC> av0, av1;
        load_a(ra, 0);
        load_b(rb0, 0);
        stage_a(ra, 0);
        load_a(ra, min(1, last));
        stage_a(ra, 1);
        load_a(ra, min(2, last));
        read_a(av0, 0);
        int c = 0;
        // The loads and LDS traffic of a half-step are issued between its
        // MFMAs (one memory instruction after every two MFMAs), so the MFMA
        // pipe is not left idle while they issue (1024 x 768 x 768: loop
        // 10.5 -> 9.1 us per wave; one per MFMA 9.5, one per three 9.7).
        constexpr int NMF = STEPS * TM * TN * BV;  // MFMAs per chunk
        constexpr int NGR = (NMF + 1) / 2;          // groups of two
        for (; c + 2 <= nfull; c += 2) {
            load_b(rb1, c + 1);
            __builtin_amdgcn_sched_barrier(0);
            compute(av0, rb0);
            read_a(av1, 1);            // A(c+1), staged a chunk ago
            stage_a(ra, 0);            // A(c+2) into the buffer chunk c used
            load_a(ra, min(c + 3, last));
            load_b(rb0, min(c + 2, last));
#pragma unroll
            for (int i = 0; i < NGR; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                  // two MFMAs
                __builtin_amdgcn_sched_group_barrier(0x020 | 0x100 | 0x200, 1, 0);  // then one VMEM read / DS op
            }
            __builtin_amdgcn_sched_barrier(0);
            compute(av1, rb1);
            read_a(av0, 0);            // A(c+2)
            stage_a(ra, 1);            // A(c+3)
            load_a(ra, min(c + 4, last));
#pragma unroll
            for (int i = 0; i < NGR; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x020 | 0x100 | 0x200, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c < nfull) compute(av0, rb0);
    }
    if (K % KC) {
        // tail chunk: k >= K loads as zero; staged through buffer 0 (every
        // earlier read of it has completed: LDS accesses of a wave are in order)
        G16A<TM, KC> ra;
        G16B<TN, BV, KC> rb;
        G16AV<TM, KC> av;
        const int k0 = nfull * KC;
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int u = 0; u < AU; u++) {
                const int e = lane + 64 * u, r = e / KQ, kq = e % KQ;
                const float *src = A + (long long)min(m0 + 16 * tm + r, M - 1) * lda;
                float t4[4];
#pragma unroll
                for (int c2 = 0; c2 < 4; c2++) {
                    const int k = k0 + 4 * kq + c2;
                    t4[c2] = k < K ? src[k] : 0.f;
                }
                ra.v[tm][u] = make_float4(t4[0], t4[1], t4[2], t4[3]);
            }
#pragma unroll
        for (int s = 0; s < STEPS; s++) {
            const int k = k0 + 4 * s + g;
#pragma unroll
            for (int tn = 0; tn < TN; tn++) {
                const int col = min(n0 + 16 * BV * tn + BV * j, N - BV);
#pragma unroll
                for (int q = 0; q < BV; q++) rb.v[s][tn].v[q] = k < K ? B[(long long)k * ldb + col + q] : 0.f;
            }
        }
        stage_a(ra, 0);
        read_a(av, 0);
        compute(av, rb);
    }

    // ---- epilogue: column scale (fmaf), activation, BV-wide stores
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            const int col = n0 + 16 * BV * tn + BV * j;
            if (col >= N) continue;
            float cs[BV], cb[BV];
#pragma unroll
            for (int q = 0; q < BV; q++) {
                cs[q] = p.col_scale ? p.col_scale[col + q] : 0.f;
                cb[q] = (p.col_scale && p.col_bias) ? p.col_bias[col + q] : 0.f;
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = m0 + 16 * tm + 4 * g + r;
                if (row >= M) continue;
                float o[BV];
#pragma unroll
                for (int q = 0; q < BV; q++) {
                    float v = acc[tm][tn * BV + q][r];
                    if (p.col_scale) v = __builtin_fmaf(v, cs[q], cb[q]);
                    o[q] = activate<ACT>(v);
                }
                if (R) {  // residual: same layout as C, BV-wide loads
                    const float *src = R + (long long)row * p.ldc + col;
                    if constexpr (BV == 4) {
                        const float4 t = *reinterpret_cast<const float4 *>(src);
                        o[0] += t.x, o[1] += t.y, o[2] += t.z, o[3] += t.w;
                    } else if constexpr (BV == 2) {
                        const float2 t = *reinterpret_cast<const float2 *>(src);
                        o[0] += t.x, o[1] += t.y;
                    } else {
#pragma unroll
                        for (int q = 0; q < BV; q++) o[q] += src[q];
                    }
                }
                float *dst = C + (long long)row * p.ldc + col;
                if constexpr (BV == 4) *reinterpret_cast<float4 *>(dst) = make_float4(o[0], o[1], o[2], o[3]);
                else if constexpr (BV == 2) *reinterpret_cast<float2 *>(dst) = make_float2(o[0], o[1]);
                else {
#pragma unroll
                    for (int q = 0; q < BV; q++) dst[q] = o[q];
                }
            }
        }
}

}  // namespace osh
