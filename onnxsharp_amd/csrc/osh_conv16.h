// osh_conv16.h -- 3x3 convolution (stride 1 or 2, any pads, C % 16 == 0) as an
// implicit GEMM on v_mfma_f32_16x16x4f32, summing in the reference's NCHWc
// order:
//
//   y[oc][p] = act( b[oc] + sum over icb, ky, kx, i (i = 0..15) of
//                           w[oc][16 icb + i][ky][kx] * x[16 icb + i][iy(p, ky)][ix(p, kx)] )
//
// (NchwcConv.Row, src/OnnxSharp/Kernels/NchwcConv.cs:533-605: bias first, then
// icb -> ky -> kx -> lane16, one fmaf per term).  The MFMA adds its four
// products in lane-group order with one rounding each, so with the four k of a
// step being four consecutive input channels of one tap, every output is that
// chain bit for bit.  Padding taps read 0 and leave the chain unchanged.
//
// GEMM view: M = output channels, N = output pixels (OH*OW, row-major), K =
// 9C in the order above.  A wave owns (16*TM) channels x (16*BV) pixels and
// runs its whole K in order; the unit of balance is the 16 x 16 output block,
// so small maps (20x20, 40x40) still spread over many SIMDs.  Waves are
// independent (no LDS, no barriers).
//
// Operands (lane (j, g) = (lane & 15, lane >> 4)), per tap and 16-channel
// block (four k4 steps s):
//   * A (weights) is packed once, per 16-channel output block and per
//     (icb, tap), as 64 lanes x 4 steps, so one 16-byte load gives a lane
//     w[oc = 16 tm + j][16 icb + 4 s + g][tap] for its four steps;
//   * B (input) is one 4-byte buffer load per pixel and step:
//     x[16 icb + 4 s + g][iy][ix]; the lane's nine tap offsets are computed
//     once, with an out-of-range offset for padding taps so the load returns 0.
// The channel-block and step offsets are scalar, so the k loop issues only
// buffer loads and MFMAs.  Loads run up to four (icb, ky) chunks -- three
// taps each -- ahead.
#pragma once

#include "osh_common.h"

namespace osh {

constexpr unsigned C16_OOB = 0x80000000u;  // buffer offset past any tensor: the load returns 0

template <int TM, int BV>
struct C16Chunk {
    float4 a[3][TM];      // per tap: the lane's 4 k4-step weights of each 16-channel output block
    float b[3][4][BV];    // per tap and k4 step: the lane's input value of each pixel
};

// One wave's tile: pixel tile pt (16*BV output pixels), output-channel tile
// mt (16*TM channels) of image n.  No barriers: any subset of a workgroup's
// waves may run it.  I2C runs the im2col chain instead (bias, then
// ic -> ky -> kx: ConvKernels.Im2Col / PackedConv, ConvKernels.cs:554-563),
// with the weights packed in that order (conv16_pack with i2c): step u of a
// channel block gives lane group g the term 4u + g = 9 ic + tap; with
// u = 9v + r its channel is 4v + (4r + g) / 9 and its tap (4r + g) % 9, so
// each lane keeps nine offsets (one per r) and 4v is a scalar offset.
template <int TM, int BV, int ACT, bool I2C = false>
__device__ __forceinline__ void conv16_wave(const osh_conv_params &p, const float *__restrict__ x,
                                            const float *__restrict__ wpk, const float *__restrict__ bias,
                                            const float *__restrict__ res, float *__restrict__ y, const int pt,
                                            const int mt, const int n) {
    const int lane = threadIdx.x & 63;
    const int j = lane & 15, g = lane >> 4;
    const int HW = p.h * p.w, OHW = p.oh * p.ow;
    const int C = p.c, M = p.m;
    const int icbs = C / 16;
    const float *xn = x + (long long)n * C * HW;
    float *yn = y + (long long)n * M * OHW;
    const float *rn = res ? res + (long long)n * M * OHW : nullptr;

    // per pixel: the nine tap offsets (bytes, lane group g's channel included;
    // with I2C offset r holds term 4r + g of a channel block)
    int off[BV][9];
#pragma unroll
    for (int q = 0; q < BV; q++) {
        int pix = pt * 16 * BV + BV * j + q;
        pix = pix < OHW ? pix : OHW - 1;  // tail pixels compute a duplicate, never stored
        const int oy = pix / p.ow, ox = pix - oy * p.ow;
        const int iy0 = oy * p.sh - p.pt, ix0 = ox * p.sw - p.pl;
#pragma unroll
        for (int r = 0; r < 9; r++) {
            const int term = 4 * r + g;
            const int tap = I2C ? term % 9 : r, ch = I2C ? term / 9 : g;
            const int iy = iy0 + tap / 3, ix = ix0 + tap % 3;
            const bool ok = (unsigned)iy < (unsigned)p.h && (unsigned)ix < (unsigned)p.w;
            off[q][r] = ok ? (ch * HW + iy * p.w + ix) * 4 : (int)C16_OOB;
        }
    }
    // packed weights: [mtile16][icb*9 + tap][64 lanes][4 steps]
    const int kgroups = icbs * 9;
    int voa[TM];
#pragma unroll
    for (int tm = 0; tm < TM; tm++) voa[tm] = (((mt * TM + tm) * kgroups) * 64 + lane) * 16;
    const int bytes_x = C * HW * 4;
    const int bytes_w = ((M + 15) / 16) * kgroups * 64 * 16;

    f32x4 acc[TM][BV];
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int oc = (mt * TM + tm) * 16 + 4 * g + r;
            const float b = (bias && oc < M) ? bias[oc] : 0.f;
#pragma unroll
            for (int q = 0; q < BV; q++) acc[tm][q][r] = b;
        }
    }

    if constexpr (TM * BV <= 2) {
        // One chunk = one 16-channel input block: its nine taps (ky, kx) x four
        // k4 steps, with every register index known at compile time.  Two
        // chunks are in flight in fixed registers (R0 holds the even blocks, R1
        // the odd ones): each tap's refill loads for the block two ahead are
        // issued right after the tap's MFMAs, and the last two blocks issue no
        // refills, so nothing is loaded that is not used and the loop carries
        // no register copies that would wait for every load.
        struct Blk {
            float4 a[9][TM];    // per tap: the lane's 4 k4-step weights of each output block
            float b[9][4][BV];  // per tap and k4 step: the lane's input value of each pixel
        };
        __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)xn, (short)0, bytes_x, 0x00020000);
        __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)wpk, (short)0, bytes_w, 0x00020000);
        auto ld = [&](Blk &R, int icb, int t) {
#pragma unroll
            for (int tm = 0; tm < TM; tm++) {
                auto v = __builtin_amdgcn_raw_buffer_load_b128(rw, voa[tm], (icb * 9 + t) * 1024, 0);
                R.a[t][tm] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                                         __uint_as_float(v[3]));
            }
#pragma unroll
            for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
                for (int q = 0; q < BV; q++) {
                    if constexpr (I2C) {
                        const int u = 4 * t + s4, v = u / 9, r = u - 9 * v;
                        R.b[t][s4][q] = __uint_as_float(
                            __builtin_amdgcn_raw_buffer_load_b32(rx, off[q][r], (icb * 16 + 4 * v) * HW * 4, 0));
                    } else {
                        R.b[t][s4][q] = __uint_as_float(
                            __builtin_amdgcn_raw_buffer_load_b32(rx, off[q][t], (icb * 16 + 4 * s4) * HW * 4, 0));
                    }
                }
        };
        auto mm = [&](const Blk &R, int t) {
#pragma unroll
            for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
                for (int tm = 0; tm < TM; tm++) {
                    const float4 &a4 = R.a[t][tm];
                    const float a = s4 == 0 ? a4.x : s4 == 1 ? a4.y : s4 == 2 ? a4.z : a4.w;
#pragma unroll
                    for (int q = 0; q < BV; q++)
                        acc[tm][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, R.b[t][s4][q], acc[tm][q], 0, 0, 0);
                }
        };
        Blk R0, R1;
#pragma unroll
        for (int t = 0; t < 9; t++) ld(R0, 0, t);
        if (icbs > 1) {
#pragma unroll
            for (int t = 0; t < 9; t++) ld(R1, 1, t);
        }
        int icb = 0;
        for (; icb + 2 <= icbs; icb += 2) {
            if (icb + 2 < icbs) {
#pragma unroll
                for (int t = 0; t < 9; t++) mm(R0, t), ld(R0, icb + 2, t);
            } else {
#pragma unroll
                for (int t = 0; t < 9; t++) mm(R0, t);
            }
            if (icb + 3 < icbs) {
#pragma unroll
                for (int t = 0; t < 9; t++) mm(R1, t), ld(R1, icb + 3, t);
            } else {
#pragma unroll
                for (int t = 0; t < 9; t++) mm(R1, t);
            }
        }
        if (icb < icbs) {
#pragma unroll
            for (int t = 0; t < 9; t++) mm(R0, t);
        }
    } else {
        static_assert(!I2C, "the im2col order runs on the one-block-per-chunk loop");
        // chunk c = icb * 3 + ky: taps (ky, 0..2) of channel block icb
        auto load = [&](C16Chunk<TM, BV> &R, int c) {
            __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)xn, (short)0, bytes_x, 0x00020000);
            __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)wpk, (short)0, bytes_w, 0x00020000);
            const int icb = c / 3, ky = c - icb * 3;
    #pragma unroll
            for (int kx = 0; kx < 3; kx++) {
                const int kg = icb * 9 + ky * 3 + kx;
    #pragma unroll
                for (int tm = 0; tm < TM; tm++) {
                    auto v = __builtin_amdgcn_raw_buffer_load_b128(rw, voa[tm], kg * 1024, 0);
                    R.a[kx][tm] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                                              __uint_as_float(v[3]));
                }
    #pragma unroll
                for (int s = 0; s < 4; s++)
    #pragma unroll
                    for (int q = 0; q < BV; q++)
                        R.b[kx][s][q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                            rx, off[q][ky * 3 + kx], (icb * 16 + 4 * s) * HW * 4, 0));
            }
        };
        auto compute = [&](const C16Chunk<TM, BV> &R) {
    #pragma unroll
            for (int kx = 0; kx < 3; kx++)
    #pragma unroll
                for (int s = 0; s < 4; s++)
    #pragma unroll
                    for (int tm = 0; tm < TM; tm++) {
                        const float4 &a4 = R.a[kx][tm];
                        const float a = s == 0 ? a4.x : s == 1 ? a4.y : s == 2 ? a4.z : a4.w;
    #pragma unroll
                        for (int q = 0; q < BV; q++)
                            acc[tm][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, R.b[kx][s][q], acc[tm][q], 0, 0, 0);
                    }
        };

        // D chunks in flight (their loads fit the 63 outstanding vector loads a
        // wave can count); the ring is unrolled so each chunk has fixed registers,
        // and prefetch indices are clamped to the last chunk (a reload, in bounds)
        // so the steady-state body has no branches.
        constexpr int L = 3 * (TM + 4 * BV);
        constexpr int D = 60 / L < 2 ? 2 : (60 / L > 4 ? 4 : 60 / L);
        const int nch = icbs * 3;
        const int last = nch - 1;
        C16Chunk<TM, BV> R[D];
    #pragma unroll
        for (int d = 0; d < D; d++) load(R[d], min(d, last));
        int c = 0;
        // a chunk's refill loads are issued between its own MFMAs (two MFMAs per
        // load; each load follows the MFMA that last reads its register), so the
        // MFMA pipe is not left idle while they issue
        constexpr int NGR = (12 * TM * BV + 1) / 2;
        for (; c + D <= nch; c += D) {
    #pragma unroll
            for (int d = 0; d < D; d++) {
                __builtin_amdgcn_sched_barrier(0);
                compute(R[d]);
                load(R[d], min(c + d + D, last));
    #pragma unroll
                for (int i = 0; i < NGR; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two MFMAs
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one VMEM read
                }
            }
        }
    #pragma unroll
        for (int d = 0; d < D; d++)
            if (c + d < nch) compute(R[d]);
    }

    // ---- epilogue: activation, stores (16 lanes = 16 consecutive pixels per channel row)
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int oc = (mt * TM + tm) * 16 + 4 * g + r;
            if (oc >= M) continue;
#pragma unroll
            for (int q = 0; q < BV; q++) {
                const int pix = pt * 16 * BV + BV * j + q;
                if (pix < OHW) {
                    float v = activate<ACT>(acc[tm][q][r]);
                    if (rn) v += rn[(long long)oc * OHW + pix];
                    yn[(long long)oc * OHW + pix] = v;
                }
            }
        }
}

// WPB waves per workgroup: 4 packs a workgroup's waves onto one CU's SIMDs;
// 1 spreads the same waves over as many CUs, which for maps with few tiles
// and deep K leaves each wave a CU's L1 bandwidth for its operand stream.
template <int TM, int BV, int ACT, int WPB = 4, bool I2C = false>
__global__ __launch_bounds__(256) void conv16_kernel(osh_conv_params p, const float *__restrict__ x,
                                                     const float *__restrict__ wpk, const float *__restrict__ bias,
                                                     const float *__restrict__ res, float *__restrict__ y,
                                                     int tiles_p) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int pt = blockIdx.x * WPB + wave;  // pixel tile
    if (pt >= tiles_p) return;             // whole wave; no barriers in the tile
    conv16_wave<TM, BV, ACT, I2C>(p, x, wpk, bias, res, y, pt, blockIdx.y, blockIdx.z);
}

// Same chain with the workgroup's weights resident in LDS: the four waves of
// a persistent workgroup share one output-channel tile, copy its packed
// weights (16*TM x 9C floats, at most CONV16L_LDS bytes) into LDS once, and
// then walk pixel tiles with a grid stride, reading A with ds_read_b128
// instead of re-streaming the weights from L2 for every tile.
constexpr int CONV16L_LDS = 147456;  // 16 * 4 * 9 * 64 floats: TM * C <= 256

template <int TM, int BV, int ACT>
__global__ __launch_bounds__(256) void conv16l_kernel(osh_conv_params p, const float *__restrict__ x,
                                                      const float *__restrict__ wpk, const float *__restrict__ bias,
                                                      const float *__restrict__ res, float *__restrict__ y,
                                                      int tiles_p) {
    __shared__ __align__(16) float wl[CONV16L_LDS / 4];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int mt = blockIdx.y;
    const int HW = p.h * p.w, OHW = p.oh * p.ow;
    const int C = p.c, M = p.m;
    const int icbs = C / 16;
    const int kgroups = icbs * 9;
    const int nblk = (M + 15) / 16;
    // copy this tile's weight blocks (those that exist) into LDS
    {
        const int blocks = min(TM, nblk - mt * TM);
        const int nf4 = blocks * kgroups * 64;  // float4 per block: kgroups * 64 lanes
        const float4 *src = reinterpret_cast<const float4 *>(wpk) + (long long)mt * TM * kgroups * 64;
        float4 *dst = reinterpret_cast<float4 *>(wl);
#pragma unroll 8
        for (int e = threadIdx.x; e < nf4; e += 256) dst[e] = src[e];
        // blocks past M read as zero
        for (int e = nf4 + threadIdx.x; e < TM * kgroups * 64; e += 256) dst[e] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();  // the only barrier: every wave reaches it before its tile loop

    float bq[TM][4];
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int oc = (mt * TM + tm) * 16 + 4 * g + r;
            bq[tm][r] = (bias && oc < M) ? bias[oc] : 0.f;
        }
    const int bytes_x = C * HW * 4;
    const int la = lane * 4;  // float offset of this lane's float4 in a k-group block

    for (int n = 0; n < p.n; n++) {
        const float *xn = x + (long long)n * C * HW;
        float *yn = y + (long long)n * M * OHW;
        const float *rn = res ? res + (long long)n * M * OHW : nullptr;
        for (int pt = blockIdx.x * 4 + wave; pt < tiles_p; pt += gridDim.x * 4) {
            int off[BV][9];
#pragma unroll
            for (int q = 0; q < BV; q++) {
                int pix = pt * 16 * BV + BV * j + q;
                pix = pix < OHW ? pix : OHW - 1;
                const int oy = pix / p.ow, ox = pix - oy * p.ow;
                const int iy0 = oy * p.sh - p.pt, ix0 = ox * p.sw - p.pl;
#pragma unroll
                for (int ky = 0; ky < 3; ky++)
#pragma unroll
                    for (int kx = 0; kx < 3; kx++) {
                        const int iy = iy0 + ky, ix = ix0 + kx;
                        const bool ok = (unsigned)iy < (unsigned)p.h && (unsigned)ix < (unsigned)p.w;
                        off[q][ky * 3 + kx] = ok ? (g * HW + iy * p.w + ix) * 4 : (int)C16_OOB;
                    }
            }
            f32x4 acc[TM][BV];
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int q = 0; q < BV; q++)
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[tm][q][r] = bq[tm][r];

            auto load = [&](C16Chunk<TM, BV> &R, int c) {
                __amdgpu_buffer_rsrc_t rx =
                    __builtin_amdgcn_make_buffer_rsrc((void *)xn, (short)0, bytes_x, 0x00020000);
                const int icb = c / 3, ky = c - icb * 3;
#pragma unroll
                for (int kx = 0; kx < 3; kx++) {
                    const int kg = icb * 9 + ky * 3 + kx;
#pragma unroll
                    for (int tm = 0; tm < TM; tm++)
                        R.a[kx][tm] = *reinterpret_cast<const float4 *>(&wl[(tm * kgroups + kg) * 256 + la]);
#pragma unroll
                    for (int s = 0; s < 4; s++)
#pragma unroll
                        for (int q = 0; q < BV; q++)
                            R.b[kx][s][q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                                rx, off[q][ky * 3 + kx], (icb * 16 + 4 * s) * HW * 4, 0));
                }
            };
            auto compute = [&](const C16Chunk<TM, BV> &R) {
#pragma unroll
                for (int kx = 0; kx < 3; kx++)
#pragma unroll
                    for (int s = 0; s < 4; s++)
#pragma unroll
                        for (int tm = 0; tm < TM; tm++) {
                            const float4 &a4 = R.a[kx][tm];
                            const float a = s == 0 ? a4.x : s == 1 ? a4.y : s == 2 ? a4.z : a4.w;
#pragma unroll
                            for (int q = 0; q < BV; q++)
                                acc[tm][q] =
                                    __builtin_amdgcn_mfma_f32_16x16x4f32(a, R.b[kx][s][q], acc[tm][q], 0, 0, 0);
                        }
            };
            constexpr int L = 3 * 4 * BV;  // vector-memory loads per chunk (weights come from LDS)
            constexpr int D = 60 / L < 2 ? 2 : (60 / L > 4 ? 4 : 60 / L);
            const int nch = icbs * 3;
            const int last = nch - 1;
            C16Chunk<TM, BV> R[D];
#pragma unroll
            for (int d = 0; d < D; d++) load(R[d], min(d, last));
            int c = 0;
            for (; c + D <= nch; c += D) {
#pragma unroll
                for (int d = 0; d < D; d++) {
                    __builtin_amdgcn_sched_barrier(0);
                    compute(R[d]);
                    __builtin_amdgcn_sched_barrier(0);
                    load(R[d], min(c + d + D, last));
                }
            }
#pragma unroll
            for (int d = 0; d < D; d++)
                if (c + d < nch) compute(R[d]);

#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int oc = (mt * TM + tm) * 16 + 4 * g + r;
                    if (oc >= M) continue;
#pragma unroll
                    for (int q = 0; q < BV; q++) {
                        const int pix = pt * 16 * BV + BV * j + q;
                        if (pix < OHW) {
                            float v = activate<ACT>(acc[tm][q][r]);
                            if (rn) v += rn[(long long)oc * OHW + pix];
                            yn[(long long)oc * OHW + pix] = v;
                        }
                    }
                }
        }
    }
}

// Pack OIHW weights (T taps per channel) into
// [ceil(M/16)][C/16 * T k-groups][64 lanes][4 steps]: lane (j, g), step s of
// k-group (icb, tap) holds w[16 mb + j][16 icb + 4 s + g][tap] (zero for output
// channels past M).  With i2c (T = 9) the k-groups of a 16-channel block run
// through its 144 (channel, tap) terms in the im2col order instead: k-group t,
// step s holds local term 16 t + 4 s + g = 9 ic + tap.
static __global__ void conv16_pack_kernel(int M, int C, int T, const float *__restrict__ w, float *__restrict__ out,
                                          int i2c) {
    const long long kgroups = (long long)(C / 16) * T;
    const long long total = (long long)((M + 15) / 16) * kgroups * 256;
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int s = (int)(idx & 3);
    const int lane = (int)((idx >> 2) & 63);
    const long long t = idx >> 8;
    const int kg = (int)(t % kgroups);
    const int mb = (int)(t / kgroups);
    const int j = lane & 15, g = lane >> 4;
    const int icb = kg / T;
    int ic, tap;
    if (i2c) {
        const int term = 16 * (kg % T) + 4 * s + g;
        ic = icb * 16 + term / 9;
        tap = term % 9;
    } else {
        ic = icb * 16 + 4 * s + g;
        tap = kg % T;
    }
    const int oc = mb * 16 + j;
    out[idx] = oc < M ? w[((long long)oc * C + ic) * T + tap] : 0.f;
}

inline bool conv16_eligible(const osh_conv_params *p) {
    return p->group == 1 && p->kh == 3 && p->kw == 3 && p->dh == 1 && p->dw == 1 && p->c % 16 == 0 &&
           (long long)p->c * p->h * p->w * 4 < (1LL << 31) && (long long)p->m * p->oh * p->ow * 4 < (1LL << 31) &&
           (long long)((p->m + 15) / 16) * (p->c / 16) * 9 * 1024 < (1LL << 31) && p->n <= 65535;
}

inline size_t conv16_packed_bytes(const osh_conv_params *p) {
    return (size_t)((p->m + 15) / 16) * (p->c / 16) * p->kh * p->kw * 256 * sizeof(float);
}

inline osh_status conv16_pack(const osh_conv_params *p, const float *w, void *out, hipStream_t st,
                              bool i2c = false) {
    const long long total = (long long)conv16_packed_bytes(p) / 4;
    OSH_LAUNCH(conv16_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, p->m, p->c,
                       p->kh * p->kw, w, static_cast<float *>(out), i2c && p->kh * p->kw == 9 ? 1 : 0);
    OSH_LAUNCH_CHECK("conv16_pack_kernel");
    return OSH_OK;
}

// Tile choice: 16*TM output channels x 16*BV pixels per wave.  Prefer the
// shape whose waves fill the SIMDs in the fewest rounds of the longest chain;
// larger tiles load fewer operands per MFMA.
template <int TM, int BV, int WPB = 4, bool I2C = false>
inline osh_status conv16_launch_t(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                                  const float *res, int act, float *y, hipStream_t st) {
    const int ohw = p->oh * p->ow;
    const int tiles_p = ceil_div(ohw, 16 * BV);
    // output-channel tiles: TM 16-blocks each; the packed weights hold ceil(M/16) blocks
    const int mtiles = ceil_div(ceil_div(p->m, 16), TM);
    dim3 grid((unsigned)ceil_div(tiles_p, WPB), (unsigned)mtiles, (unsigned)p->n);
    OSH_DISPATCH_ACT(act, ACT,
                     OSH_LAUNCH((conv16_kernel<TM, BV, ACT, WPB, I2C>), grid, dim3(64 * WPB), 0, st, *p, x, w,
                                        bias, res, y, tiles_p));
    OSH_LAUNCH_CHECK("conv16_kernel");
    return OSH_OK;
}

template <int TM, int BV>
inline osh_status conv16l_launch_t(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                                   const float *res, int act, float *y, hipStream_t st) {
    const int ohw = p->oh * p->ow;
    const int tiles_p = ceil_div(ohw, 16 * BV);
    const int mtiles = ceil_div(ceil_div(p->m, 16), TM);
    // persistent: about one workgroup per CU in total, each walking pixel tiles
    int per = ceil_div(device_cus(), mtiles);
    per = per < 1 ? 1 : per;
    per = per > ceil_div(tiles_p, 4) ? ceil_div(tiles_p, 4) : per;
    dim3 grid((unsigned)per, (unsigned)mtiles, 1);
    OSH_DISPATCH_ACT(act, ACT,
                     OSH_LAUNCH((conv16l_kernel<TM, BV, ACT>), grid, dim3(256), 0, st, *p, x, w, bias, res,
                                        y, tiles_p));
    OSH_LAUNCH_CHECK("conv16l_kernel");
    return OSH_OK;
}

struct C16Variant {
    int tm, bv, lds;
};
// 0-5: weights streamed from L2 per wave; 6-11: weights resident in LDS (TM * C <= 256)
constexpr C16Variant kC16[] = {{1, 1, 0}, {2, 1, 0}, {4, 1, 0}, {1, 2, 0}, {2, 2, 0}, {4, 2, 0},
                               {1, 1, 1}, {2, 1, 1}, {4, 1, 1}, {1, 2, 1}, {2, 2, 1}, {4, 2, 1}};
constexpr int kC16Count = sizeof(kC16) / sizeof(kC16[0]);

// The same streamed tiles with one wave per workgroup (WPB = 1).
constexpr C16Variant kC16w[] = {{1, 1, 0}, {1, 2, 0}, {2, 1, 0}, {2, 2, 0}};
constexpr int kC16wCount = sizeof(kC16w) / sizeof(kC16w[0]);

osh_status conv16w_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                          const float *res, int act, float *y, hipStream_t st, int v);

// Predicted cost: rounds of waves over the SIMDs times the MFMAs of one wave,
// inflated by its operand loads per MFMA (TM/4 weight loads and BV input
// loads feed TM*BV MFMAs per k4 step).
inline bool conv16_fits(const osh_conv_params *p, const C16Variant &v) {
    return !v.lds || (size_t)v.tm * (p->c / 16) * 9 * 256 * sizeof(float) <= (size_t)CONV16L_LDS;
}

inline double conv16_cost(const osh_conv_params *p, const C16Variant &v, int cus) {
    const long long tiles_p = ceil_div(p->oh * p->ow, 16 * v.bv);
    const long long mtiles = ceil_div(ceil_div(p->m, 16), v.tm);
    const long long waves = tiles_p * mtiles * p->n;
    const long long rounds = (waves + 4LL * cus - 1) / (4LL * cus);
    const double u = (double)v.tm * v.bv;
    // LDS weights remove the per-wave weight stream (TM/4 loads per step)
    const double loads = v.lds ? v.bv : v.tm / 4.0 + v.bv;
    return rounds * u * (9.0 * p->c / 4) * (1.0 + 0.6 * loads / u);
}

osh_status conv16_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                         const float *res, int act, float *y, hipStream_t st, int forced);

}  // namespace osh
