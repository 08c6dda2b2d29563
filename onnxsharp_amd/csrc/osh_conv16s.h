// osh_conv16s.h -- 3x3 convolution with the input patch staged in LDS: the
// same in-order 16x16x4 MFMA chain as osh_conv16.h (bias, then
// icb -> ky -> kx -> four steps of four channels; NchwcConv.Row,
// src/OnnxSharp/Kernels/NchwcConv.cs:533-605), so the same bits, with the
// operand traffic reorganised for small and mid-size maps:
//
//   * a workgroup's four waves share one output-pixel tile and take four
//     different 16*TM-channel output blocks, so the input patch of the tile is
//     read from memory once per workgroup, not once per wave;
//   * per 16-channel input block the patch ((TH-1)*S+3 rows x (TWL-1)*S+3
//     columns x 16 channels) is copied to LDS by all 256 threads, one element
//     each per pass: block icb+2 is fetched into registers and block icb+1
//     written to the second LDS buffer while block icb is multiplied;
//   * the tile is 2-D: a 16-lane MFMA column group covers (16/TWL) rows x TWL
//     columns, and BV such groups are stacked vertically, so narrow maps
//     (20, 40 wide) waste no lanes;
//   * B comes from LDS (one ds_read_b32 per step and pixel group at a
//     compile-time offset from the lane's base); A (weights, packed as for
//     conv16_kernel) from global memory with 16-byte loads, one block ahead.
// Row pitch and channel-plane pitch of the patch are padded so that the 32
// lanes of each half-wave LDS read fall in distinct banks.
//
// I2C runs the same tiles in the im2col order (bias, then ic -> ky -> kx:
// ConvKernels.Im2Col and PackedConv, src/OnnxSharp/Kernels/ConvKernels.cs:554-563,
// PackedConv.cs:420-440), the reference's chain for the 3x3 layers its NCHWc
// gate refuses: a 16-channel block holds 144 consecutive terms of that chain
// either way, so only the order within a block changes.  Step u of a block
// gives lane group g the term 4u + g = 9 ic + tap; with u = 9 v + r its channel
// is 4 v + (4 r + g) / 9, so each lane keeps nine patch offsets (one per r)
// and the rest of the address is a compile-time constant.  The weights are
// packed in the same order (conv16_pack with i2c).
#pragma once

#include "osh_conv16.h"

namespace osh {

// Whether lane groups g = 0 and 1 (one half-wave) of an LDS read at row
// pitch `pitch` and channel-plane pitch `plane` fall in 32 distinct banks.
constexpr bool c16s_conflict_free(int pitch, int plane, int twl, int s) {
    bool used[32] = {};
    for (int g = 0; g < 2; g++)
        for (int j = 0; j < 16; j++) {
            const int b = (g * plane + (j / twl) * s * pitch + (j % twl) * s) % 32;
            if (used[b]) return false;
            used[b] = true;
        }
    return true;
}

// Smallest channel-plane pitch in [base, base + 32) that is conflict-free at
// this row pitch, or -1.
constexpr int c16s_plane_for(int base, int pitch, int twl, int s) {
    for (int pl = base; pl < base + 32; pl++)
        if (c16s_conflict_free(pitch, pl, twl, s)) return pl;
    return -1;
}

// Smallest row pitch in [pc, pc + 32) that admits a conflict-free plane pitch
// (pc itself if none does: the reads then take an extra pass).
constexpr int c16s_pitch(int pc, int pr, int twl, int s) {
    for (int p = pc; p < pc + 32; p++)
        if (c16s_plane_for(pr * p, p, twl, s) >= 0) return p;
    return pc;
}

constexpr int c16s_plane(int pr, int pitch, int twl, int s) {
    return c16s_plane_for(pr * pitch, pitch, twl, s) >= 0 ? c16s_plane_for(pr * pitch, pitch, twl, s) : pr * pitch;
}

// KS x KS kernel (3, or 1 for pointwise), stride S, CB 16-channel blocks per
// staged chunk.
template <int TM, int BV, int TWL, int S, int KS, int CB, bool VEC = false>
struct C16sGeom {
    static constexpr int T = KS * KS;                             // taps
    static constexpr int THL = 16 / TWL;                          // rows per lane group
    static constexpr int TH = THL * BV;                           // tile rows
    static constexpr int PR = (TH - 1) * S + KS;                  // patch rows
    static constexpr int PC = (TWL - 1) * S + KS;                 // patch columns
    static constexpr int PITCH = c16s_pitch(PC, PR, TWL, S);      // floats per patch row
    static constexpr int PLANE = c16s_plane(PR, PITCH, TWL, S);   // floats per channel
    static constexpr int CHUNK = 16 * CB * PLANE;                 // one chunk of CB channel blocks
    static constexpr int ELEMS = 16 * CB * PR * PC;               // patch elements per chunk
    static constexpr int VW = VEC ? 4 : 1;                        // elements per staging load
    static constexpr int NE = (ELEMS / VW + 255) / 256;           // staging loads per thread
    static constexpr int NA = CB * T;                             // weight k-groups per chunk
};

// VEC: the patch is staged with 16-byte loads of four adjacent columns (a
// 1x1 stride-1 kernel on a map with W % 4 == 0 and a 16-byte aligned input).
// XB: workgroups take their tiles XCD-banded (xcd_band), so that the tiles
// one XCD runs are neighbours whose patches share halo lines in its L2.
// One workgroup's tile (bx: pixel tile, by: group of four 16*TM-channel
// output blocks, bz: image) of the conv p.
template <int TM, int BV, int TWL, int S, int KS, int CB, bool VEC, int ACT, bool I2C>
__device__ __forceinline__ void conv16s_tile(const osh_conv_params &p, const float *__restrict__ x,
                                             const float *__restrict__ wpk, const float *__restrict__ bias,
                                             const float *__restrict__ res, float *__restrict__ y, int tiles_w,
                                             const int bx, const int by, const int bz) {
    using G = C16sGeom<TM, BV, TWL, S, KS, CB, VEC>;
    static_assert(16 % TWL == 0, "a lane group covers whole rows of the tile");
    static_assert(!VEC || (KS == 1 && S == 1 && G::PC % 4 == 0 && G::PITCH % 4 == 0 && G::PLANE % 4 == 0),
                  "16-byte staging needs whole, aligned four-column groups");
    static_assert(!I2C || KS == 3, "the im2col order differs from the NCHWc order only for 3x3 kernels");
    __shared__ __align__(16) float lds[2 * G::CHUNK];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int ty = bx / tiles_w, tx = bx - ty * tiles_w;
    const int oy0 = ty * G::TH, ox0 = tx * TWL;
    const int n = bz;
    const int HW = p.h * p.w, OHW = p.oh * p.ow;
    const int C = p.c, M = p.m;
    const int icbs = C / 16;
    const int kgroups = icbs * G::T;
    const int nchunks = (icbs + CB - 1) / CB;
    const int mb0 = (by * 4 + wave) * TM;               // first 16-channel output block of this wave
    const bool active = mb0 * 16 < M;                    // uniform per wave
    const float *xn = x + (long long)n * C * HW;
    const int iy0 = oy0 * S - p.pt, ix0 = ox0 * S - p.pl;

    // staging: element e = tid + 256 i of a chunk -> (channel, patch row, patch column);
    // channels past C (a partial last chunk) lie past the buffer and read 0
    // (with VEC, e counts groups of four columns; out-of-image groups lie wholly
    // outside because W % 4 == 0 and tiles start at multiples of four)
    constexpr int PCV = G::PC / G::VW;
    int goff[G::NE], loff[G::NE];
#pragma unroll
    for (int i = 0; i < G::NE; i++) {
        const int e = tid + 256 * i;
        const int ch = e / (G::PR * PCV), rem = e - ch * (G::PR * PCV);
        const int r = rem / PCV, c = (rem - r * PCV) * G::VW;
        const int iy = iy0 + r, ix = ix0 + c;
        const bool in = e < G::ELEMS / G::VW;
        const bool ok = in && (unsigned)iy < (unsigned)p.h && (unsigned)ix < (unsigned)p.w;
        goff[i] = ok ? (ch * HW + iy * p.w + ix) * 4 : (int)C16_OOB;
        loff[i] = in ? ch * G::PLANE + r * G::PITCH + c : -1;
    }
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void *)xn, (short)0, C * HW * 4, 0x00020000);
    // two register sets: a chunk's patch is fetched two chunks before it is
    // multiplied and written to LDS one chunk before
    float sv0[G::NE * G::VW], sv1[G::NE * G::VW];
    auto stage_load = [&](float (&sv)[G::NE * G::VW], int chunk) {
        const int soff = chunk * CB * 16 * HW * 4;
#pragma unroll
        for (int i = 0; i < G::NE; i++) {
            if constexpr (VEC) {
                auto v = __builtin_amdgcn_raw_buffer_load_b128(rx, goff[i], soff, 0);
#pragma unroll
                for (int u = 0; u < 4; u++) sv[4 * i + u] = __uint_as_float(v[u]);
            } else {
                sv[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, goff[i], soff, 0));
            }
        }
    };
    auto stage_store = [&](const float (&sv)[G::NE * G::VW], int buf) {
#pragma unroll
        for (int i = 0; i < G::NE; i++) {
            if (loff[i] < 0) continue;
            if constexpr (VEC)
                *reinterpret_cast<float4 *>(lds + buf * G::CHUNK + loff[i]) =
                    make_float4(sv[4 * i], sv[4 * i + 1], sv[4 * i + 2], sv[4 * i + 3]);
            else
                lds[buf * G::CHUNK + loff[i]] = sv[i];
        }
    };

    // A: packed [mblock16][icb*T + tap][64 lanes][4 steps]; k-groups past the
    // last block lie past the buffer and read 0
    const int bytes_w = ((M + 15) / 16) * kgroups * 64 * 16;
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void *)wpk, (short)0, bytes_w, 0x00020000);
    int voa[TM];
#pragma unroll
    for (int tm = 0; tm < TM; tm++) voa[tm] = (((mb0 + tm) * kgroups) * 64 + lane) * 16;
    float4 A0[G::NA][TM], A1[G::NA][TM];
    auto load_a = [&](float4 (&A)[G::NA][TM], int chunk) {
#pragma unroll
        for (int t = 0; t < G::NA; t++)
#pragma unroll
            for (int tm = 0; tm < TM; tm++) {
                auto v = __builtin_amdgcn_raw_buffer_load_b128(rw, voa[tm], (chunk * G::NA + t) * 1024, 0);
                A[t][tm] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                                       __uint_as_float(v[3]));
            }
    };

    f32x4 acc[TM][BV];
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int oc = (mb0 + tm) * 16 + 4 * g + r;
            const float b = (bias && oc < M) ? bias[oc] : 0.f;
#pragma unroll
            for (int q = 0; q < BV; q++) acc[tm][q][r] = b;
        }

    // the lane's pixel (row j / TWL + THL q, column j % TWL) in patch coordinates
    const int lbase = g * G::PLANE + (j / TWL) * S * G::PITCH + (j % TWL) * S;
    // im2col order: the lane's patch offset of term 4 r + g (r = 0..8) of a
    // group of four channels
    int i2c_off[I2C ? 9 : 1];
    if constexpr (I2C) {
#pragma unroll
        for (int r = 0; r < 9; r++) {
            const int term = 4 * r + g, tap = term % 9;
            i2c_off[r] = (term / 9) * G::PLANE + (tap / 3) * G::PITCH + tap % 3 + lbase - g * G::PLANE;
        }
    }
    // B operand of k-group t (block cb, tap or term group), step s, pixel block q
    auto bval = [&](const float *lbuf, int cb, int t, int s, int q) -> float {
        if constexpr (I2C) {
            const int u = 4 * (t - cb * G::T) + s, v = u / 9, r = u - 9 * v;
            return lbuf[(16 * cb + 4 * v) * G::PLANE + G::THL * q * S * G::PITCH + i2c_off[r]];
        } else {
            const int tap = t - cb * G::T;
            const int ky = tap / KS, kx = tap - KS * (tap / KS);
            return lbuf[lbase + (16 * cb + 4 * s) * G::PLANE + (G::THL * q * S + ky) * G::PITCH + kx];
        }
    };
    // 3x3 tiles of four or more pixel blocks run each chunk with the B
    // operands read two k4 steps ahead and each step's reads issued just
    // before its MFMAs (pinned by scheduling barriers), instead of the
    // compiler's bursts of reads that the MFMAs then wait for: 3x3 64 -> 64
    // at 160x160 21.9 -> 21.2 us.  Tiles with one or two blocks (one or two
    // dependent chains per wave) ran slower so (3x3 s2 128 -> 256 at 80x80:
    // 14.5 -> 16.4 us) and keep the compiler's order.
    constexpr bool kPinnedReads = KS == 3 && CB == 1 && !I2C && BV >= 4;
    auto compute_pinned = [&](const float4 (&A)[G::NA][TM], const float *lb) {
        constexpr int NS = G::NA * 4, D = 2;
        float br[D][BV];
#pragma unroll
        for (int u = 0; u < D; u++)
#pragma unroll
            for (int q = 0; q < BV; q++) br[u][q] = bval(lb, 0, u / 4, u % 4, q);
#pragma unroll
        for (int u = 0; u < NS; u++) {
            const int t = u / 4, s = u % 4;
            float b[BV];
#pragma unroll
            for (int q = 0; q < BV; q++) b[q] = br[u % D][q];
            if (u + D < NS) {
#pragma unroll
                for (int q = 0; q < BV; q++) br[u % D][q] = bval(lb, 0, (u + D) / 4, (u + D) % 4, q);
            }
#pragma unroll
            for (int tm = 0; tm < TM; tm++) {
                const float4 &a4 = A[t][tm];
                const float a = s == 0 ? a4.x : s == 1 ? a4.y : s == 2 ? a4.z : a4.w;
#pragma unroll
                for (int q = 0; q < BV; q++)
                    acc[tm][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b[q], acc[tm][q], 0, 0, 0);
            }
            if (u + D < NS) __builtin_amdgcn_sched_group_barrier(0x100, BV, 0);  // the step's reads
            __builtin_amdgcn_sched_group_barrier(0x008, TM * BV, 0);               // then its MFMAs
        }
    };
    // a partial last chunk skips its missing channel blocks (no extra terms
    // enter the chain)
    auto compute = [&](const float4 (&A)[G::NA][TM], int buf, int chunk) {
        const float *lb = lds + buf * G::CHUNK;
        if constexpr (kPinnedReads) {
            compute_pinned(A, lb);
            return;
        }
#pragma unroll
        for (int t = 0; t < G::NA; t++) {
            const int cb = t / G::T;
            if (CB > 1 && chunk * CB + cb >= icbs) break;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                float b[BV];
#pragma unroll
                for (int q = 0; q < BV; q++) b[q] = bval(lb, cb, t, s, q);
#pragma unroll
                for (int tm = 0; tm < TM; tm++) {
                    const float4 &a4 = A[t][tm];
                    const float a = s == 0 ? a4.x : s == 1 ? a4.y : s == 2 ? a4.z : a4.w;
#pragma unroll
                    for (int q = 0; q < BV; q++)
                        acc[tm][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b[q], acc[tm][q], 0, 0, 0);
                }
            }
        }
    };

    // lane (j, g) holds output channels 4g + r of pixel column j of block q
    float *yn = y + (long long)n * M * OHW;
    const float *rn = res ? res + (long long)n * M * OHW : nullptr;
    auto store_block = [&](int q) {
        const int oy = oy0 + j / TWL + G::THL * q, ox = ox0 + j % TWL;
        if (oy >= p.oh || ox >= p.ow) return;
        const int pix = oy * p.ow + ox;
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int oc = (mb0 + tm) * 16 + 4 * g + r;
                if (oc >= M) continue;
                float v = activate<ACT>(acc[tm][q][r]);
                if (rn) v += rn[(long long)oc * OHW + pix];
                yn[(long long)oc * OHW + pix] = v;
            }
    };
    // For 3x3 tiles with BV <= 2 the last chunk runs the pixel blocks one
    // after another (one chain issues at the MFMA pipe's own rate) and stores
    // each block as soon as its chain ends, so the output stores drain under
    // the other block's MFMAs instead of in one burst after them (128 -> 256
    // s2 at 80x80: 15.1 -> 14.65 us).  Wider tiles keep their blocks
    // interleaved (64 -> 64 at 160x160 rose from 23.4 to 25.3 us run block by
    // block) and store after the loop, as do the pointwise tiles (slower
    // block by block too).
    auto compute_last = [&](const float4 (&A)[G::NA][TM], int buf, int chunk) {
        const float *lb = lds + buf * G::CHUNK;
#pragma unroll
        for (int q = 0; q < BV; q++) {
#pragma unroll
            for (int t = 0; t < G::NA; t++) {
                const int cb = t / G::T;
                if (CB > 1 && chunk * CB + cb >= icbs) break;
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const float b = bval(lb, cb, t, s, q);
#pragma unroll
                    for (int tm = 0; tm < TM; tm++) {
                        const float4 &a4 = A[t][tm];
                        const float a = s == 0 ? a4.x : s == 1 ? a4.y : s == 2 ? a4.z : a4.w;
                        acc[tm][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[tm][q], 0, 0, 0);
                    }
                }
            }
            store_block(q);
        }
    };

    if constexpr (KS == 1 && CB >= 8) {
        // a pointwise tile with CB >= 8 takes all of C in one chunk (the
        // launch checks C <= 16 CB): the patch and every weight block are in
        // flight together, one barrier, then the whole chain
        stage_load(sv0, 0);
        if (active) load_a(A0, 0);
        stage_store(sv0, 0);
        __syncthreads();
        if (!active) return;
        compute(A0, 0, 0);
#pragma unroll
        for (int q = 0; q < BV; q++) store_block(q);
        return;
    }
    // prologue: block 0 in LDS, block 1 in flight, block 0's weights loaded
    const int last = nchunks - 1;
    stage_load(sv0, 0);
    if (active) load_a(A0, 0);
    stage_store(sv0, 0);
    stage_load(sv1, min(1, last));
    __syncthreads();
    // trip k multiplies block k from LDS buffer k % 2 with weight set k % 2,
    // fetches block k + 2 into register set k % 2 and block k + 1's weights,
    // and writes block k + 1 (fetched during trip k - 1) into the other LDS
    // buffer.  Two trips per loop pass keep every set in fixed registers;
    // prefetch indices are clamped (reloads of the last block, never stored
    // past the patch) and every wave runs the same trips and barriers.
    for (int icb = 0; icb < nchunks; icb += 2) {
        stage_load(sv0, min(icb + 2, last));
        if (active) {
            load_a(A1, min(icb + 1, last));
            if (BV <= 2 && KS == 3 && icb == last) compute_last(A0, 0, icb);
            else compute(A0, 0, icb);
        }
        stage_store(sv1, 1);
        __syncthreads();
        if (icb + 1 >= nchunks) break;
        stage_load(sv1, min(icb + 3, last));
        if (active) {
            load_a(A0, min(icb + 2, last));
            if (BV <= 2 && KS == 3 && icb + 1 == last) compute_last(A1, 1, icb + 1);
            else compute(A1, 1, icb + 1);
        }
        stage_store(sv0, 0);
        __syncthreads();
    }
    // A 3x3 form that stages the whole patch (every channel, up to 256) in
    // LDS behind a single barrier and then runs the chain with no further
    // barrier gave the same bits but ran slower (3x3 s2 128 -> 256 at 80x80:
    // 18.3-19.3 us against 15.1 for this pipeline; the frame's tuner picked
    // it for no layer): with nothing to multiply until the whole patch has
    // arrived, the fetch latency is exposed, and the larger LDS footprint
    // leaves fewer workgroups per CU to hide it.
    if constexpr (BV > 2 || KS != 3) {
        if (!active) return;
#pragma unroll
        for (int q = 0; q < BV; q++) store_block(q);
    }
    // (otherwise compute_last has stored every block of an active wave)
}

// XB: workgroups take their tiles XCD-banded (an XCD runs a band of
// neighbouring pixel tiles of one channel group, whose patches share halo
// lines in its L2).  Banding with the channel groups of a pixel tile
// innermost instead (its four workgroups, which stage the same patch, on one
// XCD) measured slower on every shape tried (3x3 s2 128 -> 256 at 80x80:
// 16.3 us against 14.7-15.0 in launch order) and the frame's tuner never
// picked it, so it is not offered.
template <int TM, int BV, int TWL, int S, int KS, int CB, bool VEC, int ACT, bool XB = false, bool I2C = false>
__global__ __launch_bounds__(256) void conv16s_kernel(osh_conv_params p, const float *__restrict__ x,
                                                      const float *__restrict__ wpk, const float *__restrict__ bias,
                                                      const float *__restrict__ res, float *__restrict__ y,
                                                      int tiles_w) {
    int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
    if constexpr (XB) {
        const int wg = xcd_band(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z),
                                gridDim.x * gridDim.y * gridDim.z);
        bx = wg % gridDim.x, by = (wg / gridDim.x) % gridDim.y, bz = wg / (gridDim.x * gridDim.y);
    }
    conv16s_tile<TM, BV, TWL, S, KS, CB, VEC, ACT, I2C>(p, x, wpk, bias, res, y, tiles_w, bx, by, bz);
}

// Several independent convs of one tile shape in one launch (e.g. a
// detection head's three scales): workgroup b runs tile b - start[i] of conv
// i, start[i] <= b < start[i + 1], with conv i's own sizes and pointers.
// Every conv keeps its own chain, so the outputs are those of separate
// launches with the same tile.
constexpr int kConvGroupMax = 6;
struct ConvGroup {
    int count;
    int start[kConvGroupMax + 1];
    int tiles_w[kConvGroupMax], tiles[kConvGroupMax], mgroups[kConvGroupMax];
    osh_conv_params p[kConvGroupMax];
    const float *x[kConvGroupMax];
    const float *w[kConvGroupMax];
    const float *bias[kConvGroupMax];
    const float *res[kConvGroupMax];
    float *y[kConvGroupMax];
};

template <int TM, int BV, int TWL, int S, int KS, int CB, bool VEC, int ACT>
__global__ __launch_bounds__(256) void conv16s_group_kernel(ConvGroup g) {
    const int b = blockIdx.x;
    int i = 0;
    while (i + 1 < g.count && b >= g.start[i + 1]) i++;
    const int local = b - g.start[i];
    const int bx = local % g.tiles[i], rest = local / g.tiles[i];
    conv16s_tile<TM, BV, TWL, S, KS, CB, VEC, ACT, false>(g.p[i], g.x[i], g.w[i], g.bias[i], g.res[i], g.y[i],
                                                          g.tiles_w[i], bx, rest % g.mgroups[i],
                                                          rest / g.mgroups[i]);
}

// Fills the block table of g for tile <TM, BV, TWL> and launches it.  With
// `exclusive`, every workgroup also reserves more than half of a CU's LDS, so
// no two workgroups share a CU: a member with a long chain then keeps its
// SIMDs' MFMA pipes to itself instead of sharing them with the waves of
// other members that would otherwise be placed on the same CU.
constexpr int kConvGroupExclusiveLds = 84 * 1024;  // > 160 KB / 2 with any tile's own LDS
template <int TM, int BV, int TWL, int S, int KS, int CB, bool VEC>
inline osh_status conv16s_group_launch_t(ConvGroup g, int act, hipStream_t st, bool exclusive = false) {
    using G = C16sGeom<TM, BV, TWL, S, KS, CB, VEC>;
    long long total = 0;
    for (int i = 0; i < g.count; i++) {
        const osh_conv_params &p = g.p[i];
        g.tiles_w[i] = ceil_div(p.ow, TWL);
        g.tiles[i] = g.tiles_w[i] * ceil_div(p.oh, G::TH);
        g.mgroups[i] = ceil_div(ceil_div(p.m, 16), 4 * TM);
        g.start[i] = (int)total;
        total += (long long)g.tiles[i] * g.mgroups[i] * p.n;
    }
    if (total > 0x7fffffffLL) return fail(OSH_E_UNSUPPORTED, "Conv group: grid too large");
    g.start[g.count] = (int)total;
    OSH_DISPATCH_ACT(act, ACT,
                     OSH_LAUNCH((conv16s_group_kernel<TM, BV, TWL, S, KS, CB, VEC, ACT>),
                                        dim3((unsigned)total), dim3(256), exclusive ? kConvGroupExclusiveLds : 0,
                                        st, g));
    OSH_LAUNCH_CHECK("conv16s_group_kernel");
    return OSH_OK;
}

// Grouped 3x3 convs on the streamed one-block tiles (conv16_wave): workgroup
// b runs WPB waves of conv i = the member whose block-table range holds b,
// each wave its own 16*BV-pixel, 16*TM-channel tile with no barriers.  On the
// head's small maps one chain per wave loses less to staging than the
// LDS-patch tiles' barrier per 16-channel chunk.
template <int TM, int BV, int ACT, int WPB>
__global__ __launch_bounds__(256) void conv16_group_kernel(ConvGroup g) {
    const int b = blockIdx.x;
    int i = 0;
    while (i + 1 < g.count && b >= g.start[i + 1]) i++;
    const int local = b - g.start[i];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int bx = local % g.tiles[i], rest = local / g.tiles[i];
    const int pt = bx * WPB + wave;
    if (pt >= g.tiles_w[i]) return;  // tiles_w holds the member's pixel tiles
    conv16_wave<TM, BV, ACT>(g.p[i], g.x[i], g.w[i], g.bias[i], g.res[i], g.y[i], pt, rest % g.mgroups[i],
                             rest / g.mgroups[i]);
}

template <int TM, int BV, int WPB>
inline osh_status conv16_group_launch_t(ConvGroup g, int act, hipStream_t st) {
    long long total = 0;
    for (int i = 0; i < g.count; i++) {
        const osh_conv_params &p = g.p[i];
        g.tiles_w[i] = ceil_div(p.oh * p.ow, 16 * BV);  // pixel tiles
        g.tiles[i] = ceil_div(g.tiles_w[i], WPB);       // workgroups per channel tile
        g.mgroups[i] = ceil_div(ceil_div(p.m, 16), TM);
        g.start[i] = (int)total;
        total += (long long)g.tiles[i] * g.mgroups[i] * p.n;
    }
    if (total > 0x7fffffffLL) return fail(OSH_E_UNSUPPORTED, "Conv group: grid too large");
    g.start[g.count] = (int)total;
    OSH_DISPATCH_ACT(act, ACT,
                     OSH_LAUNCH((conv16_group_kernel<TM, BV, ACT, WPB>), dim3((unsigned)total),
                                        dim3(64 * WPB), 0, st, g));
    OSH_LAUNCH_CHECK("conv16_group_kernel");
    return OSH_OK;
}
// the streamed group tiles {TM, BV, waves per workgroup}
constexpr int kC16gCount = 4;

struct C16sVariant {
    int tm, bv, twl;
};
constexpr C16sVariant kC16s[] = {{1, 1, 16}, {1, 2, 16}, {1, 4, 16}, {2, 2, 16}, {1, 1, 8}, {1, 2, 8},
                                 {2, 2, 8},  {1, 2, 4},  {1, 4, 4},  {1, 4, 8},  {2, 4, 8}};
constexpr int kC16sCount = sizeof(kC16s) / sizeof(kC16s[0]);

// Stride 1 or 2 in both directions (the patch geometry is compile-time).
inline bool conv16s_eligible(const osh_conv_params *p) {
    return conv16_eligible(p) && p->sh == p->sw && (p->sh == 1 || p->sh == 2);
}

template <int TM, int BV, int TWL, int S, int KS, int CB, bool VEC, bool XB = false, bool I2C = false>
inline osh_status conv16s_launch_t(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                                   const float *res, int act, float *y, hipStream_t st) {
    using G = C16sGeom<TM, BV, TWL, S, KS, CB, VEC>;
    const int tiles_w = ceil_div(p->ow, TWL), tiles_h = ceil_div(p->oh, G::TH);
    const int mgroups = ceil_div(ceil_div(p->m, 16), 4 * TM);
    dim3 grid((unsigned)(tiles_w * tiles_h), (unsigned)mgroups, (unsigned)p->n);
    OSH_DISPATCH_ACT(act, ACT,
                     OSH_LAUNCH((conv16s_kernel<TM, BV, TWL, S, KS, CB, VEC, ACT, XB, I2C>), grid, dim3(256),
                                        0, st, *p, x, w, bias, res, y, tiles_w));
    OSH_LAUNCH_CHECK("conv16s_kernel");
    return OSH_OK;
}

template <int TM, int BV, int TWL, bool XB = false, bool I2C = false>
inline osh_status conv16s_launch_s(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                                   const float *res, int act, float *y, hipStream_t st) {
    if (p->sh == 1) return conv16s_launch_t<TM, BV, TWL, 1, 3, 1, false, XB, I2C>(p, x, w, bias, res, act, y, st);
    return conv16s_launch_t<TM, BV, TWL, 2, 3, 1, false, XB, I2C>(p, x, w, bias, res, act, y, st);
}

// The kC16s tiles in the im2col order (weights packed by conv16_pack with i2c).
osh_status conv16si_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                           const float *res, int act, float *y, hipStream_t st, int v);
// Streamed conv16 tiles in the im2col order (same packing): {TM, BV, waves
// per workgroup} = {1,1,1}, {1,1,4}, {1,2,1}, {2,1,1} -- every wave its own
// pixel tile, so a conv with 16 or fewer output channels idles no wave.
constexpr int kC16wiCount = 4;
osh_status conv16wi_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                           const float *res, int act, float *y, hipStream_t st, int v);

osh_status conv16s_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                          const float *res, int act, float *y, hipStream_t st, int v);

// XCD-banded versions of the 16-column tiles (ids after the one-wave tiles).
// BV = 7 and 8: taller tiles that spread a large map's 16x16 blocks evenly
// over the SIMDs (64 -> 64 at 160x160: 230 workgroups, one wave per SIMD with
// seven blocks, instead of 400 with four, two waves on 576 SIMDs).
constexpr C16sVariant kC16sx[] = {{1, 2, 16}, {1, 4, 16}, {2, 2, 16}, {1, 7, 16}, {1, 8, 16}};
constexpr int kC16sxCount = sizeof(kC16sx) / sizeof(kC16sx[0]);


osh_status conv16sx_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                           const float *res, int act, float *y, hipStream_t st, int v);

// ---- pointwise (1x1, stride 1, no pads): the same kernel with KS = 1 and
// CB 16-channel blocks per staged chunk; the chain is the GEMM chain over
// input channels (bias, then ic ascending), as GemmKernel.Multiply sums it.
// CB = 8 and 16 take all of C (at most 128 or 256 channels) in one chunk:
// the patch and every weight block of the wave are in flight at once and
// there is one barrier (256 -> 128 at 80x80: one chunk instead of four).
struct PW16Variant {
    int tm, bv, twl, cb;
};
constexpr PW16Variant kPW16[] = {{1, 1, 16, 4}, {1, 2, 16, 4}, {1, 4, 16, 4}, {2, 2, 16, 4}, {2, 4, 16, 4},
                                 {1, 2, 4, 4},  {1, 4, 4, 4},  {2, 4, 4, 4},  {1, 1, 16, 8}, {1, 1, 16, 16},
                                 {1, 2, 16, 8}, {1, 2, 16, 16}};
constexpr int kPW16Count = sizeof(kPW16) / sizeof(kPW16[0]);

// Whether pointwise tile `tile` takes a conv of p's input channels.
inline bool pw16_fits(const osh_conv_params *p, int tile) {
    return tile >= 0 && tile < kPW16Count && (kPW16[tile].cb < 8 || p->c <= 16 * kPW16[tile].cb);
}

inline bool pw16_eligible(const osh_conv_params *p) {
    return p->group == 1 && p->kh == 1 && p->kw == 1 && p->sh == 1 && p->sw == 1 && p->dh == 1 && p->dw == 1 &&
           p->pt == 0 && p->pl == 0 && p->oh == p->h && p->ow == p->w && p->c % 16 == 0 &&
           (long long)p->c * p->h * p->w * 4 < (1LL << 31) && (long long)p->m * p->oh * p->ow * 4 < (1LL << 31) &&
           (long long)((p->m + 15) / 16) * (p->c / 16) * 1024 < (1LL << 31) && p->n <= 65535;
}


osh_status pw16_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                       const float *res, int act, float *y, hipStream_t st, int v);

// The grouped launches (osh_conv2d_group_f32): the LDS-patch 3x3 tile `tile`
// (an index into kC16s) at stride s, or the pointwise LDS tile `tile` (an
// index into kPW16; `vec`: 16-byte input loads).
osh_status conv16s_group_launch(ConvGroup g, int act, hipStream_t st, int tile, int s);
osh_status pw16_group_launch(ConvGroup g, int act, hipStream_t st, int tile, bool vec);

}  // namespace osh
