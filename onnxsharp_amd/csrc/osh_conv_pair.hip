// osh_conv_pair.hip -- two chained 3x3 stride-1 convolutions (a bottleneck's
// cv1 -> cv2: ultralytics Bottleneck, two Conv nodes that the reference runs
// one after the other through ConvLayer.Forward, src/OnnxSharp/Ops/DnnOps.cs:411-500)
// in one launch.
//
// A workgroup owns a TH x TW tile of the second conv's output.  It computes
// the first conv over the tile and a one-pixel ring around it ((TH+2) x
// (TW+2) pixels, every channel) into LDS -- zero where the ring leaves the
// map, which is what the second conv's padding taps read -- and then the
// second conv from LDS.  The ring is computed again by the neighbouring tiles
// (the same values: every output is one lane's chain), so the intermediate
// tensor never makes a round trip through memory and the pair costs one
// launch.  Each workgroup also stores its own tile of the intermediate, so a
// reader of it sees what the two launches would have left.
//
// Both convs keep the reference's chains on the 16x16x4 MFMA: bias, then the
// NCHWc order (icb -> ky -> kx -> ic16, NchwcConv.cs:533-605) for 32 and 64
// output channels, or the im2col order (ic -> ky -> kx, ConvKernels.cs:554-563)
// for 16 -- the orders the reference's gate picks for these shapes at 1 x C x H
// x W (the host checks that the single-conv dispatch agrees).  Operands and
// packed weights are those of conv16_kernel / conv16s_kernel.
#include "osh_conv16.h"
#include "osh_conv_pair.h"

namespace osh {

// Bank-friendly pitches: rows padded to an odd count, planes to 16 mod 32
// words, so the four lane groups of a read (four channels or terms) fall in
// different bank ranges.
constexpr int pair_pitch(int w) { return w | 1; }
constexpr int pair_plane(int rows, int pitch) { return ((rows * pitch + 15) / 32) * 32 + 16; }

template <int TH, int TW, int CB1, int CB2>
struct PairGeom {
    static constexpr int EH = TH + 2, EW = TW + 2, NE = EH * EW;  // first conv's pixels (tile + ring)
    static constexpr int NBA = (NE + 15) / 16;                    // its 16-pixel blocks
    static constexpr int PH = TH + 4, PW = TW + 4;                // its input patch
    static constexpr int PITCH_X = pair_pitch(PW), PLANE_X = pair_plane(PH, PITCH_X);
    static constexpr int XCHUNK = 16 * PLANE_X;                   // one 16-channel chunk of the patch
    static constexpr int MAXCH = 4;                               // chunks staged at once (C0 <= 64)
    static constexpr int XE = 16 * PH * PW;
    static constexpr int NXE = (XE + 255) / 256;                  // staging loads per thread
    static constexpr int PITCH_M = pair_pitch(EW), PLANE_M = pair_plane(EH, PITCH_M);
    static constexpr int MSIZE = 16 * CB1 * PLANE_M;              // the intermediate
    static constexpr int NBB = (TH * TW + 15) / 16;               // output 16-pixel blocks
    // waves of one channel block step through the pixel blocks together
    static constexpr int WA = 4 / CB1, IA = (NBA + WA - 1) / WA;  // items (chains) per wave
    static constexpr int WB = 4 / CB2, IB = (NBB + WB - 1) / WB;
};

template <int TH, int TW, int CB1, int CB2, int ACT>
__global__ __launch_bounds__(256) void conv_pair_kernel(PairArgs a) {
    using G = PairGeom<TH, TW, CB1, CB2>;
    static_assert(CB1 == 1 || CB1 == 2 || CB1 == 4, "16, 32 or 64 intermediate channels");
    static_assert(CB2 == 1 || CB2 == 2 || CB2 == 4, "16, 32 or 64 output channels");
    constexpr bool I2CA = CB1 == 1, I2CB = CB2 == 1;
    __shared__ __align__(16) float lx[G::MAXCH * G::XCHUNK];
    __shared__ __align__(16) float lm[G::MSIZE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int ty = blockIdx.x / a.tiles_w, tx = blockIdx.x - ty * a.tiles_w;
    const int y0 = ty * TH, x0 = tx * TW;
    const int H = a.h, W = a.w, HW = H * W;
    const int nch = a.c0 / 16;  // 1 .. MAXCH
    const int cba = wave % CB1, pa0 = wave / CB1;  // first conv: channel block, first pixel block
    const int cbb = wave % CB2, pb0 = wave / CB2;  // second conv

    // ---- the first conv's whole input patch -- rows y0-2 .. y0+TH+1,
    // columns x0-2 .. x0+TW+1, every channel -- goes to LDS in one round
    // trip (outside the map the buffer load's offset is out of range and
    // returns 0): with few chunks, a chunk-by-chunk pipeline would wait for
    // each chunk's loads
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.x, (short)0, a.c0 * HW * 4, 0x00020000);
    int goff[G::NXE], loff[G::NXE];
#pragma unroll
    for (int i = 0; i < G::NXE; i++) {
        const int e = tid + 256 * i;
        const int ch = e / (G::PH * G::PW), rem = e - ch * (G::PH * G::PW);
        const int r = rem / G::PW, c = rem - r * G::PW;
        const int iy = y0 - 2 + r, ix = x0 - 2 + c;
        const bool ok = e < G::XE && (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
        goff[i] = ok ? (ch * HW + iy * W + ix) * 4 : (int)C16_OOB;
        loff[i] = e < G::XE ? ch * G::PLANE_X + r * G::PITCH_X + c : -1;
    }
    float sv[G::MAXCH][G::NXE];
#pragma unroll
    for (int k = 0; k < G::MAXCH; k++)
        if (k < nch)
#pragma unroll
            for (int i = 0; i < G::NXE; i++)
                sv[k][i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, goff[i], k * 16 * HW * 4, 0));

    // ---- first conv: wave -> channel block cba, pixel blocks pa0 + i * WA
    int basea[G::IA];
#pragma unroll
    for (int i = 0; i < G::IA; i++) {
        int e = (pa0 + i * G::WA) * 16 + j;
        e = e < G::NE ? e : G::NE - 1;  // lanes past the ring compute a duplicate, never stored
        const int ey = e / G::EW, ex = e - ey * G::EW;
        basea[i] = ey * G::PITCH_X + ex;
    }
    // im2col order: term 4u + g of a chunk (u = 9v + r) is channel 4v + (4r+g)/9, tap (4r+g)%9
    int i2ca[I2CA ? 9 : 1];
    if constexpr (I2CA) {
#pragma unroll
        for (int r = 0; r < 9; r++) {
            const int term = 4 * r + g, tap = term % 9;
            i2ca[r] = (term / 9) * G::PLANE_X + (tap / 3) * G::PITCH_X + tap % 3;
        }
    }
    const int kga = nch * 9;
    const __amdgpu_buffer_rsrc_t rwa =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.wa, (short)0, CB1 * kga * 1024, 0x00020000);
    const int voa = (cba * kga * 64 + lane) * 16;
    float4 wa0[9], wa1[9];
    auto load_wa = [&](float4 (&wv)[9], int chunk) {
#pragma unroll
        for (int t = 0; t < 9; t++) {
            auto v = __builtin_amdgcn_raw_buffer_load_b128(rwa, voa, (chunk * 9 + t) * 1024, 0);
            wv[t] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                                __uint_as_float(v[3]));
        }
    };
    load_wa(wa0, 0);
    if (nch > 1) load_wa(wa1, 1);
    // both biases, after the patch and the first weights (the second conv's
    // chain also starts from its bias), as buffer loads: a NULL bias is a
    // zero-sized buffer whose loads return 0, so no branch makes the loads
    // wait for one another
    float biasa[4], biasb[4];
    {
        const __amdgpu_buffer_rsrc_t rba =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.ba, (short)0, a.ba ? 64 * CB1 : 0, 0x00020000);
        const __amdgpu_buffer_rsrc_t rbb =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.bb, (short)0, a.bb ? 64 * CB2 : 0, 0x00020000);
        auto va = __builtin_amdgcn_raw_buffer_load_b128(rba, (cba * 16 + 4 * g) * 4, 0, 0);
        auto vb = __builtin_amdgcn_raw_buffer_load_b128(rbb, (cbb * 16 + 4 * g) * 4, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) biasa[r] = __uint_as_float(va[r]), biasb[r] = __uint_as_float(vb[r]);
    }
    // the residuals of the wave's output pixels, loaded now so that their
    // latency passes under both convs (out-of-map pixels and a NULL residual
    // read 0; the add in the epilogue happens only with a residual)
    float rv[G::IB][4];
    {
        const __amdgpu_buffer_rsrc_t rr =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.res, (short)0, a.res ? 16 * CB2 * HW * 4 : 0, 0x00020000);
#pragma unroll
        for (int i = 0; i < G::IB; i++) {
            const int o = (pb0 + i * G::WB) * 16 + j;
            const int oy = y0 + o / TW, ox = x0 + o % TW;
            const bool in = pb0 + i * G::WB < G::NBB && o < TH * TW && oy < H && ox < W;
#pragma unroll
            for (int r = 0; r < 4; r++)
                rv[i][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    rr, in ? ((cbb * 16 + 4 * g + r) * HW + oy * W + ox) * 4 : (int)C16_OOB, 0, 0));
        }
    }
    f32x4 acca[G::IA];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int i = 0; i < G::IA; i++) acca[i][r] = biasa[r];
    // B operands are read one tap ahead (four MFMA steps cover the LDS
    // latency): tap t's reads land in bv[t & 1] while tap t - 1 multiplies
    auto read_a = [&](float (&bv)[4][G::IA], const float *lb, int t) {
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < G::IA; i++) {
                if constexpr (I2CA) {
                    const int u = 4 * t + s, v = u / 9, r = u - 9 * v;
                    bv[s][i] = lb[4 * v * G::PLANE_X + i2ca[r] + basea[i]];
                } else {
                    bv[s][i] = lb[(4 * s + g) * G::PLANE_X + basea[i] + (t / 3) * G::PITCH_X + t % 3];
                }
            }
    };
    auto compute_a = [&](const float4 (&wv)[9], int chunk) {
        const float *lb = lx + chunk * G::XCHUNK;
        float bv[2][4][G::IA];
        read_a(bv[0], lb, 0);
#pragma unroll
        for (int t = 0; t < 9; t++) {
            if (t + 1 < 9) read_a(bv[(t + 1) & 1], lb, t + 1);
            __builtin_amdgcn_sched_barrier(0);  // the next tap's reads go out before this tap's MFMAs
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const float w4 = s == 0 ? wv[t].x : s == 1 ? wv[t].y : s == 2 ? wv[t].z : wv[t].w;
#pragma unroll
                for (int i = 0; i < G::IA; i++)
                    acca[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(w4, bv[t & 1][s][i], acca[i], 0, 0, 0);
            }
        }
    };
    // the patch into LDS (after the first weight sets went out)
#pragma unroll
    for (int k = 0; k < G::MAXCH; k++)
        if (k < nch)
#pragma unroll
            for (int i = 0; i < G::NXE; i++)
                if (loff[i] >= 0) lx[k * G::XCHUNK + loff[i]] = sv[k][i];
    // the weights of chunk k are in set k % 2, loaded two chunks ahead
    __syncthreads();
    for (int c = 0; c < nch; c += 2) {
        compute_a(wa0, c);
        if (c + 2 < nch) load_wa(wa0, c + 2);
        if (c + 1 < nch) {
            compute_a(wa1, c + 1);
            if (c + 3 < nch) load_wa(wa1, c + 3);
        }
    }

    // ---- second conv's weights, issued before the intermediate is written
    const int kgb = CB1 * 9;
    const __amdgpu_buffer_rsrc_t rwb =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.wb, (short)0, CB2 * kgb * 1024, 0x00020000);
    const int vob = (cbb * kgb * 64 + lane) * 16;
    float4 wb0[9], wb1[9];
    auto load_wb = [&](float4 (&wv)[9], int blk) {
#pragma unroll
        for (int t = 0; t < 9; t++) {
            auto v = __builtin_amdgcn_raw_buffer_load_b128(rwb, vob, (blk * 9 + t) * 1024, 0);
            wv[t] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                                __uint_as_float(v[3]));
        }
    };
    load_wb(wb0, 0);
    if (CB1 > 1) load_wb(wb1, 1);

    // ---- the intermediate: activation inside the map, 0 on the ring outside
    // it (its stores to ya come last: stores count in the same in-order
    // counter as the weight loads the second conv waits for)
#pragma unroll
    for (int i = 0; i < G::IA; i++) {
        const int e = (pa0 + i * G::WA) * 16 + j;
        if (pa0 + i * G::WA >= G::NBA || e >= G::NE) continue;
        const int ey = e / G::EW, ex = e - ey * G::EW;
        const int iy = y0 - 1 + ey, ix = x0 - 1 + ex;
        const bool in = (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int ch = cba * 16 + 4 * g + r;
            lm[ch * G::PLANE_M + ey * G::PITCH_M + ex] = in ? activate<ACT>(acca[i][r]) : 0.f;
        }
    }
    __syncthreads();

    // ---- second conv from LDS: wave -> channel block cbb, pixel blocks pbb(i)
    int baseb[G::IB];
#pragma unroll
    for (int i = 0; i < G::IB; i++) {
        int o = (pb0 + i * G::WB) * 16 + j;
        o = o < TH * TW ? o : TH * TW - 1;
        const int oy = o / TW, ox = o - oy * TW;
        baseb[i] = oy * G::PITCH_M + ox;
    }
    int i2cb[I2CB ? 9 : 1];
    if constexpr (I2CB) {
#pragma unroll
        for (int r = 0; r < 9; r++) {
            const int term = 4 * r + g, tap = term % 9;
            i2cb[r] = (term / 9) * G::PLANE_M + (tap / 3) * G::PITCH_M + tap % 3;
        }
    }
    f32x4 accb[G::IB];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int i = 0; i < G::IB; i++) accb[i][r] = biasb[r];
    auto read_b = [&](float (&bv)[4][G::IB], const float *lb, int t) {
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < G::IB; i++) {
                if constexpr (I2CB) {
                    const int u = 4 * t + s, v = u / 9, r = u - 9 * v;
                    bv[s][i] = lb[4 * v * G::PLANE_M + i2cb[r] + baseb[i]];
                } else {
                    bv[s][i] = lb[(4 * s + g) * G::PLANE_M + baseb[i] + (t / 3) * G::PITCH_M + t % 3];
                }
            }
    };
    auto compute_b = [&](const float4 (&wv)[9], int blk) {
        const float *lb = lm + blk * 16 * G::PLANE_M;
        float bv[2][4][G::IB];
        read_b(bv[0], lb, 0);
#pragma unroll
        for (int t = 0; t < 9; t++) {
            if (t + 1 < 9) read_b(bv[(t + 1) & 1], lb, t + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const float w4 = s == 0 ? wv[t].x : s == 1 ? wv[t].y : s == 2 ? wv[t].z : wv[t].w;
#pragma unroll
                for (int i = 0; i < G::IB; i++)
                    accb[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(w4, bv[t & 1][s][i], accb[i], 0, 0, 0);
            }
        }
    };
    // blocks two apart share a weight set; the next block's set is already
    // in flight (both first sets were issued before the intermediate)
#pragma unroll
    for (int blk = 0; blk < CB1; blk += 2) {
        compute_b(wb0, blk);
        if (blk + 2 < CB1) load_wb(wb0, blk + 2);
        if (blk + 1 < CB1) {
            compute_b(wb1, blk + 1);
            if (blk + 3 < CB1) load_wb(wb1, blk + 3);
        }
    }

    // ---- epilogue: activation, residual, store
#pragma unroll
    for (int i = 0; i < G::IB; i++) {
        const int o = (pb0 + i * G::WB) * 16 + j;
        if (pb0 + i * G::WB >= G::NBB || o >= TH * TW) continue;
        const int oy = y0 + o / TW, ox = x0 + o % TW;
        if (oy >= H || ox >= W) continue;
        const int pix = oy * W + ox;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int oc = cbb * 16 + 4 * g + r;
            float v = activate<ACT>(accb[i][r]);
            if (a.res) v += rv[i][r];
            a.y[oc * HW + pix] = v;
        }
    }
    // ---- the tile's own pixels of the intermediate, from LDS
    if (a.ya) {
        constexpr int OWN = 16 * CB1 * TH * TW;
        for (int e = tid; e < OWN; e += 256) {
            const int ch = e / (TH * TW), rem = e - ch * (TH * TW);
            const int oy = rem / TW, ox = rem - oy * TW;
            if (y0 + oy < H && x0 + ox < W)
                a.ya[ch * HW + (y0 + oy) * W + x0 + ox] = lm[ch * G::PLANE_M + (oy + 1) * G::PITCH_M + ox + 1];
        }
    }
}

// Tiles (TH x TW) of the launch's variant space.
struct PairTile {
    int th, tw;
};
// 2 x 2: one 16-pixel block for each conv (the ring is 4 x 4), so every wave
// runs a single chain per conv; on small maps with wide intermediates this
// spreads a pair over four times the CUs of 4 x 4, at the price of computing
// 16 pixels of each conv per 4 output pixels.
constexpr PairTile kPairTiles[] = {{4, 4}, {4, 8}, {8, 8}, {2, 2}};
constexpr int kPairTileCount = sizeof(kPairTiles) / sizeof(kPairTiles[0]);

// The pair takes SiLU convs (the bottlenecks'); exact_silu() selects the
// reference polynomial as for the single convs.
template <int TH, int TW, int CB1, int CB2>
static osh_status pair_launch_t(PairArgs a, hipStream_t st) {
    a.tiles_w = ceil_div(a.w, TW);
    const int tiles = a.tiles_w * ceil_div(a.h, TH);
    if (exact_silu())
        OSH_LAUNCH((conv_pair_kernel<TH, TW, CB1, CB2, ACT_SILU_EXACT>), dim3((unsigned)tiles), dim3(256), 0,
                           st, a);
    else
        OSH_LAUNCH((conv_pair_kernel<TH, TW, CB1, CB2, OSH_ACT_SILU>), dim3((unsigned)tiles), dim3(256), 0,
                           st, a);
    OSH_LAUNCH_CHECK("conv_pair_kernel");
    return OSH_OK;
}

template <int TH, int TW>
static osh_status pair_launch_tile(const PairArgs &a, int cb1, int cb2, hipStream_t st) {
#define OSH_PAIR_CB2(CB1)                                                         \
    switch (cb2) {                                                              \
    case 1: return pair_launch_t<TH, TW, CB1, 1>(a, st);                   \
    case 2: return pair_launch_t<TH, TW, CB1, 2>(a, st);                   \
    default: return pair_launch_t<TH, TW, CB1, 4>(a, st);                  \
    }
    switch (cb1) {
    case 1: OSH_PAIR_CB2(1)
    case 2: OSH_PAIR_CB2(2)
    default: OSH_PAIR_CB2(4)
    }
#undef OSH_PAIR_CB2
}

osh_status conv_pair_launch(const PairArgs &a, int cb1, int cb2, hipStream_t st, int tile) {
    switch (tile) {
    case 0: return pair_launch_tile<4, 4>(a, cb1, cb2, st);
    case 1: return pair_launch_tile<4, 8>(a, cb1, cb2, st);
    case 2: return pair_launch_tile<8, 8>(a, cb1, cb2, st);
    default: return pair_launch_tile<2, 2>(a, cb1, cb2, st);
    }
}

int conv_pair_tile_count() { return kPairTileCount; }

// ---------------------------------------------------------- 8-channel pair
//
// A bottleneck whose intermediate has 8 channels (YOLO11n's first C3k2 at
// 160 x 160: 16 -> 8 -> 16, shortcut added after the second conv).  The
// single-conv dispatch sums the first conv in the im2col order (8 outputs:
// ConvKernels.cs:554-563) and the second, over 8 input channels, in the
// first-layer chain ic -> ky -> kx (FirstConv.cs:344-362): both are k =
// ic*9 + ky*3 + kx ascending from the bias.  Both run on the 16x16x4 MFMA
// from LDS: the first with the im2col packing of conv16_pack (its rows 8..15
// are zero weights and a zero bias, so those rows compute zeros, stored to
// unused planes), the second over the 72 terms of its 8 channels with raw
// OIHW weights (first_conv_kernel's packing).  The first conv covers the
// tile and a one-pixel ring, block by block, each block's 36-step chain
// overlapping the activation and stores of the block before.
template <int TH, int TW, int ACT>
__global__ __launch_bounds__(256) void conv_pair8_kernel(PairArgs a) {
    constexpr int EH = TH + 2, EW = TW + 2, NE = EH * EW;      // first conv's field (tile + ring)
    constexpr int NBA = (NE + 15) / 16, IA = (NBA + 3) / 4;     // its 16-pixel blocks; per wave
    constexpr int PH = TH + 4, PW = TW + 4;                     // its input patch (16 channels)
    constexpr int PITCH_X = pair_pitch(PW), PLANE_X = pair_plane(PH, PITCH_X);
    constexpr int XE = 16 * PH * PW, NXE = (XE + 255) / 256;
    constexpr int PITCH_M = pair_pitch(EW), PLANE_M = pair_plane(EH, PITCH_M);
    constexpr int NBB = TH * TW / 16, IB = (NBB + 3) / 4;       // output blocks; per wave
    static_assert(TH * TW % 16 == 0, "whole 16-pixel output blocks");
    constexpr int XDUMMY = 16 * PLANE_X;
    __shared__ __align__(16) float lx[XDUMMY + 64];  // a dummy word per lane for staging lanes past the patch
    __shared__ __align__(16) float lm[16 * PLANE_M];  // planes 8..15: the first conv's zero rows
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int ty = blockIdx.x / a.tiles_w, tx = blockIdx.x - ty * a.tiles_w;
    const int y0 = ty * TH, x0 = tx * TW;
    const int H = a.h, W = a.w, HW = H * W;

    // ---- the first conv's input patch (rows y0-2 .. y0+TH+1, columns
    // x0-2 .. x0+TW+1, 16 channels) in one round trip; outside the map the
    // offset is out of range and the load returns 0
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.x, (short)0, 16 * HW * 4, 0x00020000);
    int loff[NXE];
    float sv[NXE];
#pragma unroll
    for (int i = 0; i < NXE; i++) {
        const int e = tid + 256 * i;
        const int ch = e / (PH * PW), rem = e - ch * (PH * PW);
        const int r = rem / PW, c = rem - r * PW;
        const int iy = y0 - 2 + r, ix = x0 - 2 + c;
        const bool ok = e < XE && (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
        loff[i] = e < XE ? ch * PLANE_X + r * PITCH_X + c : XDUMMY + lane;
        sv[i] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(rx, ok ? (ch * HW + iy * W + ix) * 4 : (int)C16_OOB, 0, 0));
    }
    // ---- weights and biases.  First conv: k-group t's float4 holds steps
    // 4t .. 4t+3 of the lane (im2col packing, one 16-row block).  Second
    // conv: lane (j, g) step s holds w[j][4s + g] (raw [16][8][3][3]).
    const __amdgpu_buffer_rsrc_t rwa =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.wa, (short)0, 9 * 1024, 0x00020000);
    float4 wa[9];
#pragma unroll
    for (int t = 0; t < 9; t++) {
        auto v = __builtin_amdgcn_raw_buffer_load_b128(rwa, lane * 16, t * 1024, 0);
        wa[t] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                            __uint_as_float(v[3]));
    }
    const __amdgpu_buffer_rsrc_t rwb =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.wb, (short)0, 16 * 72 * 4, 0x00020000);
    float wb[18];
#pragma unroll
    for (int s = 0; s < 18; s++)
        wb[s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rwb, (j * 72 + 4 * s + g) * 4, 0, 0));
    // biases as buffer loads (a NULL bias is a zero-sized buffer: loads
    // return 0); the first conv's has 8 entries, so lane groups 2 and 3 (its
    // zero rows) read past it and get 0
    float biasa[4], biasb[4];
    {
        const __amdgpu_buffer_rsrc_t rba =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.ba, (short)0, a.ba ? 32 : 0, 0x00020000);
        const __amdgpu_buffer_rsrc_t rbb =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.bb, (short)0, a.bb ? 64 : 0, 0x00020000);
        auto va = __builtin_amdgcn_raw_buffer_load_b128(rba, 16 * g, 0, 0);
        auto vb = __builtin_amdgcn_raw_buffer_load_b128(rbb, 16 * g, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) biasa[r] = __uint_as_float(va[r]), biasb[r] = __uint_as_float(vb[r]);
    }
    // operand offsets.  First conv: step u = 9v + r gives lane group g the
    // term 4u + g: channel 4v + (4r + g) / 9, tap (4r + g) % 9.  Second conv:
    // step s gives term 4s + g: channel (4s + g) / 9, tap (4s + g) % 9.
    int i2ca[9], kofb[18];
#pragma unroll
    for (int r = 0; r < 9; r++) {
        const int term = 4 * r + g, tap = term % 9;
        i2ca[r] = (term / 9) * PLANE_X + (tap / 3) * PITCH_X + tap % 3;
    }
#pragma unroll
    for (int s = 0; s < 18; s++) {
        const int term = 4 * s + g, tap = term % 9;
        kofb[s] = (term / 9) * PLANE_M + (tap / 3) * PITCH_M + tap % 3;
    }

    // the residuals of the wave's output pixels, loaded now so that their
    // latency passes under both convs (out-of-map pixels and a NULL residual
    // read 0; the add below happens only with a residual)
    float rv[IB][4];
    {
        const __amdgpu_buffer_rsrc_t rr =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.res, (short)0, a.res ? 16 * HW * 4 : 0, 0x00020000);
#pragma unroll
        for (int i = 0; i < IB; i++) {
            const int o = (wave + 4 * i) * 16 + j;
            const int oy = y0 + o / TW, ox = x0 + o % TW;
            const bool in = wave + 4 * i < NBB && oy < H && ox < W;
#pragma unroll
            for (int r = 0; r < 4; r++)
                rv[i][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    rr, in ? ((4 * g + r) * HW + oy * W + ox) * 4 : (int)C16_OOB, 0, 0));
        }
    }
#pragma unroll
    for (int i = 0; i < NXE; i++) lx[loff[i]] = sv[i];
    __syncthreads();

    // ---- first conv, block by block (pixel e = 16 wave + j + 64 i of the
    // field, stepped without a division; lanes past the field take its last
    // pixel and store the same value as that pixel's own lane)
    int ey0b, ex0b;
    {
        const int e = 16 * wave + j;
        ey0b = e / EW;
        ex0b = e - ey0b * EW;
    }
    auto pix = [&](int i, int &ey, int &ex) {
        ey = ey0b + (64 * i) / EW;
        ex = ex0b + (64 * i) % EW;
        if (ex >= EW) ex -= EW, ey++;
        if (16 * wave + j + 64 * i >= NE) ey = EH - 1, ex = EW - 1;
    };
    auto read_blk = [&](float (&bv)[36], int i) {
        int ey, ex;
        pix(i, ey, ex);
        const int base = ey * PITCH_X + ex;
#pragma unroll
        for (int u = 0; u < 36; u++) bv[u] = lx[(u / 9) * 4 * PLANE_X + i2ca[u % 9] + base];
    };
    // the intermediate: activation inside the map, +0 on the ring outside it
    auto store_blk = [&](const f32x4 &acc, int i) {
        int ey, ex;
        pix(i, ey, ex);
        const int yy = y0 - 1 + ey, xx = x0 - 1 + ex;
        const int keep = (unsigned)yy < (unsigned)H && (unsigned)xx < (unsigned)W ? -1 : 0;
        const int pos = 4 * g * PLANE_M + ey * PITCH_M + ex;
#pragma unroll
        for (int r = 0; r < 4; r++)
            lm[pos + r * PLANE_M] = __int_as_float(__float_as_int(activate<ACT>(acc[r])) & keep);
    };
    {
        // One scheduling region per block: its chain, the next block's
        // operand reads and the block before's stores, the LDS operations
        // placed one after each MFMA (left to itself the scheduler sank
        // every read to just before its MFMA, which then waited for it).
        float bv[2][36];
        f32x4 prev;
        read_blk(bv[0], 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < IA; i++) {
            if (i + 1 < IA) read_blk(bv[(i + 1) & 1], i + 1);
            f32x4 acc;
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] = biasa[r];
#pragma unroll
            for (int u = 0; u < 36; u++) {
                const float4 &w4 = wa[u / 4];
                const float wv = u % 4 == 0 ? w4.x : u % 4 == 1 ? w4.y : u % 4 == 2 ? w4.z : w4.w;
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wv, bv[i & 1][u], acc, 0, 0, 0);
            }
            if (i > 0) store_blk(prev, i - 1);  // blocks before the last exist for every wave
            prev = acc;
#pragma unroll
            for (int u = 0; u < 36; u++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100 | 0x200, 1, 0);  // then one LDS read or write
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (wave + 4 * (IA - 1) < NBA) store_blk(prev, IA - 1);  // uniform
    }
    __syncthreads();

    // ---- second conv from LDS: wave -> output blocks wave + 4 i
    int baseb[IB];
#pragma unroll
    for (int i = 0; i < IB; i++) {
        int o = (wave + 4 * i) * 16 + j;
        o = o < TH * TW ? o : TH * TW - 1;
        const int oy = o / TW, ox = o - oy * TW;
        baseb[i] = oy * PITCH_M + ox;
    }
    f32x4 accb[IB];
#pragma unroll
    for (int i = 0; i < IB; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) accb[i][r] = biasb[r];
    {
        // eight reads ahead, then one read after each MFMA
        float bv[18][IB];
#pragma unroll
        for (int s = 0; s < 18; s++)
#pragma unroll
            for (int i = 0; i < IB; i++) bv[s][i] = lm[kofb[s] + baseb[i]];
#pragma unroll
        for (int s = 0; s < 18; s++)
#pragma unroll
            for (int i = 0; i < IB; i++)
                accb[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb[s], bv[s][i], accb[i], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
        for (int q = 0; q < 18 * IB; q++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // ---- epilogue: activation, residual, store
#pragma unroll
    for (int i = 0; i < IB; i++) {
        if (wave + 4 * i >= NBB) continue;  // uniform
        const int o = (wave + 4 * i) * 16 + j;
        const int oy = y0 + o / TW, ox = x0 + o % TW;
        if (oy >= H || ox >= W) continue;
        const int pix_ = oy * W + ox;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int oc = 4 * g + r;
            float v = activate<ACT>(accb[i][r]);
            if (a.res) v += rv[i][r];
            a.y[oc * HW + pix_] = v;
        }
    }
    // ---- the tile's own pixels of the intermediate (8 channels), from LDS
    if (a.ya) {
        constexpr int OWN = 8 * TH * TW;
        for (int e = tid; e < OWN; e += 256) {
            const int ch = e / (TH * TW), rem = e - ch * (TH * TW);
            const int oy = rem / TW, ox = rem - oy * TW;
            if (y0 + oy < H && x0 + ox < W)
                a.ya[ch * HW + (y0 + oy) * W + x0 + ox] = lm[ch * PLANE_M + (oy + 1) * PITCH_M + ox + 1];
        }
    }
}

constexpr PairTile kPair8Tiles[] = {{4, 16}, {8, 16}, {2, 32}, {2, 16}};
static_assert(sizeof(kPair8Tiles) / sizeof(kPair8Tiles[0]) == kPairTileCount,
              "a forced pair_tile indexes every pair family alike");

template <int TH, int TW>
static osh_status pair8_launch_t(PairArgs a, hipStream_t st) {
    a.tiles_w = ceil_div(a.w, TW);
    const unsigned tiles = (unsigned)(a.tiles_w * ceil_div(a.h, TH));
    if (exact_silu())
        OSH_LAUNCH((conv_pair8_kernel<TH, TW, ACT_SILU_EXACT>), dim3(tiles), dim3(256), 0, st, a);
    else
        OSH_LAUNCH((conv_pair8_kernel<TH, TW, OSH_ACT_SILU>), dim3(tiles), dim3(256), 0, st, a);
    OSH_LAUNCH_CHECK("conv_pair8_kernel");
    return OSH_OK;
}

osh_status conv_pair8_launch(const PairArgs &a, hipStream_t st, int tile) {
    switch (tile) {
    case 0: return pair8_launch_t<4, 16>(a, st);
    case 1: return pair8_launch_t<8, 16>(a, st);
    case 2: return pair8_launch_t<2, 32>(a, st);
    default: return pair8_launch_t<2, 16>(a, st);
    }
}

// ------------------------------------------------------ first-layer pair
//
// A network's first conv (3x3 over c0 <= 4 colour planes, 16 outputs, stride
// SA: FirstConv.cs) and the 3x3 pad-1 conv that reads it (16 -> 16 CB2
// channels, stride S2, the NCHWc chain: NchwcConv.cs:533-605) -- YOLO11n's
// 3 -> 16 -> 32 stem, two stride-2 convs -- in one launch.  The first conv's
// 16-channel map is the largest tensor of such a network after the image and
// nothing else reads it; here it never leaves the chip.
//
// A workgroup owns a TH x TW tile of the second conv's output.  It stages
// the image patch under the tile (every plane) in LDS, computes the first
// conv over the tile's receptive field ((S2 (TH-1) + 3) x (S2 (TW-1) + 3)
// pixels, zero where that leaves the map: the second conv's padding taps),
// then the second conv from LDS.
//
// Both chains are the single convs' own, on the 16x16x4 MFMA (each step adds
// its four lane-group products one after another, each rounded like an
// fmaf):
//   * first conv: bias, then k = ic*9 + ky*3 + kx ascending -- first_conv_
//     kernel's ic -> ky -> kx chain.  A step past 9 c0 multiplies a -0 weight
//     by a +0 input: adding -0 leaves every accumulator as it is;
//   * second conv: bias, then ky -> kx -> ic16 (one 16-channel block).
// With S2 = 2 each intermediate row keeps its even columns, then its odd
// ones, so the stride-2 operand reads of 16 lanes are 16 consecutive words.
template <int TH, int TW, int SA, int S2>
struct FirstPairGeom {
    static constexpr int EH = S2 * (TH - 1) + 3, EW = S2 * (TW - 1) + 3, NE = EH * EW;  // first conv's pixels
    static constexpr int NBA = (NE + 15) / 16, IA = (NBA + 3) / 4;  // its 16-pixel blocks; per wave
    static constexpr int PH = SA * (EH - 1) + 3, PW = SA * (EW - 1) + 3;  // its input patch
    static constexpr int PITCH_X = pair_pitch(PW), PLANE_X = pair_plane(PH, PITCH_X);
    static constexpr int XE = 4 * PH * PW, NXE = (XE + 255) / 256;  // staging loads per thread (4 planes)
    static constexpr int HALF = S2 == 2 ? (EW + 1) / 2 : EW;
    static constexpr int ROW = S2 == 2 ? 2 * HALF : pair_pitch(EW);
    static constexpr int PLANE_M = (EH * ROW + 47) / 64 * 64 + 16;  // >= EH * ROW, 16 mod 64 words
    static constexpr int NBB = (TH * TW + 15) / 16;
    // LDS word of intermediate pixel (ey, ex) within a channel plane
    static __device__ __forceinline__ int mpos(int ey, int ex) {
        return S2 == 2 ? ey * ROW + (ex & 1) * HALF + (ex >> 1) : ey * ROW + ex;
    }
};

// NS: the first conv's k-steps, 7 for c0 <= 3 (past 9 c0 every term is the
// -0 x +0 identity) and 9 for c0 = 4; a compile-time count keeps the
// accumulators in place (a runtime bound had the compiler copy them at every
// step's join).  Stores of lanes with nothing to store go to dummy words past
// the input patch, so no store waits behind a branch.
template <int TH, int TW, int SA, int S2, int CB2, int NS, int ACT>
__global__ __launch_bounds__(256) void first_pair_kernel(FirstPairArgs a) {
    using G = FirstPairGeom<TH, TW, SA, S2>;
    static_assert(CB2 == 2 || CB2 == 4, "32 or 64 output channels (the NCHWc chain)");
    static_assert(TW % 16 == 0 || 16 % TW == 0, "16-pixel blocks cover whole rows or whole row sets");
    static_assert(NS == 7 || NS == 9, "up to 3 planes in 7 k-steps, 4 in 9");
    constexpr int XDUMMY = 4 * G::PLANE_X;
    __shared__ __align__(16) float lx[XDUMMY + 64];  // a dummy word per lane: no bank conflicts
    __shared__ __align__(16) float lm[16 * G::PLANE_M];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int ty = blockIdx.x / a.tiles_w, tx = blockIdx.x - ty * a.tiles_w;
    const int y0 = ty * TH, x0 = tx * TW;            // the tile, in the second conv's output
    const int ey0 = S2 * y0 - 1, ex0 = S2 * x0 - 1;  // first-conv pixel at patch (0, 0)
    const int iy0 = SA * ey0 - a.pt, ix0 = SA * ex0 - a.pl;  // image pixel at input patch (0, 0)
    const int c0 = a.c0, H = a.h, W = a.w, HW = H * W;

    // ---- the input patch, every plane, in one round trip (outside the
    // image the load's offset is out of range and returns 0)
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.x, (short)0, c0 * HW * 4, 0x00020000);
    int loff[G::NXE];
    float sv[G::NXE];
#pragma unroll
    for (int i = 0; i < G::NXE; i++) {
        const int e = tid + 256 * i;
        const int ch = e / (G::PH * G::PW), rem = e - ch * (G::PH * G::PW);
        const int r = rem / G::PW, c = rem - r * G::PW;
        const int iy = iy0 + r, ix = ix0 + c;
        // planes c0 .. 3 are staged too, as zeros: the terms past 9 c0 read them
        const bool ok = e < G::XE && ch < c0 && (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
        loff[i] = e < G::XE ? ch * G::PLANE_X + r * G::PITCH_X + c : XDUMMY + lane;
        sv[i] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(rx, ok ? (ch * HW + iy * W + ix) * 4 : (int)C16_OOB, 0, 0));
    }

    // ---- first conv's A operands: lane (j, g) holds w[j][k] for k = 4s + g
    // (raw OIHW: k = ic*9 + ky*3 + kx), -0 past K = 9 c0; kof[s] is term k's
    // patch offset (past K: a zero plane, so those terms add -0 x +0)
    const int K = 9 * c0;
    const __amdgpu_buffer_rsrc_t rwa =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.wa, (short)0, 16 * K * 4, 0x00020000);
    float wa[NS];
    int kof[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int k = 4 * s + g, ic = k / 9, t = k - 9 * ic;
        const bool valid = k < K;
        const float v = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(rwa, valid ? (j * K + k) * 4 : (int)C16_OOB, 0, 0));
        wa[s] = valid ? v : -0.0f;
        kof[s] = ic * G::PLANE_X + (t / 3) * G::PITCH_X + t % 3;  // ic <= 3 (k < 4 NS <= 36)
    }
    const int cbb = wave % CB2, pb0 = wave / CB2;
    float biasa[4], biasb[4];
    {
        const __amdgpu_buffer_rsrc_t rba =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.ba, (short)0, a.ba ? 64 : 0, 0x00020000);
        const __amdgpu_buffer_rsrc_t rbb =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.bb, (short)0, a.bb ? 64 * CB2 : 0, 0x00020000);
        auto va = __builtin_amdgcn_raw_buffer_load_b128(rba, 4 * g * 4, 0, 0);
        auto vb = __builtin_amdgcn_raw_buffer_load_b128(rbb, (cbb * 16 + 4 * g) * 4, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) biasa[r] = __uint_as_float(va[r]), biasb[r] = __uint_as_float(vb[r]);
    }

    // ---- second conv's weights (one 16-channel block: nine taps), issued
    // with the first conv's: their latency passes under the first conv
    const __amdgpu_buffer_rsrc_t rwb =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.wb, (short)0, CB2 * 9 * 1024, 0x00020000);
    float4 wb[9];
#pragma unroll
    for (int t = 0; t < 9; t++) {
        auto v = __builtin_amdgcn_raw_buffer_load_b128(rwb, (cbb * 9 * 64 + lane) * 16, t * 1024, 0);
        wb[t] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                            __uint_as_float(v[3]));
    }

    // ---- first conv: wave -> pixel blocks wave + 4 i (every channel), one
    // block after the other: block i's chain (NS dependent MFMAs) runs while
    // the VALU activates and stores block i - 1, and block i + 1's operands
    // are read from LDS
#pragma unroll
    for (int i = 0; i < G::NXE; i++) lx[loff[i]] = sv[i];
    __syncthreads();
    // block i's pixel: lane j of block wave + 4 i, e = 16 wave + j + 64 i,
    // stepped from block to block without a division.  Lanes past the field
    // take its last pixel: they compute and store the same value to the same
    // word as that pixel's own lane
    int ey0b, ex0b;
    {
        const int e = 16 * wave + j;
        ey0b = e / G::EW;
        ex0b = e - ey0b * G::EW;
    }
    auto pix = [&](int i, int &ey, int &ex) {
        ey = ey0b + (64 * i) / G::EW;
        ex = ex0b + (64 * i) % G::EW;
        if (ex >= G::EW) ex -= G::EW, ey++;
        if (16 * wave + j + 64 * i >= G::NE) ey = G::EH - 1, ex = G::EW - 1;
    };
    auto read_blk = [&](float (&bv)[NS], int i) {
        int ey, ex;
        pix(i, ey, ex);
        const int base = SA * (ey * G::PITCH_X + ex);
#pragma unroll
        for (int s = 0; s < NS; s++) bv[s] = lx[kof[s] + base];
    };
    // the intermediate: activation inside the first conv's map, +0 on the
    // field outside it (the activation's bits masked: no branch)
    auto store_blk = [&](const f32x4 &acc, int i) {
        int ey, ex;
        pix(i, ey, ex);
        const int yy = ey0 + ey, xx = ex0 + ex;
        const int keep = (unsigned)yy < (unsigned)a.ah && (unsigned)xx < (unsigned)a.aw ? -1 : 0;
        const int pos = 4 * g * G::PLANE_M + G::mpos(ey, ex);
#pragma unroll
        for (int r = 0; r < 4; r++)
            lm[pos + r * G::PLANE_M] = __int_as_float(__float_as_int(activate<ACT>(acc[r])) & keep);
    };
    {
        // one scheduling region per block: its chain, the next block's reads
        // and the block before's stores, two LDS operations after each MFMA
        // (left to itself the scheduler sinks each read to its MFMA)
        float bv[2][NS];
        f32x4 prev;
        read_blk(bv[0], 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < G::IA; i++) {
            if (i + 1 < G::IA) read_blk(bv[(i + 1) & 1], i + 1);
            f32x4 acc;
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] = biasa[r];
#pragma unroll
            for (int s = 0; s < NS; s++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[s], bv[i & 1][s], acc, 0, 0, 0);
            if (i > 0) store_blk(prev, i - 1);  // blocks before the last exist for every wave
            prev = acc;
#pragma unroll
            for (int s = 0; s < NS; s++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100 | 0x200, 2, 0);  // then up to two LDS reads / writes
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (wave + 4 * (G::IA - 1) < G::NBA) store_blk(prev, G::IA - 1);  // uniform
    }
    __syncthreads();

    // ---- second conv from LDS: wave -> channel block cbb, pixel blocks
    // pb0 + i * WB
    constexpr int WB = 4 / CB2, IB = (G::NBB + WB - 1) / WB;
    int baseb[IB];
#pragma unroll
    for (int i = 0; i < IB; i++) {
        int o = (pb0 + i * WB) * 16 + j;
        o = o < TH * TW ? o : TH * TW - 1;
        const int oy = o / TW, ox = o - oy * TW;
        baseb[i] = S2 * oy * G::ROW + ox;  // row S2 oy, column S2 ox (with S2 = 2: word ox of the even half)
    }
    auto toff = [](int t) {
        const int ky = t / 3, kx = t % 3;
        return S2 == 2 ? ky * G::ROW + (kx & 1) * G::HALF + (kx >> 1) : ky * G::ROW + kx;
    };
    f32x4 accb[IB];
#pragma unroll
    for (int i = 0; i < IB; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) accb[i][r] = biasb[r];
    auto read_b = [&](float (&bv)[4][IB], int t) {
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < IB; i++) bv[s][i] = lm[(4 * s + g) * G::PLANE_M + baseb[i] + toff(t)];
    };
    {
        float bv[2][4][IB];
        read_b(bv[0], 0);
#pragma unroll
        for (int t = 0; t < 9; t++) {
            if (t + 1 < 9) read_b(bv[(t + 1) & 1], t + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const float w4 = s == 0 ? wb[t].x : s == 1 ? wb[t].y : s == 2 ? wb[t].z : wb[t].w;
#pragma unroll
                for (int i = 0; i < IB; i++)
                    accb[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(w4, bv[t & 1][s][i], accb[i], 0, 0, 0);
            }
        }
    }

    // ---- epilogue: activation, residual, store
    const int HWB = a.bh * a.bw;
#pragma unroll
    for (int i = 0; i < IB; i++) {
        const int o = (pb0 + i * WB) * 16 + j;
        if (pb0 + i * WB >= G::NBB || o >= TH * TW) continue;
        const int oy = y0 + o / TW, ox = x0 + o % TW;
        if (oy >= a.bh || ox >= a.bw) continue;
        const int pix = oy * a.bw + ox;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int oc = cbb * 16 + 4 * g + r;
            float v = activate<ACT>(accb[i][r]);
            if (a.res) v += a.res[oc * HWB + pix];
            a.y[oc * HWB + pix] = v;
        }
    }
    // ---- the tile's own pixels of the intermediate (S2 TH x S2 TW; the
    // tiles partition the first conv's map), from LDS
    if (a.ya) {
        constexpr int OH = S2 * TH, OW = S2 * TW, OWN = 16 * OH * OW;
        const int HWA = a.ah * a.aw;
        for (int e = tid; e < OWN; e += 256) {
            const int ch = e / (OH * OW), rem = e - ch * (OH * OW);
            const int ry = rem / OW, rx = rem - ry * OW;
            const int yy = S2 * y0 + ry, xx = S2 * x0 + rx;
            if (yy < a.ah && xx < a.aw) a.ya[ch * HWA + yy * a.aw + xx] = lm[ch * G::PLANE_M + G::mpos(ry + 1, rx + 1)];
        }
    }
}

// Measured at YOLO11n's stem (3 -> 16 -> 32, 640 x 640): 4 x 16 10.9 us,
// 2 x 32 10.8, 2 x 16 11.1; 8 x 16 12.1 and 4 x 32 13.3 (fewer workgroups
// than CUs) were dropped.  As many tiles as the bottleneck pair's, so that a
// forced pair_tile means the same for both.
constexpr PairTile kFirstPairTiles[] = {{4, 16}, {2, 32}, {2, 16}, {2, 8}};
constexpr int kFirstPairTileCount = sizeof(kFirstPairTiles) / sizeof(kFirstPairTiles[0]);

template <int TH, int TW, int SA, int S2, int CB2, int NS>
static void first_pair_launch_ns(const FirstPairArgs &a, unsigned tiles, hipStream_t st) {
    if (exact_silu())
        OSH_LAUNCH((first_pair_kernel<TH, TW, SA, S2, CB2, NS, ACT_SILU_EXACT>), dim3(tiles), dim3(256), 0, st,
                           a);
    else
        OSH_LAUNCH((first_pair_kernel<TH, TW, SA, S2, CB2, NS, OSH_ACT_SILU>), dim3(tiles), dim3(256), 0, st, a);
}

template <int TH, int TW, int SA, int S2, int CB2>
static osh_status first_pair_launch_t(FirstPairArgs a, hipStream_t st) {
    a.tiles_w = ceil_div(a.bw, TW);
    const unsigned tiles = (unsigned)(a.tiles_w * ceil_div(a.bh, TH));
    if (a.c0 <= 3)
        first_pair_launch_ns<TH, TW, SA, S2, CB2, 7>(a, tiles, st);
    else
        first_pair_launch_ns<TH, TW, SA, S2, CB2, 9>(a, tiles, st);
    OSH_LAUNCH_CHECK("first_pair_kernel");
    return OSH_OK;
}

template <int TH, int TW>
static osh_status first_pair_launch_tile(const FirstPairArgs &a, int sa, int sb, int cb2, hipStream_t st) {
#define OSH_FP_CB2(SA, S2) \
    return cb2 == 2 ? first_pair_launch_t<TH, TW, SA, S2, 2>(a, st) : first_pair_launch_t<TH, TW, SA, S2, 4>(a, st);
    if (sa == 1) {
        if (sb == 1) { OSH_FP_CB2(1, 1) }
        OSH_FP_CB2(1, 2)
    }
    if (sb == 1) { OSH_FP_CB2(2, 1) }
    OSH_FP_CB2(2, 2)
#undef OSH_FP_CB2
}

osh_status first_pair_launch(const FirstPairArgs &a, int sa, int sb, int cb2, hipStream_t st, int tile) {
    switch (tile) {
    case 0: return first_pair_launch_tile<4, 16>(a, sa, sb, cb2, st);
    case 1: return first_pair_launch_tile<2, 32>(a, sa, sb, cb2, st);
    case 2: return first_pair_launch_tile<2, 16>(a, sa, sb, cb2, st);
    default: return first_pair_launch_tile<2, 8>(a, sa, sb, cb2, st);
    }
}

int first_pair_tile_count() { return kFirstPairTileCount; }
static_assert(kFirstPairTileCount == kPairTileCount, "a forced pair_tile indexes both pair families alike");

}  // namespace osh
