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
            if (a.res) v += a.res[oc * HW + pix];
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
constexpr PairTile kPairTiles[] = {{4, 4}, {4, 8}, {8, 8}};
constexpr int kPairTileCount = sizeof(kPairTiles) / sizeof(kPairTiles[0]);

// The pair takes SiLU convs (the bottlenecks'); exact_silu() selects the
// reference polynomial as for the single convs.
template <int TH, int TW, int CB1, int CB2>
static osh_status pair_launch_t(PairArgs a, hipStream_t st) {
    a.tiles_w = ceil_div(a.w, TW);
    const int tiles = a.tiles_w * ceil_div(a.h, TH);
    if (exact_silu())
        hipLaunchKernelGGL((conv_pair_kernel<TH, TW, CB1, CB2, ACT_SILU_EXACT>), dim3((unsigned)tiles), dim3(256), 0,
                           st, a);
    else
        hipLaunchKernelGGL((conv_pair_kernel<TH, TW, CB1, CB2, OSH_ACT_SILU>), dim3((unsigned)tiles), dim3(256), 0,
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
    default: return pair_launch_tile<8, 8>(a, cb1, cb2, st);
    }
}

int conv_pair_tile_count() { return kPairTileCount; }

}  // namespace osh
