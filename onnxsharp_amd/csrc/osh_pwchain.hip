// osh_pwchain.hip -- chains of pointwise convolutions in one launch.
//
// Runs of 1x1 convs that feed each other (C3k2's cv1 -> C3k cv1/cv2, the
// detection head's depthwise -> 1x1 -> 1x1 tails, C2PSA's proj -> ffn.0 ->
// ffn.1 -> cv2) go through this kernel as one launch: a workgroup takes 16
// consecutive pixels through every stage, keeping each stage's output on chip
// (LDS) for the stages that read it, and writing it to its tensor as well.
//
// Each stage computes what its conv computes alone, bit for bit:
//   * 1x1: the GEMM chain over input channels -- bias, then ic ascending, four
//     at a time through v_mfma_f32_16x16x4f32 (which adds its four products
//     in order, each rounded like an fmaf) -- as GemmKernel.Multiply sums it
//     (src/OnnxSharp/Tensors/GemmKernel.cs:1130-1207) and as the pointwise
//     LDS tiles (osh_conv16s.h, KS = 1) do; a concat input is read part by
//     part in concat order, which is the ic order of the conv;
//   * 3x3 depthwise (stage 0 only): bias, then fmaf over ky -> kx, taps off
//     the map skipped (DepthwiseConv.cs; dw_conv_at in osh_conv.hip);
//   * then the fused activation, then the residual (GraphFusion.cs:1713-1718).
//
// Layout: the MFMA output block is 16 channels x the tile's 16 pixels; lane
// (j, g) holds channels 4g + r of pixel j.  Everything a workgroup reads from
// memory is in flight from its start, so it waits for memory once: the 1x1
// stages' packed weights ([M/16][C/16][64 lanes][4 steps], the pointwise
// LDS-tile pack) go straight to LDS (global_load_lds_dwordx4), the parts and
// residuals in memory and the biases are staged into LDS, the depthwise taps
// into registers.  A comes from LDS 16 bytes a lane, B from LDS
// ([channel][16 pixels]: a half-wave read hits 32 banks), both two groups of
// PWC_KU input blocks ahead of the MFMAs.  A chain therefore needs its 1x1
// weights, staged tensors and kept outputs in 160 KB of LDS.
//
// Measured on one MI355X, a chain does not beat its convs launched one by one
// in the YOLO11n frame: a workgroup runs its stages one after another with a
// single dependent accumulator per wave (about 65 cycles per 16x16x4 MFMA
// against 32 for independent ones), while separate launches spread each
// stage over the whole chip; the frame executor keeps chains off by default.
#include "osh_common.h"
#include "osh_launch.h"

#include <cstring>

using namespace osh;

namespace osh {

constexpr int PWC_NW = 4;  // waves per workgroup
constexpr int PWC_THREADS = 64 * PWC_NW;
constexpr int PWC_TILE = 16;   // pixels per workgroup: one MFMA column block
constexpr int PWC_KU = 4;      // input blocks per unrolled MFMA step
constexpr int PWC_MAXC = 512;  // channels of a part in memory, and of a 1x1 stage's output
constexpr int PWC_SPT = 4;     // 16-byte staging loads a thread per round
constexpr int PWC_MAXSEG = 8;  // tensors a chain stages from memory
constexpr int PWC_DWC = 8;     // depthwise channels a thread per round (16 slots of 16 pixels)
static_assert(PWC_THREADS == 16 * PWC_TILE, "the depthwise lanes: 16 pixels x 16 channel slots");

struct PwcStage {
    const float *w;     // packed 1x1 weights, or the raw [m][1][3][3] depthwise weights
    const float *bias;  // [m] or nullptr
    const float *x;     // a depthwise stage's input
    const float *res;   // a depthwise stage's residual in memory, or nullptr
    float *y;
    int kind, m, act, c;
    int w_lds;  // LDS float offset of a 1x1 stage's packed weights
    // LDS float offset of 16-channel input block icb (before the lane's
    // g * 16 + j): l0 + icb * 256, plus l1 - l0 from icb = e0 on and l2 - l1
    // from icb = e1 on
    int e0, e1, l0, l1, l2;
    int bias_lds;  // the staged bias, or -1
    int res_lds;   // the residual in LDS (an earlier stage's output or a staged tensor), or -1
    int out_lds;   // this stage's output in LDS, or -1 when no later stage reads it
};

struct PwcChain {
    int h, w, hw, nstages;
    // tensors in memory that 1x1 stages read, staged into LDS at the start:
    // segment k is [channels][16 pixels] from seg_ptr[k] to LDS seg_lds[k],
    // its 16-byte elements numbered from seg_start[k] to seg_start[k + 1]
    int nseg;
    int seg_start[PWC_MAXSEG + 1];
    int seg_lds[PWC_MAXSEG];
    const float *seg_ptr[PWC_MAXSEG];
    PwcStage st[OSH_PW_MAX_STAGES];
};

struct PwcArgs {
    int count;
    int start[OSH_PW_MAX_CHAINS + 1];  // first workgroup of each chain
    PwcChain ch[OSH_PW_MAX_CHAINS];
};
static_assert(sizeof(PwcArgs) <= 4000, "kernel arguments stay below the 4 KB limit");

__device__ __forceinline__ float act_rt(int a, float v) {
    switch (a) {
    case OSH_ACT_RELU: return activate<OSH_ACT_RELU>(v);
    case OSH_ACT_SILU: return activate<OSH_ACT_SILU>(v);
    case ACT_SILU_EXACT: return activate<ACT_SILU_EXACT>(v);
    default: return v;
    }
}

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void global_cvoid;

// Copies the packed weights of every 1x1 stage into LDS with direct
// memory-to-LDS loads (global_load_lds_dwordx4: no registers, so every load
// of every stage is in flight at once).  A packed 1x1 weight buffer is M*C
// floats, a whole number of 1 KB blocks: wave w of a round takes the 1 KB
// block round * PWC_NW + w.
__device__ __forceinline__ void pwc_weights_in(const PwcChain &C, float *smem, int wave, int lane) {
#pragma unroll 1
    for (int k = 0; k < C.nstages; k++) {
        const PwcStage &S = C.st[k];
        if (S.kind != OSH_PW_1X1) continue;
        const int blocks = (S.m >> 4) * (S.c >> 4);
        const char *src = reinterpret_cast<const char *>(S.w);
#pragma unroll 4
        for (int blk = wave; blk < blocks; blk += PWC_NW)
            __builtin_amdgcn_global_load_lds((global_cvoid *)(src + (size_t)blk * 1024 + lane * 16),
                                             (lds_void *)(smem + S.w_lds + blk * 256), 16, 0, 0);
    }
}

// Stages what the chain's 1x1 stages read from memory -- input parts and
// residuals (the segments), and every stage's bias -- into LDS; the loads of
// a round (PWC_SPT a thread, and the biases with the first) are all issued
// before its LDS writes.  Pixels past the map read 0 (HW % 4 == 0, so a
// group of four is wholly in or out).
__device__ __forceinline__ void pwc_stage_in(const PwcChain &C, float *smem, int p0, int tid) {
    const int HW = C.hw, T = C.seg_start[C.nseg];
    float bv[OSH_PW_MAX_STAGES];
#pragma unroll
    for (int k = 0; k < OSH_PW_MAX_STAGES; k++) {
        const PwcStage &S = C.st[k];
        bv[k] = 0.f;
        if (k < C.nstages && S.bias_lds >= 0) {
            for (int i = tid; i < S.m; i += PWC_THREADS) {
                if (i == tid) bv[k] = S.bias[i];
                else smem[S.bias_lds + i] = S.bias[i];  // more than one value a thread: m > PWC_THREADS
            }
        }
    }
#pragma unroll 1
    for (int base = 0; base < T; base += PWC_SPT * PWC_THREADS) {
        float4 v[PWC_SPT];
        int dst[PWC_SPT];
#pragma unroll
        for (int u = 0; u < PWC_SPT; u++) {
            const int e4 = base + tid + u * PWC_THREADS;
            const float *src = C.seg_ptr[0];
            int lds = C.seg_lds[0], s0 = 0;
#pragma unroll
            for (int k = 1; k < PWC_MAXSEG; k++)
                if (k < C.nseg && e4 >= C.seg_start[k]) src = C.seg_ptr[k], lds = C.seg_lds[k], s0 = C.seg_start[k];
            const int e = e4 - s0, ch = e / (PWC_TILE / 4), q = p0 + (e % (PWC_TILE / 4)) * 4;
            dst[u] = lds + 4 * e;
            v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (e4 < T && q < HW) v[u] = *reinterpret_cast<const float4 *>(src + (long long)ch * HW + q);
        }
#pragma unroll
        for (int u = 0; u < PWC_SPT; u++)
            if (base + tid + u * PWC_THREADS < T) *reinterpret_cast<float4 *>(smem + dst[u]) = v[u];
    }
#pragma unroll
    for (int k = 0; k < OSH_PW_MAX_STAGES; k++) {
        const PwcStage &S = C.st[k];
        if (k < C.nstages && S.bias_lds >= 0 && tid < S.m) smem[S.bias_lds + tid] = bv[k];
    }
}

// The operands of PWC_KU consecutive input blocks of one output block, read
// from LDS: A (weights, 16 bytes a lane a block) and B (the four k-steps of
// the lane's pixel column a block).
struct PwcOps {
    float4 a[PWC_KU];
    float b[PWC_KU][4];
};

// Where input block kk of a stage's B lies: arithmetic on the part bounds,
// not a select (a select between the stage's members becomes a select of
// their addresses).
struct PwcParts {
    int e0, e1, l0, d1, d2;
    __device__ __forceinline__ int at(int kk) const { return l0 + (kk >= e0 ? d1 : 0) + (kk >= e1 ? d2 : 0) + kk * 256; }
};

// Reads the operands of blocks k0 .. k0 + PWC_KU - 1 (indices past the
// stage's last block are clamped: read, never used).
__device__ __forceinline__ void pwc_read(PwcOps &o, const float4 *A, const float *bl, const PwcParts &pt, int k0,
                                         int ICB) {
#pragma unroll
    for (int i = 0; i < PWC_KU; i++) {
        const int kk = k0 + i < ICB ? k0 + i : ICB - 1;
        o.a[i] = A[kk * 64];
        const float *lb = bl + pt.at(kk);
        o.b[i][0] = lb[0 * PWC_TILE];
        o.b[i][1] = lb[4 * PWC_TILE];
        o.b[i][2] = lb[8 * PWC_TILE];
        o.b[i][3] = lb[12 * PWC_TILE];
    }
}

__device__ __forceinline__ void pwc_mfma(f32x4 &acc, const PwcOps &o, int n) {
#pragma unroll
    for (int i = 0; i < PWC_KU; i++) {
        if (i < n) {
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(o.a[i].x, o.b[i][0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(o.a[i].y, o.b[i][1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(o.a[i].z, o.b[i][2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(o.a[i].w, o.b[i][3], acc, 0, 0, 0);
        }
    }
}

// The MFMA part of 1x1 stage S for one wave: output blocks mb = wave,
// wave + PWC_NW, ..., each the in-order chain over the stage's input blocks
// with A (weights) and B (input pixels) both from LDS, read two groups of
// PWC_KU blocks ahead of the MFMAs (P and Q alternate), then the epilogue:
// activation, residual, the output to LDS (if kept) and to memory.
__device__ __forceinline__ void pwc_run(const PwcStage &S, float *smem, int wave, int lane, int p, int HW) {
    const int MB = S.m >> 4, ICB = S.c >> 4;
    const int j = lane & 15, g = lane >> 4;
    PwcParts pt;
    pt.e0 = S.e0, pt.e1 = S.e1, pt.l0 = S.l0, pt.d1 = S.l1 - S.l0, pt.d2 = S.l2 - S.l1;
    const float *bl = smem + g * PWC_TILE + j;
    for (int mb = wave; mb < MB; mb += PWC_NW) {
        const float4 *A = reinterpret_cast<const float4 *>(smem + S.w_lds) + (long long)mb * ICB * 64 + lane;
        f32x4 acc;
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r] = S.bias_lds >= 0 ? smem[S.bias_lds + mb * 16 + 4 * g + r] : 0.f;
        PwcOps P, Q;
        pwc_read(P, A, bl, pt, 0, ICB);
        for (int k0 = 0; k0 < ICB; k0 += 2 * PWC_KU) {
            pwc_read(Q, A, bl, pt, k0 + PWC_KU, ICB);
            pwc_mfma(acc, P, ICB - k0);
            if (k0 + PWC_KU >= ICB) break;
            pwc_read(P, A, bl, pt, k0 + 2 * PWC_KU, ICB);
            pwc_mfma(acc, Q, ICB - k0 - PWC_KU);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int oc = mb * 16 + 4 * g + r;
            float v = act_rt(S.act, acc[r]);
            if (S.res_lds >= 0) v += smem[S.res_lds + oc * PWC_TILE + j];
            if (S.out_lds >= 0) smem[S.out_lds + oc * PWC_TILE + j] = v;
            if (p < HW) S.y[(long long)oc * HW + p] = v;
        }
    }
}

// A 3x3 depthwise stage (stage 0): lane (j, slot) of the workgroup takes
// pixel j of the tile in channels slot, slot + 16, ... (PWC_DWC of them a
// round: a load instruction then reads 16 consecutive pixels of four
// channels), loads the weights and every tap of the round first, then runs
// each output's chain; taps off the map are skipped as the standalone
// kernel skips them.
__device__ __forceinline__ void pwc_depthwise(const PwcStage &S, const PwcChain &C, float *smem, int p0, int tid) {
    const int HW = C.hw, W = C.w, H = C.h;
    const int j = tid & (PWC_TILE - 1), slot = tid / PWC_TILE;  // 16 slots
    const int q = p0 + j;
    const bool live = q < HW;
    const int oy = live ? q / W : 0, ox = live ? q - oy * W : 0;
    unsigned inb = 0;
#pragma unroll
    for (int t = 0; t < 9; t++) {
        const int iy = oy - 1 + t / 3, ix = ox - 1 + t % 3;
        inb |= (live && (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W) ? (1u << t) : 0u;
    }
    const int pix = oy * W + ox;
#pragma unroll 1
    for (int c0 = slot; c0 < S.m; c0 += 16 * PWC_DWC) {
        float wv[PWC_DWC][9], tap[PWC_DWC][9], b0[PWC_DWC];
#pragma unroll
        for (int u = 0; u < PWC_DWC; u++) {
            const int ch = c0 + 16 * u;
            const bool any = ch < S.m;
            const float *xc = S.x + (long long)(any ? ch : 0) * HW + pix;
#pragma unroll
            for (int t = 0; t < 9; t++) {
                wv[u][t] = any ? S.w[ch * 9 + t] : 0.f;
                tap[u][t] = any && (inb & (1u << t)) ? xc[(t / 3 - 1) * W + (t % 3 - 1)] : 0.f;
            }
            b0[u] = any && S.bias ? S.bias[ch] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < PWC_DWC; u++) {
            const int ch = c0 + 16 * u;
            if (ch >= S.m) continue;
            float v = 0.f;
            if (live) {
                float acc = b0[u];
#pragma unroll
                for (int t = 0; t < 9; t++)
                    if (inb & (1u << t)) acc = __builtin_fmaf(wv[u][t], tap[u][t], acc);
                v = act_rt(S.act, acc);
                if (S.res) v += S.res[(long long)ch * HW + q];
                S.y[(long long)ch * HW + q] = v;
            }
            if (S.out_lds >= 0) smem[S.out_lds + ch * PWC_TILE + j] = v;
        }
    }
}

__global__ __launch_bounds__(PWC_THREADS) void pw_chain_kernel(PwcArgs a) {
    extern __shared__ __align__(16) float smem[];
    const int b = blockIdx.x;
    int ci = 0;
    while (ci + 1 < a.count && b >= a.start[ci + 1]) ci++;
    const PwcChain &C = a.ch[ci];
    const int p0 = (b - a.start[ci]) * PWC_TILE;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int HW = C.hw;
    const int p = p0 + (lane & 15);  // this lane's pixel in the MFMA epilogue

    // everything the launch reads from memory is in flight from the start:
    // the 1x1 stages' weights (straight to LDS), the staged tensors and
    // biases, then the depthwise stage's taps
    pwc_weights_in(C, smem, wave, lane);
    pwc_stage_in(C, smem, p0, tid);
    const int s1 = C.st[0].kind == OSH_PW_DW3X3 ? 1 : 0;
    if (s1 == 1) pwc_depthwise(C.st[0], C, smem, p0, tid);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's direct-to-LDS weight loads have landed
    __syncthreads();
    for (int s = s1; s < C.nstages; s++) {
        pwc_run(C.st[s], smem, wave, lane, p, HW);
        if (s + 1 < C.nstages) __syncthreads();  // the stage's output in LDS is complete before later stages read it
    }
}

static bool overlaps(const void *a, size_t na, const void *b, size_t nb) {
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a && b && a0 < b0 + nb && b0 < a0 + na;
}

}  // namespace osh

extern "C" {

OSH_API osh_status osh_pw_chain_f32(int count, const osh_pw_chain *chains, osh_stream s) {
    if (count < 1 || count > OSH_PW_MAX_CHAINS || !chains)
        return fail(OSH_E_INVALID, "pointwise chain: %d chains (1..%d)", count, OSH_PW_MAX_CHAINS);
    PwcArgs args;
    memset(&args, 0, sizeof(args));
    args.count = count;
    long long total = 0;
    size_t lds_floats = 0;
    // every tensor a launch reads from memory, and every tensor it writes
    // a 1x1 stage reads and writes only its own tile's pixels, and a tile
    // reads everything it reads from memory before any stage writes: within
    // one chain a stage may overwrite what it or an earlier stage read (same
    // pixels: whole-plane offsets); a depthwise stage reads neighbouring
    // tiles, so nothing may write its input
    struct Span {
        const void *p;
        size_t bytes;
        int chain, stage;
        bool halo;
    };
    Span reads[OSH_PW_MAX_CHAINS * OSH_PW_MAX_STAGES * (OSH_PW_MAX_SRC + 2)];
    Span writes[OSH_PW_MAX_CHAINS * OSH_PW_MAX_STAGES];
    int nr = 0, nw = 0;
    for (int ci = 0; ci < count; ci++) {
        const osh_pw_chain &ch = chains[ci];
        PwcChain &D = args.ch[ci];
        if (ch.h <= 0 || ch.w <= 0 || ch.nstages < 1 || ch.nstages > OSH_PW_MAX_STAGES)
            return fail(OSH_E_INVALID, "pointwise chain %d: %dx%d map, %d stages (1..%d)", ci, ch.h, ch.w,
                        ch.nstages, OSH_PW_MAX_STAGES);
        const long long hw = (long long)ch.h * ch.w;
        if (hw * 512 * 4 > 0x7fffffffLL) return fail(OSH_E_UNSUPPORTED, "pointwise chain %d: map too large", ci);
        if (hw % 4 != 0) return fail(OSH_E_UNSUPPORTED, "pointwise chain %d: H*W = %lld not a multiple of 4", ci, hw);
        D.h = ch.h;
        D.w = ch.w;
        D.hw = (int)hw;
        D.nstages = ch.nstages;
        // LDS: the biases of the 1x1 stages, the tensors they read from
        // memory, then the outputs later stages read; nothing is reused
        bool kept[OSH_PW_MAX_STAGES] = {};
        for (int k = 0; k < ch.nstages; k++) {
            const osh_pw_stage &S = ch.stage[k];
            for (int i = 0; i < S.nsrc && i < OSH_PW_MAX_SRC; i++)
                if (S.src_stage[i] >= 0 && S.src_stage[i] < k) kept[S.src_stage[i]] = true;
            if (S.res_stage >= 0 && S.res_stage < k) kept[S.res_stage] = true;
        }
        int off = 0;
        int out_lds[OSH_PW_MAX_STAGES];
        int part_lds[OSH_PW_MAX_STAGES][OSH_PW_MAX_SRC] = {}, part_first[OSH_PW_MAX_STAGES][OSH_PW_MAX_SRC] = {};
        int part_src[OSH_PW_MAX_STAGES][OSH_PW_MAX_SRC] = {};
        D.nseg = 0;
        auto add_seg = [&](const float *ptr, int c) -> int {
            if (D.nseg == PWC_MAXSEG) return -1;
            D.seg_ptr[D.nseg] = ptr;
            D.seg_lds[D.nseg] = off;
            D.seg_start[D.nseg + 1] = D.seg_start[D.nseg] + c * (PWC_TILE / 4);
            D.nseg++;
            const int at = off;
            off += c * PWC_TILE;
            return at;
        };
        for (int k = 0; k < ch.nstages; k++) {
            const osh_pw_stage &S = ch.stage[k];
            PwcStage &T = D.st[k];
            if (S.kind != OSH_PW_1X1 && S.kind != OSH_PW_DW3X3)
                return fail(OSH_E_INVALID, "pointwise chain %d stage %d: unknown kind %d", ci, k, S.kind);
            if (S.m <= 0 || !S.w || !S.y)
                return fail(OSH_E_INVALID, "pointwise chain %d stage %d: m=%d, weights or output missing", ci, k, S.m);
            if (S.act != OSH_ACT_NONE && S.act != OSH_ACT_RELU && S.act != OSH_ACT_SILU)
                return fail(OSH_E_INVALID, "pointwise chain %d stage %d: unknown activation %d", ci, k, S.act);
            if (S.nsrc < 1 || S.nsrc > OSH_PW_MAX_SRC)
                return fail(OSH_E_INVALID, "pointwise chain %d stage %d: %d input parts", ci, k, S.nsrc);
            T.kind = S.kind;
            T.m = S.m;
            T.act = (S.act == OSH_ACT_SILU && exact_silu()) ? ACT_SILU_EXACT : S.act;
            T.w = static_cast<const float *>(S.w);
            T.bias = S.bias;
            T.y = S.y;
            T.bias_lds = -1;
            T.res_lds = -1;
            if (S.kind == OSH_PW_DW3X3) {
                if (S.m > 256) return fail(OSH_E_UNSUPPORTED, "pointwise chain %d: depthwise over %d channels (256 at most)", ci, S.m);
                if (k != 0 || S.nsrc != 1 || S.src_stage[0] >= 0 || S.src_c[0] != S.m || !S.src[0])
                    return fail(OSH_E_INVALID,
                                "pointwise chain %d stage %d: a depthwise stage is stage 0 over one tensor with m "
                                "channels", ci, k);
                if (S.res_stage >= 0)
                    return fail(OSH_E_INVALID, "pointwise chain %d stage %d: residual names stage %d", ci, k,
                                S.res_stage);
                T.x = S.src[0];
                T.res = S.res;
                T.c = S.m;
                reads[nr++] = Span{S.src[0], (size_t)S.m * hw * sizeof(float), ci, k, true};
                // the depthwise stage reads its residual from memory while other
                // waves write neighbouring channels of y: y may be the residual
                // itself (each element read and written by one thread), but it
                // may not overlap it anywhere else
                if (S.res) reads[nr++] = Span{S.res, (size_t)S.m * hw * sizeof(float), ci, k, S.res != S.y};
                writes[nw++] = Span{S.y, (size_t)S.m * hw * sizeof(float), ci, k, false};
                continue;
            }
            if (S.m % 16 != 0) return fail(OSH_E_INVALID, "pointwise chain %d stage %d: m=%d not a multiple of 16", ci, k, S.m);
            if (S.m > PWC_MAXC)
                return fail(OSH_E_UNSUPPORTED, "pointwise chain %d stage %d: m=%d (%d at most)", ci, k, S.m, PWC_MAXC);
            if (S.bias) {
                T.bias_lds = off;
                off += (S.m + 3) / 4 * 4;
            }
            // input parts: a part in memory is staged (its LDS offset known
            // now); a part of a stage's output is placed with the kept outputs
            int c = 0;
            for (int i = 0; i < S.nsrc; i++) {
                const int src = S.src_stage[i];
                if (S.src_c[i] <= 0 || S.src_c[i] % 16 != 0)
                    return fail(OSH_E_INVALID, "pointwise chain %d stage %d: part %d has %d channels (a positive "
                                "multiple of 16 is needed)", ci, k, i, S.src_c[i]);
                part_first[k][i] = c / 16;
                part_src[k][i] = src;
                if (src >= 0) {
                    // the whole output of stage src, or the channels of it that
                    // src[i] points at
                    long long c0 = 0;
                    if (src < k && S.src[i]) {
                        const long long d = (const float *)S.src[i] - (const float *)ch.stage[src].y;
                        c0 = d % hw == 0 ? d / hw : -1;
                    }
                    if (src >= k || c0 < 0 || c0 + S.src_c[i] > ch.stage[src].m)
                        return fail(OSH_E_INVALID, "pointwise chain %d stage %d: part %d is not within stage %d's "
                                    "output", ci, k, i, src);
                    part_lds[k][i] = (int)c0 * PWC_TILE;  // within the stage's output
                } else {
                    if (!S.src[i]) return fail(OSH_E_INVALID, "pointwise chain %d stage %d: part %d is NULL", ci, k, i);
                    if (S.src_c[i] > PWC_MAXC || (reinterpret_cast<uintptr_t>(S.src[i]) & 15) != 0)
                        return fail(OSH_E_UNSUPPORTED, "pointwise chain %d stage %d: part %d (%d channels, 16-byte "
                                    "aligned up to %d)", ci, k, i, S.src_c[i], PWC_MAXC);
                    part_lds[k][i] = add_seg(S.src[i], S.src_c[i]);
                    if (part_lds[k][i] < 0)
                        return fail(OSH_E_UNSUPPORTED, "pointwise chain %d: more than %d tensors in memory", ci,
                                    PWC_MAXSEG);
                    reads[nr++] = Span{S.src[i], (size_t)S.src_c[i] * hw * sizeof(float), ci, k, false};
                }
                c += S.src_c[i];
            }
            T.c = c;
            T.w_lds = off;  // the packed weights: M*C floats
            off += S.m * c;
            if (S.res_stage >= 0) {
                if (S.res_stage >= k || ch.stage[S.res_stage].m != S.m)
                    return fail(OSH_E_INVALID, "pointwise chain %d stage %d: residual names stage %d", ci, k,
                                S.res_stage);
                T.res = nullptr;  // T.res_lds is placed with the kept outputs
            } else if (S.res) {
                T.res_lds = add_seg(S.res, S.m);
                if (T.res_lds < 0)
                    return fail(OSH_E_UNSUPPORTED, "pointwise chain %d: more than %d tensors in memory", ci, PWC_MAXSEG);
                T.res = nullptr;
                reads[nr++] = Span{S.res, (size_t)S.m * hw * sizeof(float), ci, k, false};
            }
            osh_conv_params p{};
            p.n = 1; p.c = c; p.h = ch.h; p.w = ch.w; p.m = S.m; p.kh = 1; p.kw = 1; p.group = 1;
            p.sh = 1; p.sw = 1; p.dh = 1; p.dw = 1; p.oh = ch.h; p.ow = ch.w;
            if (!packed_for_pointwise_tiles(&p, S.w))
                return fail(OSH_E_INVALID,
                            "pointwise chain %d stage %d: weights not packed by osh_conv_pack_weights for the "
                            "1x1 conv %d -> %d at %dx%d", ci, k, c, S.m, ch.h, ch.w);
            writes[nw++] = Span{S.y, (size_t)S.m * hw * sizeof(float), ci, k, false};
        }
        for (int k = 0; k < ch.nstages; k++) {
            out_lds[k] = kept[k] ? off : -1;
            if (kept[k]) off += ch.stage[k].m * PWC_TILE;
        }
        // second pass: the LDS offsets of parts and residuals that are stage
        // outputs, and the B addressing (block icb of part i sits at
        // lds[i] + (icb - first[i]) * 256)
        for (int k = 0; k < ch.nstages; k++) {
            const osh_pw_stage &S = ch.stage[k];
            PwcStage &T = D.st[k];
            T.out_lds = out_lds[k];
            if (S.kind == OSH_PW_DW3X3) continue;
            const int np = S.nsrc;
            int lds[OSH_PW_MAX_SRC];
            for (int i = 0; i < np; i++)
                lds[i] = part_src[k][i] >= 0 ? out_lds[part_src[k][i]] + part_lds[k][i] : part_lds[k][i];
            T.e0 = np > 1 ? part_first[k][1] : 1 << 30;
            T.e1 = np > 2 ? part_first[k][2] : 1 << 30;
            T.l0 = lds[0] - part_first[k][0] * 256;
            T.l1 = np > 1 ? lds[1] - part_first[k][1] * 256 : T.l0;
            T.l2 = np > 2 ? lds[2] - part_first[k][2] * 256 : T.l1;
            if (S.res_stage >= 0) T.res_lds = out_lds[S.res_stage];
        }
        if ((size_t)off > lds_floats) lds_floats = (size_t)off;
        args.start[ci] = (int)total;
        total += (hw + PWC_TILE - 1) / PWC_TILE;
    }
    args.start[count] = (int)total;
    for (int i = 0; i < nw; i++) {
        const Span &W = writes[i];
        for (int k = 0; k < nr; k++) {
            const Span &R = reads[k];
            if (!overlaps(W.p, W.bytes, R.p, R.bytes)) continue;
            const long long plane = (long long)args.ch[W.chain].hw * sizeof(float);
            const long long d = (long long)(reinterpret_cast<uintptr_t>(W.p) - reinterpret_cast<uintptr_t>(R.p));
            if (R.halo || W.chain != R.chain || W.stage < R.stage || d % plane != 0)
                return fail(OSH_E_INVALID, "pointwise chain: an output overlaps a tensor the launch reads");
        }
        for (int k = 0; k < i; k++)
            if (overlaps(writes[i].p, writes[i].bytes, writes[k].p, writes[k].bytes))
                return fail(OSH_E_INVALID, "pointwise chain: two outputs overlap");
    }
    const size_t lds_bytes = lds_floats * sizeof(float);
    if (lds_bytes > 160 * 1024)
        return fail(OSH_E_UNSUPPORTED, "pointwise chain: %zu bytes of LDS (160 KB available)", lds_bytes);
    if (lds_bytes > 64 * 1024) {
        static std::once_flag once;
        hipError_t e = hipSuccess;
        std::call_once(once, [&] {
            e = hipFuncSetAttribute(reinterpret_cast<const void *>(pw_chain_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        });
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail(OSH_E_DEVICE, "pointwise chain: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
        }
    }
    OSH_LAUNCH(pw_chain_kernel, dim3((unsigned)total), dim3(PWC_THREADS), lds_bytes, to_stream(s), args);
    OSH_LAUNCH_CHECK("pw_chain_kernel");
    return OSH_OK;
}

}  // extern "C"
