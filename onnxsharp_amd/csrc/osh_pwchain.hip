// osh_pwchain.hip -- chains of pointwise convolutions in one launch.
//
// A YOLO11n frame is launch-bound: most of its 1x1 convs at 20x20 and 40x40
// take about the ~3.5 us a launch costs in a HIP graph whatever it does.  Runs
// of 1x1 convs that feed each other (C2PSA's proj -> ffn.0 -> ffn.1 -> cv2,
// the detection head's depthwise -> 1x1 -> 1x1 tails, C3k2's cv1 -> C3k cv1/cv2)
// go through this kernel as one launch: a workgroup takes 16 consecutive
// pixels through every stage, keeping each stage's output on chip (LDS) for
// the stages that read it, and writing it to its tensor as well.
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
// (j, g) holds channels 4g + r of pixel j.  A (weights) comes from the
// pointwise LDS-tile pack ([M/16][C/16][64 lanes][4 steps], 16 bytes a lane
// per four k-steps), B from LDS ([channel][16 pixels]: the 16 lanes of a
// group read 16 consecutive words, the four groups four rows 16 words apart,
// so a half-wave read hits 32 banks).  Parts that live in memory are staged
// into LDS first; earlier stages' outputs are already there.
#include "osh_common.h"
#include "osh_launch.h"

#include <cstring>

using namespace osh;

namespace osh {

constexpr int PWC_NW = 8;  // waves per workgroup
constexpr int PWC_THREADS = 64 * PWC_NW;
constexpr int PWC_TILE = 16;  // pixels per workgroup: one MFMA column block
constexpr int PWC_KA = 8;     // 16-channel weight blocks per load group (double-buffered)
constexpr int PWC_MAXC = 512;  // channels of a part in memory, and of a depthwise stage's input (256)
constexpr int PWC_SPT = PWC_MAXC * PWC_TILE / 4 / PWC_THREADS;  // 16-byte staging loads a thread
constexpr int PWC_DWE = 256 * PWC_TILE / PWC_THREADS;          // depthwise outputs a thread (8: half a tile row)
static_assert(PWC_TILE % PWC_DWE == 0, "a thread's depthwise outputs lie in one channel");

struct PwcPart {
    const float *ptr;  // tensor in memory (staged), or nullptr for a stage output
    int lds;           // float offset of the part's channel 0 in LDS
    int c;             // channels
};

struct PwcStage {
    const float *w;
    const float *bias;
    const float *res;
    float *y;
    PwcPart part[OSH_PW_MAX_SRC];
    int kind, m, act, nsrc, c;
    int res_lds;  // the residual's float offset in LDS (an earlier stage), or -1
    int out_lds;  // this stage's output in LDS, or -1 when no later stage reads it
};

struct PwcChain {
    int h, w, hw, nstages;
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

__global__ __launch_bounds__(PWC_THREADS) void pw_chain_kernel(PwcArgs a) {
    extern __shared__ __align__(16) float smem[];
    const int b = blockIdx.x;
    int ci = 0;
    while (ci + 1 < a.count && b >= a.start[ci + 1]) ci++;
    const PwcChain &C = a.ch[ci];
    const int p0 = (b - a.start[ci]) * PWC_TILE;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int HW = C.hw;
    const int p = p0 + j;  // this lane's pixel in the MFMA epilogue

    for (int s = 0; s < C.nstages; s++) {
        const PwcStage &S = C.st[s];
        if (S.kind == OSH_PW_DW3X3) {
            // a thread takes PWC_DWE consecutive pixels of one channel (two
            // threads a channel), loads its nine weights and every tap first,
            // then runs each output's chain; taps off the map are skipped as
            // the standalone kernel skips them
            const float *x = S.part[0].ptr;
            const float *w = static_cast<const float *>(S.w);
            const int e0 = tid * PWC_DWE, ch = e0 / PWC_TILE;
            if (ch < S.m) {
                const float *xc = x + (long long)ch * HW;
                float wv[9], tap[PWC_DWE][9];
                unsigned inb[PWC_DWE];
#pragma unroll
                for (int t = 0; t < 9; t++) wv[t] = w[ch * 9 + t];
#pragma unroll
                for (int u = 0; u < PWC_DWE; u++) {
                    const int q = p0 + (e0 + u) % PWC_TILE;
                    const bool live = q < HW;
                    const int oy = live ? q / C.w : 0, ox = live ? q - oy * C.w : 0;
                    inb[u] = 0;
#pragma unroll
                    for (int t = 0; t < 9; t++) {
                        const int iy = oy - 1 + t / 3, ix = ox - 1 + t % 3;
                        const bool in = live && (unsigned)iy < (unsigned)C.h && (unsigned)ix < (unsigned)C.w;
                        tap[u][t] = in ? xc[iy * C.w + ix] : 0.f;
                        inb[u] |= in ? (1u << t) : 0u;
                    }
                }
                const float b0 = S.bias ? S.bias[ch] : 0.f;
#pragma unroll
                for (int u = 0; u < PWC_DWE; u++) {
                    const int q = p0 + (e0 + u) % PWC_TILE;
                    float v = 0.f;
                    if (q < HW) {
                        float acc = b0;
#pragma unroll
                        for (int t = 0; t < 9; t++)
                            if (inb[u] & (1u << t)) acc = __builtin_fmaf(wv[t], tap[u][t], acc);
                        v = act_rt(S.act, acc);
                        if (S.res) v += S.res[(long long)ch * HW + q];
                        S.y[(long long)ch * HW + q] = v;
                    }
                    if (S.out_lds >= 0) smem[S.out_lds + e0 + u] = v;
                }
            }
            __syncthreads();
            continue;
        }
        // parts that live in memory come into LDS ([channel][16 pixels]) as
        // 16-byte loads, all of a part's issued before any is written; pixels
        // past the map read 0 (HW % 4 == 0, so a 4-pixel group is wholly in or out)
        for (int i = 0; i < S.nsrc; i++) {
            const PwcPart &P = S.part[i];
            if (!P.ptr) continue;
            float4 v[PWC_SPT];
#pragma unroll
            for (int u = 0; u < PWC_SPT; u++) {
                const int e4 = tid + u * PWC_THREADS;  // a group of four pixels
                const int ch = e4 / (PWC_TILE / 4), q = p0 + (e4 % (PWC_TILE / 4)) * 4;
                v[u] = (ch < P.c && q < HW) ? *reinterpret_cast<const float4 *>(P.ptr + (long long)ch * HW + q)
                                            : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < PWC_SPT; u++) {
                const int e4 = tid + u * PWC_THREADS;
                if (e4 / (PWC_TILE / 4) < P.c) *reinterpret_cast<float4 *>(smem + P.lds + 4 * e4) = v[u];
            }
        }
        __syncthreads();
        const int MB = S.m / 16, ICB = S.c / 16;
        const float4 *wpk = reinterpret_cast<const float4 *>(S.w);
        // the LDS float offset of 16-channel input block icb
        auto block_base = [&](int icb) {
            int c0 = icb * 16;
            int k = 0;
            while (k + 1 < S.nsrc && c0 >= S.part[k].c) c0 -= S.part[k].c, k++;
            return S.part[k].lds + c0 * PWC_TILE;
        };
        for (int mb = wave; mb < MB; mb += PWC_NW) {
            f32x4 acc;
            float rv[4];  // a residual in memory, loaded before the chain
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int oc = mb * 16 + 4 * g + r;
                acc[r] = S.bias ? S.bias[oc] : 0.f;
                rv[r] = (S.res_lds < 0 && S.res && p < HW) ? S.res[(long long)oc * HW + p] : 0.f;
            }
            float4 A0[PWC_KA], A1[PWC_KA];
            auto load = [&](float4 (&A)[PWC_KA], int k0) {
#pragma unroll
                for (int i = 0; i < PWC_KA; i++) {
                    const int icb = k0 + i < ICB ? k0 + i : ICB - 1;  // past the end: a block never used
                    A[i] = wpk[((long long)mb * ICB + icb) * 64 + lane];
                }
            };
            auto compute = [&](const float4 (&A)[PWC_KA], int k0) {
#pragma unroll
                for (int i = 0; i < PWC_KA; i++) {
                    if (k0 + i >= ICB) break;
                    const float *lb = smem + block_base(k0 + i) + g * PWC_TILE + j;
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[i].x, lb[0 * PWC_TILE], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[i].y, lb[4 * PWC_TILE], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[i].z, lb[8 * PWC_TILE], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[i].w, lb[12 * PWC_TILE], acc, 0, 0, 0);
                }
            };
            load(A0, 0);
            for (int k0 = 0; k0 < ICB; k0 += 2 * PWC_KA) {
                if (k0 + PWC_KA < ICB) load(A1, k0 + PWC_KA);
                compute(A0, k0);
                if (k0 + PWC_KA >= ICB) break;
                if (k0 + 2 * PWC_KA < ICB) load(A0, k0 + 2 * PWC_KA);
                compute(A1, k0 + PWC_KA);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int oc = mb * 16 + 4 * g + r;
                float v = act_rt(S.act, acc[r]);
                if (S.res_lds >= 0) v += smem[S.res_lds + oc * PWC_TILE + j];
                else if (S.res) v += rv[r];
                if (S.out_lds >= 0) smem[S.out_lds + oc * PWC_TILE + j] = v;
                if (p < HW) S.y[(long long)oc * HW + p] = v;
            }
        }
        __syncthreads();
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
    // runs its stages in order: within one chain a stage may overwrite what
    // it or an earlier stage read (same pixels: whole-plane offsets); a
    // depthwise stage reads neighbouring tiles, so nothing may write its input
    struct Span {
        const void *p;
        size_t bytes;
        int chain, stage;
        bool halo;
    };
    Span reads[OSH_PW_MAX_CHAINS * OSH_PW_MAX_STAGES * (OSH_PW_MAX_SRC + 1)];
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
        // LDS: the staging region for parts in memory at 0, then the outputs
        // later stages read
        int stage_floats = 0;
        bool kept[OSH_PW_MAX_STAGES] = {};
        for (int k = 0; k < ch.nstages; k++) {
            const osh_pw_stage &S = ch.stage[k];
            int staged = 0;
            for (int i = 0; i < S.nsrc && i < OSH_PW_MAX_SRC; i++) {
                if (S.src_stage[i] >= 0 && S.src_stage[i] < k) kept[S.src_stage[i]] = true;
                if (S.src_stage[i] < 0) staged += S.src_c[i];
            }
            if (S.res_stage >= 0 && S.res_stage < k) kept[S.res_stage] = true;
            if (S.kind == OSH_PW_1X1 && staged * PWC_TILE > stage_floats) stage_floats = staged * PWC_TILE;
        }
        int off = stage_floats;
        int out_lds[OSH_PW_MAX_STAGES];
        for (int k = 0; k < ch.nstages; k++) {
            out_lds[k] = kept[k] ? off : -1;
            if (kept[k]) off += ch.stage[k].m * PWC_TILE;
        }
        if ((size_t)off > lds_floats) lds_floats = (size_t)off;
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
            T.nsrc = S.nsrc;
            T.w = static_cast<const float *>(S.w);
            T.bias = S.bias;
            T.y = S.y;
            T.out_lds = out_lds[k];
            int c = 0, staged = 0;
            for (int i = 0; i < S.nsrc; i++) {
                const int src = S.src_stage[i];
                if (S.src_c[i] <= 0) return fail(OSH_E_INVALID, "pointwise chain %d stage %d: part %d empty", ci, k, i);
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
                    T.part[i] = PwcPart{nullptr, out_lds[src] + (int)c0 * PWC_TILE, S.src_c[i]};
                } else {
                    if (!S.src[i]) return fail(OSH_E_INVALID, "pointwise chain %d stage %d: part %d is NULL", ci, k, i);
                    if (S.src_c[i] > PWC_MAXC || (reinterpret_cast<uintptr_t>(S.src[i]) & 15) != 0)
                        return fail(OSH_E_UNSUPPORTED, "pointwise chain %d stage %d: part %d (%d channels, 16-byte "
                                    "aligned up to %d)", ci, k, i, S.src_c[i], PWC_MAXC);
                    T.part[i] = PwcPart{S.src[i], staged * PWC_TILE, S.src_c[i]};
                    staged += S.src_c[i];
                    reads[nr++] = Span{S.src[i], (size_t)S.src_c[i] * hw * sizeof(float), ci, k,
                                       S.kind == OSH_PW_DW3X3};
                }
                c += S.src_c[i];
            }
            T.c = c;
            if (S.res_stage >= 0) {
                if (S.res_stage >= k || ch.stage[S.res_stage].m != S.m)
                    return fail(OSH_E_INVALID, "pointwise chain %d stage %d: residual names stage %d", ci, k,
                                S.res_stage);
                T.res_lds = out_lds[S.res_stage];
                T.res = nullptr;
            } else {
                T.res_lds = -1;
                T.res = S.res;
                if (S.res) reads[nr++] = Span{S.res, (size_t)S.m * hw * sizeof(float), ci, k, false};
            }
            if (S.kind == OSH_PW_DW3X3) {
                if (S.m > 256) return fail(OSH_E_UNSUPPORTED, "pointwise chain %d: depthwise over %d channels (256 at most)", ci, S.m);
                if (k != 0 || S.nsrc != 1 || S.src_stage[0] >= 0 || S.src_c[0] != S.m)
                    return fail(OSH_E_INVALID,
                                "pointwise chain %d stage %d: a depthwise stage is stage 0 over one tensor with m "
                                "channels", ci, k);
                reads[nr++] = Span{S.w, (size_t)S.m * 9 * sizeof(float), ci, k, true};
            } else {
                if (S.m % 16 != 0) return fail(OSH_E_INVALID, "pointwise chain %d stage %d: m=%d not a multiple of 16", ci, k, S.m);
                for (int i = 0; i < S.nsrc; i++)
                    if (S.src_c[i] % 16 != 0)
                        return fail(OSH_E_INVALID, "pointwise chain %d stage %d: part %d has %d channels (a multiple "
                                    "of 16 is needed)", ci, k, i, S.src_c[i]);
                osh_conv_params p{};
                p.n = 1; p.c = c; p.h = ch.h; p.w = ch.w; p.m = S.m; p.kh = 1; p.kw = 1; p.group = 1;
                p.sh = 1; p.sw = 1; p.dh = 1; p.dw = 1; p.oh = ch.h; p.ow = ch.w;
                if (!packed_for_pointwise_tiles(&p, S.w))
                    return fail(OSH_E_INVALID,
                                "pointwise chain %d stage %d: weights not packed by osh_conv_pack_weights for the "
                                "1x1 conv %d -> %d at %dx%d", ci, k, c, S.m, ch.h, ch.w);
            }
            writes[nw++] = Span{S.y, (size_t)S.m * hw * sizeof(float), ci, k, false};
        }
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
    hipLaunchKernelGGL(pw_chain_kernel, dim3((unsigned)total), dim3(PWC_THREADS), lds_bytes, to_stream(s), args);
    OSH_LAUNCH_CHECK("pw_chain_kernel");
    return OSH_OK;
}

}  // extern "C"
