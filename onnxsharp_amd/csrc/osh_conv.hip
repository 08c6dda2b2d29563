// osh_conv.hip -- Conv entry points of the C ABI: shape logic of ConvLayer
// (src/OnnxSharp/Ops/DnnOps.cs:53-89,134-201,379-409) and the kernel choice
// of ConvLayer.Forward (DnnOps.cs:411-500), re-planned for gfx950.  The
// choice follows the reference's kernel chain on an AVX-512 host --
// DepthwiseConv, FirstConv, NchwcConv, Winograd, PackedConv, Im2Col, first
// gate that holds -- and every kernel sums in the order of the reference's
// kernel for that shape, so the outputs are its bits:
//
//   depthwise (group == C == M)         -> dw_conv_kernel (ky -> kx FMA chain, DepthwiseConv.cs)
//   3x3, C <= 4, M = 8/16/32, group 1   -> first_conv_kernel (the network's first layer,
//                                          FirstConv.cs: the ic -> ky -> kx FMA chain)
//   NchwcConv's gate (3x3, stride 1 or 2, pad 1, C % 16 == 0, M % 32 == 0, batch 1,
//   NchwcConv.cs:100-126)               -> in-order 16x16x4 MFMA kernels (osh_conv16.h,
//                                          osh_conv16s.h): the NCHWc chain icb -> ky -> kx -> ic16
//   Winograd's gate (3x3 s1 p1, C, M >= 8, H*W <= 4096, Winograd.cs:58-122)
//                                       -> wino_f23_kernel (osh_winograd.h): Winograd.cs's
//                                          transforms and component GEMMs
//   other 3x3, stride 1 or 2, C % 16 == 0
//                                       -> conv16s_kernel<..., I2C> (the LDS-patch tiles with the
//                                          terms of each 16-channel block in the im2col order)
//   other 3x3 with C = 8/16/32, M = 8/16/32
//                                       -> first_conv_kernel (the im2col chain per pixel)
//   1x1 / stride 1 / pad 0, C % 16 == 0 -> the LDS-tile kernel with one tap, or the GEMM tile,
//                                          tuned per shape (the GEMM chain over ic)
//   other 1x1 / stride 1 / pad 0        -> MFMA GEMM over NCHW (W[M,C] x X[C,H*W])
//   everything else                     -> MFMA implicit GEMM with an im2col gather, k in the
//                                          im2col order ic -> ky -> kx (ConvKernels.cs, PackedConv.cs)
//
// osh_config "winograd" = 0 leaves Winograd out (those shapes take the im2col
// chain), 2 puts it ahead of the NCHWc kernels (the reference's choice on a
// host without AVX-512, for the Winograd-eligible shapes).  A forced
// "conv16_variant" >= 0 runs the NCHWc-chain kernels on any 3x3 shape they fit.
//
// Bias and the fused activation (Relu / SiLU, GraphFusion.cs:1713-1718) are
// applied in registers before the single store, then an optional residual.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <map>
#include <mutex>
#include <tuple>
#include <utility>

#include "osh_conv16.h"
#include "osh_conv16s.h"
#include "osh_conv_pair.h"
#include "osh_igemm.h"
#include "osh_launch.h"
#include "osh_winograd.h"

using namespace osh;

namespace osh {

// DnnOps.cs:53-67 (ceil_mode is false for Conv).
static int spatial_out(int input, int kernel, int stride, int dilation, int pad_begin, int pad_end) {
    int effective = (kernel - 1) * dilation + 1;
    int numerator = input + pad_begin + pad_end - effective;
    return numerator / stride + 1;  // C# integer division truncates toward zero, as C does
}

// DnnOps.cs:69-89.
static void auto_pad(int mode, int input, int kernel, int stride, int dilation, int *begin, int *end) {
    int effective = (kernel - 1) * dilation + 1;
    int output = (input + stride - 1) / stride;  // ceil(input / stride) for positive sizes
    if (mode == OSH_PAD_SAME_UPPER || mode == OSH_PAD_SAME_LOWER) {
        int total = (output - 1) * stride + effective - input;
        if (total < 0) total = 0;
        int b = mode == OSH_PAD_SAME_UPPER ? total / 2 : total - total / 2;
        *begin = b;
        *end = total - b;
    } else {  // VALID
        *begin = 0;
        *end = 0;
    }
}

static osh_status check_attrs(const osh_conv_attrs *at, const int64_t x[4], const int64_t w[4]) {
    if (!at || !x || !w) return fail(OSH_E_INVALID, "Conv: NULL argument");
    if (at->n_kernel_shape < 0 || at->n_kernel_shape > 2 || at->n_strides < 0 || at->n_strides > 2 ||
        at->n_dilations < 0 || at->n_dilations > 2 || at->n_pads < 0 || at->n_pads > 4)
        return fail(OSH_E_INVALID, "Conv: attribute list length out of range for a 2-D conv");
    if (at->auto_pad < OSH_PAD_NOTSET || at->auto_pad > OSH_PAD_VALID)
        return fail(OSH_E_INVALID, "Conv: unknown auto_pad %d", at->auto_pad);
    for (int i = 0; i < 4; i++)
        if (x[i] <= 0 || w[i] <= 0 || x[i] > (1 << 30) || w[i] > (1 << 30))
            return fail(OSH_E_INVALID, "Conv: non-positive or oversized dimension");
    long long channels = x[1];
    if (at->group <= 0 || channels % at->group != 0)
        return fail(OSH_E_INVALID, "Conv: channels %lld not divisible by group %d", channels, at->group);
    if (w[1] != channels / at->group)
        return fail(OSH_E_INVALID, "Conv: weight in-channels %lld != %lld", (long long)w[1], channels / at->group);
    if (w[0] % at->group != 0)
        return fail(OSH_E_INVALID, "Conv: output channels %lld not divisible by group %d", (long long)w[0],
                    at->group);
    for (int i = 0; i < at->n_strides; i++)
        if (at->strides[i] <= 0) return fail(OSH_E_INVALID, "Conv: stride must be positive");
    for (int i = 0; i < at->n_dilations; i++)
        if (at->dilations[i] <= 0) return fail(OSH_E_INVALID, "Conv: dilation must be positive");
    for (int i = 0; i < at->n_pads; i++)
        if (at->pads[i] < 0) return fail(OSH_E_UNSUPPORTED, "Conv: negative pads are not supported");
    return OSH_OK;
}

// ---------------------------------------------------------------- depthwise

template <int ACT>
__device__ __forceinline__ void dw_conv_at(const osh_conv_params &p, const float *__restrict__ x,
                                           const float *__restrict__ w, const float *__restrict__ bias,
                                           const float *__restrict__ res, float *__restrict__ y, long long idx) {
    long long total = (long long)p.n * p.m * p.oh * p.ow;
    if (idx >= total) return;
    int ox = (int)(idx % p.ow);
    long long t = idx / p.ow;
    int oy = (int)(t % p.oh);
    t /= p.oh;
    int c = (int)(t % p.m);
    int n = (int)(t / p.m);
    const float *xc = x + ((long long)n * p.c + c) * p.h * p.w;
    const float *wc = w + (long long)c * p.kh * p.kw;
    float acc = bias ? bias[c] : 0.f;
    for (int ky = 0; ky < p.kh; ky++) {
        int iy = oy * p.sh - p.pt + ky * p.dh;
        if ((unsigned)iy >= (unsigned)p.h) continue;
        for (int kx = 0; kx < p.kw; kx++) {
            int ix = ox * p.sw - p.pl + kx * p.dw;
            if ((unsigned)ix >= (unsigned)p.w) continue;
            acc = __builtin_fmaf(wc[ky * p.kw + kx], xc[(long long)iy * p.w + ix], acc);
        }
    }
    float v = activate<ACT>(acc);
    if (res) v += res[idx];
    y[idx] = v;
}

// The 3x3 stride-S, dilation-1 case of dw_conv_at (every depthwise layer of
// YOLO11n): 32-bit indices, and the nine weights and the in-map taps loaded
// before the chain starts, so the loads are in flight together; taps off the
// map are skipped, as in dw_conv_at (an fma with a zero tap could turn a -0
// accumulator into +0).
inline bool dw3_eligible(const osh_conv_params *p) {
    return p->kh == 3 && p->kw == 3 && p->dh == 1 && p->dw == 1 && p->sh == p->sw && (p->sh == 1 || p->sh == 2) &&
           (long long)p->n * p->m * p->oh * p->ow < (1LL << 31) && (long long)p->n * p->c * p->h * p->w < (1LL << 31);
}

template <int ACT, int S>
__device__ __forceinline__ void dw3_conv_at(const osh_conv_params &p, const float *__restrict__ x,
                                            const float *__restrict__ w, const float *__restrict__ bias,
                                            const float *__restrict__ res, float *__restrict__ y, int idx) {
    const int total = p.n * p.m * p.oh * p.ow;
    if (idx >= total) return;
    const int ox = idx % p.ow;
    int t = idx / p.ow;
    const int oy = t % p.oh;
    t /= p.oh;
    const int c = t % p.m, n = t / p.m;
    const float *xc = x + (n * p.c + c) * p.h * p.w;
    const float *wc = w + c * 9;
    const int iy0 = oy * S - p.pt, ix0 = ox * S - p.pl;
    float wv[9], tap[9];
    unsigned in = 0;
#pragma unroll
    for (int k = 0; k < 9; k++) {
        const int iy = iy0 + k / 3, ix = ix0 + k % 3;
        const bool ok = (unsigned)iy < (unsigned)p.h && (unsigned)ix < (unsigned)p.w;
        in |= ok ? 1u << k : 0u;
        wv[k] = wc[k];
        tap[k] = ok ? xc[iy * p.w + ix] : 0.f;
    }
    float acc = bias ? bias[c] : 0.f;
#pragma unroll
    for (int k = 0; k < 9; k++)
        if (in & (1u << k)) acc = __builtin_fmaf(wv[k], tap[k], acc);
    float v = activate<ACT>(acc);
    if (res) v += res[idx];
    y[idx] = v;
}

template <int ACT>
__global__ __launch_bounds__(256) void dw_conv_kernel(osh_conv_params p, const float *__restrict__ x,
                                                      const float *__restrict__ w, const float *__restrict__ bias,
                                                      const float *__restrict__ res, float *__restrict__ y) {
    dw_conv_at<ACT>(p, x, w, bias, res, y, (long long)blockIdx.x * blockDim.x + threadIdx.x);
}

template <int ACT, int S>
__global__ __launch_bounds__(256) void dw3_conv_kernel(osh_conv_params p, const float *__restrict__ x,
                                                       const float *__restrict__ w, const float *__restrict__ bias,
                                                       const float *__restrict__ res, float *__restrict__ y) {
    dw3_conv_at<ACT, S>(p, x, w, bias, res, y, blockIdx.x * 256 + threadIdx.x);
}

// Several depthwise convs in one launch: workgroup b covers outputs
// 256 (b - start[i]) .. of conv i (ConvGroup's block table).  S > 0: every
// member is a 3x3 stride-S conv (dw3_eligible).
template <int ACT, int S>
__global__ __launch_bounds__(256) void dw_conv_group_kernel(ConvGroup g) {
    const int b = blockIdx.x;
    int i = 0;
    while (i + 1 < g.count && b >= g.start[i + 1]) i++;
    if constexpr (S > 0)
        dw3_conv_at<ACT, S>(g.p[i], g.x[i], g.w[i], g.bias[i], g.res[i], g.y[i], (b - g.start[i]) * 256 + threadIdx.x);
    else
        dw_conv_at<ACT>(g.p[i], g.x[i], g.w[i], g.bias[i], g.res[i], g.y[i],
                        (long long)(b - g.start[i]) * 256 + threadIdx.x);
}

// ------------------------------------------------------- small-C first layer
//
// The first layer of an image network (C = 3 colour planes): too little K for
// MFMA tiles (27 for 3x3) and HBM-bound (it reads the image once and writes M
// planes).  One thread per output pixel keeps MM accumulators in registers
// (output channels MM * blockIdx.y + 0 .. MM-1: smaller maps split M over
// the grid's y so that more CUs take part); the weight index is the same for
// every lane, so the weights are read as LDS broadcasts.  Per output
// channel the chain is bias, then fmaf over ic -> ky -> kx (the panel order of
// FirstConv.cs:344-362); padding taps add nothing.
template <int MM, int CC, int ACT>
__global__ __launch_bounds__(256) void first_conv_kernel(osh_conv_params p, const float *__restrict__ x,
                                                         const float *__restrict__ w,
                                                         const float *__restrict__ bias,
                                                         const float *__restrict__ res, float *__restrict__ y) {
    // The workgroup's weights (MM output channels x CC x 9) and biases go to
    // LDS and are read back as broadcasts: through the scalar cache an output
    // channel's weights arrived a few words at a time, each batch waited for
    // before its FMAs (the stem at 640x640: 8.2 us).  Their loads, and with
    // CC <= 8 the pixel's input taps, are all issued before the barrier.
    constexpr int NW = MM * CC * 9, NWT = (NW + 255) / 256;
    __shared__ float lw[NW];
    __shared__ float lb[MM];
    const int tid = threadIdx.x;
    const int oc0 = blockIdx.y * MM;
    float wr[NWT];
#pragma unroll
    for (int i = 0; i < NWT; i++) {
        const int e = tid + 256 * i;
        wr[i] = e < NW ? w[(long long)oc0 * CC * 9 + e] : 0.f;
    }
    const float br = tid < MM && bias ? bias[oc0 + tid] : 0.f;
    const long long idx = (long long)blockIdx.x * blockDim.x + tid;
    const long long plane = (long long)p.oh * p.ow;
    const bool live = idx < (long long)p.n * plane;
    const long long id = live ? idx : 0;  // dead lanes address pixel 0 and store nothing
    const int ox = (int)(id % p.ow);
    const long long t = id / p.ow;
    const int oy = (int)(t % p.oh);
    const int n = (int)(t / p.oh);
    const int m = p.m;
    const float *xn = x + (long long)n * CC * p.h * p.w;
    // CC <= 8: all CC*9 input taps, independent loads
    float v[CC <= 8 ? CC : 1][3][3];
    if constexpr (CC <= 8) {
#pragma unroll
        for (int ic = 0; ic < CC; ic++)
#pragma unroll
            for (int ky = 0; ky < 3; ky++) {
                const int iy = oy * p.sh - p.pt + ky;
#pragma unroll
                for (int kx = 0; kx < 3; kx++) {
                    const int ix = ox * p.sw - p.pl + kx;
                    const bool ok = (unsigned)iy < (unsigned)p.h && (unsigned)ix < (unsigned)p.w;
                    v[ic][ky][kx] = ok ? xn[((long long)ic * p.h + iy) * p.w + ix] : 0.f;
                }
            }
    }
    // the residuals too (one round trip, not one per output channel)
    const long long yo = (long long)n * m * plane + (long long)oy * p.ow + ox;
    float *yp = y + yo;
    float rv[MM];
#pragma unroll
    for (int o = 0; o < MM; o++) rv[o] = 0.f;
    if (res) {
#pragma unroll
        for (int o = 0; o < MM; o++) rv[o] = res[yo + (oc0 + o) * plane];
    }
#pragma unroll
    for (int i = 0; i < NWT; i++)
        if (tid + 256 * i < NW) lw[tid + 256 * i] = wr[i];
    if (tid < MM) lb[tid] = br;
    __syncthreads();
    if (!live) return;
    if constexpr (CC > 8) {
        // 16 or 32 channels: MM accumulators, input channels in the outer
        // loop; each output channel still sums bias, then ic -> ky -> kx
        float acc[MM];
#pragma unroll
        for (int o = 0; o < MM; o++) acc[o] = lb[o];
        for (int ic = 0; ic < CC; ic++) {
            float vi[3][3];
#pragma unroll
            for (int ky = 0; ky < 3; ky++) {
                const int iy = oy * p.sh - p.pt + ky;
#pragma unroll
                for (int kx = 0; kx < 3; kx++) {
                    const int ix = ox * p.sw - p.pl + kx;
                    const bool ok = (unsigned)iy < (unsigned)p.h && (unsigned)ix < (unsigned)p.w;
                    vi[ky][kx] = ok ? xn[((long long)ic * p.h + iy) * p.w + ix] : 0.f;
                }
            }
#pragma unroll
            for (int o = 0; o < MM; o++) {
                const float *wo = lw + (o * CC + ic) * 9;
#pragma unroll
                for (int ky = 0; ky < 3; ky++)
#pragma unroll
                    for (int kx = 0; kx < 3; kx++) acc[o] = __builtin_fmaf(wo[ky * 3 + kx], vi[ky][kx], acc[o]);
            }
        }
#pragma unroll
        for (int o = 0; o < MM; o++) {
            float r = activate<ACT>(acc[o]);
            if (res) r += rv[o];
            yp[(oc0 + o) * plane] = r;
        }
        return;
    }
    // 3x3 taps at compile-time offsets
#pragma unroll
    for (int oc = oc0; oc < oc0 + MM; oc++) {  // m = MM * gridDim.y (launch)
        float acc = lb[oc - oc0];
        const float *wo = lw + (oc - oc0) * CC * 9;
#pragma unroll
        for (int ic = 0; ic < CC; ic++)
#pragma unroll
            for (int ky = 0; ky < 3; ky++)
#pragma unroll
                for (int kx = 0; kx < 3; kx++) acc = __builtin_fmaf(wo[(ic * 3 + ky) * 3 + kx], v[ic][ky][kx], acc);
        float o = activate<ACT>(acc);
        if (res) o += rv[oc - oc0];
        yp[oc * plane] = o;
    }
}

// Also the few-channel 3x3 layers inside a network (8 input channels, e.g.
// YOLO11n's 8 -> 16 bottleneck conv at 160 x 160): the same per-pixel chain is
// the reference's im2col order for them, and cheaper than a GEMM tile whose
// M = 16 would idle most of its rows.
static bool first_conv_eligible(const osh_conv_params *p) {
    return p->group == 1 && (p->c <= 4 || p->c == 8 || p->c == 16 || p->c == 32) &&
           (p->m == 8 || p->m == 16 || p->m == 32) && p->kh == 3 && p->kw == 3 && p->dh == 1 && p->dw == 1;
}

// NchwcConv.CanUse + Dispatch + TryConv's batch test (NchwcConv.cs:100-126,
// 166-194): the shapes the reference runs through its NCHWc chain.
static bool nchwc_gate(const osh_conv_params *p) {
    const bool s2 = p->sh == 2;
    return p->group == 1 && p->kh == 3 && p->kw == 3 && p->sh == p->sw && (p->sh == 1 || s2) && p->dh == 1 &&
           p->dw == 1 && p->pt == 1 && p->pl == 1 && (!s2 || ((p->h & 1) == 0 && (p->w & 1) == 0)) &&
           p->c % 16 == 0 && p->m % 32 == 0 && p->n == 1 &&
           (s2 ? p->oh * 2 == p->h && p->ow * 2 == p->w : p->oh == p->h && p->ow == p->w);
}

enum ConvAlgo { ALGO_DEPTHWISE = 0, ALGO_POINTWISE = 1, ALGO_IM2COL = 3, ALGO_FIRST = 6, ALGO_CONV16 = 7, ALGO_PW16 = 8,
                ALGO_WINOGRAD = 9, ALGO_CONV16I = 10 };

static bool is_pointwise(const osh_conv_params *p) {
    return p->kh == 1 && p->kw == 1 && p->sh == 1 && p->sw == 1 && p->pt == 0 && p->pl == 0 && p->oh == p->h &&
           p->ow == p->w;
}

static ConvAlgo select_algo(const osh_conv_params *p) {
    if (p->group == p->c && p->group == p->m && p->group > 1) return ALGO_DEPTHWISE;
    const int v16 = conv16_variant();
    if (v16 >= 0 && conv16_eligible(p)) return ALGO_CONV16;  // a forced tile (tuning and tests)
    const int wm = winograd_mode();
    const bool wino = wm != 0 && winograd_eligible(p, winograd_max_pixels());
    if (p->c <= 4 && first_conv_eligible(p)) return ALGO_FIRST;
    if (wm == 2 && wino) return ALGO_WINOGRAD;
    if (nchwc_enabled() && nchwc_gate(p) && conv16_eligible(p)) return ALGO_CONV16;
    if (wino) return ALGO_WINOGRAD;
    if (conv16s_eligible(p)) return ALGO_CONV16I;  // the LDS-patch tiles in the im2col order
    if (first_conv_eligible(p)) return ALGO_FIRST;
    if (pointwise_variant() != -2 && pw16_eligible(p)) return ALGO_PW16;
    if (is_pointwise(p)) return ALGO_POINTWISE;
    // the implicit-im2col GEMM: k in the order ic -> ky -> kx, the
    // reference's im2col and panel chain
    return ALGO_IM2COL;
}

// ------------------------------------------------------------ conv16 tuning
//
// Every conv16 wave tile computes the same chain, so the fastest one can be
// chosen by measurement without changing any result: the first launch of a
// shape on a stream that is not being captured times each tile that fits
// (HIP events, two warm-up and ten timed launches each, in two passes over
// the tiles, writing the real output every time) and remembers the winner
// per shape.  Launches recorded
// into a graph before that use the cost model.
//
// With ONNXSHARP_HIP_TUNE_DB=<path> the choices persist: the table is read
// from that text file on first use and every new choice is appended to it,
// so a later process (a deployment, a profiler run) makes the same choices
// without timing.  The first line names the format and the size of each tile
// family; a file written for other families is started afresh.  A recorded
// tile that does not fit its shape is tuned again.
static std::mutex g_tune_mu;
using ConvKey = std::tuple<int, int, int, int, int, int, int, int, int, int, int, int, int, int>;
static std::map<std::tuple<int, ConvKey>, int> g_tuned;
static bool g_tune_db_read = false;

static ConvKey conv_key(const osh_conv_params *p) {
    return std::make_tuple(p->n, p->c, p->h, p->w, p->m, p->kh, p->kw, p->sh, p->sw, p->pt, p->pl, p->oh, p->ow,
                           p->group);
}

// One key for a group of convs: each field of the first member's key mixed
// with the others' (a collision could only pick a different, equally exact
// tile).
template <size_t... I>
static ConvKey mix_key_impl(const ConvKey &a, const ConvKey &b, std::index_sequence<I...>) {
    return std::make_tuple((int)((unsigned)std::get<I>(a) * 1000003u ^ (unsigned)std::get<I>(b))...);
}
static ConvKey mix_key(const ConvKey &a, const ConvKey &b) {
    return mix_key_impl(a, b, std::make_index_sequence<std::tuple_size<ConvKey>::value>{});
}
constexpr int kGroupTuneTag = 20;  // tuning-table tags of grouped launches (3x3, +1 pointwise)

static std::string tune_db_header() {
    char h[128];
    snprintf(h, sizeof(h), "onnxsharp-hip tune v1 conv3x3=%d pointwise=%d im2col3x3=%d pair=%d", conv16_variant_count(),
             pointwise_variant_count(), im2col3x3_variant_count(), conv_pair_tile_count());
    return h;
}

static const char *tune_db_path() {
    const char *e = getenv("ONNXSHARP_HIP_TUNE_DB");
    return (e && *e) ? e : nullptr;
}

// Reads the database once (g_tune_mu held).
static void tune_db_read_locked() {
    if (g_tune_db_read) return;
    g_tune_db_read = true;
    const char *path = tune_db_path();
    if (!path) return;
    FILE *f = fopen(path, "r");
    if (!f) return;
    char line[512];
    const std::string want = tune_db_header();
    bool ok = fgets(line, sizeof(line), f) && std::string(line).substr(0, want.size()) == want;
    int v[16];
    while (ok && fgets(line, sizeof(line), f)) {
        if (sscanf(line, "%d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d", &v[0], &v[1], &v[2], &v[3], &v[4], &v[5],
                   &v[6], &v[7], &v[8], &v[9], &v[10], &v[11], &v[12], &v[13], &v[14], &v[15]) != 16)
            continue;
        g_tuned[std::make_tuple(v[0], std::make_tuple(v[1], v[2], v[3], v[4], v[5], v[6], v[7], v[8], v[9], v[10],
                                                      v[11], v[12], v[13], v[14]))] = v[15];
    }
    fclose(f);
    if (!ok) {  // another format: start the file afresh
        FILE *w = fopen(path, "w");
        if (w) {
            fprintf(w, "%s\n", want.c_str());
            fclose(w);
        }
    }
}

// Appends one choice (g_tune_mu held).
static void tune_db_append_locked(int tag, const ConvKey &k, int v) {
    const char *path = tune_db_path();
    if (!path) return;
    FILE *probe = fopen(path, "r");
    const bool fresh = probe == nullptr;
    if (probe) fclose(probe);
    FILE *f = fopen(path, "a");
    if (!f) return;
    if (fresh) fprintf(f, "%s\n", tune_db_header().c_str());
    fprintf(f, "%d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d\n", tag, std::get<0>(k), std::get<1>(k),
            std::get<2>(k), std::get<3>(k), std::get<4>(k), std::get<5>(k), std::get<6>(k), std::get<7>(k),
            std::get<8>(k), std::get<9>(k), std::get<10>(k), std::get<11>(k), std::get<12>(k), std::get<13>(k), v);
    fclose(f);
}

// Which kernel and shape each packed weight buffer was laid out for.  The
// layout depends on the kernel choice, which the options "winograd",
// "winograd_max_pixels" and "pointwise_variant" -2 can
// change between packing and launch; a launch whose buffer was packed for
// another kernel or shape is refused instead of reading a wrong layout (or
// past its end).  Buffers this library did not pack are not checked.  An
// entry covers [address, address + bytes): packing into a range drops every
// entry it overlaps (memory reused for new weights), and osh_free /
// osh_conv_forget_pack drop the entries of a range the caller releases.
struct PackTag {
    int algo;
    ConvKey key;
    size_t bytes;
};
static std::mutex g_packs_mu;
static std::map<uintptr_t, PackTag> g_packs;  // by start address

// Erases the entries overlapping [a, a + bytes) (g_packs_mu held).
static void forget_range_locked(uintptr_t a, size_t bytes) {
    auto it = g_packs.lower_bound(a);
    if (it != g_packs.begin()) {
        auto prev = std::prev(it);
        if (prev->first + prev->second.bytes > a) it = prev;
    }
    while (it != g_packs.end() && it->first < a + (bytes ? bytes : 1)) it = g_packs.erase(it);
}

// Whether d_w holds weights this library packed for p with the pointwise
// LDS-tile layout (conv16 layout first), the layout the pointwise-chain
// kernel reads.
bool packed_for_pointwise_tiles(const osh_conv_params *p, const void *d_w) {
    if (select_algo(p) != ALGO_PW16) return false;
    std::lock_guard<std::mutex> lk(g_packs_mu);
    auto it = g_packs.find(reinterpret_cast<uintptr_t>(d_w));
    return it != g_packs.end() && it->second.algo == (int)ALGO_PW16 && it->second.key == conv_key(p);
}

static void record_pack(const osh_conv_params *p, const void *d_packed, size_t bytes) {
    std::lock_guard<std::mutex> lk(g_packs_mu);
    const uintptr_t a = reinterpret_cast<uintptr_t>(d_packed);
    forget_range_locked(a, bytes);
    g_packs[a] = PackTag{(int)select_algo(p), conv_key(p), bytes ? bytes : 1};
}

// Drops the entry that starts at d_ptr and every entry inside the
// allocation it starts (osh_free passes the allocation base).
void forget_pack(const void *d_ptr) {
    std::lock_guard<std::mutex> lk(g_packs_mu);
    const uintptr_t a = reinterpret_cast<uintptr_t>(d_ptr);
    size_t span = 1;
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, const_cast<void *>(d_ptr)) == hipSuccess &&
        reinterpret_cast<uintptr_t>(base) == a)
        span = size;
    else
        (void)hipGetLastError();
    forget_range_locked(a, span);
}

static bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone;
}

// The 3x3 variant space: ids 0 .. kC16Count-1 are conv16 / conv16l tiles,
// the next kC16sCount ids the LDS-patch kernel (stride 1 or 2 only), then
// kC16wCount conv16 tiles with one wave per workgroup, then kC16sxCount
// LDS-patch tiles with XCD-banded workgroups.  All compute the same chain.
constexpr int kC3W0 = kC16Count + kC16sCount;
constexpr int kC3X0 = kC3W0 + kC16wCount;
constexpr int kC3Count = kC3X0 + kC16sxCount;
int conv16_variant_count() { return kC3Count; }
int pointwise_variant_count() { return 1 + kPW16Count; }
int im2col3x3_variant_count() { return kC16sCount + kC16wiCount; }
// each LDS-patch tile shared, then one workgroup per CU, then the streamed tiles
int group3x3_tile_count() { return 2 * kC16sCount + kC16gCount; }
int group_pointwise_tile_count() { return kPW16Count; }

static bool c3_fits(const osh_conv_params *p, int v) {
    if (v < kC16Count) return conv16_fits(p, kC16[v]);
    if (v < kC3W0) return conv16s_eligible(p);
    if (v < kC3X0) return true;
    return conv16s_eligible(p);
}

// Predicted cost of an LDS-patch tile: rounds of waves over the SIMDs times
// one wave's MFMAs (tiles past the map edge included), inflated a little for
// the weight loads and the per-block barrier.
static double conv16s_cost(const osh_conv_params *p, const C16sVariant &v, int cus) {
    const int th = 16 / v.twl * v.bv;
    const long long tiles = (long long)ceil_div(p->ow, v.twl) * ceil_div(p->oh, th);
    const long long waves = tiles * ceil_div(ceil_div(p->m, 16), v.tm) * p->n;
    const long long rounds = (waves + 4LL * cus - 1) / (4LL * cus);
    const double u = (double)v.tm * v.bv;
    return rounds * u * (9.0 * p->c / 4) * (1.0 + 0.25 / u);
}

static osh_status c3_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                            const float *res, int act, float *y, hipStream_t st, int v) {
    if (v < 0) {  // cost model over both families
        const int cus = device_cus();
        double bc = 0;
        for (int i = 0; i < kC16Count; i++) {
            if (!conv16_fits(p, kC16[i])) continue;
            const double c = conv16_cost(p, kC16[i], cus);
            if (v < 0 || c < bc) v = i, bc = c;
        }
        if (conv16s_eligible(p))
            for (int i = 0; i < kC16sCount; i++) {
                const double c = conv16s_cost(p, kC16s[i], cus);
                if (c < bc) v = kC16Count + i, bc = c;
            }
    }
    if (v >= kC3X0 && v < kC3Count && conv16s_eligible(p))
        return conv16sx_launch(p, x, w, bias, res, act, y, st, v - kC3X0);
    if (v >= kC3W0 && v < kC3X0) return conv16w_launch(p, x, w, bias, res, act, y, st, v - kC3W0);
    if (v >= kC16Count && v < kC3W0 && conv16s_eligible(p))
        return conv16s_launch(p, x, w, bias, res, act, y, st, v - kC16Count);
    return conv16_launch(p, x, w, bias, res, act, y, st, v < kC16Count ? v : -1);
}

// Launches variant v (0 .. count-1) of a tile family, or the family's
// cost-model pick for v < 0.  Tag separates families in the tuning table.
template <class Fits, class Launch>
static osh_status tuned_launch_key(const std::tuple<int, ConvKey> &key, int count, int forced, Fits fits,
                                   Launch launch, hipStream_t st);

template <class Fits, class Launch>
static osh_status tuned_launch(const osh_conv_params *p, int tag, int count, int forced, Fits fits, Launch launch,
                               hipStream_t st) {
    return tuned_launch_key(std::make_tuple(tag, conv_key(p)), count, forced, fits, launch, st);
}

template <class Fits, class Launch>
static osh_status tuned_launch_key(const std::tuple<int, ConvKey> &key, int count, int forced, Fits fits,
                                   Launch launch, hipStream_t st) {
    if (forced >= 0 || !tuning_enabled()) return launch(forced >= 0 && forced < count && fits(forced) ? forced : -1);
    int chosen = -1;
    {
        std::lock_guard<std::mutex> lk(g_tune_mu);
        tune_db_read_locked();
        auto it = g_tuned.find(key);
        if (it != g_tuned.end()) chosen = it->second;
    }
    // launched outside the lock: a launch may itself be a tuned launch (the
    // conv pair's two-launch form runs each conv through its own choice)
    if (chosen >= 0 && chosen < count && fits(chosen)) return launch(chosen);
    if (capturing(st)) return launch(-1);
    hipEvent_t e0, e1;
    OSH_HIP_CHECK(hipEventCreate(&e0));
    if (hipEventCreate(&e1) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return fail(OSH_E_DEVICE, "hipEventCreate failed");
    }
    // two passes over all tiles, each tile keeping its faster pass, so a
    // tile timed while the clock was still rising is not ruled out
    int best = -1;
    float best_ms = 0.f;
    osh_status rc = OSH_OK;
    for (int pass = 0; pass < 2 && rc == OSH_OK; pass++)
        for (int v = 0; v < count && rc == OSH_OK; v++) {
            if (!fits(v)) continue;
            for (int r = 0; r < 2 && rc == OSH_OK; r++) rc = launch(v);
            if (rc != OSH_OK) break;
            if (hipEventRecord(e0, st) != hipSuccess) { rc = fail(OSH_E_DEVICE, "hipEventRecord failed"); break; }
            for (int r = 0; r < 10 && rc == OSH_OK; r++) rc = launch(v);
            if (rc != OSH_OK) break;
            float ms = 0.f;
            if (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                hipEventElapsedTime(&ms, e0, e1) != hipSuccess) {
                rc = fail(OSH_E_DEVICE, "conv tuning: event timing failed");
                break;
            }
            if (best < 0 || ms < best_ms) best = v, best_ms = ms;
        }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc != OSH_OK) return rc;
    {
        std::lock_guard<std::mutex> lk(g_tune_mu);
        g_tuned[key] = best;
        tune_db_append_locked(std::get<0>(key), std::get<1>(key), best);
    }
    return OSH_OK;  // y already holds the result (every tile computes the same values)
}

static osh_status conv16_tuned_launch(const osh_conv_params *p, const float *x, const float *w, const float *bias,
                                      const float *res, int act, float *y, hipStream_t st) {
    return tuned_launch(
        p, 3, kC3Count, conv16_variant(), [&](int v) { return c3_fits(p, v); },
        [&](int v) { return c3_launch(p, x, w, bias, res, act, y, st, v); }, st);
}

static osh_status check_params(const osh_conv_params *p) {
    if (!p) return fail(OSH_E_INVALID, "Conv: params is NULL");
    if (p->n <= 0 || p->c <= 0 || p->h <= 0 || p->w <= 0 || p->m <= 0 || p->kh <= 0 || p->kw <= 0 ||
        p->group <= 0 || p->sh <= 0 || p->sw <= 0 || p->dh <= 0 || p->dw <= 0 || p->oh <= 0 || p->ow <= 0)
        return fail(OSH_E_INVALID, "Conv: non-positive size in params");
    if (p->pt < 0 || p->pl < 0) return fail(OSH_E_UNSUPPORTED, "Conv: negative pads are not supported");
    if (p->c % p->group != 0 || p->m % p->group != 0)
        return fail(OSH_E_INVALID, "Conv: channels not divisible by group");
    long long cpg = p->c / p->group;
    if (cpg * p->kh * p->kw > (1LL << 30) || (long long)p->oh * p->ow > (1LL << 30) ||
        (long long)p->n * p->group > 65535)
        return fail(OSH_E_UNSUPPORTED, "Conv: problem exceeds the launch limits");
    return OSH_OK;
}

}  // namespace osh

namespace osh {
static osh_status pack_weights(const osh_conv_params *p, const float *d_w, void *d_packed, osh_stream s);
}  // namespace osh

extern "C" {

OSH_API osh_status osh_conv_infer_shape(const osh_conv_attrs *at, const int64_t x[4], const int64_t w[4],
                                        int64_t y[4]) {
    osh_status st = check_attrs(at, x, w);
    if (st != OSH_OK) return st;
    if (!y) return fail(OSH_E_INVALID, "Conv: y_dims is NULL");
    const int spatial = 2;
    y[0] = x[0];
    y[1] = w[0];
    for (int i = 0; i < spatial; i++) {
        int kernel = at->n_kernel_shape > i ? at->kernel_shape[i] : (int)w[2 + i];
        int stride = at->n_strides > i ? at->strides[i] : 1;
        int dilation = at->n_dilations > i ? at->dilations[i] : 1;
        int pad_begin = at->n_pads > i ? at->pads[i] : 0;
        // DnnOps.cs:174-175: the end pad is read only when more than 2*spatial pads are given,
        // so a 4-entry pads list makes the shape use the begin pad twice.
        int pad_end = at->n_pads > 2 * spatial ? at->pads[spatial + i] : pad_begin;
        if (at->auto_pad != OSH_PAD_NOTSET) auto_pad(at->auto_pad, (int)x[2 + i], kernel, stride, dilation, &pad_begin, &pad_end);
        int o = spatial_out((int)x[2 + i], kernel, stride, dilation, pad_begin, pad_end);
        if (o <= 0) return fail(OSH_E_INVALID, "Conv: output spatial size %d is not positive", o);
        y[2 + i] = o;
    }
    return OSH_OK;
}

OSH_API osh_status osh_conv_resolve(const osh_conv_attrs *at, const int64_t x[4], const int64_t w[4],
                                    osh_conv_params *p) {
    if (!p) return fail(OSH_E_INVALID, "Conv: out is NULL");
    int64_t y[4];
    osh_status st = osh_conv_infer_shape(at, x, w, y);
    if (st != OSH_OK) return st;
    const int spatial = 2;
    int strides[2], dil[2], pads[4];
    for (int i = 0; i < spatial; i++) {
        int kernel = at->n_kernel_shape > i ? at->kernel_shape[i] : (int)w[2 + i];
        strides[i] = at->n_strides > i ? at->strides[i] : 1;
        dil[i] = at->n_dilations > i ? at->dilations[i] : 1;
        if (at->auto_pad != OSH_PAD_NOTSET) {
            auto_pad(at->auto_pad, (int)x[2 + i], kernel, strides[i], dil[i], &pads[i], &pads[spatial + i]);
        } else {
            pads[i] = at->n_pads > i ? at->pads[i] : 0;
            pads[spatial + i] = at->n_pads > spatial + i ? at->pads[spatial + i] : pads[i];
        }
    }
    memset(p, 0, sizeof(*p));
    p->n = (int)x[0]; p->c = (int)x[1]; p->h = (int)x[2]; p->w = (int)x[3];
    // The kernels take their taps from the weight tensor (as ConvLayer's CPU kernels do).
    p->m = (int)w[0]; p->kh = (int)w[2]; p->kw = (int)w[3]; p->group = at->group;
    p->sh = strides[0]; p->sw = strides[1]; p->dh = dil[0]; p->dw = dil[1];
    p->pt = pads[0]; p->pl = pads[1]; p->pb = pads[2]; p->pr = pads[3];
    p->oh = (int)y[2]; p->ow = (int)y[3];
    return check_params(p);
}

OSH_API osh_status osh_conv_packed_weight_bytes(const osh_conv_params *p, size_t *bytes) {
    osh_status st = check_params(p);
    if (st != OSH_OK) return st;
    if (!bytes) return fail(OSH_E_INVALID, "bytes is NULL");
    size_t oihw = (size_t)p->m * (p->c / p->group) * p->kh * p->kw * sizeof(float);
    switch (select_algo(p)) {
    case ALGO_CONV16:
    case ALGO_CONV16I: *bytes = conv16_packed_bytes(p); break;
    case ALGO_WINOGRAD: *bytes = winograd_packed_bytes(p); break;
    case ALGO_PW16: *bytes = conv16_packed_bytes(p) + oihw; break;  // LDS-tile layout, then the raw GEMM operand
    default: *bytes = oihw;
    }
    return OSH_OK;
}

OSH_API osh_status osh_conv_pack_weights(const osh_conv_params *p, const float *d_w, void *d_packed,
                                         osh_stream s) {
    osh_status st = check_params(p);
    if (st != OSH_OK) return st;
    if (!d_w || !d_packed) return fail(OSH_E_INVALID, "Conv pack: NULL pointer");
    st = pack_weights(p, d_w, d_packed, s);
    if (st == OSH_OK) {
        size_t bytes = 0;
        if (osh_conv_packed_weight_bytes(p, &bytes) != OSH_OK) bytes = 1;
        record_pack(p, d_packed, bytes);
    }
    return st;
}

OSH_API osh_status osh_conv_forget_pack(const void *d_packed, size_t bytes) {
    if (!d_packed) return fail(OSH_E_INVALID, "Conv forget pack: NULL pointer");
    std::lock_guard<std::mutex> lk(g_packs_mu);
    forget_range_locked(reinterpret_cast<uintptr_t>(d_packed), bytes);
    return OSH_OK;
}

}  // extern "C"

namespace osh {

static osh_status pack_weights(const osh_conv_params *p, const float *d_w, void *d_packed, osh_stream s) {
    osh_status st = OSH_OK;
    if (select_algo(p) == ALGO_CONV16) return conv16_pack(p, d_w, d_packed, to_stream(s));
    if (select_algo(p) == ALGO_WINOGRAD) return winograd_pack(p, d_w, d_packed, to_stream(s));
    if (select_algo(p) == ALGO_CONV16I) return conv16_pack(p, d_w, d_packed, to_stream(s), true);
    if (select_algo(p) == ALGO_PW16) {
        st = conv16_pack(p, d_w, d_packed, to_stream(s));
        if (st != OSH_OK) return st;
        const size_t oihw = (size_t)p->m * p->c * sizeof(float);
        OSH_HIP_CHECK(hipMemcpyAsync(static_cast<char *>(d_packed) + conv16_packed_bytes(p), d_w, oihw,
                                     hipMemcpyDeviceToDevice, to_stream(s)));
        return OSH_OK;
    }
    size_t oihw = (size_t)p->m * (p->c / p->group) * p->kh * p->kw * sizeof(float);
    OSH_HIP_CHECK(hipMemcpyAsync(d_packed, d_w, oihw, hipMemcpyDeviceToDevice, to_stream(s)));
    return OSH_OK;
}

}  // namespace osh



namespace osh {

static osh_status igemm_conv(const osh_conv_params *p, const float *d_x, const float *w, const float *d_bias,
                             const float *d_res, int act, float *d_y, hipStream_t stream, int bmode);

// Pick among the pointwise LDS tiles without timing: on one MI355X the
// smallest tile (16 channels x 16 pixels per wave, many waves per SIMD) was
// fastest for every YOLO11n and C2f 1x1 shape measured; a map narrower than
// 16 takes the 4-wide tile instead.
static int pw16_pick(const osh_conv_params *p) { return p->ow >= 16 ? 0 : 5; }

// Launches the conv of p: y = act(conv(x) + bias) (+ res when res is not NULL;
// res has y's layout and does not overlap it).
static osh_status conv2d(const osh_conv_params *p, const float *d_x, const void *d_wpacked, const float *d_bias,
                         int act, const float *d_res, float *d_y, hipStream_t stream) {
    const float *w = static_cast<const float *>(d_wpacked);
    const long long out_hw = (long long)p->oh * p->ow;

    switch (select_algo(p)) {
    case ALGO_DEPTHWISE: {
        long long total = (long long)p->n * p->m * out_hw;
        dim3 grid((unsigned)((total + 255) / 256));
        if (dw3_eligible(p)) {
            if (p->sh == 1) {
                OSH_DISPATCH_ACT(act, ACT,
                                 OSH_LAUNCH((dw3_conv_kernel<ACT, 1>), grid, dim3(256), 0, stream, *p, d_x, w,
                                                    d_bias, d_res, d_y));
            } else {
                OSH_DISPATCH_ACT(act, ACT,
                                 OSH_LAUNCH((dw3_conv_kernel<ACT, 2>), grid, dim3(256), 0, stream, *p, d_x, w,
                                                    d_bias, d_res, d_y));
            }
            OSH_LAUNCH_CHECK("dw3_conv_kernel");
            return OSH_OK;
        }
        OSH_DISPATCH_ACT(act, ACT,
                         OSH_LAUNCH(dw_conv_kernel<ACT>, grid, dim3(256), 0, stream, *p, d_x, w, d_bias, d_res,
                                            d_y));
        OSH_LAUNCH_CHECK("dw_conv_kernel");
        return OSH_OK;
    }
    case ALGO_FIRST: {
        long long total = (long long)p->n * out_hw;
        // output channels per thread: all m, halved (down to 4) while the
        // grid has fewer workgroups than CUs (8 -> 16 at 160x160: 11.0 ->
        // 6.5 us; the 640x640 stem, already past one per CU, keeps all m)
        int og = p->m;
        const long long blocks = (total + 255) / 256;
        while (og > 4 && blocks * (p->m / og) < device_cus()) og /= 2;
        dim3 grid((unsigned)blocks, (unsigned)(p->m / og));
#define OSH_FIRST(MM, CC)                                                                                      \
    OSH_DISPATCH_ACT(act, ACT, OSH_LAUNCH((first_conv_kernel<MM, CC, ACT>), grid, dim3(256), 0, stream, \
                                                  *p, d_x, w, d_bias, d_res, d_y))
#define OSH_FIRST_C(MM)            \
    do {                           \
        switch (p->c) {            \
        case 1: OSH_FIRST(MM, 1); break; \
        case 2: OSH_FIRST(MM, 2); break; \
        case 3: OSH_FIRST(MM, 3); break; \
        case 4: OSH_FIRST(MM, 4); break; \
        case 16: OSH_FIRST(MM, 16); break; \
        case 32: OSH_FIRST(MM, 32); break; \
        default: OSH_FIRST(MM, 8); break; \
        }                          \
    } while (0)
        if (og == 4) OSH_FIRST_C(4);
        else if (og == 8) OSH_FIRST_C(8);
        else if (og == 16) OSH_FIRST_C(16);
        else OSH_FIRST_C(32);
#undef OSH_FIRST_C
#undef OSH_FIRST
        OSH_LAUNCH_CHECK("first_conv_kernel");
        return OSH_OK;
    }
    case ALGO_CONV16:
        return conv16_tuned_launch(p, d_x, w, d_bias, d_res, act, d_y, stream);
    case ALGO_CONV16I:
        return tuned_launch(
            p, 4, kC16sCount + kC16wiCount, im2col3x3_variant(), [](int) { return true; },
            [&](int v) {
                if (v < 0) {  // cost model
                    const int cus = device_cus();
                    double bc = 0;
                    for (int i = 0; i < kC16sCount; i++) {
                        const double c = conv16s_cost(p, kC16s[i], cus);
                        if (v < 0 || c < bc) v = i, bc = c;
                    }
                }
                if (v >= kC16sCount) return conv16wi_launch(p, d_x, w, d_bias, d_res, act, d_y, stream, v - kC16sCount);
                return conv16si_launch(p, d_x, w, d_bias, d_res, act, d_y, stream, v);
            },
            stream);
    case ALGO_WINOGRAD: {
        const long long tiles = (long long)p->n * ((p->h + 1) / 2) * ((p->w + 1) / 2);
        dim3 grid((unsigned)((p->m + 15) / 16), (unsigned)((tiles + 15) / 16));
        if (grid.y > 65535) return fail(OSH_E_UNSUPPORTED, "Conv: Winograd grid too large");
        const float4 *u = reinterpret_cast<const float4 *>(d_wpacked);
        OSH_DISPATCH_ACT(act, ACT,
                         OSH_LAUNCH(wino_f23_kernel<ACT>, grid, dim3(256), 0, stream, *p, d_x, u, d_bias,
                                            d_res, d_y));
        OSH_LAUNCH_CHECK("wino_f23_kernel");
        return OSH_OK;
    }
    case ALGO_PW16: {
        // 0: the GEMM tile over the raw weights; 1..: the LDS-tile kernel
        const float *wraw = reinterpret_cast<const float *>(static_cast<const char *>(d_wpacked) +
                                                            conv16_packed_bytes(p));
        return tuned_launch(
            p, 1, 1 + kPW16Count, pointwise_variant(), [p](int v) { return v == 0 || pw16_fits(p, v - 1); },
            [&](int v) {
                if (v == 0) return igemm_conv(p, d_x, wraw, d_bias, d_res, act, d_y, stream, B_DENSE);
                if (v < 0) v = 1 + pw16_pick(p);
                return pw16_launch(p, d_x, w, d_bias, d_res, act, d_y, stream, v - 1);
            },
            stream);
    }
    case ALGO_POINTWISE:
    case ALGO_IM2COL:
        return igemm_conv(p, d_x, w, d_bias, d_res, act, d_y, stream,
                          is_pointwise(p) ? B_DENSE : B_IM2COL);
    }
    return fail(OSH_E_INVALID, "Conv: no kernel");
}

// The conv as an implicit GEMM over raw OIHW weights: W[M/g][C/g*kh*kw] x
// (X dense for 1x1 s1 p0, else gathered), per image and group.
// The convs of a group in one launch when they share a kernel family the
// grouped kernels cover (LDS-patch 3x3 tiles of one stride, the pointwise
// LDS tiles, depthwise), else one launch each.  The LDS-patch tile is the one
// the cost model rates best for the group's slowest conv; every tile gives
// the same bits.
static osh_status conv2d_group(int count, const osh_conv_params *ps, const float *const *xs, const void *const *ws,
                               const float *const *bs, int act, const float *const *rs, float *const *ys,
                               hipStream_t st) {
    const ConvAlgo a0 = select_algo(&ps[0]);
    bool one = count > 1 && (a0 == ALGO_CONV16 || a0 == ALGO_PW16 || a0 == ALGO_DEPTHWISE);
    bool vec = true;
    for (int i = 0; i < count && one; i++) {
        const osh_conv_params &p = ps[i];
        one = select_algo(&p) == a0 && p.sh == ps[0].sh;
        if (a0 == ALGO_CONV16) one = one && conv16s_eligible(&p);
        if (a0 == ALGO_PW16) vec = vec && p.w % 4 == 0 && (reinterpret_cast<uintptr_t>(xs[i]) & 15) == 0;
    }
    if (!one) {
        for (int i = 0; i < count; i++) {
            osh_status r = conv2d(&ps[i], xs[i], ws[i], bs ? bs[i] : nullptr, act, rs ? rs[i] : nullptr, ys[i], st);
            if (r != OSH_OK) return r;
        }
        return OSH_OK;
    }
    // Members are laid out longest chain first (most MFMA steps a wave, C/g
    // * kh * kw): workgroups start in block order, so the deep-K member's
    // chains (the head's 256 -> 64 at 20x20: 576 dependent steps) start at
    // once and the shorter members' workgroups fill the SIMDs around them.
    int order[kConvGroupMax];
    for (int i = 0; i < count; i++) order[i] = i;
    auto steps = [&](int i) { return (long long)ps[i].c / ps[i].group * ps[i].kh * ps[i].kw; };
    for (int i = 1; i < count; i++)  // stable insertion sort, descending
        for (int k = i; k > 0 && steps(order[k]) > steps(order[k - 1]); k--) std::swap(order[k], order[k - 1]);
    ConvGroup g{};
    g.count = count;
    for (int k = 0; k < count; k++) {
        const int i = order[k];
        g.p[k] = ps[i];
        g.x[k] = xs[i];
        g.w[k] = static_cast<const float *>(ws[i]);
        g.bias[k] = bs ? bs[i] : nullptr;
        g.res[k] = rs ? rs[i] : nullptr;
        g.y[k] = ys[i];
    }
    if (a0 == ALGO_DEPTHWISE) {
        long long total = 0;
        for (int i = 0; i < count; i++) {
            g.start[i] = (int)total;
            total += ((long long)ps[i].n * ps[i].m * ps[i].oh * ps[i].ow + 255) / 256;
            if (total > 0x7fffffffLL) return fail(OSH_E_UNSUPPORTED, "Conv group: grid too large");
        }
        g.start[count] = (int)total;
        int s3 = dw3_eligible(&ps[0]) ? ps[0].sh : 0;  // every member 3x3 at one stride: the 3x3 path
        for (int i = 1; i < count; i++)
            if (!dw3_eligible(&ps[i]) || ps[i].sh != s3) s3 = 0;
        if (s3 == 1) {
            OSH_DISPATCH_ACT(act, ACT,
                             OSH_LAUNCH((dw_conv_group_kernel<ACT, 1>), dim3((unsigned)total), dim3(256), 0, st,
                                                g));
        } else if (s3 == 2) {
            OSH_DISPATCH_ACT(act, ACT,
                             OSH_LAUNCH((dw_conv_group_kernel<ACT, 2>), dim3((unsigned)total), dim3(256), 0, st,
                                                g));
        } else {
            OSH_DISPATCH_ACT(act, ACT,
                             OSH_LAUNCH((dw_conv_group_kernel<ACT, 0>), dim3((unsigned)total), dim3(256), 0, st,
                                                g));
        }
        OSH_LAUNCH_CHECK("dw_conv_group_kernel");
        return OSH_OK;
    }
    // The tile is chosen like a single conv's, by first-use timing of the
    // whole group (every tile gives every member the same bits), keyed by all
    // members' shapes; launches recorded into a graph before that use the
    // default below.
    ConvKey gk = conv_key(&ps[0]);
    for (int i = 1; i < count; i++) gk = mix_key(gk, conv_key(&ps[i]));
    if (a0 == ALGO_PW16) {  // the pointwise LDS tiles read the LDS-tile part of the packed weights
        bool narrow = false;
        for (int i = 0; i < count; i++) narrow = narrow || ps[i].ow < 16;
        const int dflt = narrow ? 5 : 0;  // {1, 2, 4} on narrow maps, else {1, 1, 16}
        auto fits = [&](int v) {
            for (int i = 0; i < count; i++)
                if (!pw16_fits(&ps[i], v)) return false;
            return true;
        };
        return tuned_launch_key(
            std::make_tuple(kGroupTuneTag + 1, gk), kPW16Count, group_pointwise_tile(), fits,
            [&](int v) { return pw16_group_launch(g, act, st, v < 0 ? dflt : v, vec); }, st);
    }
    // Default: the convs run side by side, so the slowest one bounds the
    // launch: the tile with the smallest largest cost (then the smallest total).
    const int cus = device_cus();
    int best = 0;
    double bmax = 0, bsum = 0;
    for (int v = 0; v < kC16sCount; v++) {
        double cmax = 0, csum = 0;
        for (int i = 0; i < count; i++) {
            const double c = conv16s_cost(&ps[i], kC16s[v], cus);
            cmax = c > cmax ? c : cmax;
            csum += c;
        }
        if (v == 0 || cmax < bmax || (cmax == bmax && csum < bsum)) best = v, bmax = cmax, bsum = csum;
    }
    return tuned_launch_key(
        std::make_tuple(kGroupTuneTag, gk), group3x3_tile_count(), group3x3_tile(), [](int) { return true; },
        [&](int v) { return conv16s_group_launch(g, act, st, v < 0 ? best : v, ps[0].sh); }, st);
}

static osh_status igemm_conv(const osh_conv_params *p, const float *d_x, const float *w, const float *d_bias,
                             const float *d_res, int act, float *d_y, hipStream_t stream, int bmode) {
    const int cpg = p->c / p->group, opg = p->m / p->group;
    const long long in_hw = (long long)p->h * p->w, out_hw = (long long)p->oh * p->ow;
    {
        IgemmArgs a{};
        a.M = opg;
        a.N = (int)out_hw;
        a.K = cpg * p->kh * p->kw;
        a.A = w;
        a.lda = a.K;
        a.strideA = 0;
        a.strideA_in = (long long)opg * a.K;
        a.B = d_x;
        a.ldb = (int)in_hw;
        a.strideB = (long long)p->c * in_hw;
        a.strideB_in = (long long)cpg * in_hw;
        a.C = d_y;
        a.ldc = (int)out_hw;
        a.strideC = (long long)p->m * out_hw;
        a.strideC_in = (long long)opg * out_hw;
        a.row_bias = d_bias;
        a.res = d_res;
        a.bias_stride = opg;
        a.zdiv = p->group;
        a.H = p->h; a.W = p->w; a.KH = p->kh; a.KW = p->kw;
        a.sh = p->sh; a.sw = p->sw; a.dh = p->dh; a.dw = p->dw;
        a.pt = p->pt; a.pl = p->pl; a.OW = p->ow;
        return launch_igemm(a, p->n * p->group, bmode, act, stream);
    }
}

static size_t x_bytes(const osh_conv_params *p) { return (size_t)p->n * p->c * p->h * p->w * sizeof(float); }
static size_t y_bytes(const osh_conv_params *p) { return (size_t)p->n * p->m * p->oh * p->ow * sizeof(float); }
static bool ranges_overlap(const void *a, size_t na, const void *b, size_t nb) {
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a && b && a0 < b0 + nb && b0 < a0 + na;
}

static osh_status check_launch(const osh_conv_params *p, const float *d_x, const void *d_wpacked, int act,
                                float *d_y) {
    osh_status st = check_params(p);
    if (st != OSH_OK) return st;
    if (!d_x || !d_wpacked || !d_y) return fail(OSH_E_INVALID, "Conv: NULL tensor pointer");
    if (act < OSH_ACT_NONE || act > OSH_ACT_SILU) return fail(OSH_E_INVALID, "Conv: unknown activation %d", act);
    // in place is refused: the tiles read input halos other workgroups write
    if (ranges_overlap(d_x, x_bytes(p), d_y, y_bytes(p)))
        return fail(OSH_E_INVALID, "Conv: the output overlaps the input");
    std::lock_guard<std::mutex> lk(g_packs_mu);
    auto it = g_packs.find(reinterpret_cast<uintptr_t>(d_wpacked));
    if (it != g_packs.end() && (it->second.algo != (int)select_algo(p) || it->second.key != conv_key(p)))
        return fail(OSH_E_INVALID,
                    "Conv: the weights were packed for another kernel or shape (pack them again after changing "
                    "the conv options)");
    return OSH_OK;
}

// ---- two chained 3x3 convs in one launch (osh_conv_pair.hip)

constexpr int kPairTuneTag = 30;  // tuning-table tags of the fused pair (+1 without an intermediate buffer)

// Why a pair cannot run fused, or nullptr: both convs 3x3 stride 1 pad 1 over
// one 1 x C x H x W map, the second reading the first's output, 16/32/64
// channels out of each, SiLU, and the single-conv dispatch taking for each
// the chain the pair computes (NCHWc for 32 and 64 outputs, im2col for 16).
static const char *first_pair_refusal(const osh_conv_params *pa, const osh_conv_params *pb, int act);
static const char *pair8_refusal(const osh_conv_params *pa, const osh_conv_params *pb, int act);

static const char *pair_refusal(const osh_conv_params *pa, const osh_conv_params *pb, int act) {
    if (pa->c <= 4) return first_pair_refusal(pa, pb, act);
    if (pa->m == 8) return pair8_refusal(pa, pb, act);
    auto same_map_3x3 = [](const osh_conv_params *p) {
        return p->group == 1 && p->kh == 3 && p->kw == 3 && p->sh == 1 && p->sw == 1 && p->dh == 1 &&
               p->dw == 1 && p->pt == 1 && p->pl == 1 && p->oh == p->h && p->ow == p->w;
    };
    if (!same_map_3x3(pa) || !same_map_3x3(pb)) return "both convs must be 3x3, stride 1, pad 1 on one map";
    if (pa->n != 1 || pb->n != 1) return "batch 1 only";
    if (pb->c != pa->m || pb->h != pa->h || pb->w != pa->w) return "the second conv must read the first one's output";
    if (pa->c % 16 != 0 || pa->c > 64) return "the first conv must have 16, 32, 48 or 64 input channels";
    auto cb_ok = [](int m) { return m == 16 || m == 32 || m == 64; };
    if (!cb_ok(pa->m) || !cb_ok(pb->m)) return "each conv must have 16, 32 or 64 output channels";
    if (act != OSH_ACT_SILU) return "the fused pair takes SiLU convs";
    if ((long long)pa->c * pa->h * pa->w * 4 >= (1LL << 31)) return "input too large";
    if (select_algo(pa) != (pa->m == 16 ? ALGO_CONV16I : ALGO_CONV16) ||
        select_algo(pb) != (pb->m == 16 ? ALGO_CONV16I : ALGO_CONV16))
        return "the single-conv dispatch takes another chain for one of the convs";
    return nullptr;
}

// The 8-channel pair (conv_pair8_kernel): 16 -> 8 -> 16, both 3x3 stride 1
// pad 1 on one map, the first in the im2col order and the second in the
// first-layer chain, as the single-conv dispatch takes them.
static const char *pair8_refusal(const osh_conv_params *pa, const osh_conv_params *pb, int act) {
    auto same_map_3x3 = [](const osh_conv_params *p) {
        return p->group == 1 && p->kh == 3 && p->kw == 3 && p->sh == 1 && p->sw == 1 && p->dh == 1 &&
               p->dw == 1 && p->pt == 1 && p->pl == 1 && p->oh == p->h && p->ow == p->w;
    };
    if (!same_map_3x3(pa) || !same_map_3x3(pb)) return "both convs must be 3x3, stride 1, pad 1 on one map";
    if (pa->n != 1 || pb->n != 1) return "batch 1 only";
    if (pb->c != pa->m || pb->h != pa->h || pb->w != pa->w) return "the second conv must read the first one's output";
    if (pa->c != 16 || pb->m != 16) return "an 8-channel intermediate pairs 16 -> 8 -> 16 only";
    if (act != OSH_ACT_SILU) return "the fused pair takes SiLU convs";
    if (16LL * pa->h * pa->w * 4 >= (1LL << 31)) return "input too large";
    if (select_algo(pa) != ALGO_CONV16I || select_algo(pb) != ALGO_FIRST)
        return "the single-conv dispatch takes another chain for one of the convs";
    return nullptr;
}

// The first-layer pair (first_pair_kernel): a 3x3 undilated conv of stride 1
// or 2 over c <= 4 planes with 16 outputs, which the single-conv dispatch
// runs as first_conv_kernel, then a 3x3 conv over exactly its output that the
// dispatch runs in the NCHWc order (32 or 64 outputs, stride 1 or 2, pad 1).
static const char *first_pair_refusal(const osh_conv_params *pa, const osh_conv_params *pb, int act) {
    if (pa->group != 1 || pa->kh != 3 || pa->kw != 3 || pa->dh != 1 || pa->dw != 1 || pa->sh != pa->sw ||
        (pa->sh != 1 && pa->sh != 2))
        return "a first-layer conv must be 3x3, undilated, stride 1 or 2";
    if (pa->n != 1 || pb->n != 1) return "batch 1 only";
    if (pa->m != 16) return "a first-layer conv must have 16 output channels";
    if (pb->c != 16 || pb->h != pa->oh || pb->w != pa->ow) return "the second conv must read the first one's output";
    if (pb->m != 32 && pb->m != 64) return "after a first-layer conv the second conv must have 32 or 64 outputs";
    if (act != OSH_ACT_SILU) return "the fused pair takes SiLU convs";
    if ((long long)pa->c * pa->h * pa->w * 4 >= (1LL << 31) || (long long)pb->m * pb->oh * pb->ow * 4 >= (1LL << 31))
        return "tensors too large";
    if (select_algo(pa) != ALGO_FIRST || !nchwc_enabled() || !nchwc_gate(pb) || select_algo(pb) != ALGO_CONV16)
        return "the single-conv dispatch takes another chain for one of the convs";
    return nullptr;
}

static osh_status check_pack(const void *d_wpacked, const osh_conv_params *p) {
    std::lock_guard<std::mutex> lk(g_packs_mu);
    auto it = g_packs.find(reinterpret_cast<uintptr_t>(d_wpacked));
    if (it != g_packs.end() && (it->second.algo != (int)select_algo(p) || it->second.key != conv_key(p)))
        return fail(OSH_E_INVALID, "Conv pair: weights packed for another kernel or shape");
    return OSH_OK;
}

}  // namespace osh

extern "C" {

OSH_API osh_status osh_conv2d_f32(const osh_conv_params *p, const float *d_x, const void *d_wpacked,
                                  const float *d_bias, int act, float *d_y, osh_stream s) {
    osh_status st = check_launch(p, d_x, d_wpacked, act, d_y);
    if (st != OSH_OK) return st;
    return conv2d(p, d_x, d_wpacked, d_bias, act, nullptr, d_y, to_stream(s));
}

OSH_API osh_status osh_conv2d_group_f32(int count, const osh_conv_params *ps, const float *const *d_xs,
                                        const void *const *d_ws, const float *const *d_biases, int act,
                                        const float *const *d_res, float *const *d_ys, osh_stream s) {
    if (count < 1 || count > kConvGroupMax) return fail(OSH_E_INVALID, "Conv group: %d convs (1..%d)", count,
                                                        kConvGroupMax);
    if (!ps || !d_xs || !d_ws || !d_ys) return fail(OSH_E_INVALID, "Conv group: NULL array");
    for (int i = 0; i < count; i++) {
        osh_status st = check_launch(&ps[i], d_xs[i], d_ws[i], act, d_ys[i]);
        if (st != OSH_OK) return st;
    }
    // The members run side by side in one launch: no output may overlap any
    // member's input, residual or output (the own input is checked above).
    for (int i = 0; i < count; i++)
        for (int j = 0; j < count; j++) {
            const float *rj = d_res ? d_res[j] : nullptr;
            if (ranges_overlap(d_ys[i], y_bytes(&ps[i]), rj, y_bytes(&ps[j])))
                return fail(OSH_E_INVALID, "Conv group: output %d overlaps the residual of conv %d", i, j);
            if (i != j && (ranges_overlap(d_ys[i], y_bytes(&ps[i]), d_xs[j], x_bytes(&ps[j])) ||
                           ranges_overlap(d_ys[i], y_bytes(&ps[i]), d_ys[j], y_bytes(&ps[j]))))
                return fail(OSH_E_INVALID, "Conv group: output %d overlaps the input or output of conv %d", i, j);
        }
    return conv2d_group(count, ps, d_xs, d_ws, d_biases, act, d_res, d_ys, to_stream(s));
}

OSH_API osh_status osh_conv2d_add_f32(const osh_conv_params *p, const float *d_x, const void *d_wpacked,
                                      const float *d_bias, int act, const float *d_res, float *d_y, osh_stream s) {
    osh_status st = check_launch(p, d_x, d_wpacked, act, d_y);
    if (st != OSH_OK) return st;
    if (!d_res) return fail(OSH_E_INVALID, "Conv+Add: residual is NULL");
    if (ranges_overlap(d_res, y_bytes(p), d_y, y_bytes(p)))
        return fail(OSH_E_INVALID, "Conv+Add: the residual overlaps the output");
    return conv2d(p, d_x, d_wpacked, d_bias, act, d_res, d_y, to_stream(s));
}

OSH_API osh_status osh_conv2d_pair_check(const osh_conv_params *pa, const osh_conv_params *pb, int act) {
    if (!pa || !pb) return fail(OSH_E_INVALID, "Conv pair: params is NULL");
    osh_status st = check_params(pa);
    if (st == OSH_OK) st = check_params(pb);
    if (st != OSH_OK) return st;
    if (const char *why = pair_refusal(pa, pb, act)) return fail(OSH_E_UNSUPPORTED, "Conv pair: %s", why);
    return OSH_OK;
}

OSH_API osh_status osh_conv2d_pair_f32(const osh_conv_params *pa, const osh_conv_params *pb, const float *d_x,
                                       const void *d_wa, const float *d_bias_a, const void *d_wb,
                                       const float *d_bias_b, int act, const float *d_res, float *d_ya, float *d_y,
                                       osh_stream s) {
    osh_status st = osh_conv2d_pair_check(pa, pb, act);
    if (st != OSH_OK) return st;
    if (!d_x || !d_wa || !d_wb || !d_y) return fail(OSH_E_INVALID, "Conv pair: NULL tensor pointer");
    if ((st = check_pack(d_wa, pa)) != OSH_OK || (st = check_pack(d_wb, pb)) != OSH_OK) return st;
    // every workgroup reads input rows that neighbouring workgroups' outputs
    // would cover if they overlapped; a residual inside the output would be
    // added again by every launch of first-use timing
    const size_t xb = x_bytes(pa), yab = y_bytes(pa), yb = y_bytes(pb);
    if (ranges_overlap(d_y, yb, d_x, xb) || (d_ya && ranges_overlap(d_ya, yab, d_x, xb)) ||
        (d_ya && ranges_overlap(d_ya, yab, d_y, yb)))
        return fail(OSH_E_INVALID, "Conv pair: an output overlaps the input or the other output");
    if (d_res && ranges_overlap(d_res, yb, d_y, yb))
        return fail(OSH_E_INVALID, "Conv pair: the residual overlaps the output");
    if (d_res && d_ya && ranges_overlap(d_res, yb, d_ya, yab))
        return fail(OSH_E_INVALID, "Conv pair: the residual overlaps the intermediate");
    hipStream_t stream = to_stream(s);
    if (pa->c <= 4) {
        // the first-layer pair: its tiles, then (with an intermediate buffer)
        // the two convs as separate launches; tile 0 before first-use timing
        FirstPairArgs f{};
        f.h = pa->h;
        f.w = pa->w;
        f.c0 = pa->c;
        f.pt = pa->pt;
        f.pl = pa->pl;
        f.ah = pa->oh;
        f.aw = pa->ow;
        f.bh = pb->oh;
        f.bw = pb->ow;
        f.x = d_x;
        f.wa = static_cast<const float *>(d_wa);
        f.ba = d_bias_a;
        f.wb = static_cast<const float *>(d_wb);
        f.bb = d_bias_b;
        f.res = d_res;
        f.ya = d_ya;
        f.y = d_y;
        const int nft = first_pair_tile_count();
        const auto key = std::make_tuple(kPairTuneTag + 2 + (d_ya ? 0 : 1), mix_key(conv_key(pa), conv_key(pb)));
        return tuned_launch_key(
            key, nft + 1, pair_tile(), [&](int v) { return v < nft || d_ya != nullptr; },
            [&](int v) {
                if (v < 0) v = 0;
                if (v == nft) {
                    osh_status st = conv2d(pa, d_x, d_wa, d_bias_a, act, nullptr, d_ya, stream);
                    return st != OSH_OK ? st : conv2d(pb, d_ya, d_wb, d_bias_b, act, d_res, d_y, stream);
                }
                return first_pair_launch(f, pa->sh, pb->sh, pb->m / 16, stream, v);
            },
            stream);
    }
    PairArgs a{};
    a.h = pa->h;
    a.w = pa->w;
    a.c0 = pa->c;
    a.x = d_x;
    a.wa = static_cast<const float *>(d_wa);
    a.ba = d_bias_a;
    a.wb = static_cast<const float *>(d_wb);
    a.bb = d_bias_b;
    a.res = d_res;
    a.ya = d_ya;
    a.y = d_y;
    const int cb1 = pa->m / 16, cb2 = pb->m / 16;
    const bool eight = pa->m == 8;  // conv_pair8_kernel
    // Variants: the pair kernel's tiles, then (when the intermediate has a
    // buffer) the two convs as separate launches -- the pair's ring
    // recompute runs on one CU's four MFMA pipes, which loses to two
    // launches on small maps and wide intermediates.  First-use timing picks;
    // before it (graph capture) the pair runs on maps of 80x80 and more with
    // at most 32 intermediate channels.
    const int ntile = conv_pair_tile_count();
    const auto key = std::make_tuple(kPairTuneTag + (d_ya ? 0 : 1), mix_key(conv_key(pa), conv_key(pb)));
    return tuned_launch_key(
        key, ntile + 1, pair_tile(), [&](int v) { return v < ntile || d_ya != nullptr; },
        [&](int v) {
            if (v < 0) v = (pa->h * pa->w >= 6400 && pa->m <= 32) || !d_ya ? 2 : ntile;
            if (v == ntile) {
                osh_status st = conv2d(pa, d_x, d_wa, d_bias_a, act, nullptr, d_ya, stream);
                return st != OSH_OK ? st : conv2d(pb, d_ya, d_wb, d_bias_b, act, d_res, d_y, stream);
            }
            return eight ? conv_pair8_launch(a, stream, v) : conv_pair_launch(a, cb1, cb2, stream, v);
        },
        stream);
}

}  // extern "C"
