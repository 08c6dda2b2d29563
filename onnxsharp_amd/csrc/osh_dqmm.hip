// osh_dqmm.hip -- DynamicQuantizeMatMul and DynamicQuantizeLinear on gfx950.
//
// Reference: DynamicQuantizeMatMulLayer.Forward (src/OnnxSharp/Ops/QuantizedMatMulOps.cs:115-201),
// Quantizer.MinMax (src/OnnxSharp/Tensors/Quantization.cs:109-181), QuantizeAndWiden
// (QuantizedMatMulOps.cs:280-335) and the zero-point identity of PackedInt8Weights
// (src/OnnxSharp/Kernels/Int8Gemm.cs:66-70).
//
// Pipeline (three launches, all on the caller's stream; by default 2 and 3
// run as one launch, dqmm_fused_kernel):
//   1. dqmm_minmax_kernel   grid-stride min/max of A (0 included, NaN skipped) into per-block
//                           partials.
//   2. dqmm_quantize_kernel every block reduces the partials to scale = (max-min)/255 (1 if
//                           not > 0), zp = clamp(rne(-min/scale)), inv = 1/scale -- single IEEE
//                           ops, no contraction -- then q = clamp(rne(x*inv) + zp, 0, 255); stores
//                           a'' = q - 128 as s8 in the MFMA operand layout, the per-row sums of
//                           a'', and a per-row flag for x*inv = NaN (the reference's q is then
//                           NaN and its whole output row is NaN).
//   3. dqmm_gemm_kernel     v_mfma_i32_32x32x32_i8 over a'' x w'' (both s8), then the exact
//                           integer correction
//                             acc = sum a''w'' + off_j*rowsum_i + alpha*colsum_j + K*alpha*off_j
//                           with alpha = 128 - zp and w' = w'' + off_j (w'' is the raw s8
//                           weight, or w - 128 for u8 weights; off_j = (u8 ? 128 : 0) - w_zp_j),
//                           which equals sum (q - zp)(w - w_zp) exactly; then
//                           out = fmaf((float)acc, scale * w_scale[j], bias[j]).
//
// Operand layout (both operands): fragment f = (tile, kstep) holds 64 lanes x 16 bytes;
// lane l carries row/column (l & 31) of the tile and k = kstep*32 + 16*(l >> 5) + byte.
// A and B use the same k assignment, so the MFMA pairs matching k regardless of the
// hardware's internal k order.
#include "osh_common.h"

using namespace osh;

namespace osh {

constexpr int DQ_MINMAX_BLOCKS = 256;
constexpr int DQ_THREADS = 256;
constexpr int DQ_KC = 16;  // k-steps of 32 per GEMM load chunk (K = 512 in one chunk)

struct DqScratch {  // layout of the caller's scratch buffer
    float partial_min[DQ_MINMAX_BLOCKS];
    float partial_max[DQ_MINMAX_BLOCKS];
    int zp;
    float scale;
    float inv;
    int alpha;  // a - a_zp = a'' + alpha for the packed a'' (128 - zp for quantized u8)
    int pad[60];
    // followed by: int rowsum[mpad]; int rownan[mpad]; int8 a_packed[mpad * kpad]
};

__host__ __device__ static inline int pad32(int v) { return (v + 31) & ~31; }

static size_t scratch_bytes(int m, int k) {
    return sizeof(DqScratch) + (size_t)pad32(m) * 8 + (size_t)pad32(m) * pad32(k);
}

__device__ __forceinline__ float wave_min(float v) {
    for (int o = 32; o > 0; o >>= 1) v = __builtin_fminf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o));
    return v;
}

// Block-level min/max of (lo, hi) into thread 0's return values (NW waves).
template <int NW = DQ_THREADS / 64>
__device__ void block_minmax(float &lo, float &hi) {
    __shared__ float smin[NW], smax[NW];
    lo = wave_min(lo);
    hi = wave_max(hi);
    int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        smin[w] = lo;
        smax[w] = hi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < NW; i++) {
            lo = __builtin_fminf(lo, smin[i]);
            hi = __builtin_fmaxf(hi, smax[i]);
        }
    }
}

__global__ __launch_bounds__(DQ_THREADS) void dqmm_minmax_kernel(const float *__restrict__ a, long long n,
                                                                  DqScratch *__restrict__ sc) {
    float lo = 0.f, hi = 0.f;  // 0 is always inside the range (Quantization.cs:115-116)
    long long stride = (long long)gridDim.x * blockDim.x;
    // XCD-banded block ids: the workgroups of one XCD read one contiguous band
    // of A, which the fused kernel's workgroups on the same XCD (banded the
    // same way, row tiles first) then find in that XCD's L2.  Min and max are
    // exact in any order, so the partials' assignment does not matter.
    long long i = (long long)xcd_band(blockIdx.x, gridDim.x) * blockDim.x + threadIdx.x;
    // 16-byte loads when the base is aligned (all callers pass tensor bases)
    long long n4 = (reinterpret_cast<uintptr_t>(a) & 15) == 0 ? n / 4 : 0;
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    for (long long j = i; j < n4; j += stride) {
        float4 v = a4[j];
        // NaN lanes are skipped (compare-false keeps the running value)
        lo = v.x < lo ? v.x : lo; hi = v.x > hi ? v.x : hi;
        lo = v.y < lo ? v.y : lo; hi = v.y > hi ? v.y : hi;
        lo = v.z < lo ? v.z : lo; hi = v.z > hi ? v.z : hi;
        lo = v.w < lo ? v.w : lo; hi = v.w > hi ? v.w : hi;
    }
    for (long long j = n4 * 4 + i; j < n; j += stride) {
        float v = a[j];
        lo = v < lo ? v : lo;
        hi = v > hi ? v : hi;
    }
    block_minmax(lo, hi);
    if (threadIdx.x == 0) {
        sc->partial_min[blockIdx.x] = lo;
        sc->partial_max[blockIdx.x] = hi;
    }
}

// scale = (max-min)/255 (1 if not > 0), zp = clamp(rne(-min/scale)),
// inv = 1/scale: single IEEE ops, no contraction (QuantizedMatMulOps.cs:151-155;
// QuantizeAndWiden multiplies by the reciprocal, :282).
__device__ __forceinline__ void dq_param_values(float lo, float hi, float &scale, int &zp, float &inv) {
    scale = (hi - lo) / 255.0f;
    if (!(scale > 0.0f)) scale = 1.0f;
    const float zf = __builtin_rintf(-lo / scale);
    zp = (int)zf;
    zp = zp < 0 ? 0 : (zp > 255 ? 255 : zp);
    inv = 1.0f / scale;
}

// The parameters for later launches and the caller.
__device__ __forceinline__ void dq_publish_params(DqScratch *__restrict__ sc, int *__restrict__ qparams, float scale,
                                                  int zp, float inv) {
    sc->scale = scale;
    sc->zp = zp;
    sc->inv = inv;
    sc->alpha = 128 - zp;
    if (qparams) {
        qparams[0] = __float_as_int(scale);
        qparams[1] = zp;
    }
}

// Every consumer block reduces the per-block partials itself (a few hundred
// floats from L2), so no grid-wide counter is needed and the scratch needs no
// initialisation.  One block (`publish`) stores the parameters for later
// launches and the caller.
template <int NW = DQ_THREADS / 64>
__device__ void dq_finish(DqScratch *__restrict__ sc, float lo, float hi, int *__restrict__ qparams,
                          bool publish, float &inv_out, int &zp_out, float *scale_out) {
    __shared__ float s_inv, s_scale;
    __shared__ int s_zp;
    block_minmax<NW>(lo, hi);
    if (threadIdx.x == 0) {
        float scale, inv;
        int zp;
        dq_param_values(lo, hi, scale, zp, inv);
        s_inv = inv;
        s_scale = scale;
        s_zp = zp;
        if (publish) dq_publish_params(sc, qparams, scale, zp, inv);
    }
    __syncthreads();
    inv_out = s_inv;
    zp_out = s_zp;
    if (scale_out) *scale_out = s_scale;
}

__device__ void dq_params(DqScratch *__restrict__ sc, int nparts, int *__restrict__ qparams, bool publish,
                          float &inv_out, int &zp_out) {
    float lo = 0.f, hi = 0.f;
    for (int b = threadIdx.x; b < nparts; b += blockDim.x) {
        lo = __builtin_fminf(lo, sc->partial_min[b]);
        hi = __builtin_fmaxf(hi, sc->partial_max[b]);
    }
    dq_finish(sc, lo, hi, qparams, publish, inv_out, zp_out, nullptr);
}

// q = clamp(rne(x * inv) + zp, 0, 255) as QuantizeAndWiden computes it in float.
// A NaN product yields 0 here; callers flag it (the reference's q is NaN then).
__device__ __forceinline__ int quantize_one(float x, float inv, float zpf) {
    float q = __builtin_rintf(x * inv) + zpf;
    q = __builtin_fminf(255.0f, __builtin_fmaxf(0.0f, q));
    return (int)q;
}

// One wave per row of A (padded rows write zeros): each lane quantizes 4
// consecutive k per step (one 16-byte load, one 4-byte store into the lane's
// operand slot), and the row sum of a'' and the NaN flag are wave reductions,
// so the kernel needs no atomics and no zeroed scratch.
struct Quad {
    float v[4];
};

// x[kk .. kk+3] of one row (zeros past k or for padding rows).
__device__ __forceinline__ Quad load_quad(const float *__restrict__ src, int kk, int k, bool live, bool vec) {
    Quad q = {{0.f, 0.f, 0.f, 0.f}};
    if (live && kk < k) {
        if (vec) {
            float4 v = *reinterpret_cast<const float4 *>(src + kk);
            q.v[0] = v.x; q.v[1] = v.y; q.v[2] = v.z; q.v[3] = v.w;
        } else {
#pragma unroll
            for (int b = 0; b < 4; b++) q.v[b] = kk + b < k ? src[kk + b] : 0.f;
        }
    }
    return q;
}

constexpr int DQ_QPRE = 4;  // row chunks of 256 loaded before the parameter reduction

__global__ __launch_bounds__(DQ_THREADS) void dqmm_quantize_kernel(const float *__restrict__ a, int m, int k,
                                                                    DqScratch *__restrict__ sc, int nparts,
                                                                    int *__restrict__ qparams,
                                                                    int *__restrict__ rowsum,
                                                                    int8_t *__restrict__ apk) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (DQ_THREADS / 64) + (threadIdx.x >> 6);
    const int kpad = pad32(k), mpad = pad32(m);
    const bool live = row < m;
    const float *src = a + (long long)(live ? row : 0) * k;
    const bool vec = (k & 3) == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0;
    // The first chunks of the row are in flight while the block reduces the
    // min/max partials.
    Quad pre[DQ_QPRE];
#pragma unroll
    for (int c = 0; c < DQ_QPRE; c++) pre[c] = load_quad(src, 4 * lane + 256 * c, k, live, vec);
    float inv;
    int zp;
    dq_params(sc, nparts, qparams, blockIdx.x == 0, inv, zp);
    if (row >= mpad) return;
    const float zpf = (float)zp;
    int *dst = reinterpret_cast<int *>(apk) + (long long)(row >> 5) * (kpad / 32) * 256 + (row & 31) * 4;
    int sum = 0;
    bool nan = false;
    auto emit = [&](const Quad &x, int kk) {
        unsigned packed = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            int v = 0;  // padding rows/columns carry a'' = 0
            if (live && kk + b < k) {
                float p = x.v[b] * inv;
                nan |= !(p == p);
                v = quantize_one(x.v[b], inv, zpf) - 128;
                sum += v;
            }
            packed |= (unsigned)(v & 0xff) << (8 * b);
        }
        // fragment (row/32, kk/32); lane slot (row & 31) + 32 * ((kk >> 4) & 1); byte kk & 15
        dst[(kk >> 5) * 256 + ((kk >> 4) & 1) * 128 + ((kk & 15) >> 2)] = (int)packed;
    };
#pragma unroll
    for (int c = 0; c < DQ_QPRE; c++) {
        const int kk = 4 * lane + 256 * c;
        if (kk < kpad) emit(pre[c], kk);
    }
    for (int kk = 4 * lane + 256 * DQ_QPRE; kk < kpad; kk += 256) emit(load_quad(src, kk, k, live, vec), kk);
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    const bool any_nan = __any(nan);
    if (lane == 0) {
        rowsum[row] = sum;
        rowsum[mpad + row] = any_nan ? 1 : 0;
    }
}

// MatMulInteger's activations: one wave per row turns u8 (a - 128) or s8 (a)
// into the s8 a'' of the MFMA layout and sums each row; block 0 publishes
// alpha = (u8 ? 128 : 0) - a_zp so that a - a_zp = a'' + alpha.
__global__ __launch_bounds__(DQ_THREADS) void mmi_pack_a_kernel(const uint8_t *__restrict__ a, int m, int k,
                                                                 int a_signed, int a_zp, DqScratch *__restrict__ sc,
                                                                 int *__restrict__ rowsum, int8_t *__restrict__ apk) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (DQ_THREADS / 64) + (threadIdx.x >> 6);
    const int kpad = pad32(k), mpad = pad32(m);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        sc->alpha = (a_signed ? 0 : 128) - a_zp;
        sc->scale = 1.0f;
        sc->zp = a_zp;
    }
    if (row >= mpad) return;
    const bool live = row < m;
    const uint8_t *src = a + (long long)(live ? row : 0) * k;
    int *dst = reinterpret_cast<int *>(apk) + (long long)(row >> 5) * (kpad / 32) * 256 + (row & 31) * 4;
    int sum = 0;
    for (int kk = 4 * lane; kk < kpad; kk += 256) {
        unsigned packed = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            int v = 0;  // padding rows/columns carry a'' = 0
            if (live && kk + b < k) {
                const int raw = src[kk + b];
                v = a_signed ? (int)(int8_t)raw : raw - 128;
                sum += v;
            }
            packed |= (unsigned)(v & 0xff) << (8 * b);
        }
        dst[(kk >> 5) * 256 + ((kk >> 4) & 1) * 128 + ((kk & 15) >> 2)] = (int)packed;
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    if (lane == 0) {
        rowsum[row] = sum;
        rowsum[mpad + row] = 0;
    }
}

// DynamicQuantizeLinear output: u8 q in the input's own layout.
__global__ __launch_bounds__(DQ_THREADS) void dql_quantize_kernel(const float *__restrict__ x, long long n,
                                                                   DqScratch *__restrict__ sc, int nparts,
                                                                   int *__restrict__ qparams,
                                                                   uint8_t *__restrict__ q) {
    float inv;
    int zp;
    dq_params(sc, nparts, qparams, blockIdx.x == 0, inv, zp);
    const float zpf = (float)zp;
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long stride = (long long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) q[i] = (uint8_t)quantize_one(x[i], inv, zpf);
}

// Packed weight buffer: int8 fragments [npad/32][kpad/32][64][16], then int colsum[npad],
// then int off[npad].
static size_t packed_w_bytes(int k, int n) { return (size_t)pad32(n) * pad32(k) + (size_t)pad32(n) * 8; }

__global__ void dqmm_pack_kernel(int k, int n, const void *__restrict__ w, int w_signed,
                                 const int *__restrict__ wzp, int n_wzp, int8_t *__restrict__ out,
                                 int *__restrict__ colsum, int *__restrict__ off) {
    // one thread per column
    int j = blockIdx.x * blockDim.x + threadIdx.x;
    int npad = pad32(n), kpad = pad32(k);
    if (j >= npad) return;
    int zp = (j < n && n_wzp > 0) ? (n_wzp == 1 ? wzp[0] : wzp[j]) : 0;
    int o = (w_signed ? 0 : 128) - zp;
    int s = 0;
    for (int kk = 0; kk < kpad; kk++) {
        int v = 0;
        if (j < n && kk < k) {
            long long idx = (long long)kk * n + j;
            v = w_signed ? (int)reinterpret_cast<const int8_t *>(w)[idx]
                         : (int)reinterpret_cast<const uint8_t *>(w)[idx] - 128;
            s += v;
        }
        long long frag = (long long)(j >> 5) * (kpad / 32) + (kk >> 5);
        int lane = (j & 31) + 32 * ((kk >> 4) & 1);
        out[(frag * 64 + lane) * 16 + (kk & 15)] = (int8_t)v;
    }
    colsum[j] = s;
    off[j] = j < n ? o : 0;
}

// Wave tile 32 x 32, 4 waves per block as 2 x 2 -> 64 x 64 outputs per block.
__global__ __launch_bounds__(256) void dqmm_gemm_kernel(int m, int k, int n, const int8_t *__restrict__ apk,
                                                        const int8_t *__restrict__ wpk,
                                                        const int *__restrict__ colsum, const int *__restrict__ off,
                                                        const int *__restrict__ rowsum,
                                                        const DqScratch *__restrict__ sc,
                                                        const float *__restrict__ wscale, int n_wscale,
                                                        const float *__restrict__ bias, float *__restrict__ out,
                                                        int *__restrict__ acc_out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int mt = blockIdx.y * 2 + (wave >> 1);
    const int nt = blockIdx.x * 2 + (wave & 1);
    const int kpad = pad32(k), ks = kpad / 32;
    if (mt * 32 >= pad32(m) || nt * 32 >= pad32(n)) return;
    const i32x4 *A = reinterpret_cast<const i32x4 *>(apk) + (long long)mt * ks * 64 + lane;
    const i32x4 *B = reinterpret_cast<const i32x4 *>(wpk) + (long long)nt * ks * 64 + lane;
    // Epilogue operands are loaded before the k loop so their latency overlaps it.
    // The lane's 16 rows are 4 runs of 4 consecutive rows: their row sums and
    // NaN flags are 8 int4 loads (rows are padded to mpad, columns to npad).
    const int j = nt * 32 + (lane & 31);
    const int mpad = pad32(m);
    int4 rs[4], rn[4];
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const int i0 = mt * 32 + 8 * g + 4 * (lane >> 5);
        rs[g] = *reinterpret_cast<const int4 *>(rowsum + i0);
        rn[g] = *reinterpret_cast<const int4 *>(rowsum + mpad + i0);
    }
    // two's-complement wrap-around below is exact as long as the final sum fits in int32
    const unsigned offj = (unsigned)off[j];
    const int csum = colsum[j];
    const float ws = (wscale && j < n) ? (n_wscale == 1 ? wscale[0] : wscale[j]) : 0.0f;
    const float bj = (bias && j < n) ? bias[j] : 0.0f;
    const int aalpha = sc->alpha;
    const float ascale = sc->scale;
    // k in chunks of DQ_KC steps: the next chunk's 2*DQ_KC loads are in flight
    // while the current chunk's MFMAs run.
    i32x16 acc = {};
    i32x4 a[DQ_KC], b[DQ_KC];
    const int full = ks / DQ_KC;
    if (full > 0) {
#pragma unroll
        for (int t = 0; t < DQ_KC; t++) {
            a[t] = A[t * 64];
            b[t] = B[t * 64];
        }
    }
    for (int c = 0; c < full; c++) {
        i32x4 na[DQ_KC], nb[DQ_KC];
        const bool more = c + 1 < full;
        if (more) {
#pragma unroll
            for (int t = 0; t < DQ_KC; t++) {
                na[t] = A[((c + 1) * DQ_KC + t) * 64];
                nb[t] = B[((c + 1) * DQ_KC + t) * 64];
            }
        }
#pragma unroll
        for (int t = 0; t < DQ_KC; t++) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[t], b[t], acc, 0, 0, 0);
        if (more) {
#pragma unroll
            for (int t = 0; t < DQ_KC; t++) {
                a[t] = na[t];
                b[t] = nb[t];
            }
        }
    }
    for (int s = full * DQ_KC; s < ks; s++)
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[s * 64], B[s * 64], acc, 0, 0, 0);

    if (j >= n) return;
    const unsigned alpha = (unsigned)aalpha;
    const unsigned colterm = alpha * (unsigned)csum + (unsigned)k * alpha * offj;
    const float comb = ascale * ws;  // CombinedScale, QuantizedMatMulOps.cs:203-221
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int i = mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int4 s4 = rs[r >> 2], n4 = rn[r >> 2];
        const int rsum = (r & 3) == 0 ? s4.x : (r & 3) == 1 ? s4.y : (r & 3) == 2 ? s4.z : s4.w;
        const int rnan = (r & 3) == 0 ? n4.x : (r & 3) == 1 ? n4.y : (r & 3) == 2 ? n4.z : n4.w;
        if (i < m) {
            int v = (int)((unsigned)acc[r] + offj * (unsigned)rsum + colterm);
            if (acc_out) acc_out[(long long)i * n + j] = v;
            if (out) {
                float o = __builtin_fmaf((float)v, comb, bj);
                if (rnan) o = __builtin_nanf("");
                out[(long long)i * n + j] = o;
            }
        }
    }
}

// Quantize + GEMM in one launch, after dqmm_minmax_kernel.  A workgroup owns
// 32 rows of A and DQF_WAVES column tiles of 32.  Its 256 threads load the
// rows' floats (thread -> row tid/8, four consecutive k at 32*i + 4*(tid%8))
// and each wave its column tile's B fragments for a pass of DQF_KS k-steps,
// all issued at once behind the min/max partials and the epilogue's column
// operands.  The threads quantize with the parameters every workgroup reduces
// from the partials and store a'' = q - 128 in the MFMA A-operand order in
// LDS; after one barrier each wave runs its v_mfma_i32_32x32x32_i8 chain.  The
// row sums of a'' (v_dot4 over the packed bytes) and the NaN flags come from
// the same registers; nothing but the parameters goes through global scratch.
// Arithmetic (quantization, zero-point correction, epilogue) is the
// three-launch pipeline's, so both give identical bits.
//
// Time line of one launch at C5's size (512 x 512 x 2048; per-workgroup
// s_memrealtime stamps in a copy of the kernel, medians): workgroups start
// over 0.7 us; the first loads return after ~2 us (a cold first load takes
// that long even with nothing else in flight); quantization 0.9 us; the MFMA
// chain 1.0 us; the output stores 1.2 us, near the HBM write rate for 4 MB.
constexpr int DQF_WAVES = 4;
constexpr int DQF_KS = 16;  // k-steps of 32 per pass: K = 512 in one pass
constexpr int DQF_GM = 4;   // row tiles per group of the tile order
static_assert(DQ_MINMAX_BLOCKS <= 256, "one min/max partial per thread of a 256-thread workgroup");

// Four elements of one row, quantized: returns the packed a'' bytes
// (q - 128 as s8) and adds their sum and NaN flag.  `live_mask` bit e says
// whether element e is a real element (else its a'' is 0).  v_cvt_pk_u8_f32
// converts with round-to-nearest-even and saturates to [0, 255] (a NaN gives
// 0), so on the integer-valued q = rne(x * inv) + zp it is the clamp of
// QuantizeAndWiden; both facts were checked on the device for every integer
// from -1000 to 1300, the .25/.5/.75 fractions, +-inf and NaN, and the
// pipelines' bit equality is tested.
__device__ __forceinline__ unsigned quantize4(const Quad &x, float inv, float zpf, unsigned live_mask, int &sum,
                                              bool &nan) {
    unsigned packed = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float p = x.v[e] * inv;
        const float q = __builtin_rintf(p) + zpf;
        if (live_mask & (1u << e)) {
            nan |= !(p == p);
            packed = __builtin_amdgcn_cvt_pk_u8_f32(q, e, packed);
        } else {
            packed |= 128u << (8 * e);  // q = 128 <-> a'' = 0
        }
    }
    packed ^= 0x80808080u;  // q -> q - 128, byte by byte
    sum = __builtin_amdgcn_sdot4((int)packed, 0x01010101, sum, false);
    return packed;
}

// FULL: m % 32 == 0, n % 128 == 0, k % 512 == 0 and A 16-byte aligned, so
// every row, column and k-step is live and no load or store needs a check.
// The host picks it whenever it applies; the kernel then has no divergent
// paths, so the compiler issues all operand loads before the first wait
// (with the checks, the registers of the two load paths are merged by copies
// that wait for every A load before any B load is issued).
//
// A and W are not declared __restrict__: the operand loads must stay ahead of
// the barriers that follow them (the compiler may otherwise sink loads of
// restrict read-only memory to their first use).
template <bool FULL>
__global__ __launch_bounds__(64 * DQF_WAVES) void dqmm_fused_kernel(
    int m, int k, int n, const float *a, DqScratch *__restrict__ sc, int nparts, int *__restrict__ qparams,
    const int8_t *wpk, const int *__restrict__ colsum, const int *__restrict__ off,
    const float *__restrict__ wscale, int n_wscale, const float *__restrict__ bias, float *__restrict__ out,
    int *__restrict__ acc_out) {
    __shared__ __attribute__((aligned(16))) int lds_a[DQF_KS * 256];  // [kstep][64 lanes][16 bytes]
    __shared__ int lds_rs[32], lds_rn[32];
    const int tid = threadIdx.x, lane = tid & 63, wt = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kpad = pad32(k), ks = kpad / 32, npad = pad32(n);
    // Tiles: XCD-banded ids, then groups of DQF_GM row tiles x all column
    // blocks, so one XCD's L2 holds a few row tiles of A and part of W.
    const int ncb = (npad / 32 + DQF_WAVES - 1) / DQF_WAVES, nmt = pad32(m) / 32;
    const int id = xcd_band(blockIdx.x, gridDim.x);
    const int grp = id / (DQF_GM * ncb), gl = id % (DQF_GM * ncb);
    const int mt0 = grp * DQF_GM;
    const int gm = nmt - mt0 < DQF_GM ? nmt - mt0 : DQF_GM;
    const int mt = mt0 + gl % gm;
    const int nt = (gl / gm) * DQF_WAVES + wt;
    const bool col_live = FULL || nt * 32 < npad;
    const int r = tid >> 3, c8 = tid & 7;
    const int row = mt * 32 + r;
    const bool live = FULL || row < m;
    const float *src = a + (long long)(live ? row : 0) * k;
    const bool vec = FULL || ((k & 3) == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0);
    // all 32 rows live and 16-byte loads: passes inside k need no per-element checks
    const bool rows_full = FULL || (vec && mt * 32 + 32 <= m);
    const int npass = (ks + DQF_KS - 1) / DQF_KS;
    const i32x4 *B = reinterpret_cast<const i32x4 *>(wpk) + (long long)(col_live ? nt : 0) * ks * 64 + lane;

    // nparts <= 256: one partial per thread (threads past nparts repeat
    // partial 0), consumed after the operand loads are issued
    const int pidx = tid < nparts ? tid : 0;
    const float pmin = sc->partial_min[pidx], pmax = sc->partial_max[pidx];
    // the epilogue's column operands, loaded now so their latency hides under the pass
    const int j = nt * 32 + (lane & 31);
    const bool jlive = col_live && (FULL || j < n);
    const int offj_raw = jlive ? off[j] : 0;
    const int csum = jlive ? colsum[j] : 0;
    const float ws = jlive ? (n_wscale == 1 ? wscale[0] : wscale[j]) : 0.0f;
    const float bj = (jlive && bias) ? bias[j] : 0.0f;

    Quad x[DQF_KS];
    i32x4 b[DQF_KS];
    auto load_pass = [&](int s0) {
        if (FULL || (rows_full && (s0 + DQF_KS) * 32 <= k)) {
#pragma unroll
            for (int i = 0; i < DQF_KS; i++) {
                const float4 v = *reinterpret_cast<const float4 *>(src + (s0 + i) * 32 + 4 * c8);
                x[i].v[0] = v.x; x[i].v[1] = v.y; x[i].v[2] = v.z; x[i].v[3] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < DQF_KS; i++) x[i] = load_quad(src, (s0 + i) * 32 + 4 * c8, k, live, vec);
        }
        if (FULL) {
#pragma unroll
            for (int t = 0; t < DQF_KS; t++) b[t] = B[(s0 + t) * 64];
        } else if (col_live) {
#pragma unroll
            for (int t = 0; t < DQF_KS; t++)
                if (s0 + t < ks) b[t] = B[(s0 + t) * 64];
        }
    };
    load_pass(0);
    // nothing below moves above this point: every load is out before the
    // first wait
    __builtin_amdgcn_sched_barrier(0);

    float inv, scale;
    int zp;
    dq_finish(sc, __builtin_fminf(0.f, pmin), __builtin_fmaxf(0.f, pmax), qparams, blockIdx.x == 0, inv, zp,
              &scale);
    const float zpf = (float)zp;

    // The MFMA chain runs as two interleaved chains (even and odd k-steps)
    // summed at the end; int32 sums are exact in any order.
    int sum = 0;
    bool nan = false;
    i32x16 acc0 = {}, acc1 = {};
    int *dst = lds_a + (r + 32 * (c8 >> 2)) * 4 + (c8 & 3);
    for (int ps = 0; ps < npass; ps++) {
        const int s0 = ps * DQF_KS;
        if (FULL || (rows_full && (s0 + DQF_KS) * 32 <= k)) {
#pragma unroll
            for (int i = 0; i < DQF_KS; i++) dst[i * 256] = (int)quantize4(x[i], inv, zpf, 0xfu, sum, nan);
        } else {
#pragma unroll
            for (int i = 0; i < DQF_KS; i++) {
                const int kk = (s0 + i) * 32 + 4 * c8;
                if (kk < kpad) {
                    unsigned lm = 0;
#pragma unroll
                    for (int e = 0; e < 4; e++) lm |= (live && kk + e < k) ? (1u << e) : 0u;
                    dst[i * 256] = (int)quantize4(x[i], inv, zpf, lm, sum, nan);
                }
            }
        }
        __syncthreads();
        if (col_live) {
            const int *srcl = lds_a + lane * 4;
            if (FULL || s0 + DQF_KS <= ks) {
                i32x4 av[DQF_KS];
#pragma unroll
                for (int t = 0; t < DQF_KS; t++) av[t] = *reinterpret_cast<const i32x4 *>(srcl + t * 256);
#pragma unroll
                for (int t = 0; t < DQF_KS; t += 2) {
                    acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[t], b[t], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[t + 1], b[t + 1], acc1, 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int t = 0; t < DQF_KS; t++) {
                    if (s0 + t < ks) {
                        const i32x4 av = *reinterpret_cast<const i32x4 *>(srcl + t * 256);
                        if (t & 1) acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b[t], acc1, 0, 0, 0);
                        else acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b[t], acc0, 0, 0, 0);
                    }
                }
            }
        }
        if (ps + 1 < npass) {
            // the next pass's loads go out after this pass's MFMAs, whose b
            // registers they reuse
            __builtin_amdgcn_sched_barrier(0);
            load_pass(s0 + DQF_KS);  // x and b are free: the pass is quantized and multiplied
            __syncthreads();         // every wave's MFMAs have read the pass before it is rewritten
        }
    }
    const i32x16 acc = acc0 + acc1;
    // a row's 8 threads are consecutive lanes of one wave
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        sum += __shfl_xor(sum, o);
        const int other = __shfl_xor(nan ? 1 : 0, o);
        nan = nan || other != 0;
    }
    if (c8 == 0) {
        lds_rs[r] = sum;
        lds_rn[r] = nan ? 1 : 0;
    }
    __syncthreads();
    if (!jlive) return;
    const unsigned offj = (unsigned)offj_raw;
    const unsigned alpha = (unsigned)(128 - zp);
    const unsigned colterm = alpha * (unsigned)csum + (unsigned)k * alpha * offj;
    const float comb = scale * ws;  // CombinedScale, QuantizedMatMulOps.cs:203-221
    if constexpr (FULL) {
        // Float output only, 16-byte aligned: the wave's 32 x 32 tile goes
        // through its own 4 KB of lds_a (every wave's A reads ended before
        // the barrier above) so that each lane stores four 16-byte vectors
        // -- eight lanes a 128-byte row -- instead of 16 single words.  The
        // values are the ones the loop below computes.
        if (out && !acc_out && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {  // uniform
            float *tl = reinterpret_cast<float *>(lds_a) + wt * 1024;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int il = 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
                const int v = (int)((unsigned)acc[q] + offj * (unsigned)lds_rs[il] + colterm);
                float o = __builtin_fmaf((float)v, comb, bj);
                if (lds_rn[il]) o = __builtin_nanf("");
                tl[il * 32 + (lane & 31)] = o;
            }
            // the lanes of this wave read what the others wrote (LDS accesses
            // of a wave are in order; this keeps the compiler from moving them)
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
            for (int pass = 0; pass < 4; pass++) {
                const int rr = pass * 8 + (lane >> 3), c4 = (lane & 7) * 4;
                const float4 v4 = *reinterpret_cast<const float4 *>(tl + rr * 32 + c4);
                *reinterpret_cast<float4 *>(out + (long long)(mt * 32 + rr) * n + nt * 32 + c4) = v4;
            }
            return;
        }
    }
#pragma unroll
    for (int q = 0; q < 16; q++) {
        const int il = 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
        const int i = mt * 32 + il;
        if (FULL || i < m) {
            const int rs = lds_rs[il], rn = lds_rn[il];
            const int v = (int)((unsigned)acc[q] + offj * (unsigned)rs + colterm);
            if (acc_out) acc_out[(long long)i * n + j] = v;
            if (out) {
                float o = __builtin_fmaf((float)v, comb, bj);
                if (rn) o = __builtin_nanf("");
                out[(long long)i * n + j] = o;
            }
        }
    }
}

// The fused kernel on 16 x 16 output tiles (v_mfma_i32_16x16x64_i8), for
// the full-tile case (m % 32 == 0, n % 128 == 0, k % 512 == 0, A 16-byte
// aligned).  Same workgroup tile (32 rows x 128 columns), same quantization
// and arithmetic as dqmm_fused_kernel, so the same bits; what differs is the
// schedule after the quantization barrier.  A wave's 32 x 32 block is four
// 16 x 16 tiles, each an 8-step chain over K = 512, run one after another:
// the integer correction, dequantization and stores of one tile are issued
// between the next tile's MFMAs, so the epilogue's VALU work and the output
// writes overlap the matrix core instead of following it.  The row sums and
// NaN flags are reduced before the barrier, so every tile's epilogue can run
// as soon as its chain ends.
//
// Operands: A (16 rows x 64 k per step) lane l holds row l & 15 and k =
// 64 s + 16 (l >> 4) + byte.  B is read straight from the 32 x 32 x 32
// packing: lane l of 16-column subtile c takes packed lane
// 16 c + (l & 15) + 32 ((l >> 4) & 1) of fragment 2 s + (l >> 5), whose k
// is the same 64 s + 16 (l >> 4) + byte, so A and B pair matching k.  The
// output tile's lane l holds column l & 15 and rows 4 (l >> 4) + v,
// v = 0..3.  ACC: the int32 accumulators are stored too.
//
// Tried and slower: the second half of K quantized between the first half's
// MFMAs, behind one more barrier (7.33 -> 7.65 us per op).
template <bool ACC>
__global__ __launch_bounds__(64 * DQF_WAVES) void dqmm_fused16_kernel(
    int m, int k, int n, const float *a, DqScratch *__restrict__ sc, int nparts, int *__restrict__ qparams,
    const int8_t *wpk, const int *__restrict__ colsum, const int *__restrict__ off,
    const float *__restrict__ wscale, int n_wscale, const float *__restrict__ bias, float *__restrict__ out,
    int *__restrict__ acc_out) {
    __shared__ __attribute__((aligned(16))) int lds_a[DQF_KS * 256];  // [kstep64 8][row tile 2][64 lanes][16 bytes]
    __shared__ __attribute__((aligned(16))) int lds_rs[32];
    __shared__ __attribute__((aligned(16))) int lds_rn[32];
    const int tid = threadIdx.x, lane = tid & 63, wt = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ks = k / 32;
    const int ncb = n / 32 / DQF_WAVES, nmt = m / 32;
    const int id = xcd_band(blockIdx.x, gridDim.x);
    const int grp = id / (DQF_GM * ncb), gl = id % (DQF_GM * ncb);
    const int mt0 = grp * DQF_GM;
    const int gm = nmt - mt0 < DQF_GM ? nmt - mt0 : DQF_GM;
    const int mt = mt0 + gl % gm;
    const int nt = (gl / gm) * DQF_WAVES + wt;
    const int r = tid >> 3, c8 = tid & 7;
    const float *src = a + (long long)(mt * 32 + r) * k;
    const int npass = ks / DQF_KS;
    // B: this lane's 16 bytes of packed lane 16 c + (lane & 15) + 32 ((lane >> 4) & 1)
    // of fragment (nt, 2 s + (lane >> 5)); subtile c adds 16 lanes (256 bytes)
    const int8_t *bl = wpk + ((long long)nt * ks + (lane >> 5)) * 1024 + ((lane & 15) + 32 * ((lane >> 4) & 1)) * 16;

    const int pidx = tid < nparts ? tid : 0;
    const float pmin = sc->partial_min[pidx], pmax = sc->partial_max[pidx];
    // the epilogue's column operands of both 16-column subtiles
    int offj_raw[2], csum[2];
    float ws[2], bj[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const int j = nt * 32 + 16 * c + (lane & 15);
        offj_raw[c] = off[j];
        csum[c] = colsum[j];
        ws[c] = n_wscale == 1 ? wscale[0] : wscale[j];
        bj[c] = bias ? bias[j] : 0.0f;
    }

    Quad x[DQF_KS];
    i32x4 b[2][DQF_KS / 2];
    auto load_pass = [&](int s0) {
#pragma unroll
        for (int i = 0; i < DQF_KS; i++) {
            const float4 v = *reinterpret_cast<const float4 *>(src + (s0 + i) * 32 + 4 * c8);
            x[i].v[0] = v.x; x[i].v[1] = v.y; x[i].v[2] = v.z; x[i].v[3] = v.w;
        }
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int s = 0; s < DQF_KS / 2; s++)
                b[c][s] = *reinterpret_cast<const i32x4 *>(bl + (long long)(s0 + 2 * s) * 1024 + c * 256);
    };
    load_pass(0);
    __builtin_amdgcn_sched_barrier(0);

    float inv, scale;
    int zp;
    dq_finish(sc, __builtin_fminf(0.f, pmin), __builtin_fmaxf(0.f, pmax), qparams, blockIdx.x == 0, inv, zp,
              &scale);
    const float zpf = (float)zp;
    const unsigned alpha = (unsigned)(128 - zp);

    int sum = 0;
    bool nan = false;
    i32x4 acc[2][2] = {};
    i32x4 av[2][DQF_KS / 2];
    // quad i of this thread: k = 32 i + 4 c8 -> step i / 2, lane group 2 (i & 1) + c8 / 4
    int *dst = lds_a + ((r >> 4) * 64 + (r & 15) + 16 * (c8 >> 2)) * 4 + (c8 & 3);
    auto quantize_pass = [&]() {
#pragma unroll
        for (int i = 0; i < DQF_KS; i++)
            dst[(i >> 1) * 512 + (i & 1) * 128] = (int)quantize4(x[i], inv, zpf, 0xfu, sum, nan);
    };
    auto read_a = [&]() {
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int s = 0; s < DQF_KS / 2; s++)
                av[rt][s] = *reinterpret_cast<const i32x4 *>(lds_a + ((s * 2 + rt) * 64 + lane) * 4);
    };
    auto chain = [&](int t) {
#pragma unroll
        for (int s = 0; s < DQF_KS / 2; s++)
            acc[t >> 1][t & 1] =
                __builtin_amdgcn_mfma_i32_16x16x64_i8(av[t >> 1][s], b[t & 1][s], acc[t >> 1][t & 1], 0, 0, 0);
    };
    for (int ps = 0; ps + 1 < npass; ps++) {  // passes before the last (K > 512)
        quantize_pass();
        __syncthreads();
        read_a();
#pragma unroll
        for (int t = 0; t < 4; t++) chain(t);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // every wave has read this pass's a'' before it is rewritten
        load_pass((ps + 1) * DQF_KS);
    }
    quantize_pass();
    // row sums and NaN flags: a row's 8 threads are consecutive lanes
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        sum += __shfl_xor(sum, o);
        const int other = __shfl_xor(nan ? 1 : 0, o);
        nan = nan || other != 0;
    }
    if (c8 == 0) {
        lds_rs[r] = sum;
        lds_rn[r] = nan ? 1 : 0;
    }
    __syncthreads();
    read_a();
    // the lane's row sums and NaN flags (rows 16 rt + 4 (lane >> 4) + v)
    int4 rs4[2], rn4[2];
#pragma unroll
    for (int rt = 0; rt < 2; rt++) {
        rs4[rt] = *reinterpret_cast<const int4 *>(lds_rs + 16 * rt + 4 * (lane >> 4));
        rn4[rt] = *reinterpret_cast<const int4 *>(lds_rn + 16 * rt + 4 * (lane >> 4));
    }
    auto epilogue = [&](int t) {
        const int rt = t >> 1, c = t & 1;
        const int j = nt * 32 + 16 * c + (lane & 15);
        const unsigned offj = (unsigned)offj_raw[c];
        const unsigned colterm = alpha * (unsigned)csum[c] + (unsigned)k * alpha * offj;
        const float comb = scale * ws[c];  // CombinedScale, QuantizedMatMulOps.cs:203-221
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int il = 16 * rt + 4 * (lane >> 4) + v;
            const int rsv = v == 0 ? rs4[rt].x : v == 1 ? rs4[rt].y : v == 2 ? rs4[rt].z : rs4[rt].w;
            const int rnv = v == 0 ? rn4[rt].x : v == 1 ? rn4[rt].y : v == 2 ? rn4[rt].z : rn4[rt].w;
            const int val = (int)((unsigned)acc[rt][c][v] + offj * (unsigned)rsv + colterm);
            const long long o_idx = (long long)(mt * 32 + il) * n + j;
            if constexpr (ACC) acc_out[o_idx] = val;
            const float o = __builtin_fmaf((float)val, comb, bj[c]);
            out[o_idx] = rnv ? __builtin_nanf("") : o;
        }
    };
    // tile t's chain, with tile t - 1's epilogue issued between its MFMAs:
    // the epilogue's VALU work and stores overlap the matrix core
    chain(0);
#pragma unroll
    for (int t = 1; t < 4; t++) {
        chain(t);
        epilogue(t - 1);
#pragma unroll
        for (int q = 0; q < DQF_KS / 2; q++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // five VALU
            __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);  // one global store
        }
    }
    epilogue(3);
}

static osh_status run_minmax(const float *a, long long count, DqScratch *sc, int *nparts, hipStream_t st) {
    long long blocks = (count / 4 + DQ_THREADS - 1) / DQ_THREADS;
    if (blocks < 1) blocks = 1;
    if (blocks > DQ_MINMAX_BLOCKS) blocks = DQ_MINMAX_BLOCKS;
    OSH_LAUNCH(dqmm_minmax_kernel, dim3((unsigned)blocks), dim3(DQ_THREADS), 0, st, a, count, sc);
    *nparts = (int)blocks;
    OSH_LAUNCH_CHECK("dqmm_minmax_kernel");
    return OSH_OK;
}

static thread_local int t_dqmm_launches = 0;
int dqmm_last_launches() { return t_dqmm_launches; }

static osh_status dqmm_run(int m, int k, int n, const float *d_a, const void *d_wpacked, const float *d_wscale,
                           int n_wscale, const float *d_bias, float *d_out, int32_t *d_acc, int32_t *d_qparams,
                           void *d_scratch, hipStream_t st) {
    DqScratch *sc = static_cast<DqScratch *>(d_scratch);
    int *rowsum = reinterpret_cast<int *>(sc + 1);
    int8_t *apk = reinterpret_cast<int8_t *>(rowsum + 2 * pad32(m));
    const int8_t *frag = static_cast<const int8_t *>(d_wpacked);
    const int *colsum = reinterpret_cast<const int *>(frag + (size_t)pad32(n) * pad32(k));
    const int *off = colsum + pad32(n);
    const long long fblocks = (long long)((pad32(n) / 32 + DQF_WAVES - 1) / DQF_WAVES) * (pad32(m) / 32);
    const long long total = (long long)m * k;
    int nparts = 0;
    osh_status r = run_minmax(d_a, total, sc, &nparts, st);
    if (r != OSH_OK) return r;
    const bool full = m % 32 == 0 && n % 128 == 0 && k % (32 * DQF_KS) == 0 &&
                      (reinterpret_cast<uintptr_t>(d_a) & 15) == 0;
    const int variant = dqmm_variant();
    if (variant != 1 && fblocks <= 0x7fffffffLL) {
        if (full && variant == 0 && d_acc)
            OSH_LAUNCH(dqmm_fused16_kernel<true>, dim3((unsigned)fblocks), dim3(64 * DQF_WAVES), 0, st, m, k, n,
                       d_a, sc, nparts, (int *)d_qparams, frag, colsum, off, d_wscale, n_wscale, d_bias, d_out,
                       (int *)d_acc);
        else if (full && variant == 0)
            OSH_LAUNCH(dqmm_fused16_kernel<false>, dim3((unsigned)fblocks), dim3(64 * DQF_WAVES), 0, st, m, k, n,
                       d_a, sc, nparts, (int *)d_qparams, frag, colsum, off, d_wscale, n_wscale, d_bias, d_out,
                       (int *)d_acc);
        else if (full)
            OSH_LAUNCH(dqmm_fused_kernel<true>, dim3((unsigned)fblocks), dim3(64 * DQF_WAVES), 0, st, m, k, n,
                               d_a, sc, nparts, (int *)d_qparams, frag, colsum, off, d_wscale, n_wscale, d_bias, d_out,
                               (int *)d_acc);
        else
            OSH_LAUNCH(dqmm_fused_kernel<false>, dim3((unsigned)fblocks), dim3(64 * DQF_WAVES), 0, st, m, k,
                               n, d_a, sc, nparts, (int *)d_qparams, frag, colsum, off, d_wscale, n_wscale, d_bias,
                               d_out, (int *)d_acc);
        OSH_LAUNCH_CHECK("dqmm_fused_kernel");
        t_dqmm_launches = 2;
        return OSH_OK;
    }
    const int rows_per_block = DQ_THREADS / 64;
    OSH_LAUNCH(dqmm_quantize_kernel, dim3((unsigned)((pad32(m) + rows_per_block - 1) / rows_per_block)),
                       dim3(DQ_THREADS), 0, st, d_a, m, k, sc, nparts, (int *)d_qparams, rowsum, apk);
    OSH_LAUNCH_CHECK("dqmm_quantize_kernel");
    dim3 grid((pad32(n) / 32 + 1) / 2, (pad32(m) / 32 + 1) / 2);
    OSH_LAUNCH(dqmm_gemm_kernel, grid, dim3(256), 0, st, m, k, n, apk, frag, colsum, off, rowsum, sc,
                       d_wscale, n_wscale, d_bias, d_out, (int *)d_acc);
    OSH_LAUNCH_CHECK("dqmm_gemm_kernel");
    t_dqmm_launches = 3;
    return OSH_OK;
}

static osh_status dqmm_check(int m, int k, int n, const float *d_a, const void *d_wpacked, const float *d_wscale,
                             int n_wscale, float *d_out) {
    if (m < 0 || k <= 0 || n <= 0) return fail(OSH_E_INVALID, "DQM: bad size m=%d k=%d n=%d", m, k, n);
    if (m == 0) return OSH_OK;
    if (!d_a || !d_wpacked || !d_wscale || !d_out) return fail(OSH_E_INVALID, "DQM: NULL pointer");
    if (n_wscale != 1 && n_wscale != n) return fail(OSH_E_INVALID, "DQM: w_scale has %d entries", n_wscale);
    if ((long long)k * 255 * 255 > 2147483647LL)
        return fail(OSH_E_UNSUPPORTED, "DQM: K=%d can overflow the int32 accumulator", k);
    if (pad32(m) / 32 > 2 * 65535) return fail(OSH_E_UNSUPPORTED, "DQM: m too large");
    return OSH_OK;
}

// The no-allocation variant's scratch: one array per GPU, held until the
// process ends.  `scratch` names the host-side stand-in; kernels take the
// device address hipGetSymbolAddress returns for the current device.
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kNoAllocMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kNoAllocMaxDevices];

// Resolves (once per device, with that device current) the device address of
// `scratch`; osh_init calls it, and the entry point calls it on its first
// call on a device that osh_init did not set up.
osh_status noalloc_scratch_setup(int dev) {
    if (dev < 0 || dev >= kNoAllocMaxDevices)
        return fail(OSH_E_UNSUPPORTED, "DQM (no allocation): device %d beyond %d devices", dev, kNoAllocMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev]) return OSH_OK;
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        return fail(OSH_E_DEVICE, "DQM (no allocation): hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                    hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = ptr;
    return OSH_OK;
}

}  // namespace osh

extern "C" {

OSH_API osh_status osh_dqmm_packed_weight_bytes(int k, int n, size_t *bytes) {
    if (k <= 0 || n <= 0 || !bytes) return fail(OSH_E_INVALID, "DQM: bad size");
    *bytes = packed_w_bytes(k, n);
    return OSH_OK;
}

OSH_API osh_status osh_dqmm_scratch_bytes(int m, int k, size_t *bytes) {
    if (m < 0 || k <= 0 || !bytes) return fail(OSH_E_INVALID, "DQM: bad size");
    *bytes = scratch_bytes(m, k);
    return OSH_OK;
}

OSH_API osh_status osh_dqmm_pack_weights(int k, int n, const void *d_w, int w_signed, const int32_t *h_wzp,
                                         int n_wzp, void *d_packed, osh_stream s) {
    if (k <= 0 || n <= 0 || !d_w || !d_packed) return fail(OSH_E_INVALID, "DQM pack: bad argument");
    if (n_wzp != 0 && n_wzp != 1 && n_wzp != n)
        return fail(OSH_E_INVALID, "DQM pack: w_zero_point has %d entries (need 1 or %d)", n_wzp, n);
    if (n_wzp > 0 && !h_wzp) return fail(OSH_E_INVALID, "DQM pack: w_zero_point is NULL");
    if ((long long)k * 255 * 255 > 2147483647LL)
        return fail(OSH_E_UNSUPPORTED, "DQM: K=%d can overflow the int32 accumulator", k);
    // a zero point has the weights' element type (ONNX MatMulInteger /
    // DynamicQuantizeMatMul), so |w - w_zp| <= 255 and K * 255 * 255 bounds
    // the accumulator (checked above)
    const int zlo = w_signed ? -128 : 0, zhi = w_signed ? 127 : 255;
    for (int i = 0; i < n_wzp; i++)
        if (h_wzp[i] < zlo || h_wzp[i] > zhi)
            return fail(OSH_E_INVALID, "DQM pack: weight zero point %d outside the %s range [%d, %d]", h_wzp[i],
                        w_signed ? "int8" : "uint8", zlo, zhi);
    hipStream_t st = to_stream(s);
    int *d_zp = nullptr;
    if (n_wzp > 0) {
        OSH_HIP_CHECK(hipMalloc((void **)&d_zp, sizeof(int) * n_wzp));
        hipError_t e = hipMemcpyAsync(d_zp, h_wzp, sizeof(int) * n_wzp, hipMemcpyHostToDevice, st);
        if (e != hipSuccess) {
            (void)hipFree(d_zp);
            return fail(OSH_E_DEVICE, "DQM pack: copy of zero points failed: %s", hipGetErrorString(e));
        }
    }
    int8_t *frag = static_cast<int8_t *>(d_packed);
    int *colsum = reinterpret_cast<int *>(frag + (size_t)pad32(n) * pad32(k));
    int *off = colsum + pad32(n);
    OSH_LAUNCH(dqmm_pack_kernel, dim3((pad32(n) + 63) / 64), dim3(64), 0, st, k, n, d_w, w_signed, d_zp,
                       n_wzp, frag, colsum, off);
    hipError_t le = hipGetLastError();
    hipError_t se = hipStreamSynchronize(st);
    if (d_zp) (void)hipFree(d_zp);
    if (le != hipSuccess) return fail(OSH_E_DEVICE, "dqmm_pack_kernel launch failed: %s", hipGetErrorString(le));
    if (se != hipSuccess) return fail(OSH_E_DEVICE, "DQM pack failed: %s", hipGetErrorString(se));
    return OSH_OK;
}

OSH_API osh_status osh_dqmm_u8s8(int m, int k, int n, const float *d_a, const void *d_wpacked,
                                 const float *d_wscale, int n_wscale, const float *d_bias, float *d_out,
                                 int32_t *d_acc, int32_t *d_qparams, void *d_scratch, osh_stream s) {
    osh_status st = dqmm_check(m, k, n, d_a, d_wpacked, d_wscale, n_wscale, d_out);
    if (st != OSH_OK || m == 0) return st;
    if (!d_scratch) return fail(OSH_E_INVALID, "DQM: NULL pointer");
    return dqmm_run(m, k, n, d_a, d_wpacked, d_wscale, n_wscale, d_bias, d_out, d_acc, d_qparams, d_scratch,
                    to_stream(s));
}

OSH_API osh_status osh_dqmm_u8s8_noalloc(int m, int k, int n, const float *d_a, const void *d_wpacked,
                                         const float *d_wscale, int n_wscale, const float *d_bias, float *d_out,
                                         int32_t *d_acc, int32_t *d_qparams, osh_stream s) {
    osh_status st = dqmm_check(m, k, n, d_a, d_wpacked, d_wscale, n_wscale, d_out);
    if (st != OSH_OK || m == 0) return st;
    if (scratch_bytes(m, k) > kNoAllocScratchBytes)
        return fail(OSH_E_UNSUPPORTED,
                    "DQM (no allocation): m=%d, k=%d need %zu scratch bytes; the static scratch holds %zu", m, k,
                    scratch_bytes(m, k), kNoAllocScratchBytes);
    int dev = 0;
    OSH_HIP_CHECK(hipGetDevice(&dev));
    void *ptr = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (dev >= 0 && dev < kNoAllocMaxDevices) ptr = g_scratch_ptr[dev];
    }
    if (!ptr) {
        st = noalloc_scratch_setup(dev);
        if (st != OSH_OK) return st;
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        ptr = g_scratch_ptr[dev];
    }
    return dqmm_run(m, k, n, d_a, d_wpacked, d_wscale, n_wscale, d_bias, d_out, d_acc, d_qparams, ptr,
                    to_stream(s));
}

OSH_API osh_status osh_matmul_integer(int m, int k, int n, const void *d_a, int a_signed, int a_zp,
                                      const void *d_wpacked, int32_t *d_c, void *d_scratch, osh_stream s) {
    if (m < 0 || k <= 0 || n <= 0) return fail(OSH_E_INVALID, "MatMulInteger: bad size m=%d k=%d n=%d", m, k, n);
    if (m == 0) return OSH_OK;
    if (!d_a || !d_wpacked || !d_c || !d_scratch) return fail(OSH_E_INVALID, "MatMulInteger: NULL pointer");
    if (a_zp < (a_signed ? -128 : 0) || a_zp > (a_signed ? 127 : 255))
        return fail(OSH_E_INVALID, "MatMulInteger: a_zero_point %d outside the %s range", a_zp,
                    a_signed ? "int8" : "uint8");
    if ((long long)k * 255 * 255 > 2147483647LL)
        return fail(OSH_E_UNSUPPORTED, "MatMulInteger: K=%d can overflow the int32 accumulator", k);
    if (pad32(m) / 32 > 2 * 65535) return fail(OSH_E_UNSUPPORTED, "MatMulInteger: m too large");
    hipStream_t st = to_stream(s);
    DqScratch *sc = static_cast<DqScratch *>(d_scratch);
    int *rowsum = reinterpret_cast<int *>(sc + 1);
    int8_t *apk = reinterpret_cast<int8_t *>(rowsum + 2 * pad32(m));
    const int rows_per_block = DQ_THREADS / 64;
    OSH_LAUNCH(mmi_pack_a_kernel, dim3((unsigned)((pad32(m) + rows_per_block - 1) / rows_per_block)),
                       dim3(DQ_THREADS), 0, st, static_cast<const uint8_t *>(d_a), m, k, a_signed, a_zp, sc, rowsum,
                       apk);
    OSH_LAUNCH_CHECK("mmi_pack_a_kernel");
    const int8_t *frag = static_cast<const int8_t *>(d_wpacked);
    const int *colsum = reinterpret_cast<const int *>(frag + (size_t)pad32(n) * pad32(k));
    const int *off = colsum + pad32(n);
    dim3 grid((pad32(n) / 32 + 1) / 2, (pad32(m) / 32 + 1) / 2);
    OSH_LAUNCH(dqmm_gemm_kernel, grid, dim3(256), 0, st, m, k, n, apk, frag, colsum, off, rowsum, sc,
                       static_cast<const float *>(nullptr), 1, static_cast<const float *>(nullptr),
                       static_cast<float *>(nullptr), (int *)d_c);
    OSH_LAUNCH_CHECK("dqmm_gemm_kernel");
    return OSH_OK;
}

OSH_API osh_status osh_dynamic_quantize_linear(int64_t n, const float *d_x, uint8_t *d_q, int32_t *d_qparams,
                                               void *d_scratch, osh_stream s) {
    if (n <= 0 || !d_x || !d_q || !d_scratch) return fail(OSH_E_INVALID, "DQL: bad argument");
    hipStream_t st = to_stream(s);
    DqScratch *sc = static_cast<DqScratch *>(d_scratch);
    int nparts = 0;
    osh_status r = run_minmax(d_x, n, sc, &nparts, st);
    if (r != OSH_OK) return r;
    long long blocks = (n + DQ_THREADS - 1) / DQ_THREADS;
    if (blocks > 4096) blocks = 4096;
    OSH_LAUNCH(dql_quantize_kernel, dim3((unsigned)blocks), dim3(DQ_THREADS), 0, st, d_x, n, sc, nparts,
                       (int *)d_qparams, d_q);
    OSH_LAUNCH_CHECK("dql_quantize_kernel");
    return OSH_OK;
}

}  // extern "C"
