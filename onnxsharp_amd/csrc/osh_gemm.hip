// osh_gemm.hip -- MatMul (+ fused column bias) entry points of the C ABI.
//
// Replaces GemmKernel.Multiply / MultiplyPacked / MultiplyBatched
// (src/OnnxSharp/Tensors/GemmKernel.cs:131-269,284-405,675-852) and the shape
// rules of MatMulLayer (src/OnnxSharp/Ops/DnnOps.cs:2789-3103).
#include <algorithm>

#include "osh_gemm16.h"
#include "osh_igemm.h"
#include "osh_launch.h"

using namespace osh;

namespace osh {

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Wave tiles of gemm16_kernel: (16*TM) x (16*BV*TN) outputs per wave.
struct G16Variant {
    int tm, tn, bv, kc;
};
static const G16Variant kG16[] = {
    {1, 1, 1, 32},  // 0: 16 x 16, 32-k chunks
    {1, 1, 2, 32},  // 1: 16 x 32, 32-k chunks
    {1, 1, 3, 32},  // 2: 16 x 48, 32-k chunks
    {1, 1, 4, 32},  // 3: 16 x 64, 32-k chunks
    {2, 1, 2, 32},  // 4: 32 x 32, 32-k chunks
    {2, 1, 3, 32},  // 5: 32 x 48, 32-k chunks
    {2, 1, 4, 32},  // 6: 32 x 64, 32-k chunks
    {1, 1, 3, 64},  // 7: 16 x 48, 64-k chunks
    {1, 1, 4, 64},  // 8: 16 x 64, 64-k chunks
    {1, 1, 1, 64},  // 9: 16 x 16, 64-k chunks
    {1, 1, 2, 64},  // 10: 16 x 32, 64-k chunks
};
constexpr int kG16Count = sizeof(kG16) / sizeof(kG16[0]);

}  // namespace osh

int osh::gemm16_variant_count() { return kG16Count; }

namespace osh {

static bool aligned_to(const void *p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// Operand constraints of a wave tile (see osh_gemm16.h): 16-byte A rows,
// BV-wide B loads and C stores on BV-aligned rows, N a multiple of BV, and
// 32-bit buffer offsets.
static bool g16_fits(const IgemmArgs &a, const G16Variant &v) {
    const int bv = v.bv;
    const int al = bv == 3 ? 1 : bv;  // 12-byte accesses need 4-byte alignment only
    if (a.K < 1 || a.N < bv || a.N % bv) return false;
    if (a.lda % 4 || !aligned_to(a.A, 16) || a.strideA % 4 || a.strideA_in % 4) return false;
    if (a.ldb % al || !aligned_to(a.B, 4 * al) || a.strideB % al || a.strideB_in % al) return false;
    if (a.ldc % al || !aligned_to(a.C, 4 * al) || a.strideC % al || a.strideC_in % al) return false;
    if (a.res && !aligned_to(a.res, 4 * al)) return false;  // residual rows share C's strides
    if (((long long)(a.M - 1) * a.lda + a.K) * 4 >= (1LL << 31)) return false;
    if (((long long)(a.K - 1) * a.ldb + a.N) * 4 >= (1LL << 31)) return false;
    return true;
}

// Predicted cost: rounds of waves over the SIMDs times the MFMAs of one wave
// tile, inflated by the operand traffic per MFMA (TN B loads and about TM/2
// A loads feed TM*TN*BV MFMAs per k4 step).
static double g16_cost(const IgemmArgs &a, int zcount, const G16Variant &v, int cus) {
    const long long waves = (long long)ceil_div(a.M, 16 * v.tm) * ceil_div(a.N, 16 * v.bv * v.tn) * zcount;
    const long long rounds = (waves + 4LL * cus - 1) / (4LL * cus);
    const double u = (double)v.tm * v.tn * v.bv;
    return rounds * u * ceil_div(a.K, 4) * (1.0 + 0.5 * (v.tn + 0.5 * v.tm) / u);
}

template <int TM, int TN, int BV, int KC>
static osh_status g16_launch(const IgemmArgs &a, int zcount, int act, hipStream_t st) {
    const int tiles_m = ceil_div(a.M, 16 * TM), tiles_n = ceil_div(a.N, 16 * BV * TN);
    const long long blocks = (long long)ceil_div(tiles_m, 4) * tiles_n;
    if (blocks > 0x7fffffffLL) return fail(OSH_E_UNSUPPORTED, "GEMM grid too large");
    dim3 grid((unsigned)blocks, zcount);
    OSH_DISPATCH_ACT(act, ACT,
                     OSH_LAUNCH((gemm16_kernel<TM, TN, BV, KC, ACT>), grid, dim3(256), 0, st, a, tiles_m));
    OSH_LAUNCH_CHECK("gemm16_kernel");
    return OSH_OK;
}

// Returns true when a gemm16 tile took the problem (*status = its launch status).
static bool launch_gemm16(const IgemmArgs &a, int zcount, int act, hipStream_t st, osh_status *status) {
    const int forced = gemm_variant();
    if (forced == -2 || zcount > 65535) return false;
    int best = -1;
    if (forced >= 0) {
        if (forced < kG16Count && g16_fits(a, kG16[forced])) best = forced;
    } else {
        const int cus = device_cus();
        double bc = 0;
        for (int i = 0; i < kG16Count; i++) {
            if (!g16_fits(a, kG16[i])) continue;
            const double c = g16_cost(a, zcount, kG16[i], cus);
            if (best < 0 || c < bc) best = i, bc = c;
        }
    }
    switch (best) {
    case 0: *status = g16_launch<1, 1, 1, 32>(a, zcount, act, st); return true;
    case 1: *status = g16_launch<1, 1, 2, 32>(a, zcount, act, st); return true;
    case 2: *status = g16_launch<1, 1, 3, 32>(a, zcount, act, st); return true;
    case 3: *status = g16_launch<1, 1, 4, 32>(a, zcount, act, st); return true;
    case 4: *status = g16_launch<2, 1, 2, 32>(a, zcount, act, st); return true;
    case 5: *status = g16_launch<2, 1, 3, 32>(a, zcount, act, st); return true;
    case 6: *status = g16_launch<2, 1, 4, 32>(a, zcount, act, st); return true;
    case 7: *status = g16_launch<1, 1, 3, 64>(a, zcount, act, st); return true;
    case 8: *status = g16_launch<1, 1, 4, 64>(a, zcount, act, st); return true;
    case 9: *status = g16_launch<1, 1, 1, 64>(a, zcount, act, st); return true;
    case 10: *status = g16_launch<1, 1, 2, 64>(a, zcount, act, st); return true;
    default: return false;
    }
}

osh_status launch_igemm(const IgemmArgs &a, int zcount, int bmode, int act, hipStream_t st) {
    if (a.M <= 0 || a.N <= 0 || zcount <= 0) return OSH_OK;
    osh_status g16_status = OSH_OK;
    if (bmode == B_DENSE && launch_gemm16(a, zcount, act, st, &g16_status)) return g16_status;
    const bool vec_a = a.K % 4 == 0 && a.lda % 4 == 0 && aligned16(a.A) && a.strideA % 4 == 0 &&
                       a.strideA_in % 4 == 0;
    const bool vec_b = bmode == B_DENSE && a.ldb % 4 == 0 && aligned16(a.B) && a.strideB % 4 == 0 &&
                       a.strideB_in % 4 == 0;
    // Small-M problems (conv with few output channels) take a 32-row tile.
    const bool small_m = a.M <= 32;
    dim3 block(256);
#define OSH_IG_LAUNCH(BM, BN, WM, WN, BMODE, VA, VB)                                                   \
    do {                                                                                              \
        dim3 grid(ceil_div(a.N, BN), ceil_div(a.M, BM), zcount);                                      \
        OSH_DISPATCH_ACT(act, ACT,                                                                    \
            OSH_LAUNCH((igemm_f32_kernel<BM, BN, WM, WN, BMODE, VA, VB, ACT>), grid, block, 0, \
                               st, a));                                                               \
    } while (0)
#define OSH_IG_SHAPE(BMODE, VA, VB)                                \
    do {                                                          \
        if (small_m) OSH_IG_LAUNCH(32, 128, 1, 4, BMODE, VA, VB); \
        else OSH_IG_LAUNCH(64, 64, 2, 2, BMODE, VA, VB);          \
    } while (0)
    if (bmode == B_IM2COL) {
        if (vec_a) OSH_IG_SHAPE(B_IM2COL, true, false);
        else OSH_IG_SHAPE(B_IM2COL, false, false);
    } else {
        if (vec_a && vec_b) OSH_IG_SHAPE(B_DENSE, true, true);
        else if (vec_a) OSH_IG_SHAPE(B_DENSE, true, false);
        else if (vec_b) OSH_IG_SHAPE(B_DENSE, false, true);
        else OSH_IG_SHAPE(B_DENSE, false, false);
    }
#undef OSH_IG_SHAPE
#undef OSH_IG_LAUNCH
    OSH_LAUNCH_CHECK("igemm_f32_kernel");
    return OSH_OK;
}

// y = alpha * y (alpha != 1), then y += beta * c (beta != 0 and C given): the
// reference's two separately rounded steps (AttnOps.cs:111-131), no contraction.
__global__ __launch_bounds__(256) void gemm_ex_epilogue_kernel(float *__restrict__ y, int m, int n, float alpha,
                                                               int scale, float beta, const float *__restrict__ c,
                                                               long long c_len) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)m * n;
    if (idx >= total) return;
    const int j = (int)(idx % n);
    float v = y[idx];
    if (scale) v = alpha * v;
    if (c) {
        const float cv = c_len >= total ? c[idx] : (c_len == 1 ? c[0] : c[j % c_len]);
        v = v + beta * cv;
    }
    y[idx] = v;
}

}  // namespace osh

extern "C" {

OSH_API osh_status osh_gemm_ex_workspace_bytes(int trans_a, int trans_b, int m, int n, int k, size_t *bytes) {
    if (!bytes || m < 0 || n < 0 || k < 0) return fail(OSH_E_INVALID, "Gemm: bad argument");
    size_t b = 0;
    if (trans_a) b += ((size_t)m * k * sizeof(float) + 255) & ~(size_t)255;
    if (trans_b) b += (size_t)k * n * sizeof(float);
    *bytes = b;
    return OSH_OK;
}

OSH_API osh_status osh_gemm_ex_f32(int trans_a, int trans_b, int m, int n, int k, float alpha, const float *d_a,
                                   const float *d_b, float beta, const float *d_c, int64_t c_len, float *d_y,
                                   void *d_workspace, osh_stream s) {
    if (m < 0 || n < 0 || k < 0) return fail(OSH_E_INVALID, "Gemm: negative size");
    if (m == 0 || n == 0) return OSH_OK;
    if (!d_a || !d_b || !d_y) return fail(OSH_E_INVALID, "Gemm: A, B and Y must be non-NULL");
    if ((trans_a || trans_b) && !d_workspace) return fail(OSH_E_INVALID, "Gemm: transposes need the workspace");
    if (d_c && c_len <= 0) return fail(OSH_E_INVALID, "Gemm: C given with %lld elements", (long long)c_len);
    hipStream_t st = to_stream(s);
    const float *a = d_a, *b = d_b;
    char *ws = static_cast<char *>(d_workspace);
    if (trans_a) {  // A is [k, m]
        float *t = reinterpret_cast<float *>(ws);
        osh_status r = osh_transpose_f32(1, k, m, d_a, 0, t, 0, s);
        if (r != OSH_OK) return r;
        a = t;
        ws += ((size_t)m * k * sizeof(float) + 255) & ~(size_t)255;
    }
    if (trans_b) {  // B is [n, k]
        float *t = reinterpret_cast<float *>(ws);
        osh_status r = osh_transpose_f32(1, n, k, d_b, 0, t, 0, s);
        if (r != OSH_OK) return r;
        b = t;
    }
    osh_status r = osh_gemm_f32(m, n, k, a, k, b, n, nullptr, nullptr, nullptr, OSH_ACT_NONE, d_y, n, s);
    if (r != OSH_OK) return r;
    const bool scale = alpha != 1.0f;
    const bool bias = beta != 0.0f && d_c && c_len > 0;
    if (!scale && !bias) return OSH_OK;
    const long long total = (long long)m * n;
    OSH_LAUNCH(gemm_ex_epilogue_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, d_y, m, n,
                       alpha, scale ? 1 : 0, beta, bias ? d_c : nullptr, (long long)c_len);
    OSH_LAUNCH_CHECK("gemm_ex_epilogue_kernel");
    return OSH_OK;
}

OSH_API osh_status osh_gemm_f32_batched(int batch, int m, int n, int k, const float *d_a, int lda,
                                        int64_t stride_a, const float *d_b, int ldb, int64_t stride_b,
                                        const float *d_col_bias, int act, float *d_c, int ldc,
                                        int64_t stride_c, osh_stream s) {
    if (batch < 0 || m < 0 || n < 0 || k < 0) return fail(OSH_E_INVALID, "negative GEMM size");
    if (batch == 0 || m == 0 || n == 0) return OSH_OK;
    if (!d_a || !d_b || !d_c) return fail(OSH_E_INVALID, "A, B and C must be non-NULL");
    if (lda < k || ldb < n || ldc < n) return fail(OSH_E_INVALID, "leading dimension smaller than the row");
    if (batch > 65535) return fail(OSH_E_UNSUPPORTED, "batch %d exceeds the grid limit", batch);
    IgemmArgs a{};
    a.M = m; a.N = n; a.K = k;
    a.A = d_a; a.lda = lda; a.strideA = stride_a;
    a.B = d_b; a.ldb = ldb; a.strideB = stride_b;
    a.C = d_c; a.ldc = ldc; a.strideC = stride_c;
    a.col_bias = d_col_bias;
    a.zdiv = 1;
    return launch_igemm(a, batch, B_DENSE, act, to_stream(s));
}

OSH_API osh_status osh_gemm_f32(int m, int n, int k, const float *d_a, int lda, const float *d_b, int ldb,
                                const float *d_col_bias, const float *d_row_bias, const float *d_col_scale,
                                int act, float *d_c, int ldc, osh_stream s) {
    if (m < 0 || n < 0 || k < 0) return fail(OSH_E_INVALID, "negative GEMM size");
    if (m == 0 || n == 0) return OSH_OK;
    if (!d_a || !d_b || !d_c) return fail(OSH_E_INVALID, "A, B and C must be non-NULL");
    if (lda < k || ldb < n || ldc < n) return fail(OSH_E_INVALID, "leading dimension smaller than the row");
    IgemmArgs a{};
    a.M = m; a.N = n; a.K = k;
    a.A = d_a; a.lda = lda;
    a.B = d_b; a.ldb = ldb;
    a.C = d_c; a.ldc = ldc;
    a.col_bias = d_col_bias;
    a.row_bias = d_row_bias;
    a.col_scale = d_col_scale;
    a.zdiv = 1;
    return launch_igemm(a, 1, B_DENSE, act, to_stream(s));
}

// MatMul numpy broadcast (MatMulLayer.GetMemoryShapes, src/OnnxSharp/Ops/DnnOps.cs:2840-2900):
// rank-1 operands are promoted ([k] -> [1,k] for A, [k] -> [k,1] for B) and the
// promoted axis is dropped from the output; batch axes align right and take
// the larger extent.
OSH_API osh_status osh_matmul_infer_shape(const int64_t *a_dims, int ra, const int64_t *b_dims, int rb,
                                          int64_t *y_dims, int *ry) {
    if (!a_dims || !b_dims || !y_dims || !ry) return fail(OSH_E_INVALID, "NULL argument");
    if (ra < 1 || rb < 1 || ra > 8 || rb > 8) return fail(OSH_E_INVALID, "MatMul rank out of range");
    int64_t A[8], B[8];
    int na = ra, nb = rb;
    for (int i = 0; i < ra; i++) A[i] = a_dims[i];
    for (int i = 0; i < rb; i++) B[i] = b_dims[i];
    bool a1 = ra == 1, b1 = rb == 1;
    if (a1) { A[1] = A[0]; A[0] = 1; na = 2; }
    if (b1) { B[1] = 1; nb = 2; }
    int64_t m = A[na - 2], k = A[na - 1], k2 = B[nb - 2], n = B[nb - 1];
    if (k != k2) return fail(OSH_E_INVALID, "MatMul: K mismatch (%lld vs %lld)", (long long)k, (long long)k2);
    int batch_rank = std::max(na, nb) - 2;
    int out = 0;
    for (int i = 0; i < batch_rank; i++) {
        int ia = i - (batch_rank - (na - 2)), ib = i - (batch_rank - (nb - 2));
        int64_t da = ia >= 0 ? A[ia] : 1, db = ib >= 0 ? B[ib] : 1;
        if (da != db && da != 1 && db != 1)
            return fail(OSH_E_INVALID, "MatMul: batch dims %lld and %lld do not broadcast", (long long)da,
                        (long long)db);
        y_dims[out++] = std::max(da, db);
    }
    if (!a1) y_dims[out++] = m;
    if (!b1) y_dims[out++] = n;
    *ry = out;
    return OSH_OK;
}

}  // extern "C"
