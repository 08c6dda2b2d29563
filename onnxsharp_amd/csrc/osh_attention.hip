// osh_attention.hip -- the attention core of a YOLO11n C2PSA block in one
// launch.  The reference runs this as its exported node sequence: its
// attention fusion (GraphFusion.FuseAttention, src/OnnxSharp/Core/
// GraphFusion.cs:950-1150) wants MatMul(Softmax(.), Transpose[0,2,1,3](V))
// (lines 996-1005), while C2PSA multiplies V by the transposed probabilities:
//
//   S = MatMul(Transpose(q), k)        GemmKernel chain over d from 0
//   S = Mul(S, scale)                  one rounding
//   P = Softmax(S, axis = -1)          VectorMath.SoftmaxRow
//   y = MatMul(v, Transpose(P))        GemmKernel chain over j from 0
//
// per head h, with q = qkv[h][0, kd), k = qkv[h][kd, 2kd), v =
// qkv[h][2kd, 2kd + hd) as rows of N = H*W values.  This kernel keeps every
// one of those orders, so it returns the node sequence's bits:
//   * a workgroup owns 16 query rows of one head; each of its four waves
//     computes 16 x 16 score tiles with v_mfma_f32_16x16x4f32, d in order
//     (k-slot g = d % 4), into LDS;
//   * the softmax runs in SoftmaxRow's order: scale, row max (any order: only
//     v - max reaches the exponential), exponentials, eight lane sums over
//     columns 8j + k in order of j, the lane sums added to 0 in lane order,
//     then e * (1 / sum) (N % 16 == 0 leaves no tail);
//   * each wave then takes 16 of the head's hd output channels and runs the
//     chain over j in order, A = v rows staged through LDS, B = the
//     probabilities from LDS.
// The chain of N / 4 dependent MFMAs bounds the launch (about 40 ns a step);
// the v rows are loaded at the start so that only LDS latency meets it.
#include "osh_common.h"

using namespace osh;

namespace osh {

constexpr int ATT_ROWS = 16;     // query rows per workgroup
constexpr int ATT_MAX_KS = 16;   // key_dim / 4 k-steps held in registers (key_dim <= 64)
constexpr int ATT_MAX_N = 480;   // score rows and v chunks within 64 KiB of LDS
constexpr int ATT_VC = 64;       // v columns (j) per staged chunk
constexpr int ATT_VP = 66;       // LDS pitch of a staged v row
constexpr int ATT_MAX_CH = (ATT_MAX_N + ATT_VC - 1) / ATT_VC;  // v chunks a lane holds
constexpr unsigned ATT_BUF_WORD3 = 0x00020000;

// LDS row pitch of the scores: pitch % 32 == 2 puts the probability reads of
// a half-wave in the last phase (lanes jl = 0..15, g = 0..1 at jl * pitch + g)
// in 32 banks; ATT_VP does the same for the staged v rows.
__host__ __device__ constexpr int att_pitch(int n) { return n + (34 - n % 32) % 32; }
__host__ __device__ constexpr size_t att_lds_bytes(int n) {
    return ((size_t)ATT_ROWS * att_pitch(n) + 4 * 2 * 16 * ATT_VP) * sizeof(float);
}

__device__ __forceinline__ float att_load(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0));
}

// Operands come through raw buffer loads, whose range check returns 0 past
// the operand, and no load sits under a condition (the compiler would sink
// it into the branch and wait for every load in flight there):
//   * the scores run KS k-steps for every key_dim <= 4 KS; steps past
//     key_dim / 4 multiply zeros, which can only turn a zero score's sign,
//     and the sign of a zero score never reaches the output (exp of
//     +-0 - max and of -max are the same values);
//   * score tiles past n / 16 are computed from whatever lies there and
//     never stored;
//   * v chunks past n are loaded and never staged.
template <int KS>
__global__ __launch_bounds__(256) void attention_kernel(int kd, int hd, int n, float scale,
                                                        const float *__restrict__ qkv, long long head_stride,
                                                        float *__restrict__ y) {
    // [ATT_ROWS][pitch] scores, then exponentials; after them 2 x [16][ATT_VP]
    // staged v per wave
    extern __shared__ float S[];
    __shared__ float s_inv[ATT_ROWS];
    constexpr int TB = KS <= 8 ? 8 : 4;  // score tiles per load batch (8 per wave cover n <= 512)
    const int pitch = att_pitch(n);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int jl = lane & 15, g = lane >> 4;
    const int h = blockIdx.y;
    const int i0 = blockIdx.x * ATT_ROWS;
    const int nt = n >> 4, ncb = hd >> 4;
    const float *q = qkv + h * head_stride;
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc((void *)q, (short)0, kd * n * 4, ATT_BUF_WORD3);
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc((void *)(q + (long long)kd * n), (short)0, kd * n * 4, ATT_BUF_WORD3);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void *)(q + 2LL * kd * n), (short)0, hd * n * 4, ATT_BUF_WORD3);

    // scores S[i][j] = fold over d of fmaf(q[d][i0 + i], k[d][j], .) from 0;
    // lane (jl, g) holds q[4s + g][i0 + jl] and k[4s + g][16 jt + jl] for
    // the wave's column tiles jt = wave + 4u, which run side by side
    float aq[KS];
#pragma unroll
    for (int s = 0; s < KS; s++) aq[s] = att_load(rq, ((4 * s + g) * n + i0 + jl) * 4);

    // The v rows of the wave's 16 output channels reach the last phase's
    // chain through two LDS chunks of ATT_VC columns.  Lane: rows lane / 16
    // + 4 r, columns 4 (lane % 16) + 0..3 of each chunk, all loaded (16 bytes
    // a load) right after the first score operands, so that their latency
    // passes under the scores and the softmax.
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int srow = lane >> 4, scol = (lane & 15) * 4;
    f4 vv[ATT_MAX_CH][4];
    auto load_v = [&](int cb) {
#pragma unroll
        for (int c = 0; c < ATT_MAX_CH; c++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int off = ((cb * 16 + srow + 4 * r) * n + c * ATT_VC + scol) * 4;
                const auto v4 = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
                vv[c][r] = f4{__uint_as_float(v4[0]), __uint_as_float(v4[1]), __uint_as_float(v4[2]),
                              __uint_as_float(v4[3])};
            }
    };

    load_v(wave);  // past the operand when wave >= hd / 16: reads return 0, never used

    for (int u0 = 0; u0 < 8 && wave + 4 * u0 < nt; u0 += TB) {
        float bk[TB][KS];
#pragma unroll
        for (int u = 0; u < TB; u++) {
            const int col = (wave + 4 * (u0 + u)) * 16 + jl;
#pragma unroll
            for (int s = 0; s < KS; s++) bk[u][s] = att_load(rk, ((4 * s + g) * n + col) * 4);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load in flight before the first MFMA waits
        f32x4 acc[TB];
#pragma unroll
        for (int u = 0; u < TB; u++) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; s++)
#pragma unroll
            for (int u = 0; u < TB; u++)
                acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(aq[s], bk[u][s], acc[u], 0, 0, 0);
#pragma unroll
        for (int u = 0; u < TB; u++) {
            const int jt = wave + 4 * (u0 + u);
            if (jt < nt)
#pragma unroll
                for (int r = 0; r < 4; r++) S[(4 * g + r) * pitch + jt * 16 + jl] = acc[u][r];
        }
    }

    __syncthreads();

    // softmax, 16 threads of one wave per row, thread t holding columns
    // t + 16 i: the Mul node's rounding, the row max, the exponentials
    {
        constexpr int NE = ATT_MAX_N / 16;
        const int row = tid >> 4, t = tid & 15;
        float *sr = S + row * pitch + t;
        float e[NE];
        float m = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < NE; i++) {
            e[i] = sr[16 * min(i, nt - 1)] * scale;  // repeats of the last column leave the max alone
            m = __builtin_fmaxf(m, e[i]);
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, o));
#pragma unroll
        for (int i = 0; i < NE; i++)
            if (i < nt) {
                e[i] = exp_ref(e[i] - m);
                sr[16 * i] = e[i];
            }
        // lane sum k (thread t = k < 8) adds columns 8 j + k in order of j:
        // even j from its own columns, odd j from thread k + 8's
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < NE; i++) {
            const float other = __shfl_xor(e[i], 8);
            if (i < nt) part = (part + e[i]) + other;
        }
        float sum = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 8; kk++) sum = sum + __shfl(part, kk, 16);
        if (t == 0) s_inv[row] = 1.0f / sum;
    }
    __syncthreads();

    // y[h][c][i0 + i] = fold over j of fmaf(v[c][j], P[i][j], .) from 0 with
    // P[i][j] = e[i][j] * inv[i]; a wave owns 16 output channels.
    const float inv = s_inv[jl];
    const float *pr = S + jl * pitch + g;  // lane: e[jl][j + g]
    float *vbuf = S + ATT_ROWS * pitch + wave * 2 * 16 * ATT_VP;  // two chunks of [16][ATT_VP]
    const int nch = (n + ATT_VC - 1) / ATT_VC;
    auto stage = [&](int c) {
        float *buf = vbuf + (c & 1) * 16 * ATT_VP;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float *d = buf + (srow + 4 * r) * ATT_VP + scol;  // 8-byte aligned (ATT_VP even)
            *reinterpret_cast<float2 *>(d) = float2{vv[c][r][0], vv[c][r][1]};
            *reinterpret_cast<float2 *>(d + 2) = float2{vv[c][r][2], vv[c][r][3]};
        }
        // other lanes of this wave read what this lane wrote: keep the
        // compiler from moving those reads above these writes
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    };
    // a whole chunk's operands, read one chunk ahead (right after that chunk
    // is staged) so that the chain of the chunk before hides their latency
    float a[2][ATT_VC / 4], b[2][ATT_VC / 4];
    auto read_chunk = [&](int c) {
        const float *va = vbuf + (c & 1) * 16 * ATT_VP + jl * ATT_VP + g;  // lane: v[16 cb + jl][64 c + 4 t + g]
        const float *pb = pr + c * ATT_VC;
#pragma unroll
        for (int w = 0; w < ATT_VC / 4; w++) {
            a[c & 1][w] = va[4 * w];
            b[c & 1][w] = pb[4 * w];
        }
    };
    for (int cb = wave; cb < ncb; cb += 4) {
        if (cb != wave) load_v(cb);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        stage(0);
        if (n >= ATT_VC) read_chunk(0);
#pragma unroll
        for (int c = 0; c < ATT_MAX_CH; c++) {
            if (c >= nch) break;
            if (c + 1 < nch) {
                stage(c + 1);  // the other buffer, read by the chunk before
                if (n - (c + 1) * ATT_VC >= ATT_VC) read_chunk(c + 1);
            }
            const float *va = vbuf + (c & 1) * 16 * ATT_VP + jl * ATT_VP + g;  // lane: v[16 cb + jl][64 c + 4 t + g]
            const float *pb = pr + c * ATT_VC;
            const int steps = min(ATT_VC, n - c * ATT_VC) / 4;  // a multiple of 4 (n % 16 == 0)
            if (steps == ATT_VC / 4) {  // a whole chunk: its operands were read a chunk ahead
                __builtin_amdgcn_sched_barrier(0);  // keep the next chunk's reads ahead of this chain
#pragma unroll
                for (int w = 0; w < ATT_VC / 4; w++)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c & 1][w], b[c & 1][w] * inv, acc, 0, 0, 0);
            } else {
                for (int t = 0; t < steps; t += 4)
#pragma unroll
                    for (int w = t; w < t + 4; w++)
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(va[4 * w], pb[4 * w] * inv, acc, 0, 0, 0);
            }
        }
        float *yo = y + ((long long)h * hd + cb * 16) * n + i0 + jl;
#pragma unroll
        for (int r = 0; r < 4; r++) yo[(long long)(4 * g + r) * n] = acc[r];
    }
}

}  // namespace osh

extern "C" {

OSH_API osh_status osh_attention_f32(int heads, int key_dim, int head_dim, int n, float scale, const float *d_qkv,
                                     int64_t head_stride, float *d_y, osh_stream s) {
    if (heads <= 0 || key_dim <= 0 || head_dim <= 0 || n <= 0)
        return fail(OSH_E_INVALID, "Attention: bad sizes");
    if (head_dim > 65536) return fail(OSH_E_UNSUPPORTED, "Attention: head size too large");
    if (!d_qkv || !d_y) return fail(OSH_E_INVALID, "Attention: NULL pointer");
    if (head_stride < (long long)(2 * key_dim + head_dim) * n)
        return fail(OSH_E_INVALID, "Attention: head stride below (2 key_dim + head_dim) * n");
    if (key_dim % 4 || key_dim > 4 * ATT_MAX_KS || head_dim % 16 || n % 16 || heads > 65535)
        return fail(OSH_E_UNSUPPORTED,
                    "Attention: needs key_dim %% 4 == 0, key_dim <= %d, head_dim %% 16 == 0, n %% 16 == 0",
                    4 * ATT_MAX_KS);
    if (n > ATT_MAX_N) return fail(OSH_E_UNSUPPORTED, "Attention: n = %d above %d", n, ATT_MAX_N);
    const size_t lds = att_lds_bytes(n);
    if ((long long)heads * head_stride >= (1LL << 31))
        return fail(OSH_E_UNSUPPORTED, "Attention: qkv too large");
    {
        // other workgroups still read v while one writes y
        const char *a0 = reinterpret_cast<const char *>(d_qkv);
        const char *a1 = a0 + ((heads - 1) * (long long)head_stride + (2LL * key_dim + head_dim) * n) * 4;
        const char *b0 = reinterpret_cast<const char *>(d_y);
        const char *b1 = b0 + (long long)heads * head_dim * n * 4;
        if (a0 < b1 && b0 < a1) return fail(OSH_E_INVALID, "Attention: y overlaps qkv");
    }
    dim3 grid((unsigned)(n / ATT_ROWS), (unsigned)heads);
    const int ks = key_dim / 4;
#define OSH_ATT_LAUNCH(KS) \
    OSH_LAUNCH(attention_kernel<KS>, grid, dim3(256), lds, to_stream(s), key_dim, head_dim, n, scale, d_qkv, \
               (long long)head_stride, d_y)
    if (ks <= 4)
        OSH_ATT_LAUNCH(4);
    else if (ks <= 8)
        OSH_ATT_LAUNCH(8);
    else
        OSH_ATT_LAUNCH(16);
#undef OSH_ATT_LAUNCH
    OSH_LAUNCH_CHECK("attention_kernel");
    return OSH_OK;
}

}  // extern "C"
