/*
 * osh_oracle.c -- CPU restatement of OnnxSharp's dense-contraction arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library in onnxsharp_amd/csrc: tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py are the only callers.  Nothing in the product
 * path links or calls it.
 *
 * Every function restates the arithmetic of the C# reference (paths below are
 * relative to the OnnxSharp source tree) in the same per-element operation
 * order, so that where the reference is a single FMA chain the restatement is
 * bit-exact, and elsewhere the difference is a documented rounding choice.
 *
 *   orc_gemm_f32        src/OnnxSharp/Tensors/GemmKernel.cs:1070-1241 (MR12/6/4 micro-kernels:
 *                       accumulator starts at the bias, k-ascending fmaf chain, fused
 *                       column-scale epilogue fmaf(acc, scale, bias)); unfused tails
 *                       GemmKernel.cs:1594-1608,1645-1690
 *   orc_conv2d_f32      order ORC_ORDER_IM2COL: ConvKernels.cs:554-563 + GemmKernel.cs:1156-1207
 *                       (ic -> ky -> kx fmaf chain from the bias; also PackedConv.cs:420-440,
 *                       Pointwise ConvKernels.cs:464-514, FirstConv.cs:351-420)
 *                       order ORC_ORDER_NCHWC: NchwcConv.cs:533-605 (icb -> ky -> kx -> lane16)
 *   orc_nchwc_conv_avx512  NchwcConv.cs:247-665 (blocked layouts, 2 output blocks x 8 pixels
 *                       per step, AVX-512; the same chain as ORC_ORDER_NCHWC)
 *   orc_conv2d_f64      ConvKernels.cs:656-754 (textbook direct conv, in double)
 *   orc_conv_dw_f32     DepthwiseConv.cs:95-185 (bias, then ky -> kx fmaf)
 *   orc_winograd_f23    Winograd.cs:125-166 (G g G^T), :414-443 (B^T d B), :234-258 (16 GEMMs),
 *                       :497-513 (A^T M A + bias)
 *   orc_exp_ref         VectorMath.cs:21-43 (clamp, Cody-Waite 2-term split, degree-6 Horner)
 *   orc_silu_ref        VectorMath.cs:70-77 (x * (1 / (1 + exp(-x))))
 *   orc_minmax          Quantization.cs:109-181 (0 always included, NaN skipped)
 *   orc_dql_params      QuantizedMatMulOps.cs:151-155
 *   orc_quantize_u8     QuantizedMatMulOps.cs:280-335, Quantization.cs:68-103
 *   orc_dqmm            QuantizedMatMulOps.cs:115-201 (+ Int8F32Gemm.cs:124-174 weight widening)
 *   orc_matmul_integer  Int8Gemm.cs:212-236 (int64 sum of (a - a_zp)(b - b_zp[col]))
 *   orc_softmax_f32     DnnOps.cs:2547-2675 + VectorMath.cs:282-287 (Mul by the constant, then per
 *                       row: max, e = exp(x - max) summed, scale by 1/sum; the sum runs
 *                       sequentially here, in 8 vector lanes there: parity unpinned at that
 *                       rounding)
 *   orc_maxpool2d_f32   DnnOps.cs:1335-1580 (scalar path :1564-1579: -inf, then v > best)
 *   orc_resize_nearest  DnnOps.cs:2215-2330 (nearest, integer factor: source index dst / factor)
 *   orc_sigmoid_ref     VectorMath.cs:64-68 (1 / (1 + Exp(x * -1)), vector path)
 *   orc_dfl_f32         DflOps.cs:97-240 (softmax over bins, expectation of the bin index)
 *
 * Build: see oracle/Makefile (gcc, -O3 -ffp-contract=off; fmaf is explicit).
 */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))
#define HOT

/* ------------------------------------------------------------------ threads */

static int g_threads = 1;

/* The build uses -mavx2 -mfma (fmaf then vectorises along the output row);
 * the loader checks this before the first call. */
ORC_API int orc_cpu_ok(void)
{
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

/* Whether this host runs the AVX-512 paths (the NCHWc kernel, the blocked
 * GEMM, the vector activations); each is bit-identical to its scalar loop. */
static int g_avx512 = -1;
static int have_avx512(void)
{
    if (g_avx512 < 0) {
        __builtin_cpu_init();
        g_avx512 = __builtin_cpu_supports("avx512f") ? 1 : 0;
    }
    return g_avx512;
}

ORC_API void orc_set_threads(int t) { g_threads = t < 1 ? 1 : t; }
ORC_API int orc_get_threads(void) { return g_threads; }

typedef void (*range_fn)(void *ctx, long begin, long end);

typedef struct {
    range_fn fn;
    void *ctx;
    long begin, end;
} job_t;

/* A persistent pool of worker threads (as ParallelRange keeps its workers,
 * src/OnnxSharp/Threading/ParallelRange.cs:15-373): created on first use,
 * woken per parallel_for by a generation counter, joined by a countdown.
 * Creating threads per call cost tens of microseconds each, which the many
 * small layers of a whole network paid a hundred times per frame. */
#define POOL_MAX 256
static pthread_mutex_t pool_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_mutex_t pool_call_mu = PTHREAD_MUTEX_INITIALIZER; /* one parallel_for at a time */
static pthread_cond_t pool_wake = PTHREAD_COND_INITIALIZER;
static pthread_cond_t pool_done = PTHREAD_COND_INITIALIZER;
static int pool_started = 0;  /* workers 1 .. pool_started exist */
static long pool_gen = 0;
static int pool_active = 0;   /* threads of the current job, the caller included */
static int pool_pending = 0;  /* workers of the current job not finished */
static job_t pool_jobs[POOL_MAX];

static void *pool_worker(void *arg)
{
    const int id = (int)(intptr_t)arg;
    long seen = 0;
    pthread_mutex_lock(&pool_mu);
    for (;;) {
        while (pool_gen == seen) pthread_cond_wait(&pool_wake, &pool_mu);
        seen = pool_gen;
        if (id >= pool_active) continue;
        job_t j = pool_jobs[id];
        pthread_mutex_unlock(&pool_mu);
        j.fn(j.ctx, j.begin, j.end);
        pthread_mutex_lock(&pool_mu);
        if (--pool_pending == 0) pthread_cond_signal(&pool_done);
    }
    return NULL;
}

/* Split [0, n) into contiguous chunks over g_threads threads.  Each output
 * element is computed by exactly one thread with the same per-element order,
 * so the result does not depend on the thread count. */
static void parallel_for(long n, range_fn fn, void *ctx)
{
    int t = g_threads;
    if (t <= 1 || n < 2) {
        fn(ctx, 0, n);
        return;
    }
    if (t > n) t = (int)n;
    if (t > POOL_MAX) t = POOL_MAX;
    pthread_mutex_lock(&pool_call_mu);
    pthread_mutex_lock(&pool_mu);
    while (pool_started < t - 1) {
        pthread_t th;
        if (pthread_create(&th, NULL, pool_worker, (void *)(intptr_t)(pool_started + 1)) != 0) break;
        pthread_detach(th);
        pool_started++;
    }
    if (t > pool_started + 1) t = pool_started + 1;
    long base = n / t, rem = n % t, at = 0;
    for (int i = 0; i < t; i++) {
        long len = base + (i < rem ? 1 : 0);
        pool_jobs[i].fn = fn;
        pool_jobs[i].ctx = ctx;
        pool_jobs[i].begin = at;
        pool_jobs[i].end = at + len;
        at += len;
    }
    pool_active = t;
    pool_pending = t - 1;
    pool_gen++;
    pthread_cond_broadcast(&pool_wake);
    job_t j0 = pool_jobs[0];
    pthread_mutex_unlock(&pool_mu);
    j0.fn(j0.ctx, j0.begin, j0.end);
    pthread_mutex_lock(&pool_mu);
    while (pool_pending > 0) pthread_cond_wait(&pool_done, &pool_mu);
    pthread_mutex_unlock(&pool_mu);
    pthread_mutex_unlock(&pool_call_mu);
}

/* --------------------------------------------------------------------- GEMM */

typedef struct {
    int m, k, n, lda, ldb, ldc, fused;
    const float *a, *b, *row_bias, *col_bias, *col_scale;
    float *c;
} gemm_ctx;

/* One row: acc[j] = init; acc[j] = fmaf(a[i,t], b[t,j], acc[j]) for t ascending.
 * Init follows Multiply12Rows (GemmKernel.cs:1113-1152): column scale present
 * -> 0; else column bias -> col_bias[j]; else row bias -> row_bias[i]; else 0. */
HOT static void gemm_rows(void *p, long r0, long r1)
{
    gemm_ctx *g = (gemm_ctx *)p;
    const int k = g->k, n = g->n;
    for (long i = r0; i < r1; i++) {
        float *acc = g->c + i * (long)g->ldc;
        const float *arow = g->a + i * (long)g->lda;
        if (g->col_scale)
            for (int j = 0; j < n; j++) acc[j] = 0.0f;
        else if (g->col_bias)
            for (int j = 0; j < n; j++) acc[j] = g->col_bias[j];
        else {
            float rb = g->row_bias ? g->row_bias[i] : 0.0f;
            for (int j = 0; j < n; j++) acc[j] = rb;
        }
        for (int t = 0; t < k; t++) {
            const float av = arow[t];
            const float *brow = g->b + (long)t * g->ldb;
            for (int j = 0; j < n; j++) acc[j] = fmaf(av, brow[j], acc[j]);
        }
        if (g->col_scale) {
            for (int j = 0; j < n; j++) {
                float bb = g->col_bias ? g->col_bias[j] : 0.0f;
                acc[j] = g->fused ? fmaf(acc[j], g->col_scale[j], bb)
                                  : (g->col_bias ? acc[j] * g->col_scale[j] + bb
                                                 : acc[j] * g->col_scale[j]);
            }
        }
    }
}

/* The same chain register-blocked on AVX-512, as the reference's MR12
 * micro-kernel runs it over packed B panels (GemmKernel.cs:418-526,
 * 1070-1207): a task is one 32-column block of C; its B columns are copied
 * into a contiguous [k][32] panel once, then every 8-row block of C runs
 * against it with 16 accumulators of 16 lanes initialised from the bias --
 * per k step two 16-wide panel rows against eight broadcast values of A, one
 * fused multiply-add each (from 0 with a column scale, then its epilogue).
 * Every element is the fmaf chain gemm_rows computes, so the same bits.
 * Column tails use masked lanes. */
__attribute__((target("avx512f,fma"))) static void gemm_blocks(void *p, long t0, long t1)
{
    const gemm_ctx *g = (const gemm_ctx *)p;
    const int k = g->k;
    float *panel = (float *)aligned_alloc(64, sizeof(float) * 32 * (size_t)(k > 0 ? k : 1));
    for (long t = t0; t < t1; t++) {
        const int j0 = (int)t * 32;
        const int c0 = g->n - j0 < 16 ? g->n - j0 : 16, c1 = g->n - j0 - 16 < 16 ? g->n - j0 - 16 : 16;
        const __mmask16 m0 = c0 >= 16 ? 0xFFFF : (__mmask16)((1u << c0) - 1);
        const __mmask16 m1 = c1 <= 0 ? 0 : c1 >= 16 ? 0xFFFF : (__mmask16)((1u << c1) - 1);
        for (int kk = 0; kk < k; kk++) {
            const float *brow = g->b + (long)kk * g->ldb + j0;
            _mm512_store_ps(panel + (long)kk * 32, _mm512_maskz_loadu_ps(m0, brow));
            _mm512_store_ps(panel + (long)kk * 32 + 16, _mm512_maskz_loadu_ps(m1, brow + 16));
        }
        __m512 s0 = _mm512_setzero_ps(), s1 = _mm512_setzero_ps(), cb0 = s0, cb1 = s0;
        if (g->col_scale) {
            s0 = _mm512_maskz_loadu_ps(m0, g->col_scale + j0);
            s1 = _mm512_maskz_loadu_ps(m1, g->col_scale + j0 + 16);
            if (g->col_bias) {
                cb0 = _mm512_maskz_loadu_ps(m0, g->col_bias + j0);
                cb1 = _mm512_maskz_loadu_ps(m1, g->col_bias + j0 + 16);
            }
        }
        for (int i0 = 0; i0 < g->m; i0 += 8) {
            const int rows = g->m - i0 < 8 ? g->m - i0 : 8;
            __m512 acc0[8], acc1[8];
            const float *arow[8];
#pragma GCC unroll 8
            for (int r = 0; r < 8; r++) {
                arow[r] = g->a + (long)(i0 + (r < rows ? r : 0)) * g->lda;
                if (g->col_scale) {
                    acc0[r] = acc1[r] = _mm512_setzero_ps();
                } else if (g->col_bias) {
                    acc0[r] = _mm512_maskz_loadu_ps(m0, g->col_bias + j0);
                    acc1[r] = _mm512_maskz_loadu_ps(m1, g->col_bias + j0 + 16);
                } else {
                    const float rb = (g->row_bias && r < rows) ? g->row_bias[i0 + r] : 0.0f;
                    acc0[r] = acc1[r] = _mm512_set1_ps(rb);
                }
            }
            for (int kk = 0; kk < k; kk++) {
                const __m512 b0 = _mm512_load_ps(panel + (long)kk * 32), b1 = _mm512_load_ps(panel + (long)kk * 32 + 16);
#pragma GCC unroll 8
                for (int r = 0; r < 8; r++) {
                    const __m512 av = _mm512_set1_ps(arow[r][kk]);
                    acc0[r] = _mm512_fmadd_ps(av, b0, acc0[r]);
                    acc1[r] = _mm512_fmadd_ps(av, b1, acc1[r]);
                }
            }
            if (g->col_scale)  /* the column-scale epilogue, fused or as the ScaleColumns tail */
                for (int r = 0; r < rows; r++) {
                    if (g->fused) {
                        acc0[r] = _mm512_fmadd_ps(acc0[r], s0, cb0);
                        acc1[r] = _mm512_fmadd_ps(acc1[r], s1, cb1);
                    } else {
                        acc0[r] = _mm512_mul_ps(acc0[r], s0);
                        acc1[r] = _mm512_mul_ps(acc1[r], s1);
                        if (g->col_bias) {
                            acc0[r] = _mm512_add_ps(acc0[r], cb0);
                            acc1[r] = _mm512_add_ps(acc1[r], cb1);
                        }
                    }
                }
            for (int r = 0; r < rows; r++) {
                float *crow = g->c + (long)(i0 + r) * g->ldc + j0;
                _mm512_mask_storeu_ps(crow, m0, acc0[r]);
                _mm512_mask_storeu_ps(crow + 16, m1, acc1[r]);
            }
        }
    }
    free(panel);
}

/* C[m,n] (ldc) = A[m,k] (lda) * B[k,n] (ldb) with the reference's bias and
 * column-scale epilogue.  fused=1 is the micro-kernel epilogue (one fmaf),
 * fused=0 the ScaleColumns tail (multiply, then add).  The register-blocked
 * AVX-512 path runs where the host has AVX-512. */
ORC_API void orc_gemm_f32(int m, int k, int n, const float *a, int lda, const float *b, int ldb,
                          const float *row_bias, const float *col_bias, const float *col_scale,
                          float *c, int ldc, int fused)
{
    gemm_ctx g = {m, k, n, lda, ldb, ldc, fused, a, b, row_bias, col_bias, col_scale, c};
    if (have_avx512()) {
        parallel_for((n + 31) / 32, gemm_blocks, &g);
        return;
    }
    parallel_for(m, gemm_rows, &g);
}

/* The same product on the scalar loop only (gemm_rows), for checking the
 * blocked path against it. */
ORC_API void orc_gemm_f32_rows(int m, int k, int n, const float *a, int lda, const float *b, int ldb,
                               const float *row_bias, const float *col_bias, const float *col_scale,
                               float *c, int ldc, int fused)
{
    gemm_ctx g = {m, k, n, lda, ldb, ldc, fused, a, b, row_bias, col_bias, col_scale, c};
    parallel_for(m, gemm_rows, &g);
}

/* Double-precision naive product (the reference tests' "naive" oracle,
 * tests/OnnxSharp.Tests/GemmKernelTests.cs:174-180,205-214). */
ORC_API void orc_gemm_f64(int m, int k, int n, const float *a, const float *b, const float *col_bias,
                          const float *row_bias, double *c)
{
    for (int i = 0; i < m; i++)
        for (int j = 0; j < n; j++) {
            double s = col_bias ? col_bias[j] : (row_bias ? row_bias[i] : 0.0);
            for (int t = 0; t < k; t++) s += (double)a[(long)i * k + t] * b[(long)t * n + j];
            c[(long)i * n + j] = s;
        }
}

/* --------------------------------------------------------------------- conv */

enum { ORC_ORDER_IM2COL = 0, ORC_ORDER_NCHWC = 1 };

typedef struct {
    int N, C, H, W, M, KH, KW, group, sh, sw, dh, dw, pt, pl, OH, OW;
} conv_shape;

typedef struct {
    conv_shape s;
    int order, Hp, Wp;
    const float *xpad; /* [N][C][Hp][Wp], zero halo */
    const float *w, *bias;
    float *y;
} conv_ctx;

/* Zero-padded copy of the input so that every tap reads a value (padding
 * positions read 0, as the reference's im2col / blocked buffers do). */
static float *pad_input(const conv_shape *s, const float *x, int *Hp_out, int *Wp_out)
{
    long needH = (long)(s->OH - 1) * s->sh + (long)(s->KH - 1) * s->dh + 1;
    long needW = (long)(s->OW - 1) * s->sw + (long)(s->KW - 1) * s->dw + 1;
    long Hp = s->pt + s->H, Wp = s->pl + s->W;
    if (needH > Hp) Hp = needH;
    if (needW > Wp) Wp = needW;
    float *xp = (float *)calloc((size_t)s->N * s->C * Hp * Wp, sizeof(float));
    for (long nc = 0; nc < (long)s->N * s->C; nc++)
        for (int yy = 0; yy < s->H; yy++)
            memcpy(xp + (nc * Hp + yy + s->pt) * Wp + s->pl, x + (nc * s->H + yy) * (long)s->W,
                   sizeof(float) * s->W);
    *Hp_out = (int)Hp;
    *Wp_out = (int)Wp;
    return xp;
}

HOT static void conv_planes(void *p, long t0, long t1)
{
    conv_ctx *cx = (conv_ctx *)p;
    const conv_shape *s = &cx->s;
    const int cpg = s->C / s->group, opg = s->M / s->group;
    const int OW = s->OW;
    float *acc = (float *)malloc(sizeof(float) * OW);
    float *xv = (float *)malloc(sizeof(float) * OW);
    for (long t = t0; t < t1; t++) { /* t = (n * M + oc) * OH + oy */
        int oy = (int)(t % s->OH);
        long nm = t / s->OH;
        int oc = (int)(nm % s->M), n = (int)(nm / s->M);
        int g = oc / opg;
        float b0 = cx->bias ? cx->bias[oc] : 0.0f;
        for (int ox = 0; ox < OW; ox++) acc[ox] = b0;
        const float *wo = cx->w + (long)oc * cpg * s->KH * s->KW;
        if (cx->order == ORC_ORDER_NCHWC) {
            for (int ib = 0; ib < cpg / 16; ib++)
                for (int ky = 0; ky < s->KH; ky++)
                    for (int kx = 0; kx < s->KW; kx++)
                        for (int lane = 0; lane < 16; lane++) {
                            int ic = ib * 16 + lane;
                            float wv = wo[((long)ic * s->KH + ky) * s->KW + kx];
                            const float *row = cx->xpad +
                                (((long)n * s->C + g * cpg + ic) * cx->Hp + (long)oy * s->sh + (long)ky * s->dh) * cx->Wp +
                                (long)kx * s->dw;
                            for (int ox = 0; ox < OW; ox++) xv[ox] = row[(long)ox * s->sw];
                            for (int ox = 0; ox < OW; ox++) acc[ox] = fmaf(xv[ox], wv, acc[ox]);
                        }
        } else {
            for (int ic = 0; ic < cpg; ic++)
                for (int ky = 0; ky < s->KH; ky++)
                    for (int kx = 0; kx < s->KW; kx++) {
                        float wv = wo[((long)ic * s->KH + ky) * s->KW + kx];
                        const float *row = cx->xpad +
                            (((long)n * s->C + g * cpg + ic) * cx->Hp + (long)oy * s->sh + (long)ky * s->dh) * cx->Wp +
                            (long)kx * s->dw;
                        if (s->sw == 1)
                            for (int ox = 0; ox < OW; ox++) acc[ox] = fmaf(wv, row[ox], acc[ox]);
                        else {
                            for (int ox = 0; ox < OW; ox++) xv[ox] = row[(long)ox * s->sw];
                            for (int ox = 0; ox < OW; ox++) acc[ox] = fmaf(wv, xv[ox], acc[ox]);
                        }
                    }
        }
        memcpy(cx->y + t * (long)OW, acc, sizeof(float) * OW);
    }
    free(acc);
    free(xv);
}

/* NCHW conv with explicit begin pads; the output size is given (the caller
 * resolved it as ConvLayer.GetMemoryShapes does).  Returns -1 if the NCHWc
 * order is asked for a shape it does not cover (C/group not a multiple of 16). */
ORC_API int orc_conv2d_f32(int order, int N, int C, int H, int W, int M, int KH, int KW, int group, int sh,
                           int sw, int dh, int dw, int pt, int pl, int OH, int OW, const float *x,
                           const float *w, const float *bias, float *y)
{
    conv_shape s = {N, C, H, W, M, KH, KW, group, sh, sw, dh, dw, pt, pl, OH, OW};
    if (order == ORC_ORDER_NCHWC && (C / group) % 16 != 0) return -1;
    conv_ctx cx;
    cx.s = s;
    cx.order = order;
    float *xp = pad_input(&s, x, &cx.Hp, &cx.Wp);
    cx.xpad = xp;
    cx.w = w;
    cx.bias = bias;
    cx.y = y;
    parallel_for((long)N * M * OH, conv_planes, &cx);
    free(xp);
    return 0;
}

/* ------------------------------------------------ NCHWc blocked, AVX-512 */

/* The reference's NchwcConv as it runs on an AVX-512 host (NchwcConv.cs:247-665),
 * restated with AVX-512 intrinsics: the cpu_baseline's fast path for the
 * shapes the NCHWc gate takes, bit-identical to orc_conv2d_f32's
 * ORC_ORDER_NCHWC (the same per-element fused multiply-add chain from the
 * bias, ib -> ky -> kx -> input lane; checked by the CPU tests).
 *   weights  [M/16][C/16][ky*3 + kx][input lane 16][output lane 16], packed once
 *            (NchwcConv.PackWeights, :247-274; the reference caches it on the
 *            weight tensor);
 *   input    [C/16][H + pad][W + pad][16], pad 2 at stride 1 (a zero ring), 1 at
 *            stride 2 (top row and left column), repacked per call (PackInput,
 *            :289-368);
 *   output   [M/16][OH][OW][16], then back to NCHW (UnpackOutput, :370-412);
 *   kernel   per (pair of output blocks, output row): groups of 8 pixels x 2
 *            output blocks = 16 accumulators of 16 lanes, each lane step one
 *            broadcast input value against a 16-wide weight row (Row, :508-665);
 *            the last OW % 8 pixels one at a time.
 * Threads split (block pair, row) tasks as ParallelRange.For does in Conv
 * (:462-505).  Built only into functions with the avx512f target; callers
 * check orc_nchwc_avx512_ok() first. */

ORC_API int orc_nchwc_avx512_ok(void)
{
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f");
}

/* w: OIHW [M][C][3][3] -> wp [M/16][C/16][9][16][16] */
ORC_API void orc_nchwc_pack_weights(int C, int M, const float *w, float *wp)
{
    const int ib = C / 16;
    for (int o = 0; o < M; o++)
        for (int i = 0; i < C; i++)
            for (int kp = 0; kp < 9; kp++)
                wp[((((long)(o / 16) * ib + i / 16) * 9 + kp) * 16 + i % 16) * 16 + o % 16] =
                    w[((long)o * C + i) * 9 + kp];
}

typedef struct {
    int C, H, W, M, stride, OH, OW, pad, Hp, Wp;
    const float *x, *wp, *bias;
    float *xb, *yb, *y;
} nchwc_ctx;

/* task = (input block, padded row): NCHW rows into the blocked buffer, halo zero */
__attribute__((target("avx512f,fma"))) static void nchwc_pack_rows(void *p, long t0, long t1)
{
    nchwc_ctx *c = (nchwc_ctx *)p;
    const long plane = (long)c->H * c->W;
    for (long t = t0; t < t1; t++) {
        const int cb = (int)(t / c->Hp), r = (int)(t % c->Hp);
        float *dst = c->xb + ((long)cb * c->Hp + r) * c->Wp * 16;
        const int y = r - 1;
        if (y < 0 || y >= c->H) {
            memset(dst, 0, sizeof(float) * 16 * c->Wp);
            continue;
        }
        _mm512_storeu_ps(dst, _mm512_setzero_ps());
        if (c->pad == 2) _mm512_storeu_ps(dst + (long)(c->W + 1) * 16, _mm512_setzero_ps());
        const float *src = c->x + (long)cb * 16 * plane + (long)y * c->W;
        for (int xx = 0; xx < c->W; xx++) {
            float *d = dst + (long)(xx + 1) * 16;
            for (int lane = 0; lane < 16; lane++) d[lane] = src[lane * plane + xx];
        }
    }
}

/* task = (output block pair, output row) */
__attribute__((target("avx512f,fma"))) static void nchwc_rows(void *p, long t0, long t1)
{
    nchwc_ctx *c = (nchwc_ctx *)p;
    const int icb = c->C / 16, s = c->stride, OW = c->OW, OH = c->OH;
    const long wblk = (long)icb * 9 * 256; /* floats of one output block's weights */
    for (long t = t0; t < t1; t++) {
        const int row = (int)(t % OH), ob = (int)(t / OH) * 2;
        const __m512 b0 = c->bias ? _mm512_loadu_ps(c->bias + (long)ob * 16) : _mm512_setzero_ps();
        const __m512 b1 = c->bias ? _mm512_loadu_ps(c->bias + (long)(ob + 1) * 16) : _mm512_setzero_ps();
        const float *w0 = c->wp + (long)ob * wblk, *w1 = w0 + wblk;
        float *o0 = c->yb + ((long)ob * OH + row) * OW * 16, *o1 = o0 + (long)OH * OW * 16;
        const int groups = OW / 8;
        for (int g = 0; g < groups; g++) {
            __m512 a0[8], a1[8];
            for (int q = 0; q < 8; q++) a0[q] = b0, a1[q] = b1;
            for (int ib = 0; ib < icb; ib++)
                for (int ky = 0; ky < 3; ky++) {
                    const float *rin = c->xb + (((long)ib * c->Hp + (long)row * s + ky) * c->Wp + (long)g * 8 * s) * 16;
                    for (int kx = 0; kx < 3; kx++) {
                        const float *wp0 = w0 + (long)(ib * 9 + ky * 3 + kx) * 256;
                        const float *wp1 = w1 + (long)(ib * 9 + ky * 3 + kx) * 256;
                        const float *px = rin + kx * 16;
                        for (int lane = 0; lane < 16; lane++) {
                            const __m512 wv0 = _mm512_loadu_ps(wp0 + lane * 16);
                            const __m512 wv1 = _mm512_loadu_ps(wp1 + lane * 16);
                            for (int q = 0; q < 8; q++) {
                                const __m512 xv = _mm512_set1_ps(px[(long)q * s * 16 + lane]);
                                a0[q] = _mm512_fmadd_ps(xv, wv0, a0[q]);
                                a1[q] = _mm512_fmadd_ps(xv, wv1, a1[q]);
                            }
                        }
                    }
                }
            for (int q = 0; q < 8; q++) {
                _mm512_storeu_ps(o0 + ((long)g * 8 + q) * 16, a0[q]);
                _mm512_storeu_ps(o1 + ((long)g * 8 + q) * 16, a1[q]);
            }
        }
        for (int col = groups * 8; col < OW; col++) {
            __m512 a = b0, b = b1;
            for (int ib = 0; ib < icb; ib++)
                for (int ky = 0; ky < 3; ky++)
                    for (int kx = 0; kx < 3; kx++) {
                        const float *wp0 = w0 + (long)(ib * 9 + ky * 3 + kx) * 256;
                        const float *wp1 = w1 + (long)(ib * 9 + ky * 3 + kx) * 256;
                        const float *px =
                            c->xb + (((long)ib * c->Hp + (long)row * s + ky) * c->Wp + (long)col * s + kx) * 16;
                        for (int lane = 0; lane < 16; lane++) {
                            const __m512 xv = _mm512_set1_ps(px[lane]);
                            a = _mm512_fmadd_ps(xv, _mm512_loadu_ps(wp0 + lane * 16), a);
                            b = _mm512_fmadd_ps(xv, _mm512_loadu_ps(wp1 + lane * 16), b);
                        }
                    }
            _mm512_storeu_ps(o0 + (long)col * 16, a);
            _mm512_storeu_ps(o1 + (long)col * 16, b);
        }
    }
}

/* task = (output block, output row): blocked rows back to NCHW */
static void nchwc_unpack_rows(void *p, long t0, long t1)
{
    nchwc_ctx *c = (nchwc_ctx *)p;
    const long plane = (long)c->OH * c->OW;
    for (long t = t0; t < t1; t++) {
        const int ob = (int)(t / c->OH), row = (int)(t % c->OH);
        const float *src = c->yb + ((long)ob * c->OH + row) * c->OW * 16;
        float *dst = c->y + (long)ob * 16 * plane + (long)row * c->OW;
        for (int lane = 0; lane < 16; lane++)
            for (int col = 0; col < c->OW; col++) dst[lane * plane + col] = src[(long)col * 16 + lane];
    }
}

/* Bytes of the blocked input and output buffers the conv needs. */
ORC_API void orc_nchwc_scratch_floats(int C, int H, int W, int M, int stride, int OH, int OW, long *xb, long *yb)
{
    const int pad = stride == 2 ? 1 : 2;
    *xb = (long)C * (H + pad) * (W + pad);
    *yb = (long)M * OH * OW;
}

/* Batch-1 NCHW conv through the blocked kernel.  Returns -1 outside the
 * reference's NCHWc gate (NchwcConv.Dispatch, :129-143) or without AVX-512. */
ORC_API int orc_nchwc_conv_avx512(int C, int H, int W, int M, int stride, int OH, int OW, const float *x,
                                  const float *wp, const float *bias, float *y, float *xb, float *yb)
{
    if (!orc_nchwc_avx512_ok() || C % 16 || M % 32 || (stride != 1 && stride != 2)) return -1;
    if (stride == 2 ? (H % 2 || W % 2 || OH * 2 != H || OW * 2 != W) : (OH != H || OW != W)) return -1;
    nchwc_ctx c = {C, H, W, M, stride, OH, OW, stride == 2 ? 1 : 2, 0, 0, x, wp, bias, xb, yb, y};
    c.Hp = H + c.pad;
    c.Wp = W + c.pad;
    parallel_for((long)(C / 16) * c.Hp, nchwc_pack_rows, &c);
    parallel_for((long)(M / 32) * OH, nchwc_rows, &c);
    parallel_for((long)(M / 16) * OH, nchwc_unpack_rows, &c);
    return 0;
}

/* Textbook direct conv in double (ConvKernels.Direct semantics). */
ORC_API void orc_conv2d_f64(int N, int C, int H, int W, int M, int KH, int KW, int group, int sh, int sw,
                            int dh, int dw, int pt, int pl, int OH, int OW, const float *x, const float *w,
                            const float *bias, double *y)
{
    int cpg = C / group, opg = M / group;
    for (int n = 0; n < N; n++)
        for (int oc = 0; oc < M; oc++) {
            int g = oc / opg;
            for (int oy = 0; oy < OH; oy++)
                for (int ox = 0; ox < OW; ox++) {
                    double s = bias ? bias[oc] : 0.0;
                    for (int ic = 0; ic < cpg; ic++)
                        for (int ky = 0; ky < KH; ky++) {
                            int iy = oy * sh - pt + ky * dh;
                            if (iy < 0 || iy >= H) continue;
                            for (int kx = 0; kx < KW; kx++) {
                                int ix = ox * sw - pl + kx * dw;
                                if (ix < 0 || ix >= W) continue;
                                s += (double)x[(((long)n * C + g * cpg + ic) * H + iy) * W + ix] *
                                     w[(((long)oc * cpg + ic) * KH + ky) * KW + kx];
                            }
                        }
                    y[(((long)n * M + oc) * OH + oy) * OW + ox] = s;
                }
        }
}

/* Depthwise conv (group == C == M, one input channel per group): the
 * accumulator starts at the bias and runs ky -> kx with fmaf (the reference's
 * vector path; its stride>1 path is unfused, a rounding-only difference). */
typedef struct {
    int C, H, W, KH, KW, sh, sw, dh, dw, pt, pl, OH, OW;
    const float *x, *w, *bias;
    float *y;
} dw_ctx;

/* task = (image, channel) plane; per output: bias, then ky -> kx fmaf, taps
 * off the map skipped */
static void dw_planes(void *p, long t0, long t1)
{
    const dw_ctx *d = (const dw_ctx *)p;
    for (long t = t0; t < t1; t++) {
        const int c = (int)(t % d->C);
        const float *xp = d->x + t * (long)d->H * d->W;
        const float *wc = d->w + (long)c * d->KH * d->KW;
        float *yp = d->y + t * (long)d->OH * d->OW;
        for (int oy = 0; oy < d->OH; oy++)
            for (int ox = 0; ox < d->OW; ox++) {
                float acc = d->bias ? d->bias[c] : 0.0f;
                for (int ky = 0; ky < d->KH; ky++) {
                    int iy = oy * d->sh - d->pt + ky * d->dh;
                    if (iy < 0 || iy >= d->H) continue;
                    for (int kx = 0; kx < d->KW; kx++) {
                        int ix = ox * d->sw - d->pl + kx * d->dw;
                        if (ix < 0 || ix >= d->W) continue;
                        acc = fmaf(wc[ky * d->KW + kx], xp[(long)iy * d->W + ix], acc);
                    }
                }
                yp[(long)oy * d->OW + ox] = acc;
            }
    }
}

ORC_API void orc_conv_dw_f32(int N, int C, int H, int W, int KH, int KW, int sh, int sw, int dh, int dw,
                             int pt, int pl, int OH, int OW, const float *x, const float *w,
                             const float *bias, float *y)
{
    dw_ctx d = {C, H, W, KH, KW, sh, sw, dh, dw, pt, pl, OH, OW, x, w, bias, y};
    parallel_for((long)N * C, dw_planes, &d);
}

/* Winograd F(2x2, 3x3), stride 1, pad 1 (Winograd.cs).  Output size == input size. */
ORC_API void orc_winograd_f23(int N, int C, int H, int W, int M, const float *x, const float *w,
                              const float *bias, float *y)
{
    int tilesY = (H + 1) / 2, tilesX = (W + 1) / 2, tiles = tilesY * tilesX;
    float *U = (float *)malloc(sizeof(float) * 16 * (size_t)M * C);
    float *V = (float *)malloc(sizeof(float) * 16 * (size_t)C * tiles);
    float *Mc = (float *)malloc(sizeof(float) * 16 * (size_t)M * tiles);
    for (int oc = 0; oc < M; oc++)
        for (int ic = 0; ic < C; ic++) {
            const float *g = w + ((long)oc * C + ic) * 9;
            float s[12], u[16];
            for (int j = 0; j < 3; j++) {
                float g0 = g[j], g1 = g[3 + j], g2 = g[6 + j];
                s[j] = g0;
                s[3 + j] = (g0 + g1 + g2) * 0.5f;
                s[6 + j] = (g0 - g1 + g2) * 0.5f;
                s[9 + j] = g2;
            }
            for (int i = 0; i < 4; i++) {
                float a = s[i * 3], b = s[i * 3 + 1], c = s[i * 3 + 2];
                u[i * 4] = a;
                u[i * 4 + 1] = (a + b + c) * 0.5f;
                u[i * 4 + 2] = (a - b + c) * 0.5f;
                u[i * 4 + 3] = c;
            }
            for (int comp = 0; comp < 16; comp++) U[(long)comp * M * C + (long)oc * C + ic] = u[comp];
        }
    for (int n = 0; n < N; n++) {
        const float *xn = x + (long)n * C * H * W;
        for (int c = 0; c < C; c++)
            for (int ty = 0; ty < tilesY; ty++)
                for (int tx = 0; tx < tilesX; tx++) {
                    float d[16], t[16];
                    int y0 = ty * 2 - 1, x0 = tx * 2 - 1;
                    for (int i = 0; i < 4; i++)
                        for (int j = 0; j < 4; j++) {
                            int yy = y0 + i, xx = x0 + j;
                            d[i * 4 + j] = (yy >= 0 && yy < H && xx >= 0 && xx < W)
                                               ? xn[((long)c * H + yy) * W + xx] : 0.0f;
                        }
                    for (int j = 0; j < 4; j++) {
                        float d0 = d[j], d1 = d[4 + j], d2 = d[8 + j], d3 = d[12 + j];
                        t[j] = d0 - d2;
                        t[4 + j] = d1 + d2;
                        t[8 + j] = d2 - d1;
                        t[12 + j] = d1 - d3;
                    }
                    long tile = (long)ty * tilesX + tx;
                    for (int i = 0; i < 4; i++) {
                        float a = t[i * 4], b = t[i * 4 + 1], c2 = t[i * 4 + 2], d3 = t[i * 4 + 3];
                        V[((long)(i * 4) * C + c) * tiles + tile] = a - c2;
                        V[((long)(i * 4 + 1) * C + c) * tiles + tile] = b + c2;
                        V[((long)(i * 4 + 2) * C + c) * tiles + tile] = c2 - b;
                        V[((long)(i * 4 + 3) * C + c) * tiles + tile] = b - d3;
                    }
                }
        for (int comp = 0; comp < 16; comp++)
            orc_gemm_f32(M, C, tiles, U + (long)comp * M * C, C, V + (long)comp * C * tiles, tiles, NULL, NULL,
                         NULL, Mc + (long)comp * M * tiles, tiles, 1);
        for (int oc = 0; oc < M; oc++) {
            float b = bias ? bias[oc] : 0.0f;
            for (int ty = 0; ty < tilesY; ty++)
                for (int tx = 0; tx < tilesX; tx++) {
                    long tile = (long)ty * tilesX + tx;
                    float t[8];
                    for (int j = 0; j < 4; j++) {
                        float m0 = Mc[((long)j * M + oc) * tiles + tile];
                        float m1 = Mc[((long)(4 + j) * M + oc) * tiles + tile];
                        float m2 = Mc[((long)(8 + j) * M + oc) * tiles + tile];
                        float m3 = Mc[((long)(12 + j) * M + oc) * tiles + tile];
                        t[j] = m0 + m1 + m2;
                        t[4 + j] = m1 - m2 - m3;
                    }
                    float y00 = t[0] + t[1] + t[2] + b;
                    float y01 = t[1] - t[2] - t[3] + b;
                    float y10 = t[4] + t[5] + t[6] + b;
                    float y11 = t[5] - t[6] - t[7] + b;
                    int oy = ty * 2, ox = tx * 2;
                    float *yc = y + ((long)n * M + oc) * H * W;
                    if (oy < H) {
                        if (ox < W) yc[(long)oy * W + ox] = y00;
                        if (ox + 1 < W) yc[(long)oy * W + ox + 1] = y01;
                    }
                    if (oy + 1 < H) {
                        if (ox < W) yc[(long)(oy + 1) * W + ox] = y10;
                        if (ox + 1 < W) yc[(long)(oy + 1) * W + ox + 1] = y11;
                    }
                }
        }
    }
    free(U);
    free(V);
    free(Mc);
}

/* --------------------------------------------------------------- activations */

/* exp polynomial of the reference vector path (VectorMath.Exp). */
static float exp_ref(float x)
{
    x = fminf(fmaxf(x, -87.3f), 88.7f);
    float n = nearbyintf(x * 1.4426950408889634f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.4286067653e-6f, r);
    float p = 1.0f / 720.0f;
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int32_t bits = ((int32_t)n + 127) << 23;
    float two_n;
    memcpy(&two_n, &bits, 4);
    return p * two_n;
}

/* exp_ref on 16 lanes: the same single IEEE operations (max/min against
 * the constants return the constant for a NaN lane, as fmaxf/fminf do; the
 * rounding is round-to-nearest-even; n is integral, so its conversion to int
 * is exact). */
__attribute__((target("avx512f,fma"))) static __m512 exp_ref16(__m512 x)
{
    x = _mm512_min_ps(_mm512_max_ps(x, _mm512_set1_ps(-87.3f)), _mm512_set1_ps(88.7f));
    const __m512 n = _mm512_roundscale_ps(_mm512_mul_ps(x, _mm512_set1_ps(1.4426950408889634f)),
                                          _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m512 r = _mm512_fmadd_ps(n, _mm512_set1_ps(-0.693145751953125f), x);
    r = _mm512_fmadd_ps(n, _mm512_set1_ps(-1.4286067653e-6f), r);
    __m512 p = _mm512_set1_ps(1.0f / 720.0f);
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(1.0f / 120.0f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(1.0f / 24.0f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(1.0f / 6.0f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(0.5f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(1.0f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(1.0f));
    const __m512i bits = _mm512_slli_epi32(_mm512_add_epi32(_mm512_cvtps_epi32(n), _mm512_set1_epi32(127)), 23);
    return _mm512_mul_ps(p, _mm512_castsi512_ps(bits));
}

enum { UNARY_EXP = 0, UNARY_SILU = 1, UNARY_SIGMOID = 2 };

typedef struct {
    int op;
    const float *x;
    float *y;
    long n;
} unary_ctx;

static float unary1(int op, float v)
{
    if (op == UNARY_EXP) return exp_ref(v);
    const float e = exp_ref(v * -1.0f);
    return op == UNARY_SILU ? v * (1.0f / (1.0f + e)) : 1.0f / (1.0f + e);
}

__attribute__((target("avx512f,fma"))) static void unary_avx512(const unary_ctx *u, long i0, long i1)
{
    const __m512 one = _mm512_set1_ps(1.0f), neg = _mm512_set1_ps(-1.0f);
    long i = i0;
    for (; i + 16 <= i1; i += 16) {
        const __m512 v = _mm512_loadu_ps(u->x + i);
        __m512 r;
        if (u->op == UNARY_EXP) {
            r = exp_ref16(v);
        } else {
            const __m512 q = _mm512_div_ps(one, _mm512_add_ps(one, exp_ref16(_mm512_mul_ps(v, neg))));
            r = u->op == UNARY_SILU ? _mm512_mul_ps(v, q) : q;
        }
        _mm512_storeu_ps(u->y + i, r);
    }
    for (; i < i1; i++) u->y[i] = unary1(u->op, u->x[i]);
}

/* chunk c of 8192 elements (TensorOps.ElementWiseUnary splits large tensors
 * into parallel chunks, TensorOps.cs:281-298; every element's bits are the
 * same whichever lane or thread computes it) */
static void unary_chunks(void *p, long c0, long c1)
{
    const unary_ctx *u = (const unary_ctx *)p;
    const long i0 = c0 * 8192, i1 = c1 * 8192 < u->n ? c1 * 8192 : u->n;
    if (have_avx512()) {
        unary_avx512(u, i0, i1);
        return;
    }
    for (long i = i0; i < i1; i++) u->y[i] = unary1(u->op, u->x[i]);
}

static void unary_run(int op, long n, const float *x, float *y)
{
    unary_ctx u = {op, x, y, n};
    parallel_for((n + 8191) / 8192, unary_chunks, &u);
}

ORC_API void orc_exp_ref(long n, const float *x, float *y) { unary_run(UNARY_EXP, n, x, y); }

/* The scalar loop alone (op 0 exp, 1 SiLU, 2 sigmoid), for checking the
 * vector path against it. */
ORC_API void orc_unary_scalar(int op, long n, const float *x, float *y)
{
    for (long i = 0; i < n; i++) y[i] = unary1(op, x[i]);
}

/* SiLU of the vector path: x * (1 / (1 + exp(x * -1))). */
ORC_API void orc_silu_ref(long n, const float *x, float *y) { unary_run(UNARY_SILU, n, x, y); }

/* SiLU of the scalar tail (MathF.Exp; here the C library's expf, whose last
 * bit is not pinned against .NET). */
ORC_API void orc_silu_scalar(long n, const float *x, float *y)
{
    for (long i = 0; i < n; i++) y[i] = x[i] * (1.0f / (1.0f + expf(-x[i])));
}

/* MathF.Max: NaN if either operand is NaN; +0 over -0. */
static float dotnet_max(float a, float b)
{
    if (a != a || b != b) return NAN;
    if (a > b) return a;
    if (b > a) return b;
    return signbit(a) ? b : a; /* equal: +0 over -0 */
}

/* Sigmoid of the vector path (VectorMath.cs:64-68): 1 / (1 + exp(x * -1)). */
ORC_API void orc_sigmoid_ref(long n, const float *x, float *y) { unary_run(UNARY_SIGMOID, n, x, y); }

/* DflSoftmax (DflOps.cs:97-240): x [B][sides*bins][N] -> y [B][sides][N],
 * y = sum_b softmax_b(x[side*bins + b]) * b.  The reference works on blocks of
 * 256 columns, 8 at a time (:108-146,168-240):
 *   max  = Avx.Max(max, row)  -- maxps: the row value unless max > row;
 *   e_b  = VectorMath.Exp(row - max), sum = sum + e_b in bin order;
 *   inv  = 1 / sum;  w = fma(e_b * inv, b, w) from 0 in bin order.
 * The last width % 8 columns of a block take the scalar lines: MathF.Max
 * (NaN if either is NaN), MathF.Exp (here exp_ref: its bits are not pinned
 * against .NET), and w += e_b * inv * b with three roundings. */

ORC_API void orc_dfl_f32(int batches, int sides, int bins, int pixels, const float *x, float *y)
{
    for (int bt = 0; bt < batches; bt++)
        for (int s = 0; s < sides; s++) {
            const float *src = x + ((long)bt * sides + s) * bins * pixels;
            float *dst = y + ((long)bt * sides + s) * pixels;
            for (int n = 0; n < pixels; n++) {
                const int col = n % 256, width = (pixels - (n - col)) < 256 ? pixels - (n - col) : 256;
                const int tail = col >= (width & ~7);
                float m = -INFINITY;
                for (int b = 0; b < bins; b++) {
                    const float v = src[(long)b * pixels + n];
                    m = tail ? dotnet_max(m, v) : (m > v ? m : v);
                }
                float total = 0.0f;
                for (int b = 0; b < bins; b++) total = total + exp_ref(src[(long)b * pixels + n] - m);
                const float inv = 1.0f / total;
                float w = 0.0f;
                for (int b = 0; b < bins; b++) {
                    const float p = exp_ref(src[(long)b * pixels + n] - m) * inv;
                    if (tail) {
                        const float t = p * (float)b;
                        w = w + t;
                    } else {
                        w = fmaf(p, (float)b, w);
                    }
                }
                dst[n] = w;
            }
        }
}

ORC_API void orc_relu(long n, const float *x, float *y)
{
    for (long i = 0; i < n; i++) y[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

/* ------------------------------------------------- segment-continuity ops */


/* VectorMath.SoftmaxRow (VectorMath.cs:172-204,246-287) on rows of the
 * scaled input (the Mul node runs first, so v = x * scale is rounded):
 *   max: MaxRow -- eight lanes, lane k folding v[8j + k] with Avx.Max (maxps:
 *        the later value unless the running one is greater), the lanes
 *        combined as max(max(l0,l4), max(l2,l6)) vs max(max(l1,l5), max(l3,l7))
 *        through MathF.Max, then the tail with MathF.Max; rows shorter than 8
 *        fold MathF.Max from -inf;
 *   sum: SumExp -- lane k sums e = Exp(v - max) over v[8j + k] in order; the
 *        eight lane sums are added in lane order to 0, then the tail values
 *        (MathF.Exp in the reference, its bits not pinned; exp_ref here);
 *   y = e * (1 / sum). */
static float maxps1(float a, float b) { return a > b ? a : b; }

ORC_API void orc_softmax_f32(long rows, int cols, float scale, const float *x, float *y)
{
    for (long r = 0; r < rows; r++) {
        const float *xr = x + r * cols;
        float *yr = y + r * cols;
        const int vec = cols & ~7;
        float mx = -INFINITY;
        if (cols >= 8) {
            float acc[8];
            for (int k = 0; k < 8; k++) acc[k] = xr[k] * scale;
            for (int i = 8; i <= cols - 8; i += 8)
                for (int k = 0; k < 8; k++) acc[k] = maxps1(acc[k], xr[i + k] * scale);
            float lo[4];
            for (int q = 0; q < 4; q++) lo[q] = maxps1(acc[q], acc[q + 4]);
            const float l0 = maxps1(lo[0], lo[2]), l1 = maxps1(lo[1], lo[3]);
            mx = dotnet_max(l0, l1);
            for (int i = vec; i < cols; i++) mx = dotnet_max(mx, xr[i] * scale);
        } else {
            for (int i = 0; i < cols; i++) mx = dotnet_max(mx, xr[i] * scale);
        }
        float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int i = 0; i < vec; i += 8)
            for (int k = 0; k < 8; k++) {
                const float e = exp_ref(xr[i + k] * scale - mx);
                yr[i + k] = e;
                lane[k] = lane[k] + e;
            }
        float sum = 0.0f;
        for (int k = 0; k < 8; k++) sum = sum + lane[k];
        for (int i = vec; i < cols; i++) {
            const float e = exp_ref(xr[i] * scale - mx);
            yr[i] = e;
            sum = sum + e;
        }
        const float inv = 1.0f / sum;
        for (int c = 0; c < cols; c++) yr[c] = yr[c] * inv;
    }
}

ORC_API void orc_maxpool2d_f32(int N, int C, int H, int W, int kh, int kw, int sh, int sw, int pt, int pl,
                               int OH, int OW, const float *x, float *y)
{
    for (long pl_ = 0; pl_ < (long)N * C; pl_++) {
        const float *xp = x + pl_ * H * W;
        float *yp = y + pl_ * OH * OW;
        for (int oy = 0; oy < OH; oy++)
            for (int ox = 0; ox < OW; ox++) {
                /* the scalar path of the reference (DnnOps.cs:1564-1579): start at
                 * -inf, keep v when v > best, so NaN inputs are never taken */
                float m = -INFINITY;
                for (int ky = 0; ky < kh; ky++) {
                    int iy = oy * sh - pt + ky;
                    if (iy < 0 || iy >= H) continue;
                    for (int kx = 0; kx < kw; kx++) {
                        int ix = ox * sw - pl + kx;
                        if (ix < 0 || ix >= W) continue;
                        float v = xp[(long)iy * W + ix];
                        if (v > m) m = v;
                    }
                }
                yp[(long)oy * OW + ox] = m;
            }
    }
}

ORC_API void orc_resize_nearest(int N, int C, int H, int W, int fh, int fw, const float *x, float *y)
{
    int OH = H * fh, OW = W * fw;
    for (long pl_ = 0; pl_ < (long)N * C; pl_++)
        for (int oy = 0; oy < OH; oy++)
            for (int ox = 0; ox < OW; ox++)
                y[(pl_ * OH + oy) * OW + ox] = x[(pl_ * H + oy / fh) * W + ox / fw];
}

/* ------------------------------------------------------------------ int8 DQM */

ORC_API void orc_minmax(long n, const float *x, float *mn, float *mx)
{
    float lo = 0.0f, hi = 0.0f;
    for (long i = 0; i < n; i++) {
        float v = x[i];
        if (isnan(v)) continue;
        if (v < lo) lo = v;
        if (v > hi) hi = v;
    }
    *mn = lo;
    *mx = hi;
}

ORC_API void orc_dql_params(float mn, float mx, float *scale, int *zp)
{
    float s = (mx - mn) / 255.0f;
    if (!(s > 0.0f)) s = 1.0f;
    float z = nearbyintf(-mn / s);
    int zi = (int)z;
    if (zi < 0) zi = 0;
    if (zi > 255) zi = 255;
    *scale = s;
    *zp = zi;
}

static inline float quant1(float x, float inv, float zpf)
{
    float q = nearbyintf(x * inv) + zpf;
    return fminf(255.0f, fmaxf(0.0f, q));
}

ORC_API void orc_quantize_u8(long n, const float *x, float scale, int zp, uint8_t *q)
{
    float inv = 1.0f / scale, zpf = (float)zp;
    for (long i = 0; i < n; i++) q[i] = (uint8_t)quant1(x[i], inv, zpf);
}

/* DynamicQuantizeLinear (QuantOps.cs:166-227): q, scale, zero point. */
ORC_API void orc_dynamic_quantize_linear(long n, const float *x, uint8_t *q, float *scale, int *zp)
{
    float mn, mx;
    orc_minmax(n, x, &mn, &mx);
    orc_dql_params(mn, mx, scale, zp);
    orc_quantize_u8(n, x, *scale, *zp, q);
}

static inline int wval(const void *w, int w_signed, long idx)
{
    return w_signed ? (int)((const int8_t *)w)[idx] : (int)((const uint8_t *)w)[idx];
}

typedef struct {
    int m, k, n, w_signed, n_wzp, n_wscale, fused, zp;
    const uint8_t *q;
    const void *w;
    const int *wzp;
    const float *wscale, *bias;
    float scale;
    float *out;
    int32_t *acc;
    float *acc_f32;
} dqmm_ctx;

static void dqmm_rows(void *p, long r0, long r1)
{
    dqmm_ctx *d = (dqmm_ctx *)p;
    for (long i = r0; i < r1; i++)
        for (int j = 0; j < d->n; j++) {
            int zpw = d->wzp ? (d->n_wzp == 1 ? d->wzp[0] : d->wzp[j]) : 0;
            int64_t s = 0;
            float sf = 0.0f;
            for (int t = 0; t < d->k; t++) {
                int qa = (int)d->q[i * (long)d->k + t] - d->zp;
                int qw = wval(d->w, d->w_signed, (long)t * d->n + j) - zpw;
                s += (int64_t)qa * qw;
                sf = fmaf((float)qa, (float)qw, sf);
            }
            if (d->acc) d->acc[i * (long)d->n + j] = (int32_t)s;
            if (d->acc_f32) d->acc_f32[i * (long)d->n + j] = sf;
            float ws = d->wscale ? (d->n_wscale == 1 ? d->wscale[0] : d->wscale[j]) : 1.0f;
            float comb = d->scale * ws;
            float b = d->bias ? d->bias[j] : 0.0f;
            /* The reference epilogue consumes its FP32 accumulator. */
            float acc = sf;
            d->out[i * (long)d->n + j] = d->fused ? fmaf(acc, comb, b)
                                                  : (d->bias ? acc * comb + b : acc * comb);
        }
}

/* DynamicQuantizeMatMul with inputs [A, W, w_zp, w_scale, bias]:
 *   per-tensor u8 quantization of A, (q - zp)(w - w_zp) summed (exact int64
 *   into acc_i32; the reference's FP32 fmaf chain into acc_f32), then
 *   out = fmaf(acc_f32, a_scale * w_scale[j], bias[j]) (fused=1) or the
 *   unfused tail form (fused=0).  scale/zp are returned.  */
ORC_API void orc_dqmm(int m, int k, int n, const float *a, const void *w, int w_signed, const int *wzp,
                      int n_wzp, const float *wscale, int n_wscale, const float *bias, float *out,
                      int32_t *acc_i32, float *acc_f32, int fused, float *scale_out, int *zp_out)
{
    float mn, mx, scale;
    int zp;
    orc_minmax((long)m * k, a, &mn, &mx);
    orc_dql_params(mn, mx, &scale, &zp);
    uint8_t *q = (uint8_t *)malloc((size_t)m * k);
    orc_quantize_u8((long)m * k, a, scale, zp, q);
    dqmm_ctx d = {m, k, n, w_signed, n_wzp, n_wscale, fused, zp, q, w, wzp, wscale, bias, scale,
                  out, acc_i32, acc_f32};
    parallel_for(m, dqmm_rows, &d);
    free(q);
    if (scale_out) *scale_out = scale;
    if (zp_out) *zp_out = zp;
}

/* MatMulInteger: int64 sum of (a - a_zp)(b - b_zp[col]) (Int8Gemm.MultiplyIntegerScalar). */
/* a_signed: s8 activations read as signed values (Int8F32Gemm.WidenActivation(sbyte),
 * Int8F32Gemm.cs:109-125, and the ONNX definition); u8 otherwise. */
ORC_API void orc_matmul_integer(int m, int k, int n, const void *a, int a_signed, int a_zp, const void *b,
                                int b_signed, const int *b_zp, int n_bzp, int32_t *c)
{
    for (int i = 0; i < m; i++)
        for (int j = 0; j < n; j++) {
            int zp = b_zp ? (n_bzp == 1 ? b_zp[0] : b_zp[j]) : 0;
            int64_t s = 0;
            for (int t = 0; t < k; t++)
                s += (int64_t)(wval(a, a_signed, (long)i * k + t) - a_zp) * (wval(b, b_signed, (long)t * n + j) - zp);
            c[(long)i * n + j] = (int32_t)s;
        }
}
