/*
 * osh_hip.h -- C ABI of libosh_hip.so, the MI355X (gfx950) backend for
 * OnnxSharp's dense-contraction operators: Conv (+ fused Relu/SiLU),
 * MatMul with a fused column bias, and DynamicQuantizeMatMul.
 *
 * One P/Invoke surface: device, memory, copies, streams/events, one-time
 * weight packing, operator launches and operator-level shape logic.  Plain
 * pointers and sizes only.  Every entry point returns an osh_status (0 = OK,
 * negative = error) and leaves a message for osh_last_error() on the calling
 * thread.  Launch entry points are asynchronous on the given stream (NULL =
 * the device's default stream); pointers named d_* are device memory.
 *
 * Reference citations are relative to the OnnxSharp source tree.
 */
#ifndef OSH_HIP_H
#define OSH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(_WIN32)
#define OSH_API __declspec(dllexport)
#else
#define OSH_API __attribute__((visibility("default")))
#endif

typedef int osh_status;
enum {
    OSH_OK = 0,
    OSH_E_INVALID = -1,     /* bad argument or shape (reference: OnnxSharpException) */
    OSH_E_UNSUPPORTED = -2, /* shape/attribute the backend does not take (reference: NotSupportedException;
                               an emitter refusing an op, src/OnnxSharp.Vulkan/VkOpRegistry.cs:168-180) */
    OSH_E_DEVICE = -3,      /* HIP runtime error (reference: VkDeviceLostException) */
    OSH_E_NOMEM = -4        /* device allocation failed */
};

typedef void *osh_stream; /* hipStream_t */
typedef void *osh_event;  /* hipEvent_t */

/* Fused activation of a Conv, UnaryOpKind subset that
 * GraphFusion.FuseActivationIntoProducer moves into a producer
 * (src/OnnxSharp/Core/GraphFusion.cs:1713-1718). */
enum { OSH_ACT_NONE = 0, OSH_ACT_RELU = 1, OSH_ACT_SILU = 2, OSH_ACT_SIGMOID = 3 };

/* ONNX auto_pad (src/OnnxSharp/Ops/DnnOps.cs:69-89). */
enum { OSH_PAD_NOTSET = 0, OSH_PAD_SAME_UPPER = 1, OSH_PAD_SAME_LOWER = 2, OSH_PAD_VALID = 3 };

/* ------------------------------------------------------------------ errors */

/* Message of the last failing call on this thread ("" if none). */
OSH_API const char *osh_last_error(void);

/* ------------------------------------------------------------------ device */

typedef struct osh_device_info {
    char name[64];
    char arch[32];          /* e.g. "gfx950" */
    int compute_units;
    int clock_khz;
    size_t total_mem;
    size_t lds_per_block;
} osh_device_info;

/* Select device `dev` for the calling thread and report it (info may be NULL).
 * Replaces VkDevice creation (src/OnnxSharp.Vulkan/VkDevice.cs:9-120). */
OSH_API osh_status osh_init(int dev, osh_device_info *info);
OSH_API osh_status osh_device_count(int *count);
OSH_API osh_status osh_device_synchronize(void);

/* Launch log: the kernels the calling thread launched since the last reset,
 * one "name<template arguments>" per line in launch order (the names
 * rocprofv3 prints), so a caller can tell which kernel and tile each call ran
 * after first-use tuning.  *count (may be NULL) receives the number of
 * launches; buf (may be NULL) receives the names, NUL-terminated
 * (OSH_E_INVALID if `bytes` is too small); reset != 0 clears the log
 * afterwards.  Launches recorded into a graph are logged when recorded, not
 * when replayed.  The per-op kernel names of the reference's profiler
 * (Net.ProfileAll, src/OnnxSharp/Core/Net.cs:282-332) are its counterpart. */
OSH_API osh_status osh_kernel_log(int reset, char *buf, size_t bytes, int *count);

/* Backend options (the reference reads its kernel switches from ONNXSHARP_*
 * environment variables, e.g. src/OnnxSharp/Kernels/NchwcConv.cs:39-40).
 *   "exact_silu": 0 (default) = fused SiLU epilogues use exp2/rcp (relative
 *                 difference to the reference polynomial < 2e-6);
 *                 1 = the reference polynomial and IEEE division bit for bit
 *                 (src/OnnxSharp/Tensors/VectorMath.cs:21-77).  Initial value
 *                 from ONNXSHARP_HIP_EXACT_SILU.
 *   "gemm_variant": -1 (default) = dense GEMMs (MatMul, 1x1 conv) pick their
 *                 wave tile from the problem size; 0..N-1 forces one tile
 *                 where the operands allow it (tuning and tests); -2 = always
 *                 use the LDS-staged GEMM tile.  Every choice sums k in the
 *                 same order.  Initial value from ONNXSHARP_HIP_GEMM_VARIANT.
 *   "gemm_variants" (get only): N, the number of wave tiles.
 *   "conv16_variant": -1 (default) = 3x3 convolutions that pass the
 *                 reference's NCHWc gate (stride 1 or 2, pad 1, C % 16 == 0,
 *                 M % 32 == 0, batch 1; NchwcConv.cs:100-126) run the in-order
 *                 16x16x4 MFMA kernel (the reference's NCHWc chain, bit for
 *                 bit) with a wave tile picked per shape; 0..N-1 forces a tile
 *                 on any 3x3 shape with C % 16 == 0 it fits (6..11:
 *                 weights held in LDS; 12..22: input patch staged in LDS
 *                 and shared by a workgroup's four waves, stride 1 or 2;
 *                 23..26: tiles 0, 3, 1, 4 with one wave per workgroup;
 *                 27..N-1: XCD-banded 16-column tiles, TM x BV = 1x2, 1x4,
 *                 2x2, 1x7, 1x8).
 *                 Initial value from ONNXSHARP_HIP_CONV16_VARIANT.
 *   "conv16_variants" (get only): N, the number of 3x3 tiles.
 *   "pointwise_variant": -1 (default) = 1x1 stride-1 convolutions with
 *                 C % 16 == 0 pick, by the same first-use timing, between the
 *                 GEMM tile over raw weights (0) and the LDS-tile kernel's
 *                 tiles (1..N-1); all sum in the GEMM chain's order.  -2 = the
 *                 GEMM path only.  Initial value from
 *                 ONNXSHARP_HIP_POINTWISE_VARIANT.
 *   "group3x3_tile": -1 (default) = grouped 3x3 launches
 *                 (osh_conv2d_group_f32) pick their tile by first-use timing
 *                 of the whole group; 0..N-1 forces a tile: with T
 *                 LDS-patch tiles, 0..T-1 those, T..2T-1 the same with one
 *                 workgroup per CU (a long member's chain keeps its SIMDs),
 *                 2T..N-1 the streamed one-block tiles; all give the same
 *                 bits.
 *   "group3x3_tiles" (get only): N.
 *   "group_pointwise_tile", "group_pointwise_tiles": the same for grouped
 *                 pointwise launches (the pointwise LDS tiles that fit every
 *                 member; a forced tile that does not fit takes the default).
 *   "pair_tile", "pair_tiles": the same for osh_conv2d_pair_f32: its
 *                 output tiles (bottleneck pairs 4x4, 4x8, 8x8, 2x2;
 *                 8-channel pairs 4x16, 8x16, 2x32, 2x16; first-layer pairs
 *                 4x16, 2x32, 2x16, 2x8), then N-1 = the two convs as
 *                 separate launches (only with an intermediate buffer).
 *   "pointwise_variants" (get only): N.
 *                 The -2 setting of "pointwise_variant" changes the packed
 *                 weight layout: pack again after changing it.
 *   Environment: ONNXSHARP_HIP_TUNE_DB=<path> keeps the first-use tile
 *                 choices in a text file: read on first use, each new choice
 *                 appended, so later processes choose the same tiles without
 *                 timing them.
 *   "dqmm_variant": 0 (default) = osh_dqmm_u8s8 runs a min/max launch and
 *                 then one launch that quantizes A and multiplies (on 16x16
 *                 tiles whose epilogue overlaps the MFMAs where every tile is
 *                 full); 1 = min/max, quantize and GEMM as three launches;
 *                 2 = as 0 with 32x32 tiles for full tiles.  All give
 *                 identical outputs.  Initial value from
 *                 ONNXSHARP_HIP_DQMM_VARIANT.
 *   "dqmm_launches" (get only): kernel launches (2 or 3) of the calling
 *                 thread's last osh_dqmm_u8s8 / osh_dqmm_u8s8_noalloc call.
 *   "im2col3x3_variant": -1 (default) = 3x3 stride-1/2 convolutions with
 *                 C % 16 == 0 that neither the NCHWc nor the Winograd gate
 *                 takes run in the reference's im2col order
 *                 (ConvKernels.cs:554-563) on the LDS-patch tiles or the
 *                 streamed one-block tiles (the last four ids), tile picked
 *                 by first-use timing; 0..N-1 forces a tile.  Initial value from
 *                 ONNXSHARP_HIP_IM2COL3X3_VARIANT.
 *   "im2col3x3_variants" (get only): N.
 *   "winograd": 1 (default) = 3x3 stride-1 convolutions that pass the
 *                 reference's Winograd gate (Winograd.TryConv3x3,
 *                 src/OnnxSharp/Kernels/Winograd.cs:58-122) but not its NCHWc
 *                 gate (NchwcConv.cs:100-126) run Winograd F(2x2,3x3) in the
 *                 reference's arithmetic -- the reference's own choice on an
 *                 AVX-512 host; 2 = Winograd for every shape that passes its
 *                 gate, ahead of the NCHWc kernels; 0 = never (those shapes
 *                 take the im2col chain).  Initial value from
 *                 ONNXSHARP_HIP_WINOGRAD.  Changes the packed weight layout:
 *                 pack again after changing it.
 *   "winograd_max_pixels": the largest output map (H*W) Winograd takes;
 *                 initial value from the reference's ONNXSHARP_WINO_MAX, else
 *                 4096.  Also changes the packed layout.
 *   "nchwc": 1 (default) = the reference host runs its NCHWc 3x3 kernel (an
 *                 AVX-512 host, NchwcConv.Enabled && IsSupported,
 *                 src/OnnxSharp/Kernels/NchwcConv.cs:38-43), so the shapes its
 *                 gate takes sum in the NCHWc chain; 0 = it does not (an
 *                 AVX2-only host, or ONNXSHARP_NCHWC=0): those shapes take
 *                 what ConvLayer.Forward falls back to (DnnOps.cs:475-482):
 *                 Winograd where its gate holds, else the panel / im2col
 *                 chain.  Initial value from the reference's own
 *                 ONNXSHARP_NCHWC (anything but "0" is on).  Changes the
 *                 packed weight layout: pack again after changing it.
 *   "tune": 1 (default) = the first launch of a 3x3 conv shape on a stream
 *                 that is not capturing times every conv16 tile (they all give
 *                 identical outputs) and keeps the fastest for that shape;
 *                 0 = pick tiles by the cost model only.  Initial value from
 *                 ONNXSHARP_HIP_TUNE. */
OSH_API osh_status osh_config_set(const char *key, int value);
OSH_API osh_status osh_config_get(const char *key, int *value);

/* ------------------------------------------------------------------ memory */

/* Device buffers: the C# side pools them by (kind, bytes) as VkBufferPool does
 * (src/OnnxSharp.Vulkan/VkBufferPool.cs:20-190). */
OSH_API osh_status osh_malloc(void **d_ptr, size_t bytes);
OSH_API osh_status osh_free(void *d_ptr);
/* Pinned host staging (hipHostMalloc; replaces VkSegment staging buffers,
 * src/OnnxSharp.Vulkan/VkSegment.cs:370,462). */
OSH_API osh_status osh_host_alloc(void **h_ptr, size_t bytes);
OSH_API osh_status osh_host_free(void *h_ptr);

/* ------------------------------------------------------------------ copies */

OSH_API osh_status osh_memcpy_h2d(void *d_dst, const void *h_src, size_t bytes, osh_stream s);
OSH_API osh_status osh_memcpy_d2h(void *h_dst, const void *d_src, size_t bytes, osh_stream s);
OSH_API osh_status osh_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes, osh_stream s);
/* Byte fill by a kernel (safe inside captured graphs). */
OSH_API osh_status osh_memset_d8(void *d_dst, int value, size_t bytes, osh_stream s);

/* --------------------------------------------------------- streams / events */

OSH_API osh_status osh_stream_create(osh_stream *s);
OSH_API osh_status osh_stream_destroy(osh_stream s);
/* One sync per segment, as VkSegment.Execute waits one fence
 * (src/OnnxSharp.Vulkan/VkSegment.cs:598-599). */
OSH_API osh_status osh_stream_sync(osh_stream s);
OSH_API osh_status osh_event_create(osh_event *e);
OSH_API osh_status osh_event_destroy(osh_event e);
OSH_API osh_status osh_event_record(osh_event e, osh_stream s);
OSH_API osh_status osh_event_elapsed_ms(osh_event start, osh_event stop, float *ms);
/* Make stream s wait for the work recorded in event e before its later work
 * (fork/join between the streams of one segment; captured into a graph as a
 * dependency edge). */
OSH_API osh_status osh_stream_wait_event(osh_stream s, osh_event e);

/* ------------------------------------------------------------ Conv (A1-A8) */

/* Conv attributes as ConvLayer reads them (src/OnnxSharp/Ops/DnnOps.cs:116-132):
 * an absent list has n_* = 0. */
typedef struct osh_conv_attrs {
    int group;
    int auto_pad;            /* OSH_PAD_* */
    int n_kernel_shape, kernel_shape[2];
    int n_strides, strides[2];
    int n_pads, pads[4];
    int n_dilations, dilations[2];
} osh_conv_attrs;

/* Resolved 2-D conv launch (the fields of Conv2DParams,
 * src/OnnxSharp.Vulkan/VkConv.cs:24-51). */
typedef struct osh_conv_params {
    int n, c, h, w;          /* input NCHW */
    int m, kh, kw, group;    /* weight OIHW: [m, c/group, kh, kw] */
    int sh, sw, dh, dw;      /* strides, dilations */
    int pt, pl, pb, pr;      /* pads (top, left, bottom, right) */
    int oh, ow;              /* output spatial size */
} osh_conv_params;

/* ConvLayer.GetMemoryShapes (src/OnnxSharp/Ops/DnnOps.cs:134-201): output
 * dims of a 4-D (NCHW) input.  Keeps the reference's rule that the shape uses
 * the begin pad as the end pad unless more than 2*spatial pads are given. */
OSH_API osh_status osh_conv_infer_shape(const osh_conv_attrs *attrs, const int64_t x_dims[4],
                                        const int64_t w_dims[4], int64_t y_dims[4]);

/* ConvLayer.Resolve + output shape (src/OnnxSharp/Ops/DnnOps.cs:379-409). */
OSH_API osh_status osh_conv_resolve(const osh_conv_attrs *attrs, const int64_t x_dims[4],
                                    const int64_t w_dims[4], osh_conv_params *out);

/* Bytes of the packed weight buffer osh_conv_pack_weights writes for p. */
OSH_API osh_status osh_conv_packed_weight_bytes(const osh_conv_params *p, size_t *bytes);

/* One-time weight packing on the device (replaces NchwcConv.PackWeights,
 * src/OnnxSharp/Kernels/NchwcConv.cs:247-274, and PackedConv.PackWeights,
 * src/OnnxSharp/Kernels/PackedConv.cs:155-182).  d_w is OIHW f32. */
OSH_API osh_status osh_conv_pack_weights(const osh_conv_params *p, const float *d_w, void *d_packed,
                                         osh_stream s);

/* The library remembers which kernel and shape each packed buffer was laid out
 * for and refuses a launch with a mismatching one.  A caller that releases or
 * reuses memory it allocated itself (not through osh_malloc, whose osh_free
 * does this) calls osh_conv_forget_pack on the range so that the record does
 * not outlive the buffer.  No counterpart in the reference (its packed weights
 * are managed objects). */
OSH_API osh_status osh_conv_forget_pack(const void *d_packed, size_t bytes);

/* Conv forward, NCHW f32 in and out, bias (length m) optional, fused
 * activation act (ConvLayer.Forward, src/OnnxSharp/Ops/DnnOps.cs:411-500).
 * d_wpacked is the output of osh_conv_pack_weights for the same p.  The
 * output must not overlap the input (OSH_E_INVALID). */
OSH_API osh_status osh_conv2d_f32(const osh_conv_params *p, const float *d_x, const void *d_wpacked,
                                  const float *d_bias, int act, float *d_y, osh_stream s);

/* Conv followed by a residual Add in one launch: y = act(conv(x) + bias) + res,
 * res laid out as y (NCHW [n, m, oh, ow]) and not overlapping it.  This is the
 * ONNX pair Conv(+fused activation) -> Add(shortcut, conv output) of a
 * bottleneck block (ConvLayer.Forward, src/OnnxSharp/Ops/DnnOps.cs:411-500,
 * then the same-shape Add of NaryEltwiseLayer.Forward, src/OnnxSharp/Ops/NaryEltwiseLayer.cs:41),
 * with the same two roundings: the activation output, then the sum. */
OSH_API osh_status osh_conv2d_add_f32(const osh_conv_params *p, const float *d_x, const void *d_wpacked,
                                      const float *d_bias, int act, const float *d_res, float *d_y,
                                      osh_stream s);

/* Up to 6 independent convs in one launch: conv i is ps[i] on d_xs[i] with
 * packed weights d_ws[i], bias d_biases[i] (d_biases may be NULL), residual
 * d_res[i] (d_res may be NULL), output d_ys[i]; one fused activation for all.
 * No single reference function: it stands for that many ConvLayer.Forward
 * calls (src/OnnxSharp/Ops/DnnOps.cs:411-500) of layers that do not depend on
 * each other, e.g. the detection head's three scales.  Outputs are those of
 * separate osh_conv2d_f32 / osh_conv2d_add_f32 calls, bit for bit.  Convs
 * that share a kernel family the grouped kernels cover (NCHWc-chain 3x3 of
 * one stride, pointwise, depthwise) run as one launch; other groups run one
 * launch per conv. */
OSH_API osh_status osh_conv2d_group_f32(int count, const osh_conv_params *ps, const float *const *d_xs,
                                        const void *const *d_ws, const float *const *d_biases, int act,
                                        const float *const *d_res, float *const *d_ys, osh_stream s);

/* Two chained 3x3 convs in one launch: pb reads pa's output, as a
 * bottleneck's cv1 -> cv2 (two Conv nodes the reference runs one after the
 * other through ConvLayer.Forward, src/OnnxSharp/Ops/DnnOps.cs:411-500; the
 * C3k2 / C3k blocks of YOLO11n).  d_wa / d_wb are each conv's weights packed
 * by osh_conv_pack_weights; the result is that of osh_conv2d_f32(pa) into
 * d_ya followed by osh_conv2d_f32 / osh_conv2d_add_f32(pb) into d_y (with the
 * residual d_res, which may be NULL), bit for bit: each conv
 * keeps its chain, and the intermediate stays on chip (it is still written to
 * d_ya unless d_ya is NULL).  First-use timing chooses between the fused
 * kernel's tiles and, when d_ya is given, two separate launches, whichever
 * is faster for the shapes.  Takes two kinds of pair of SiLU convs, batch 1,
 * in the chain orders the single-conv dispatch takes for them:
 *   - bottleneck pairs: 3x3 stride-1 pad-1 convs on one 1 x C x H x W map,
 *     C = 16 / 32 / 48 / 64, 16 / 32 / 64 output channels each, or
 *     16 -> 8 -> 16 (an 8-channel intermediate: the im2col chain, then the
 *     first-layer chain);
 *   - first-layer pairs: a 3x3 stride-1 or -2 conv over C <= 4 planes with
 *     16 outputs (the first_conv chain; a network's first layer, e.g.
 *     YOLO11n's 3 -> 16 stem, FirstConv.cs), then a 3x3 pad-1 conv of stride
 *     1 or 2 over its output with 32 or 64 outputs (the NCHWc chain).
 * Anything else returns OSH_E_UNSUPPORTED (run the two convs separately).
 * No output may overlap d_x or the other output, and the residual may not
 * overlap d_y. */
OSH_API osh_status osh_conv2d_pair_f32(const osh_conv_params *pa, const osh_conv_params *pb, const float *d_x,
                                       const void *d_wa, const float *d_bias_a, const void *d_wb,
                                       const float *d_bias_b, int act, const float *d_res, float *d_ya, float *d_y,
                                       osh_stream s);

/* OSH_OK if osh_conv2d_pair_f32 takes (pa, pb, act), else OSH_E_UNSUPPORTED
 * with the reason in osh_last_error(). */
OSH_API osh_status osh_conv2d_pair_check(const osh_conv_params *pa, const osh_conv_params *pb, int act);

/* ------------------------------------------------- MatMul + bias (A9, A10) */

/* C[m,n] (row stride ldc) = A[m,k] (lda) * B[k,n] (ldb)
 *   + col_bias[j] (MatMulLayer's FusedBias, src/OnnxSharp/Ops/DnnOps.cs:2817,3009-3022)
 *   or + row_bias[i] (Conv-style per-row bias, GemmKernel.Multiply's `bias`),
 * column bias taking precedence as in GemmKernel.cs:1113-1152; then act.
 * With col_scale: C = col_scale[j] * (A*B) + col_bias[j] in one fmaf
 * (GemmKernel.cs:1210-1241).  Any pointer except A, B, C may be NULL.
 * Replaces GemmKernel.Multiply / MultiplyPacked
 * (src/OnnxSharp/Tensors/GemmKernel.cs:131-269,675-852). */
OSH_API osh_status osh_gemm_f32(int m, int n, int k, const float *d_a, int lda, const float *d_b, int ldb,
                                const float *d_col_bias, const float *d_row_bias, const float *d_col_scale,
                                int act, float *d_c, int ldc, osh_stream s);

/* Batched form of the same (MatMulLayer broadcast with per-batch strides,
 * GemmKernel.MultiplyBatched, src/OnnxSharp/Tensors/GemmKernel.cs:284-405);
 * stride 0 broadcasts an operand. */
OSH_API osh_status osh_gemm_f32_batched(int batch, int m, int n, int k, const float *d_a, int lda,
                                        int64_t stride_a, const float *d_b, int ldb, int64_t stride_b,
                                        const float *d_col_bias, int act, float *d_c, int ldc,
                                        int64_t stride_c, osh_stream s);

/* MatMulLayer.GetMemoryShapes numpy broadcast (src/OnnxSharp/Ops/DnnOps.cs:2789-2900):
 * output dims of A (rank ra) x B (rank rb); returns the output rank in *ry. */
OSH_API osh_status osh_matmul_infer_shape(const int64_t *a_dims, int ra, const int64_t *b_dims, int rb,
                                          int64_t *y_dims, int *ry);

/* ONNX Gemm (GemmLayer, src/OnnxSharp/Ops/AttnOps.cs:31-135):
 *   Y[m,n] = alpha * (A' B') + beta * C,   A' = transA ? A^T : A, B' = transB ? B^T : B
 * with A stored [m,k] ([k,m] if trans_a), B [k,n] ([n,k] if trans_b), dense rows.
 * As in the reference: the transposes are materialized (into d_workspace,
 * osh_gemm_ex_workspace_bytes), the product is the FMA chain from 0, then
 * each element takes alpha * y (if alpha != 1) and + beta * c (if beta != 0 and
 * C is given), each rounded on its own.  C has c_len elements: m*n (full),
 * 1 (scalar) or any other length, indexed by column j % c_len. */
OSH_API osh_status osh_gemm_ex_workspace_bytes(int trans_a, int trans_b, int m, int n, int k, size_t *bytes);
OSH_API osh_status osh_gemm_ex_f32(int trans_a, int trans_b, int m, int n, int k, float alpha, const float *d_a,
                                   const float *d_b, float beta, const float *d_c, int64_t c_len, float *d_y,
                                   void *d_workspace, osh_stream s);

/* ------------------------------------------------ pointwise conv chains */

/* A chain of convolutions over the same H x W map run as one launch, each
 * workgroup taking 16 consecutive pixels through every stage: stage k is a
 * 1x1 conv (stride 1, no pads, group 1) whose input channels are the concat,
 * in order, of up to OSH_PW_MAX_SRC parts -- tensors in memory or outputs of
 * earlier stages -- or, as stage 0 only, a 3x3 depthwise conv (stride 1,
 * pad 1).  Every stage computes exactly what osh_conv2d_f32 / osh_conv2d_add_f32
 * compute for it (same chain, activation, residual), writes its whole output
 * to y, and keeps its pixels on chip for the later stages, so a chain gives
 * the bits of its convs launched one after another with one launch instead
 * of several.  This is a launch fusion with no counterpart in the reference,
 * for the frame executor (OnnxSharp's graph keeps the nodes; the backend
 * fuses their launches).
 *
 * Conditions (OSH_E_INVALID otherwise): batch 1; a 1x1 stage's weights packed
 * by osh_conv_pack_weights for that conv (the pointwise LDS-tile layout, so
 * C % 16 == 0), m % 16 == 0 and every part's channel count a multiple of 16;
 * a depthwise stage's weights are the raw [m][1][3][3] of a conv with m == c;
 * every y non-NULL; no y overlaps another y.  A workgroup reads everything it
 * reads from memory before any stage writes, and a 1x1 stage reads and
 * writes only its own 16 pixels, so within one chain a stage's y may overlap
 * a tensor the same or an earlier stage reads from memory (at whole channel
 * planes: e.g. writing over the shortcut a previous stage added); any other
 * overlap of a y with a tensor the launch reads -- another chain's, a later
 * stage's, a depthwise stage's input -- is refused.  OSH_E_UNSUPPORTED: H*W
 * not a multiple of 4, a 1x1 stage of more than 512 channels, a part in
 * memory of more than 512 channels, a depthwise stage of more than 256, more
 * than 8 tensors a chain reads from memory, or a chain whose 1x1 weights,
 * staged tensors and kept outputs exceed 160 KB of LDS. */
#define OSH_PW_MAX_SRC 3
#define OSH_PW_MAX_STAGES 5
#define OSH_PW_MAX_CHAINS 3
enum { OSH_PW_1X1 = 0, OSH_PW_DW3X3 = 1 };

typedef struct {
    int kind;                             /* OSH_PW_1X1 or OSH_PW_DW3X3 */
    int m;                                /* output channels */
    int act;                              /* OSH_ACT_NONE / RELU / SILU */
    int nsrc;                             /* input parts, concat order */
    int src_stage[OSH_PW_MAX_SRC];        /* -1: the tensor src[i]; k >= 0: stage k's output */
    const float *src[OSH_PW_MAX_SRC];     /* [c_i, H, W] when src_stage[i] == -1; for k >= 0 NULL (the
                                             whole output) or a pointer into stage k's y at a channel */
    int src_c[OSH_PW_MAX_SRC];            /* channels of part i */
    const void *w;                        /* packed weights (1x1) or raw [m][1][3][3] (depthwise) */
    const float *bias;                    /* [m] or NULL */
    int res_stage;                        /* -1: res (may be NULL); k >= 0: stage k's output */
    const float *res;                     /* [m, H, W] added after the activation */
    float *y;                             /* [m, H, W] */
} osh_pw_stage;

typedef struct {
    int h, w;                             /* map size (batch 1) */
    int nstages;
    osh_pw_stage stage[OSH_PW_MAX_STAGES];
} osh_pw_chain;

/* Runs `count` independent chains (1..OSH_PW_MAX_CHAINS) in one launch. */
OSH_API osh_status osh_pw_chain_f32(int count, const osh_pw_chain *chains, osh_stream s);

/* ------------------------------------------- DynamicQuantizeMatMul (A13-A15) */

/* Bytes of the packed int8 weight buffer and of the scratch buffer that
 * osh_dqmm_u8s8 needs for (m, k, n). */
OSH_API osh_status osh_dqmm_packed_weight_bytes(int k, int n, size_t *bytes);
OSH_API osh_status osh_dqmm_scratch_bytes(int m, int k, size_t *bytes);

/* One-time packing of W [k,n] (int8 when w_signed, else uint8) and its zero
 * point(s) (n_wzp = 0: none, 1: per-tensor, n: per-column) into the
 * MFMA-ready layout, with per-column sums and zero-point offsets.  A zero
 * point has the weights' element type: OSH_E_INVALID outside [-128, 127]
 * (int8) or [0, 255] (uint8).  OSH_E_UNSUPPORTED when k * 255 * 255 exceeds
 * INT32_MAX (the int32 accumulator could overflow).
 * (Int8F32Gemm.WidenWeights + GemmKernel.Pack,
 * src/OnnxSharp/Ops/QuantizedMatMulOps.cs:261-277.) */
OSH_API osh_status osh_dqmm_pack_weights(int k, int n, const void *d_w, int w_signed, const int32_t *h_wzp,
                                         int n_wzp, void *d_packed, osh_stream s);

/* DynamicQuantizeMatMulLayer.Forward (src/OnnxSharp/Ops/QuantizedMatMulOps.cs:115-201):
 *   per-tensor u8 quantization of A [m,k] (min/max including 0, NaN skipped;
 *   scale = (max-min)/255, zp = clamp(rne(-min/scale)); q = clamp(rne(x*(1/scale))+zp)),
 *   int32 accumulation of (q - zp)(w - w_zp), then
 *   out[i,j] = fmaf(acc, scale * w_scale[j], bias[j]).
 * w_scale has n_wscale = 1 or n entries; bias may be NULL; d_acc (m*n int32)
 * may be NULL, else receives the exact accumulators; d_qparams (may be NULL)
 * receives {scale as float bits, zp}.  d_scratch has osh_dqmm_scratch_bytes. */
OSH_API osh_status osh_dqmm_u8s8(int m, int k, int n, const float *d_a, const void *d_wpacked,
                                 const float *d_wscale, int n_wscale, const float *d_bias, float *d_out,
                                 int32_t *d_acc, int32_t *d_qparams, void *d_scratch, osh_stream s);

/* osh_dqmm_u8s8 for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): no
 * counterpart in the reference.  Same arguments, results and kernels as
 * osh_dqmm_u8s8, minus d_scratch: the scratch is a static 4 MiB array in the
 * library, one per GPU, held until the process ends, so the call allocates
 * nothing.  Sizes whose osh_dqmm_scratch_bytes(m, k) exceeds 4 MiB
 * (e.g. m = k = 2048) fail with OSH_E_UNSUPPORTED.  Every call on one GPU
 * shares that GPU's array: calls that overlap in time on one GPU (on
 * different streams or host threads) race and must not be issued. */
OSH_API osh_status osh_dqmm_u8s8_noalloc(int m, int k, int n, const float *d_a, const void *d_wpacked,
                                         const float *d_wscale, int n_wscale, const float *d_bias, float *d_out,
                                         int32_t *d_acc, int32_t *d_qparams, osh_stream s);

/* DynamicQuantizeLinear (src/OnnxSharp/Ops/QuantOps.cs:166-227) on the device:
 * q (u8, n values), scale and zero point into d_qparams {scale bits, zp}. */
/* MatMulInteger (MatMulIntegerLayer, src/OnnxSharp/Ops/QuantOps.cs:235-428):
 *   C[i,j] = sum_k (a[i,k] - a_zp) * (w[k,j] - w_zp[j])   exactly, int32
 * A is u8 (a_signed = 0) or s8 [m,k] (s8 read as signed values, as the
 * reference's widening path does, Int8F32Gemm.cs:109-125; its VNNI path reads
 * the same bytes as u8); W packed by osh_dqmm_pack_weights (u8/s8, per-column
 * zero points); d_scratch has osh_dqmm_scratch_bytes(m, k). */
OSH_API osh_status osh_matmul_integer(int m, int k, int n, const void *d_a, int a_signed, int a_zp,
                                      const void *d_wpacked, int32_t *d_c, void *d_scratch, osh_stream s);

OSH_API osh_status osh_dynamic_quantize_linear(int64_t n, const float *d_x, uint8_t *d_q, int32_t *d_qparams,
                                               void *d_scratch, osh_stream s);

/* ------------------------------------------------------ elementwise helpers */

/* Activation pass, d_y may equal d_x (TensorOps.ElementWiseUnary,
 * src/OnnxSharp/Tensors/TensorOps.cs:267-300): Relu, SiLU and Sigmoid in the
 * reference's vector-path arithmetic (VectorMath.Silu / Sigmoid,
 * src/OnnxSharp/Tensors/VectorMath.cs:21-77).  OSH_ACT_SIGMOID is taken here
 * only, not as a fused conv/GEMM epilogue (the reference fuses Relu and SiLU). */
OSH_API osh_status osh_activation_f32(int64_t n, const float *d_x, int act, float *d_y, osh_stream s);

/* DflSoftmax, the Detect head's distribution decode (DflLayer.Forward,
 * src/OnnxSharp/Ops/DflOps.cs:97-240): x [batches][sides * bins][pixels] ->
 * y [batches][sides][pixels], y = sum over b of softmax_b(x[side*bins + b]) * b,
 * in the reference's arithmetic: the max over bins, exp by the reference
 * polynomial of (x - max), the sum in bin order, inv = 1 / sum, then
 * fma(e_b * inv, b, acc) from 0 in bin order.  The reference processes 256
 * columns at a time, 8 per vector; the last (width % 8) columns of each
 * 256-column block take its scalar lines, which are restated too.  Batch i
 * reads d_x + i * x_batch_stride and writes d_y + i * y_batch_stride
 * (elements), so x may be the first sides*bins channels of a head tensor. */
OSH_API osh_status osh_dfl_f32(int batches, int sides, int bins, int pixels, const float *d_x,
                               int64_t x_batch_stride, float *d_y, int64_t y_batch_stride, osh_stream s);

/* ------------------------------------------ segment-continuity ops (NCHW) */
/* These keep a run of convolutions on the device between the ops a segment
 * would otherwise hand back to the CPU.  Concat and Split along channels of a
 * batch-1 NCHW tensor need no kernel: producers write into, and consumers read
 * from, channel slices (pointer offsets) of one buffer (ConcatLayer
 * src/OnnxSharp/Ops/ShapeOps.cs:211, SplitLayer :302). */

/* y = a + b elementwise, same shape (NaryEltwiseLayer Add,
 * src/OnnxSharp/Ops/NaryEltwiseLayer.cs:7-20).  y may alias a or b. */
OSH_API osh_status osh_add_f32(int64_t n, const float *d_a, const float *d_b, float *d_y, osh_stream s);

typedef struct osh_pool_params {
    int n, c, h, w;     /* input */
    int kh, kw, sh, sw; /* window and strides */
    int pt, pl;         /* leading pads (positions outside the input are skipped) */
    int oh, ow;         /* output */
} osh_pool_params;

/* MaxPool 2-D over NCHW (MaxPoolLayer, src/OnnxSharp/Ops/DnnOps.cs:1335-1480):
 * y[n][c][oy][ox] = max over the window rows oy*sh - pt + ky, columns
 * ox*sw - pl + kx that fall inside the input. */
OSH_API osh_status osh_maxpool2d_f32(const osh_pool_params *p, const float *d_x, float *d_y, osh_stream s);

/* The SPPF block's three chained MaxPools (k x k, stride 1, pad k/2; k = 3, 5
 * or 7) in one launch: y1 = pool(x), y2 = pool(y1), y3 = pool(y2), each the
 * same result as osh_maxpool2d_f32 (MaxPoolLayer, DnnOps.cs:1335-1480) applied
 * in turn.  All tensors are [n, c, h, w] planes; x_batch_stride and
 * y_batch_stride (elements) step between images, so the outputs may be
 * channel slices of one concat buffer.  The outputs must not overlap x. */
OSH_API osh_status osh_maxpool_chain3_f32(int n, int c, int h, int w, int k, const float *d_x,
                                          int64_t x_batch_stride, float *d_y1, float *d_y2, float *d_y3,
                                          int64_t y_batch_stride, osh_stream s);

/* Nearest-neighbour upsampling by integer factors (ResizeLayer mode "nearest",
 * src/OnnxSharp/Ops/DnnOps.cs:2215-2330): y[n][c][oy][ox] = x[n][c][oy/fh][ox/fw],
 * the index both "asymmetric"/"floor" and "half_pixel"/"round_prefer_floor"
 * give for an integer factor.  Output plane n starts at d_y + n * y_batch_stride
 * (c*oh*ow for a dense output; larger to write into a channel slice). */
OSH_API osh_status osh_resize_nearest_f32(int n, int c, int h, int w, int fh, int fw, const float *d_x, float *d_y,
                                          int64_t y_batch_stride, osh_stream s);

/* Swap the last two axes: y[b][j][i] = x[b][i][j] for x [batch][rows][cols]
 * (TransposeLayer with perm (..., -1, -2), src/OnnxSharp/Ops/ShapeOps.cs:394).
 * Batch b reads d_x + b * x_batch_stride and writes d_y + b * y_batch_stride. */
OSH_API osh_status osh_transpose_f32(int batch, int rows, int cols, const float *d_x, int64_t x_batch_stride,
                                     float *d_y, int64_t y_batch_stride, osh_stream s);

/* Softmax along rows of x [rows][cols] after a constant scale (the Mul that
 * precedes it in attention): y = e / sum(e), e = exp(scale*x - max(scale*x))
 * (SoftmaxLayer + VectorMath.SoftmaxRow, src/OnnxSharp/Ops/DnnOps.cs:2547-2675,
 * src/OnnxSharp/Tensors/VectorMath.cs:282-287; exp is the reference polynomial). */
OSH_API osh_status osh_softmax_f32(int64_t rows, int cols, float scale, const float *d_x, float *d_y, osh_stream s);

/* The attention core of a YOLO11n C2PSA block in one launch, equal bit for bit
 * to the node sequence the reference runs for it (its attention fusion,
 * src/OnnxSharp/Core/GraphFusion.cs:950-1150, does not match this form):
 * MatMul(Transpose(q), k) -> Mul(scale) -> Softmax(-1) -> MatMul(v, Transpose(P))
 * (MatMulLayer src/OnnxSharp/Ops/DnnOps.cs:2789, SoftmaxLayer DnnOps.cs:2547-2675).
 * Head h reads q = rows [0, key_dim), k = rows [key_dim, 2 key_dim) and
 * v = rows [2 key_dim, 2 key_dim + head_dim) of n values at
 * d_qkv + h * head_stride and writes y[h][c][i] (head_dim x n per head, dense).
 * Needs key_dim % 4 == 0, key_dim <= 64, head_dim % 16 == 0, n % 16 == 0 and n <= 480
 * (OSH_E_UNSUPPORTED otherwise: run the five-launch sequence); y must not
 * overlap qkv. */
OSH_API osh_status osh_attention_f32(int heads, int key_dim, int head_dim, int n, float scale, const float *d_qkv,
                                     int64_t head_stride, float *d_y, osh_stream s);

/* ----------------------------------------------------------- HIP graphs */
/* A segment's launches recorded once and replayed per Forward, the role of
 * the Vulkan backend's recorded command buffers (src/OnnxSharp.Vulkan/VkSegment.cs:324-600).
 * Capture runs on a stream from osh_stream_create (not the legacy default
 * stream); nothing may allocate or memset on it while capturing. */
typedef void *osh_graph; /* hipGraphExec_t */
OSH_API osh_status osh_graph_begin(osh_stream s);
OSH_API osh_status osh_graph_end(osh_stream s, osh_graph *g);
OSH_API osh_status osh_graph_launch(osh_graph g, osh_stream s);
OSH_API osh_status osh_graph_destroy(osh_graph g);

/* Building a graph whose nodes run concurrently where the segment's data
 * allows: each op is captured on its own (osh_graph_begin on a stream, the op's
 * launches, then osh_graph_add_captured), becomes one child-graph node, and
 * depends on the nodes listed in deps.  osh_graph_instantiate turns the
 * builder into a launchable osh_graph; the builder is destroyed separately. */
typedef void *osh_graph_builder; /* hipGraph_t */
typedef void *osh_graph_node;    /* hipGraphNode_t */
OSH_API osh_status osh_graph_builder_create(osh_graph_builder *b);
OSH_API osh_status osh_graph_add_captured(osh_graph_builder b, osh_stream s, const osh_graph_node *deps, int ndeps,
                                          osh_graph_node *node);
/* As osh_graph_add_captured, but the captured launches (a serial chain of
 * kernels) are added to the builder as kernel nodes of their own, in order,
 * the first one depending on deps; *first and *last receive the chain's ends
 * (a dependent segment lists *last).  No child graph: the builder is one flat
 * DAG of kernel nodes.  OSH_E_UNSUPPORTED (nothing added) when the capture
 * holds anything but a chain of kernel launches. */
OSH_API osh_status osh_graph_add_captured_flat(osh_graph_builder b, osh_stream s, const osh_graph_node *deps,
                                               int ndeps, osh_graph_node *first, osh_graph_node *last);
OSH_API osh_status osh_graph_instantiate(osh_graph_builder b, osh_graph *g);
OSH_API osh_status osh_graph_builder_destroy(osh_graph_builder b);

#ifdef __cplusplus
}
#endif

#endif /* OSH_HIP_H */
