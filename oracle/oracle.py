"""numpy front end of the CPU oracle (oracle/osh_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the thing
measured or shipped.  Each function names the reference routine it restates
(paths relative to the OnnxSharp source tree).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "liboracle.so")
_lib = None

ORDER_IM2COL = 0  # ic -> ky -> kx (ConvKernels.Im2Col / PackedConv / Pointwise / FirstConv)
ORDER_NCHWC = 1  # icb -> ky -> kx -> lane16 (NchwcConv.Row, AVX-512 hosts)

_fp = C.POINTER(C.c_float)
_dp = C.POINTER(C.c_double)
_ip = C.POINTER(C.c_int)
_i32p = C.POINTER(C.c_int32)
_u8p = C.POINTER(C.c_uint8)
_vp = C.c_void_p


def build() -> None:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        l = C.CDLL(_LIB_PATH)
        if not l.orc_cpu_ok():
            raise RuntimeError("oracle build needs an AVX2+FMA host")
        l.orc_gemm_f32.argtypes = [C.c_int, C.c_int, C.c_int, _fp, C.c_int, _fp, C.c_int, _fp, _fp, _fp,
                                   _fp, C.c_int, C.c_int]
        l.orc_gemm_f64.argtypes = [C.c_int, C.c_int, C.c_int, _fp, _fp, _fp, _fp, _dp]
        l.orc_conv2d_f32.argtypes = [C.c_int] + [C.c_int] * 16 + [_fp, _fp, _fp, _fp]
        l.orc_conv2d_f32.restype = C.c_int
        l.orc_conv2d_f64.argtypes = [C.c_int] * 16 + [_fp, _fp, _fp, _dp]
        l.orc_conv_dw_f32.argtypes = [C.c_int] * 14 + [_fp, _fp, _fp, _fp]
        l.orc_winograd_f23.argtypes = [C.c_int] * 5 + [_fp, _fp, _fp, _fp]
        for f in (l.orc_exp_ref, l.orc_silu_ref, l.orc_silu_scalar, l.orc_relu, l.orc_sigmoid_ref):
            f.argtypes = [C.c_long, _fp, _fp]
        l.orc_dfl_f32.argtypes = [C.c_int] * 4 + [_fp, _fp]
        l.orc_softmax_f32.argtypes = [C.c_long, C.c_int, C.c_float, _fp, _fp]
        l.orc_maxpool2d_f32.argtypes = [C.c_int] * 12 + [_fp, _fp]
        l.orc_resize_nearest.argtypes = [C.c_int] * 6 + [_fp, _fp]
        l.orc_minmax.argtypes = [C.c_long, _fp, _fp, _fp]
        l.orc_dql_params.argtypes = [C.c_float, C.c_float, _fp, _ip]
        l.orc_quantize_u8.argtypes = [C.c_long, _fp, C.c_float, C.c_int, _u8p]
        l.orc_dynamic_quantize_linear.argtypes = [C.c_long, _fp, _u8p, _fp, _ip]
        l.orc_dqmm.argtypes = [C.c_int, C.c_int, C.c_int, _fp, _vp, C.c_int, _ip, C.c_int, _fp, C.c_int, _fp,
                               _fp, _i32p, _fp, C.c_int, _fp, _ip]
        l.orc_matmul_integer.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, _ip, C.c_int, _i32p]
        l.orc_set_threads.argtypes = [C.c_int]
        l.orc_gemm_f32_rows.argtypes = l.orc_gemm_f32.argtypes
        l.orc_unary_scalar.argtypes = [C.c_int, C.c_long, _fp, _fp]
        l.orc_nchwc_pack_weights.argtypes = [C.c_int, C.c_int, _fp, _fp]
        l.orc_nchwc_scratch_floats.argtypes = [C.c_int] * 7 + [C.POINTER(C.c_long)] * 2
        l.orc_nchwc_conv_avx512.argtypes = [C.c_int] * 7 + [_fp] * 6
        l.orc_nchwc_conv_avx512.restype = C.c_int
        _lib = l
    return _lib


def set_threads(t: int) -> None:
    lib().orc_set_threads(int(t))


def _f(a):
    return None if a is None else a.ctypes.data_as(_fp)


def _c32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- GEMM

def gemm_f32(a, b, row_bias=None, col_bias=None, col_scale=None, fused=True):
    """GemmKernel.Multiply / MultiplyPacked (GemmKernel.cs:1070-1241): FMA chain from the bias."""
    a, b = _c32(a), _c32(b)
    row_bias, col_bias, col_scale = _c32(row_bias), _c32(col_bias), _c32(col_scale)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().orc_gemm_f32(m, k, n, _f(a), k, _f(b), n, _f(row_bias), _f(col_bias), _f(col_scale), _f(c), n,
                       1 if fused else 0)
    return c


def gemm_f32_rows(a, b, row_bias=None, col_bias=None, col_scale=None, fused=True):
    """gemm_f32 on the scalar row loop only (the blocked AVX-512 path of
    gemm_f32 gives the same bits; this is its check)."""
    a, b = _c32(a), _c32(b)
    row_bias, col_bias, col_scale = _c32(row_bias), _c32(col_bias), _c32(col_scale)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().orc_gemm_f32_rows(m, k, n, _f(a), k, _f(b), n, _f(row_bias), _f(col_bias), _f(col_scale), _f(c), n,
                            1 if fused else 0)
    return c


def unary_scalar(op, x):
    """exp_ref (op 0), SiLU (1) or sigmoid (2) on the scalar loop only."""
    x = _c32(x)
    y = np.empty_like(x)
    lib().orc_unary_scalar(op, x.size, _f(x), _f(y))
    return y


def gemm_ex(a, b, c=None, alpha=1.0, beta=1.0, trans_a=False, trans_b=False):
    """ONNX Gemm as GemmLayer.Forward (AttnOps.cs:82-131): materialized transposes,
    the FMA chain from 0, then alpha * y and + beta * c, each rounded in float."""
    a = _c32(a).T.copy() if trans_a else _c32(a)
    b = _c32(b).T.copy() if trans_b else _c32(b)
    y = gemm_f32(a, b)
    alpha, beta = np.float32(alpha), np.float32(beta)
    if alpha != 1:
        y = (alpha * y).astype(np.float32)
    if beta != 0 and c is not None and np.size(c) > 0:
        c = _c32(c).ravel()
        m, n = y.shape
        if c.size >= m * n:
            cv = c[:m * n].reshape(m, n)
        elif c.size == 1:
            cv = np.full((m, n), c[0], np.float32)
        else:
            cv = np.broadcast_to(c[np.arange(n) % c.size], (m, n))
        y = (y + (beta * cv).astype(np.float32)).astype(np.float32)
    return y


def gemm_f64(a, b, col_bias=None, row_bias=None):
    """Double-precision naive product (GemmKernelTests' naive loop)."""
    a, b = _c32(a), _c32(b)
    col_bias, row_bias = _c32(col_bias), _c32(row_bias)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float64)
    lib().orc_gemm_f64(m, k, n, _f(a), _f(b), _f(col_bias), _f(row_bias), c.ctypes.data_as(_dp))
    return c


# ---------------------------------------------------------------- conv

def conv2d_f32(x, w, bias, strides, pads, dilations, group, out_hw, order=ORDER_IM2COL):
    """NCHW conv, reference accumulation order `order`; pads are the begin pads (top, left)."""
    x, w, bias = _c32(x), _c32(w), _c32(bias)
    N, Cc, H, W = x.shape
    M, _, KH, KW = w.shape
    OH, OW = out_hw
    y = np.empty((N, M, OH, OW), np.float32)
    rc = lib().orc_conv2d_f32(order, N, Cc, H, W, M, KH, KW, group, strides[0], strides[1], dilations[0],
                              dilations[1], pads[0], pads[1], OH, OW, _f(x), _f(w), _f(bias), _f(y))
    if rc != 0:
        raise ValueError("NCHWc order needs C/group % 16 == 0")
    return y


def nchwc_avx512_ok() -> bool:
    """Whether this host runs the AVX-512 restatement of NchwcConv."""
    return bool(lib().orc_nchwc_avx512_ok())


_nchwc_packs = {}    # id(weights) -> (weakref to the weights, packed copy)
_nchwc_scratch = {}  # (role, element count) -> reusable blocked buffer


def _nchwc_packed(w):
    """The weights in NchwcConv.PackWeights' layout, packed once per weight
    array (the reference caches the packing on the weight tensor; weights
    are not changed in place)."""
    import weakref
    hit = _nchwc_packs.get(id(w))
    if hit is not None and hit[0]() is w:
        return hit[1]
    M, Cc = w.shape[:2]
    wp = np.empty(M * Cc * 9, np.float32)
    lib().orc_nchwc_pack_weights(Cc, M, _f(_c32(w)), _f(wp))
    try:
        _nchwc_packs[id(w)] = (weakref.ref(w), wp)
    except TypeError:  # an array that takes no weak reference: packed each time
        pass
    return wp


def _scratch(role, n):
    """A reusable float buffer of n elements (the reference's temp pool)."""
    buf = _nchwc_scratch.get((role, n))
    if buf is None:
        buf = _nchwc_scratch[(role, n)] = np.empty(max(1, n), np.float32)
    return buf


def conv_nchwc_avx512(x, w, bias, stride, out_hw):
    """The NCHWc chain through the blocked AVX-512 restatement of NchwcConv
    (orc_nchwc_conv_avx512): bit-identical to conv2d_f32(order=ORDER_NCHWC)
    for the shapes the reference's NCHWc gate takes (batch 1, 3x3, pad 1,
    stride 1 or 2); the input and output reorders run per call, the weight
    packing once, as in the reference."""
    x, bias = _c32(x), _c32(bias)
    _, Cc, H, W = x.shape
    M = w.shape[0]
    OH, OW = out_hw
    nx, ny = C.c_long(), C.c_long()
    lib().orc_nchwc_scratch_floats(Cc, H, W, M, stride, OH, OW, C.byref(nx), C.byref(ny))
    y = np.empty((1, M, OH, OW), np.float32)
    rc = lib().orc_nchwc_conv_avx512(Cc, H, W, M, stride, OH, OW, _f(x), _f(_nchwc_packed(w)), _f(bias), _f(y),
                                     _f(_scratch("in", nx.value)), _f(_scratch("out", ny.value)))
    if rc != 0:
        raise ValueError("NCHWc AVX-512 kernel: shape outside the NCHWc gate, or no AVX-512")
    return y


def conv2d_f64(x, w, bias, strides, pads, dilations, group, out_hw):
    """Textbook direct conv in double (ConvKernels.Direct semantics)."""
    x, w, bias = _c32(x), _c32(w), _c32(bias)
    N, Cc, H, W = x.shape
    M, _, KH, KW = w.shape
    OH, OW = out_hw
    y = np.empty((N, M, OH, OW), np.float64)
    lib().orc_conv2d_f64(N, Cc, H, W, M, KH, KW, group, strides[0], strides[1], dilations[0], dilations[1],
                         pads[0], pads[1], OH, OW, _f(x), _f(w), _f(bias), y.ctypes.data_as(_dp))
    return y


def conv_dw_f32(x, w, bias, strides, pads, dilations, out_hw):
    """DepthwiseConv (group == C == M)."""
    x, w, bias = _c32(x), _c32(w), _c32(bias)
    N, Cc, H, W = x.shape
    KH, KW = w.shape[2], w.shape[3]
    OH, OW = out_hw
    y = np.empty((N, Cc, OH, OW), np.float32)
    lib().orc_conv_dw_f32(N, Cc, H, W, KH, KW, strides[0], strides[1], dilations[0], dilations[1], pads[0],
                          pads[1], OH, OW, _f(x), _f(w), _f(bias), _f(y))
    return y


def winograd_f23(x, w, bias):
    """Winograd F(2x2,3x3), stride 1, pad 1 (Winograd.cs)."""
    x, w, bias = _c32(x), _c32(w), _c32(bias)
    N, Cc, H, W = x.shape
    M = w.shape[0]
    y = np.empty((N, M, H, W), np.float32)
    lib().orc_winograd_f23(N, Cc, H, W, M, _f(x), _f(w), _f(bias), _f(y))
    return y


KERNEL_DEPTHWISE = "depthwise"
KERNEL_NCHWC = "nchwc"
KERNEL_WINOGRAD = "winograd"
KERNEL_IM2COL = "im2col"


def conv_reference_kernel(x_shape, w_shape, strides, pads, dilations, group, out_hw, winograd=1,
                          wino_max=4096, nchwc=1):
    """The kernel ConvLayer.Forward (src/OnnxSharp/Ops/DnnOps.cs:437-482) runs
    for a 2-D conv on an AVX-512 host, first gate that holds:
    DepthwiseConv.TryConv (group == C == M, one input channel per group,
    DepthwiseConv.cs:25-60); FirstConv (C <= 3; its ic -> ky -> kx chain is
    the im2col order, so it is reported as KERNEL_IM2COL); NchwcConv.TryConv
    (NchwcConv.cs:100-126,166-194); Winograd.TryConv3x3 (Winograd.cs:58-122);
    else PackedConv / Im2Col, both the im2col chain.  winograd = 0 leaves
    Winograd out and 2 puts it ahead of NCHWc, as the backend's option of the
    same name does.  nchwc = 0 is a host that does not run NchwcConv
    (NchwcConv.Enabled false, ONNXSHARP_NCHWC=0, or no AVX-512:
    NchwcConv.cs:38-43): its shapes then fall to Winograd or the im2col
    chain.  Without AVX-512 FirstConv is off too and PackedConv takes its
    shapes, in the same ic -> ky -> kx order.  pads are the begin pads (top,
    left)."""
    n, c, h, w = x_shape
    m, cpg, kh, kw = w_shape
    sh, sw = strides
    pt, pl = pads
    dh, dw = dilations
    oh, ow = out_hw
    if group == c and m == c and cpg == 1 and group > 1:
        return KERNEL_DEPTHWISE
    if c <= 3 and group == 1:
        return KERNEL_IM2COL
    wino = (winograd != 0 and group == 1 and (kh, kw) == (3, 3) and (sh, sw) == (1, 1) and (dh, dw) == (1, 1)
            and (pt, pl) == (1, 1) and c >= 8 and m >= 8 and (oh, ow) == (h, w) and h >= 6 and w >= 6
            and h * w <= wino_max and m * c * 16 <= (1 << 24))
    if winograd == 2 and wino:
        return KERNEL_WINOGRAD
    s2 = sh == 2
    gate = (nchwc != 0 and group == 1 and (kh, kw) == (3, 3) and sh == sw and sh in (1, 2) and (dh, dw) == (1, 1)
            and (pt, pl) == (1, 1) and (not s2 or (h % 2 == 0 and w % 2 == 0)) and c % 16 == 0
            and m % 32 == 0 and n == 1 and ((oh * 2, ow * 2) == (h, w) if s2 else (oh, ow) == (h, w)))
    if gate:
        return KERNEL_NCHWC
    if wino:
        return KERNEL_WINOGRAD
    return KERNEL_IM2COL


def conv_reference(x, w, bias, strides, pads, dilations, group, out_hw, winograd=1, wino_max=4096, nchwc=1,
                   fast=True):
    """Conv output (before the fused activation) of the reference kernel
    conv_reference_kernel picks for the shape.  With `fast` the NCHWc shapes
    run the blocked AVX-512 restatement where the host has AVX-512 (the same
    bits as the scalar NCHWc-order loop, which fast=False runs)."""
    k = conv_reference_kernel(x.shape, w.shape, strides, pads, dilations, group, out_hw, winograd, wino_max, nchwc)
    if k == KERNEL_NCHWC and fast and nchwc_avx512_ok():
        return conv_nchwc_avx512(x, w, bias, strides[0], out_hw)
    if (k == KERNEL_IM2COL and fast and group == 1 and w.shape[2:] == (1, 1) and tuple(strides) == (1, 1)
            and tuple(pads) == (0, 0) and tuple(out_hw) == tuple(x.shape[2:])):
        # a pointwise conv is GemmKernel.Multiply(W[M x C], X[C x HW], rowBias)
        # (ConvKernels.cs:464-514): the GEMM chain, the same bits as the
        # im2col loop over input channels
        n, cin, h, wd = x.shape
        wm = _c32(w.reshape(w.shape[0], cin))
        xs = _c32(x).reshape(n, cin, h * wd)
        return np.stack([gemm_f32(wm, xs[i], row_bias=bias) for i in range(n)]).reshape(n, w.shape[0], h, wd)
    if k == KERNEL_DEPTHWISE:
        return conv_dw_f32(x, w, bias, strides, pads, dilations, out_hw)
    if k == KERNEL_WINOGRAD:
        return winograd_f23(x, w, bias)
    return conv2d_f32(x, w, bias, strides, pads, dilations, group, out_hw,
                      order=ORDER_NCHWC if k == KERNEL_NCHWC else ORDER_IM2COL)


# ---------------------------------------------------------------- activations

def _unary(fn, x):
    x = _c32(x)
    y = np.empty_like(x)
    fn(x.size, _f(x), _f(y))
    return y


def exp_ref(x):
    """VectorMath.Exp polynomial."""
    return _unary(lib().orc_exp_ref, x)


def silu_ref(x):
    """VectorMath.Silu vector path."""
    return _unary(lib().orc_silu_ref, x)


def sigmoid_ref(x):
    """VectorMath.Sigmoid vector path."""
    return _unary(lib().orc_sigmoid_ref, x)


def dfl(x, bins=16):
    """DflSoftmax: x [B, sides*bins, N] -> [B, sides, N] (DflOps.cs)."""
    x = _c32(x)
    b, c, n = x.shape
    y = np.empty((b, c // bins, n), np.float32)
    lib().orc_dfl_f32(b, c // bins, bins, n, _f(x), _f(y))
    return y


def silu_scalar(x):
    """TensorOps scalar SiLU tail (C library expf in place of MathF.Exp)."""
    return _unary(lib().orc_silu_scalar, x)


def relu(x):
    return _unary(lib().orc_relu, x)


def softmax(x, scale=1.0):
    """Mul by a constant then Softmax over the last axis (SoftmaxLayer, VectorMath.SoftmaxRow)."""
    x = _c32(x)
    y = np.empty_like(x)
    cols = x.shape[-1]
    lib().orc_softmax_f32(x.size // cols, cols, scale, _f(x), _f(y))
    return y


def maxpool2d(x, k, s, p):
    """MaxPool 2-D, symmetric pads p (MaxPoolLayer)."""
    x = _c32(x)
    n, c, h, w = x.shape
    oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    y = np.empty((n, c, oh, ow), np.float32)
    lib().orc_maxpool2d_f32(n, c, h, w, k, k, s, s, p, p, oh, ow, _f(x), _f(y))
    return y


def resize_nearest(x, f):
    """Nearest upsampling by an integer factor (ResizeLayer, mode nearest)."""
    x = _c32(x)
    n, c, h, w = x.shape
    y = np.empty((n, c, h * f, w * f), np.float32)
    lib().orc_resize_nearest(n, c, h, w, f, f, _f(x), _f(y))
    return y


# ---------------------------------------------------------------- int8

def minmax(x):
    x = _c32(x)
    mn, mx = C.c_float(), C.c_float()
    lib().orc_minmax(x.size, _f(x), C.byref(mn), C.byref(mx))
    return mn.value, mx.value


def dql_params(mn, mx):
    s, z = C.c_float(), C.c_int()
    lib().orc_dql_params(mn, mx, C.byref(s), C.byref(z))
    return np.float32(s.value), z.value


def quantize_u8(x, scale, zp):
    x = _c32(x)
    q = np.empty(x.shape, np.uint8)
    lib().orc_quantize_u8(x.size, _f(x), float(scale), int(zp), q.ctypes.data_as(_u8p))
    return q


def dynamic_quantize_linear(x):
    x = _c32(x)
    q = np.empty(x.shape, np.uint8)
    s, z = C.c_float(), C.c_int()
    lib().orc_dynamic_quantize_linear(x.size, _f(x), q.ctypes.data_as(_u8p), C.byref(s), C.byref(z))
    return q, np.float32(s.value), z.value


def _zp_arr(zp):
    if zp is None:
        return None, 0
    z = np.ascontiguousarray(np.atleast_1d(zp), dtype=np.int32)
    return z, z.size


def dqmm(a, w, w_zp=None, w_scale=None, bias=None, fused=True):
    """DynamicQuantizeMatMul [A, W, w_zp, w_scale, bias] (QuantizedMatMulOps.cs:115-201).

    Returns (out f32, acc int32 exact, acc f32 reference chain, scale, zp)."""
    a = _c32(a)
    m, k = a.reshape(-1, a.shape[-1]).shape
    w = np.ascontiguousarray(w)
    assert w.dtype in (np.int8, np.uint8) and w.shape[0] == k
    n = w.shape[1]
    z, nz = _zp_arr(w_zp)
    ws = None if w_scale is None else np.ascontiguousarray(np.atleast_1d(w_scale), np.float32)
    bias = _c32(bias)
    out = np.empty((m, n), np.float32)
    acc = np.empty((m, n), np.int32)
    accf = np.empty((m, n), np.float32)
    s, zz = C.c_float(), C.c_int()
    lib().orc_dqmm(m, k, n, _f(a), w.ctypes.data, 1 if w.dtype == np.int8 else 0,
                   None if z is None else z.ctypes.data_as(_ip), nz, _f(ws), 0 if ws is None else ws.size,
                   _f(bias), _f(out), acc.ctypes.data_as(_i32p), _f(accf), 1 if fused else 0, C.byref(s),
                   C.byref(zz))
    return out, acc, accf, np.float32(s.value), zz.value


_dqmm_widened = {}  # id(weights) -> (weakref, widened weights, zero points)


def dqmm_widened_gemm(a, w, w_zp=None, w_scale=None, bias=None):
    """DynamicQuantizeMatMul as the reference computes it on the CPU
    (QuantizedMatMulOps.cs:115-201): Quantizer.MinMax and QuantizeAndWiden
    of A, then the F32 GEMM of the widened operands (weights widened once,
    w - w_zp, as GetPackedWeights caches them) with the column-scale
    epilogue fmaf(acc, a_scale * w_scale[j], bias[j]).  The output only; the
    same bits as dqmm(...)[0] (a CPU test checks), on the blocked GEMM."""
    import weakref
    a = _c32(a)
    m, k = a.shape
    n = w.shape[1]
    zps, _ = _zp_arr(w_zp)
    hit = _dqmm_widened.get(id(w))
    if hit is not None and hit[0]() is w and ((hit[2] is None and zps is None) or
                                               (hit[2] is not None and zps is not None and
                                                np.array_equal(hit[2], zps))):
        wf = hit[1]
    else:
        zcol = np.zeros(n, np.int32) if zps is None else np.broadcast_to(zps.astype(np.int32), (n,))
        wf = (w.astype(np.int32) - zcol[None, :]).astype(np.float32)
        try:
            _dqmm_widened[id(w)] = (weakref.ref(w), wf, zps)
        except TypeError:
            pass
    mn, mx = minmax(a)
    scale, zp = dql_params(mn, mx)
    q = quantize_u8(a, scale, zp)
    af = (q.astype(np.int32) - zp).astype(np.float32)
    ws = np.ones(n, np.float32) if w_scale is None else np.broadcast_to(np.asarray(w_scale, np.float32), (n,))
    comb = (np.float32(scale) * ws).astype(np.float32)
    return gemm_f32(af, wf, col_bias=bias, col_scale=comb, fused=True)


def matmul_integer(a, b, a_zp=0, b_zp=None):
    """MatMulInteger (Int8Gemm.MultiplyIntegerScalar; s8 A read as signed): exact int32."""
    a = np.ascontiguousarray(a)
    if a.dtype != np.int8:
        a = a.astype(np.uint8)
    b = np.ascontiguousarray(b)
    m, k = a.shape
    n = b.shape[1]
    z, nz = _zp_arr(b_zp)
    c = np.empty((m, n), np.int32)
    lib().orc_matmul_integer(m, k, n, a.ctypes.data, 1 if a.dtype == np.int8 else 0, int(a_zp), b.ctypes.data,
                             1 if b.dtype == np.int8 else 0, None if z is None else z.ctypes.data_as(_ip), nz,
                             c.ctypes.data_as(_i32p))
    return c
