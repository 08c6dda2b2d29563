"""CPU tests that pin the oracle (oracle/osh_oracle.c) before it is trusted.

Each check is chosen so that a plausible slip in the restatement (a dropped
term, a transposed operand, a wrong rounding mode or order) fails it:
known answers from the reference's own tests, closed forms in float64,
brute force on small inputs, and invariants of the integer algebra.
"""
import json
import math
import os

import numpy as np
import pytest

from onnxsharp_amd import synth

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


# ----------------------------------------------------------- known answers

def test_dynamic_quantize_linear_known_answer(oracle):
    g = GOLD["dynamic_quantize_linear"]
    q, s, z = oracle.dynamic_quantize_linear(np.array(g["x"], np.float32))
    assert s == np.float32(3) / np.float32(255)
    assert z == g["zero_point"]
    assert q.tolist() == g["q"]


def test_matmul_integer_known_answer(oracle):
    g = GOLD["matmul_integer"]
    c = oracle.matmul_integer(np.array(g["a"], np.uint8), np.array(g["b"], np.uint8))
    assert c.tolist() == g["c"]


def test_quantize_u8_known_answer(oracle):
    g = GOLD["quantize_u8"]
    q = oracle.quantize_u8(np.array(g["x"], np.float32), g["scale"], g["zero_point"])
    assert q.tolist() == g["q"]


def test_conv_same_upper_window_sums(oracle):
    g = GOLD["conv_same_upper_s2"]
    x = np.arange(1, 100, dtype=np.float32).reshape(1, 1, 9, 11)
    w = np.ones((1, 1, 3, 3), np.float32)
    y = oracle.conv2d_f32(x, w, None, (2, 2), (1, 1), (1, 1), 1, (5, 6))
    xp = np.pad(x[0, 0].astype(np.int64), 1)
    brute = np.array([[xp[2 * i:2 * i + 3, 2 * j:2 * j + 3].sum() for j in range(6)] for i in range(5)])
    assert (brute == np.array(g["y"])).all()
    assert (y[0, 0] == brute).all()


# ----------------------------------------------------------- GEMM

@pytest.mark.parametrize("m,k,n", [(257, 64, 257), (64, 64, 64), (5, 17, 33), (17, 1, 257), (1, 257, 64),
                                   (96, 320, 1280)])
def test_gemm_chain_matches_float64(oracle, m, k, n):
    # GemmKernelTests.Check: |d| / max(1, |x|) <= 1e-4 against a double-precision naive product
    rng = np.random.default_rng(m * 31 + k * 7 + n)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    cb = rng.uniform(-1, 1, n).astype(np.float32)
    c = oracle.gemm_f32(a, b, col_bias=cb)
    ref = oracle.gemm_f64(a, b, col_bias=cb)
    assert (np.abs(c - ref) / np.maximum(1.0, np.abs(ref))).max() <= 1e-4
    assert np.allclose(ref, a.astype(np.float64) @ b.astype(np.float64) + cb, rtol=1e-12, atol=1e-9)


def test_gemm_chain_is_sequential_fma(oracle):
    # one output by hand: acc = bias; acc = fma(a_t, b_t, acc) for t ascending
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, (3, 50)).astype(np.float32)
    b = rng.uniform(-1, 1, (50, 4)).astype(np.float32)
    cb = rng.uniform(-1, 1, 4).astype(np.float32)
    c = oracle.gemm_f32(a, b, col_bias=cb)
    for i in range(3):
        for j in range(4):
            acc = np.float32(cb[j])
            for t in range(50):
                # float64 product of two float32 is exact; adding it in float64 and rounding once is an fma
                acc = np.float32(np.float64(acc) + np.float64(a[i, t]) * np.float64(b[t, j]))
            assert c[i, j] == acc


def test_gemm_row_bias_and_column_scale(oracle):
    rng = np.random.default_rng(2)
    a = rng.uniform(-1, 1, (7, 33)).astype(np.float32)
    b = rng.uniform(-1, 1, (33, 45)).astype(np.float32)
    rb = rng.uniform(-1, 1, 7).astype(np.float32)
    cs = rng.uniform(1e-4, 1e-2, 45).astype(np.float32)
    cb = rng.uniform(-1, 1, 45).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert np.abs(oracle.gemm_f32(a, b, row_bias=rb) - (ref + rb[:, None])).max() < 1e-4
    fused = oracle.gemm_f32(a, b, col_bias=cb, col_scale=cs)
    plain = oracle.gemm_f32(a, b)
    # GemmKernelTests.PackedScaleBiasMatchesEpilogue: fused epilogue == GEMM then *scale + bias
    exp = plain.astype(np.float64) * cs + cb
    assert (np.abs(fused - exp) / np.maximum(1, np.abs(exp))).max() <= 1e-5
    unf = oracle.gemm_f32(a, b, col_bias=cb, col_scale=cs, fused=False)
    assert (unf == (plain * cs + cb).astype(np.float32)).all()


# ----------------------------------------------------------- conv

CONV_CASES = [
    # (N, C, H, W, M, KH, KW, group, strides, pads(t,l), dil, out)
    (1, 16, 12, 13, 8, 3, 3, 1, (1, 1), (1, 1), (1, 1), (12, 13)),
    (1, 32, 10, 10, 16, 3, 3, 1, (2, 2), (1, 1), (1, 1), (5, 5)),
    (2, 8, 9, 7, 6, 3, 3, 2, (1, 2), (0, 1), (1, 1), (7, 4)),
    (1, 4, 11, 11, 5, 3, 3, 1, (1, 1), (2, 2), (2, 2), (11, 11)),
    (1, 3, 17, 17, 16, 3, 3, 1, (2, 2), (1, 1), (1, 1), (9, 9)),
    (1, 24, 6, 6, 12, 1, 1, 1, (1, 1), (0, 0), (1, 1), (6, 6)),
    (1, 5, 8, 9, 7, 5, 5, 1, (1, 1), (2, 2), (1, 1), (8, 9)),
]


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_orders_match_direct(oracle, case):
    N_, Cc, H, W, M, KH, KW, g, s, p, d, o = case
    x = synth.uniform(11, (N_, Cc, H, W))
    w = synth.normal(12, (M, Cc // g, KH, KW), 0, 0.05)
    b = synth.normal(13, (M,), 0, 0.01)
    ref = oracle.conv2d_f64(x, w, b, s, p, d, g, o)
    # independent float64 conv by explicit zero padding + einsum over windows
    xp = np.zeros((N_, Cc, H + 2 * p[0] + KH * d[0], W + 2 * p[1] + KW * d[1]))
    xp[:, :, p[0]:p[0] + H, p[1]:p[1] + W] = x
    ind = np.zeros((N_, M) + o)
    for oc in range(M):
        gi = oc // (M // g)
        for ky in range(KH):
            for kx in range(KW):
                win = xp[:, gi * (Cc // g):(gi + 1) * (Cc // g),
                         ky * d[0]: ky * d[0] + o[0] * s[0]: s[0], kx * d[1]: kx * d[1] + o[1] * s[1]: s[1]]
                ind[:, oc] += np.einsum("nchw,c->nhw", win[:, :, :o[0], :o[1]], w[oc, :, ky, kx])
        ind[:, oc] += b[oc]
    assert np.allclose(ref, ind, rtol=0, atol=1e-9)
    y = oracle.conv2d_f32(x, w, b, s, p, d, g, o, order=oracle.ORDER_IM2COL)
    assert np.abs(y - ref).max() <= 1e-5
    if (Cc // g) % 16 == 0:
        yn = oracle.conv2d_f32(x, w, b, s, p, d, g, o, order=oracle.ORDER_NCHWC)
        assert np.abs(yn - ref).max() <= 1e-5


def test_nchwc_order_differs_from_im2col_order_only_by_rounding(oracle):
    # the two ISA orders are different FMA chains: same value to rounding, not bit-equal in general
    x = synth.uniform(21, (1, 32, 20, 20))
    w = synth.normal(22, (32, 32, 3, 3), 0, 0.05)
    b = synth.normal(23, (32,), 0, 0.01)
    a = oracle.conv2d_f32(x, w, b, (1, 1), (1, 1), (1, 1), 1, (20, 20), order=oracle.ORDER_IM2COL)
    c = oracle.conv2d_f32(x, w, b, (1, 1), (1, 1), (1, 1), 1, (20, 20), order=oracle.ORDER_NCHWC)
    assert not np.array_equal(a, c)
    assert np.abs(a - c).max() < 1e-5


def test_depthwise_matches_grouped_direct(oracle):
    x = synth.uniform(31, (1, 12, 15, 14))
    w = synth.normal(32, (12, 1, 3, 3), 0, 0.05)
    b = synth.normal(33, (12,), 0, 0.01)
    for s in ((1, 1), (2, 2)):
        o = ((15 + 2 - 3) // s[0] + 1, (14 + 2 - 3) // s[1] + 1)
        ref = oracle.conv2d_f64(x, w, b, s, (1, 1), (1, 1), 12, o)
        y = oracle.conv_dw_f32(x, w, b, s, (1, 1), (1, 1), o)
        assert np.abs(y - ref).max() <= 1e-6


@pytest.mark.parametrize("hw", [(6, 6), (13, 9), (20, 20)])
def test_winograd_matches_direct(oracle, hw):
    x = synth.uniform(41, (1, 8, *hw))
    w = synth.normal(42, (9, 8, 3, 3), 0, 0.05)
    b = synth.normal(43, (9,), 0, 0.01)
    ref = oracle.conv2d_f64(x, w, b, (1, 1), (1, 1), (1, 1), 1, hw)
    y = oracle.winograd_f23(x, w, b)
    assert np.abs(y - ref).max() <= 1e-5


def test_winograd_exact_on_integer_data(oracle):
    # With small integers every Winograd step is exact in float32 (the 1/2
    # factors of G g G^T give quarters at most), so the result must equal the
    # direct conv exactly: a wrong sign, index or factor in any of the three
    # transforms shows up as an integer error.
    rng = np.random.default_rng(44)
    for (c, m, h, w) in [(8, 8, 6, 6), (11, 9, 7, 10), (16, 24, 9, 8)]:
        x = rng.integers(-4, 5, (1, c, h, w)).astype(np.float32)
        wt = rng.integers(-4, 5, (m, c, 3, 3)).astype(np.float32)
        b = rng.integers(-8, 9, (m,)).astype(np.float32)
        ref = oracle.conv2d_f64(x, wt, b, (1, 1), (1, 1), (1, 1), 1, (h, w))
        assert np.array_equal(oracle.winograd_f23(x, wt, b).astype(np.float64), ref)


def _yolo_conv_kernels(oracle, size, nchwc=1, detail=False):
    from onnxsharp_amd import yolo11n
    kinds, seen = [], set()
    for op in yolo11n.build(size).ops:
        # the C2PSA positional conv runs as one depthwise op per head
        if isinstance(op, yolo11n.ConvOp) and op.name.split("#")[0] not in seen:
            seen.add(op.name.split("#")[0])
            pad = op.k // 2
            kind = oracle.conv_reference_kernel(
                (1, op.x.c, op.x.h, op.x.w), (op.y.c, op.x.c // op.group, op.k, op.k), (op.s, op.s),
                (pad, pad), (1, 1), op.group, (op.y.h, op.y.w), nchwc=nchwc)
            kinds.append((kind, op.k, op.s, op.group > 1, op.y.h * op.y.w) if detail else (kind, op.k))
    return kinds


def test_reference_dispatch_of_the_yolo11n_frame(oracle):
    # ConvLayer.Forward's chain on an AVX-512 host for the 87 convs at 640x640:
    # 30 NCHWc calls (the reference's profile of this network, bench.md:2330),
    # 7 depthwise, no Winograd (every small-map 3x3 passes NCHWc's gate), and
    # the stem, four 3x3 bottleneck convs (16->8, 8->16 at 160, 32->16 at 80,
    # twice) and the 45 pointwise convs on the im2col / GEMM chain.
    kinds = _yolo_conv_kernels(oracle, 640)
    count = lambda k, ks=None: sum(1 for kind, kk in kinds if kind == k and (ks is None or kk == ks))
    assert len(kinds) == 87
    assert count(oracle.KERNEL_NCHWC) == 30
    assert count(oracle.KERNEL_DEPTHWISE) == 7
    assert count(oracle.KERNEL_WINOGRAD) == 0
    assert count(oracle.KERNEL_IM2COL, 1) == 45
    assert count(oracle.KERNEL_IM2COL, 3) == 5
    # at 128x128 the small maps bring Winograd in for the 3x3 convs NCHWc refuses
    assert sum(1 for kind, _ in _yolo_conv_kernels(oracle, 128) if kind == oracle.KERNEL_WINOGRAD) >= 4


def test_reference_dispatch_of_the_yolo11n_frame_without_nchwc(oracle):
    # A host that does not run NchwcConv (AVX2 only, or ONNXSHARP_NCHWC=0):
    # the reference's own family profile of this network on such a host
    # (bench.md:1747-1755) is 35 3x3 stride-1 layers (Winograd only where the
    # map is at most 4096 pixels, i.e. 40x40 and 20x20; the 160x160 and
    # 80x80 ones on im2col), 7 3x3 stride-2 layers (PackedConv: the im2col
    # order) and 45 1x1 layers (the im2col GEMM).
    kinds = _yolo_conv_kernels(oracle, 640, nchwc=0, detail=True)
    assert len(kinds) == 87
    s1 = [k for k in kinds if k[1] == 3 and k[2] == 1]
    s2 = [k for k in kinds if k[1] == 3 and k[2] == 2]
    assert (len(s1), len(s2), sum(1 for k in kinds if k[1] == 1)) == (35, 7, 45)
    assert not any(k[0] == oracle.KERNEL_NCHWC for k in kinds)
    assert all(k[0] == oracle.KERNEL_IM2COL for k in s2)  # the stem included (FirstConv needs AVX-512 too)
    dense_s1 = [k for k in s1 if not k[3]]
    assert all(k[0] == (oracle.KERNEL_WINOGRAD if k[4] <= 4096 else oracle.KERNEL_IM2COL) for k in dense_s1)
    # 20 Winograd calls (10 at 40x40, 10 at 20x20) and 8 im2col ones (160x160, 80x80)
    assert sum(1 for k in dense_s1 if k[0] == oracle.KERNEL_WINOGRAD) == 20
    assert sum(1 for k in dense_s1 if k[0] == oracle.KERNEL_IM2COL) == 8
    assert all(k[0] == oracle.KERNEL_DEPTHWISE for k in s1 if k[3])
    # the 30 NCHWc layers of the AVX-512 host are exactly the ones that move
    on = _yolo_conv_kernels(oracle, 640, nchwc=1)
    moved = [a[0] for a, b in zip(on, kinds) if a[0] != b[0]]
    assert moved == [oracle.KERNEL_NCHWC] * 30


def test_reference_dispatch_gates(oracle):
    K = oracle.conv_reference_kernel
    s1, p1, d1 = (1, 1), (1, 1), (1, 1)
    assert K((1, 64, 20, 20), (64, 64, 3, 3), s1, p1, d1, 1, (20, 20)) == oracle.KERNEL_NCHWC
    assert K((1, 64, 20, 20), (64, 64, 3, 3), s1, p1, d1, 1, (20, 20), winograd=2) == oracle.KERNEL_WINOGRAD
    assert K((1, 64, 20, 20), (48, 64, 3, 3), s1, p1, d1, 1, (20, 20)) == oracle.KERNEL_WINOGRAD  # M % 32
    assert K((2, 64, 20, 20), (64, 64, 3, 3), s1, p1, d1, 1, (20, 20)) == oracle.KERNEL_WINOGRAD  # batch 2
    assert K((1, 64, 20, 20), (48, 64, 3, 3), s1, p1, d1, 1, (20, 20), winograd=0) == oracle.KERNEL_IM2COL
    assert K((1, 64, 80, 80), (48, 64, 3, 3), s1, p1, d1, 1, (80, 80)) == oracle.KERNEL_IM2COL  # > 4096 px
    assert K((1, 64, 80, 80), (48, 64, 3, 3), s1, p1, d1, 1, (80, 80), wino_max=6400) == oracle.KERNEL_WINOGRAD
    assert K((1, 64, 41, 40), (64, 64, 3, 3), (2, 2), p1, d1, 1, (21, 20)) == oracle.KERNEL_IM2COL  # odd H, s2
    assert K((1, 64, 40, 40), (64, 64, 3, 3), (2, 2), p1, d1, 1, (20, 20)) == oracle.KERNEL_NCHWC
    assert K((1, 7, 20, 20), (64, 7, 3, 3), s1, p1, d1, 1, (20, 20)) == oracle.KERNEL_IM2COL  # C < 8
    assert K((1, 8, 5, 20), (8, 8, 3, 3), s1, p1, d1, 1, (5, 20)) == oracle.KERNEL_IM2COL  # H < 6
    assert K((1, 32, 20, 20), (32, 1, 3, 3), s1, p1, d1, 32, (20, 20)) == oracle.KERNEL_DEPTHWISE
    assert K((1, 3, 64, 64), (16, 3, 3, 3), (2, 2), p1, d1, 1, (32, 32)) == oracle.KERNEL_IM2COL
    # without NchwcConv: Winograd where its gate holds, else the im2col chain
    assert K((1, 64, 20, 20), (64, 64, 3, 3), s1, p1, d1, 1, (20, 20), nchwc=0) == oracle.KERNEL_WINOGRAD
    assert K((1, 64, 160, 160), (64, 64, 3, 3), s1, p1, d1, 1, (160, 160), nchwc=0) == oracle.KERNEL_IM2COL
    assert K((1, 64, 40, 40), (64, 64, 3, 3), (2, 2), p1, d1, 1, (20, 20), nchwc=0) == oracle.KERNEL_IM2COL
    assert K((1, 64, 20, 20), (64, 64, 3, 3), s1, p1, d1, 1, (20, 20), winograd=0, nchwc=0) == oracle.KERNEL_IM2COL
    assert K((1, 32, 20, 20), (32, 1, 3, 3), s1, p1, d1, 32, (20, 20), nchwc=0) == oracle.KERNEL_DEPTHWISE


# ----------------------------------------------------------- activations

def test_exp_polynomial_accuracy(oracle):
    x = np.linspace(-87.0, 88.0, 200001, dtype=np.float32)
    e = oracle.exp_ref(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    assert (np.abs(e - ref) / ref).max() < 4e-7  # VectorMath.cs:20 claims ~1e-7 relative
    # clamping: beyond the range the polynomial saturates at the clamp values
    big = oracle.exp_ref(np.array([200.0, -200.0], np.float32))
    assert big[0] == oracle.exp_ref(np.array([88.7], np.float32))[0]
    assert big[1] == oracle.exp_ref(np.array([-87.3], np.float32))[0]


def test_silu_matches_float64(oracle):
    x = synth.uniform(51, (100000,), -20, 20)
    y = oracle.silu_ref(x).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd / (1.0 + np.exp(-xd))
    assert (np.abs(y - ref) <= 1e-6 * np.maximum(1, np.abs(ref))).all()
    assert oracle.silu_ref(np.array([0.0], np.float32))[0] == 0.0
    s = oracle.silu_scalar(x).astype(np.float64)
    assert np.abs(s - ref).max() < 1e-5


def test_relu(oracle):
    x = np.array([-1, -0.0, 0, 2.5, np.nan], np.float32)
    assert oracle.relu(x).tolist() == [0.0, 0.0, 0.0, 2.5, 0.0]


# ----------------------------------------------------------- int8

def test_minmax_includes_zero_and_skips_nan(oracle):
    assert oracle.minmax(np.array([1, 2, 3], np.float32)) == (0.0, 3.0)
    assert oracle.minmax(np.array([-4, np.nan, -1], np.float32)) == (-4.0, 0.0)
    x = synth.normal(61, (4097,))
    assert oracle.minmax(x) == (min(0.0, float(x.min())), max(0.0, float(x.max())))


def test_dql_params_follow_the_formula(oracle):
    for mn, mx in [(-1.0, 2.0), (0.0, 0.0), (-3.3, 0.0), (0.0, 7.1), (-0.37, 0.91)]:
        s, z = oracle.dql_params(mn, mx)
        es = np.float32(np.float32(mx) - np.float32(mn)) / np.float32(255)
        if not es > 0:
            es = np.float32(1)
        assert s == es
        assert z == int(np.clip(np.rint(np.float32(-np.float32(mn)) / es), 0, 255))


def test_quantize_rounds_half_to_even(oracle):
    q = oracle.quantize_u8(np.array([0.25, 0.75, 1.25, -0.25, -0.75], np.float32), 0.5, 10)
    assert q.tolist() == [10, 12, 12, 10, 8]


def test_dqmm_accumulators_are_exact_integers(oracle):
    m, k, n = 64, 512, 96
    a = synth.normal(71, (m, k))
    w = synth.randint(72, (k, n), -127, 127, np.int8)
    ws = synth.uniform(73, (n,), 0.001, 0.02)
    bias = synth.normal(74, (n,), 0, 0.01)
    out, acc, accf, s, z = oracle.dqmm(a, w, None, ws, bias)
    q, s2, z2 = oracle.dynamic_quantize_linear(a)
    assert (s, z) == (s2, z2)
    brute = (q.astype(np.int64) - z) @ w.astype(np.int64)
    assert (acc == brute).all()
    # the reference's FP32 chain is exact here (|partial sums| < 2^24), so it equals the integer
    assert (accf == acc.astype(np.float32)).all()
    comb = (s * ws).astype(np.float32)
    expect = (acc.astype(np.float64) * comb.astype(np.float64) + bias)
    assert np.abs(out - expect).max() <= 1e-5 * np.abs(expect).max()


def test_dqmm_weight_zero_points_and_u8_weights(oracle):
    m, k, n = 9, 40, 13
    a = synth.normal(81, (m, k))
    for wdt, lo, hi in ((np.uint8, 0, 255), (np.int8, -128, 127)):
        w = synth.randint(82, (k, n), lo, hi, wdt)
        zp = synth.randint(83, (n,), -20, 20, np.int32) + (128 if wdt == np.uint8 else 0)
        out, acc, accf, s, z = oracle.dqmm(a, w, zp, np.float32(0.01), None)
        q, _, _ = oracle.dynamic_quantize_linear(a)
        brute = (q.astype(np.int64) - z) @ (w.astype(np.int64) - zp[None, :])
        assert (acc == brute).all()
        mi = oracle.matmul_integer(q, w, z, zp)
        assert (mi == brute).all()


def test_planted_mistake_is_caught(oracle):
    # a transposed weight (a plausible layout slip) must fail the float64 comparison used above
    x = synth.uniform(91, (1, 4, 7, 7))
    w = synth.normal(92, (4, 4, 3, 3), 0, 0.05)
    ref = oracle.conv2d_f64(x, w, None, (1, 1), (1, 1), (1, 1), 1, (7, 7))
    bad = oracle.conv2d_f32(x, np.ascontiguousarray(w.transpose(0, 1, 3, 2)), None, (1, 1), (1, 1), (1, 1), 1, (7, 7))
    assert np.abs(bad - ref).max() > 1e-3


# ---- segment-continuity ops (YOLO11n glue): pinned by closed forms

def test_softmax_matches_float64(oracle):
    x = np.random.default_rng(5).standard_normal((37, 401)).astype(np.float32) * 4
    scale = np.float32(32.0 ** -0.5)
    y = oracle.softmax(x, float(scale))
    v = (x * scale).astype(np.float64)
    e = np.exp(v - v.max(axis=1, keepdims=True))
    ref = e / e.sum(axis=1, keepdims=True)
    assert np.abs(y - ref).max() <= 2e-6 + 1e-5 * np.abs(ref).max()
    # the product is rounded to float before the row max (the Mul node runs first)
    assert oracle.softmax(np.array([[1.0, 2.0]], np.float32), 3.0).argmax() == 1


def test_maxpool_matches_brute_force(oracle):
    x = np.random.default_rng(6).standard_normal((2, 3, 11, 9)).astype(np.float32)
    for k, s, p in [(5, 1, 2), (3, 2, 1), (2, 2, 0)]:
        y = oracle.maxpool2d(x, k, s, p)
        xp = np.pad(x, ((0, 0), (0, 0), (p, p), (p, p)), constant_values=-np.inf)
        oh, ow = y.shape[2:]
        ref = np.empty_like(y)
        for i in range(oh):
            for j in range(ow):
                ref[:, :, i, j] = xp[:, :, i * s:i * s + k, j * s:j * s + k].max(axis=(2, 3))
        assert np.array_equal(y, ref), (k, s, p)


def test_maxpool_skips_nans_like_the_scalar_path(oracle):
    # DnnOps.cs:1564-1579: best = -inf; best = v when v > best.  A NaN never
    # wins, wherever it sits in the window; a window of NaNs only stays -inf.
    x = np.array([[[[np.nan, 1.0, -2.0], [np.nan, np.nan, np.nan], [3.0, np.nan, -5.0]]]], np.float32)
    y = oracle.maxpool2d(x, 3, 1, 1)
    xp = np.pad(x[0, 0], 1, constant_values=-np.inf)
    expect = np.array([[np.nanmax(xp[i:i + 3, j:j + 3]) for j in range(3)] for i in range(3)], np.float32)
    assert np.array_equal(y[0, 0], expect)
    assert y[0, 0, 0, 0] == 1.0 and y[0, 0, 2, 0] == 3.0 and y[0, 0, 2, 2] == -5.0
    z = oracle.maxpool2d(np.full((1, 1, 2, 2), np.nan, np.float32), 1, 1, 0)
    assert (z == -np.inf).all()


def test_resize_nearest_is_repeat(oracle):
    x = np.random.default_rng(7).standard_normal((1, 4, 5, 3)).astype(np.float32)
    assert np.array_equal(oracle.resize_nearest(x, 2), x.repeat(2, axis=2).repeat(2, axis=3))


def test_gemm_ex_against_float64(oracle):
    # ONNX Gemm restated: transposes, chain from 0, alpha * y + beta * c -- checked
    # against a float64 evaluation of the definition for every transpose pair
    rng = np.random.default_rng(9)
    m, k, n = 13, 29, 7
    for ta in (False, True):
        for tb in (False, True):
            a = rng.uniform(-1, 1, (k, m) if ta else (m, k)).astype(np.float32)
            b = rng.uniform(-1, 1, (n, k) if tb else (k, n)).astype(np.float32)
            c = rng.uniform(-1, 1, (n,)).astype(np.float32)
            y = oracle.gemm_ex(a, b, c, 0.5, 2.0, ta, tb)
            a64 = a.T.astype(np.float64) if ta else a.astype(np.float64)
            b64 = b.T.astype(np.float64) if tb else b.astype(np.float64)
            ref = 0.5 * (a64 @ b64) + 2.0 * c[None, :]
            assert np.abs(y - ref).max() < 1e-5, (ta, tb)
    # C indexing: full, scalar, and the reference's j % len for other lengths
    a = rng.uniform(-1, 1, (4, 3)).astype(np.float32)
    b = rng.uniform(-1, 1, (3, 6)).astype(np.float32)
    base = oracle.gemm_ex(a, b)
    cs = np.arange(4, dtype=np.float32)
    y = oracle.gemm_ex(a, b, cs, 1.0, 1.0)
    assert np.array_equal(y, (base + cs[np.arange(6) % 4][None, :]).astype(np.float32))
    y = oracle.gemm_ex(a, b, np.float32([3.0]), 1.0, 1.0)
    assert np.array_equal(y, base + np.float32(3.0))


def test_dfl_against_float64_and_known_answers(oracle):
    # DflOps.cs: y = sum_b softmax_b(x) * b over each side's bins
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 64, 300)).astype(np.float32) * 3
    y = oracle.dfl(x)
    xd = x.astype(np.float64).reshape(2, 4, 16, 300)
    p = np.exp(xd - xd.max(2, keepdims=True))
    p /= p.sum(2, keepdims=True)
    ref = (p * np.arange(16)[None, None, :, None]).sum(2)
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    # equal logits: every e_b is exactly 1, the sum 16, each p 1/16 -> 7.5 exactly
    assert (oracle.dfl(np.full((1, 16, 20), 0.25, np.float32)) == 7.5).all()
    # one bin far above the rest: the expectation is that bin's index (bin 0
    # keeps the other bins' e^-40 weights, ~5e-16)
    hot = np.zeros((1, 16, 11), np.float32)
    hot[0, np.arange(11) % 16, np.arange(11)] = 40.0
    got = oracle.dfl(hot)[0, 0]
    assert np.array_equal(got[1:], np.arange(1, 11, dtype=np.float32)) and 0 < got[0] < 1e-12


def test_dfl_subtracts_the_column_max(oracle):
    # shifting a column's bins by an exactly representable constant leaves
    # every (x - max) and so every output bit unchanged
    rng = np.random.default_rng(12)
    x = (rng.integers(-40, 40, (1, 32, 50)) / 8.0).astype(np.float32)
    shifted = (x + np.float32(3.0)).astype(np.float32)
    assert np.array_equal(oracle.dfl(x), oracle.dfl(shifted))


def test_sigmoid_against_float64(oracle):
    x = np.linspace(-30, 30, 20001).astype(np.float32)
    y = oracle.sigmoid_ref(x)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.abs(y - ref).max() <= 2e-7
    assert oracle.sigmoid_ref(np.zeros(3, np.float32))[0] == 0.5


# ----------------------------------------------------------- summation order, pinned by planted magnitudes
#
# A 3x3 conv over a 32-channel 3x3 map (one output pixel, no padding).  Each
# product term is planted: +2^24 first, -2^24 at a chosen tap, and small powers
# of two elsewhere.  In float32 a term below 1 added to an accumulator of
# magnitude 2^24 is lost (the spacing there is 2), and an accumulator of small
# terms added to 2^24 is lost too, so the output is exactly the sum of the
# small terms that the chain adds AFTER the -2^24 term.  Which taps those are
# depends only on the order of the chain, so each order gives a different,
# hand-derived result.  Orders, as (ic, ky, kx) visiting sequences:
#   NCHWc  (NchwcConv.Row, src/OnnxSharp/Kernels/NchwcConv.cs:555-605):
#          channel block ib -> ky -> kx -> lane (ic = 16 ib + lane)
#   im2col (ConvKernels.cs:554-563; PackedConv.cs:420-440): ic -> ky -> kx
# and two plausible mistakes that must NOT reproduce the NCHWc result:
#   lane before kx (ib -> ky -> lane -> kx) and kx before ky (ib -> kx -> ky -> lane).

BIG = np.float32(2.0 ** 24)


def _order(kind, cin=32):
    if kind == "nchwc":
        return [(16 * ib + l, ky, kx) for ib in range(cin // 16) for ky in range(3) for kx in range(3) for l in range(16)]
    if kind == "im2col":
        return [(ic, ky, kx) for ic in range(cin) for ky in range(3) for kx in range(3)]
    if kind == "lane_before_kx":
        return [(16 * ib + l, ky, kx) for ib in range(cin // 16) for ky in range(3) for l in range(16) for kx in range(3)]
    if kind == "kx_before_ky":
        return [(16 * ib + l, ky, kx) for ib in range(cin // 16) for kx in range(3) for ky in range(3) for l in range(16)]
    raise ValueError(kind)


def _fma32(a, b, c):
    """float32 fmaf(a, b, c) with one rounding: the exact value is formed in
    rationals, checked to be exact in float64, then rounded once to float32."""
    from fractions import Fraction
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    d = float(exact)
    assert Fraction(d) == exact, "planted values must keep the exact sum inside float64"
    return np.float32(d)


def _planted(terms, cin=32):
    """x = 1 at every planted tap, w = the term: each product is exactly the term."""
    x = np.zeros((1, cin, 3, 3), np.float32)
    w = np.zeros((1, cin, 3, 3), np.float32)
    for (ic, ky, kx), v in terms.items():
        x[0, ic, ky, kx] = 1.0
        w[0, ic, ky, kx] = v
    return x, w


def _chain(kind, x, w, bias):
    acc = np.float32(bias)
    for ic, ky, kx in _order(kind, x.shape[1]):
        acc = _fma32(x[0, ic, ky, kx], w[0, ic, ky, kx], acc)
    return acc


# (planted terms, hand-derived output per order)
PLANTED = [
    # -2^24 at (ic 1, ky 0, kx 0): NCHWc visits it 2nd (ib 0, tap 0, lane 1), im2col 10th.
    # 0.5 at (0, 0, 1) comes after it in NCHWc (tap 1) but before it in im2col and
    # with lane before kx; 0.25 at (2, 0, 0) and 0.125 at (17, 0, 0) come after in all.
    ({(0, 0, 0): BIG, (1, 0, 0): -BIG, (0, 0, 1): 0.5, (2, 0, 0): 0.25, (17, 0, 0): 0.125},
     {"nchwc": 0.875, "im2col": 0.375, "lane_before_kx": 0.375, "kx_before_ky": 0.875}),
    # -2^24 at (0, 1, 0): NCHWc tap 3, with kx before ky tap 1.  0.5 at (5, 0, 2) is
    # NCHWc tap 2 (before: lost) but tap 6 with kx before ky (after); im2col
    # visits ic 5 after ic 0 (kept); lane before kx visits it in row ky 0 (lost).
    # 0.25 in the second channel block is kept by every order.
    ({(0, 0, 0): BIG, (0, 1, 0): -BIG, (5, 0, 2): 0.5, (20, 0, 0): 0.25},
     {"nchwc": 0.25, "im2col": 0.75, "lane_before_kx": 0.25, "kx_before_ky": 0.75}),
    # the two channel blocks: -2^24 at (16, 2, 2) is the last NCHWc term but one
    # (lane 0 of the last tap of block 1); only 0.5 at (31, 2, 2) follows it.
    # im2col reaches (16, 2, 2) at index 152, after which ic 17..31 follow.
    ({(0, 0, 0): BIG, (16, 2, 2): -BIG, (31, 2, 2): 0.5, (20, 0, 0): 0.25, (15, 2, 2): 0.125},
     {"nchwc": 0.5, "im2col": 0.75, "lane_before_kx": 0.5, "kx_before_ky": 0.5}),
]


@pytest.mark.parametrize("case", range(len(PLANTED)))
def test_conv_chain_order_pinned_by_planted_magnitudes(oracle, case):
    terms, want = PLANTED[case]
    x, w = _planted(terms)
    b = np.zeros(1, np.float32)
    for kind, v in want.items():
        assert _chain(kind, x, w, 0.0) == np.float32(v), kind  # the hand derivation
    got_nchwc = oracle.conv2d_f32(x, w, b, (1, 1), (0, 0), (1, 1), 1, (1, 1), order=oracle.ORDER_NCHWC)
    got_im2col = oracle.conv2d_f32(x, w, b, (1, 1), (0, 0), (1, 1), 1, (1, 1), order=oracle.ORDER_IM2COL)
    assert got_nchwc[0, 0, 0, 0] == np.float32(want["nchwc"])
    assert got_im2col[0, 0, 0, 0] == np.float32(want["im2col"])
    # the order is what the test sees: each case separates NCHWc from at least one wrong order
    assert any(want[k] != want["nchwc"] for k in ("lane_before_kx", "kx_before_ky", "im2col"))


def test_planted_cases_separate_every_wrong_order():
    # over the three cases, each wrong order differs from NCHWc somewhere
    for wrong in ("im2col", "lane_before_kx", "kx_before_ky"):
        assert any(w[wrong] != w["nchwc"] for _, w in PLANTED), wrong


def test_conv_chain_starts_at_the_bias(oracle):
    # bias 2^24, then two terms of 1: bias-first loses each 1 (2^24 + 1 is a tie,
    # rounded to the even 2^24), bias-last would give 2^24 + 2
    x, w = _planted({(3, 1, 1): 1.0, (20, 2, 0): 1.0})
    b = np.array([BIG], np.float32)
    for order in (oracle.ORDER_NCHWC, oracle.ORDER_IM2COL):
        y = oracle.conv2d_f32(x, w, b, (1, 1), (0, 0), (1, 1), 1, (1, 1), order=order)
        assert y[0, 0, 0, 0] == BIG
    assert _chain("nchwc", x, w, BIG) == BIG
    assert np.float32(np.float32(2.0) + BIG) == BIG + 2


def test_planted_mistake_in_the_order_is_caught(oracle):
    # the same harness with the oracle's loop order changed (here: the
    # im2col chain asked to stand in for the NCHWc one) fails case 0
    terms, want = PLANTED[0]
    x, w = _planted(terms)
    wrong = oracle.conv2d_f32(x, w, np.zeros(1, np.float32), (1, 1), (0, 0), (1, 1), 1, (1, 1),
                              order=oracle.ORDER_IM2COL)
    assert wrong[0, 0, 0, 0] != np.float32(want["nchwc"])


# ----------------------------------------------------------- C2PSA attention core

def _attention_f64(qkv, heads, key_dim, head_dim, n, scale, swap_qk=False):
    """float64 attention from the definition (ultralytics Attention.forward as
    exported: attn = softmax(scale * q^T k) over keys, y = v attn^T); with
    swap_qk the planted mistake k^T q."""
    q3 = qkv.reshape(heads, 2 * key_dim + head_dim, n).astype(np.float64)
    out = []
    for h in range(heads):
        q, k, v = q3[h, :key_dim], q3[h, key_dim:2 * key_dim], q3[h, 2 * key_dim:]
        s = (k.T @ q if swap_qk else q.T @ k) * scale
        e = np.exp(s - s.max(axis=1, keepdims=True))
        p = e / e.sum(axis=1, keepdims=True)
        out.append(v @ p.T)
    return np.concatenate(out, axis=0)


def test_attention_matches_float64_and_catches_a_qk_swap(oracle):
    from types import SimpleNamespace as NS
    from oracle import yolo_frame
    heads, key_dim, head_dim, hw = 2, 32, 64, (8, 10)
    n = hw[0] * hw[1]
    qkv = synth.normal(51, (1, heads * (2 * key_dim + head_dim), *hw), 0, 1.0)
    op = NS(qkv=NS(h=hw[0], w=hw[1]), heads=heads, key_dim=key_dim, head_dim=head_dim,
            scale=key_dim ** -0.5, y=NS(c=heads * head_dim, h=hw[0], w=hw[1]))
    got = yolo_frame.attention(oracle, op, qkv).reshape(heads * head_dim, n).astype(np.float64)
    ref = _attention_f64(qkv, heads, key_dim, head_dim, n, op.scale)
    d = np.abs(got - ref)
    assert (d <= 1e-5 + 1e-4 * np.abs(ref)).all(), d.max()
    # the planted mistake: q and k exchanged gives attn^T's softmax, far off
    bad = _attention_f64(qkv, heads, key_dim, head_dim, n, op.scale, swap_qk=True)
    assert np.abs(got - bad).max() > 1e-2


# ----------------------------------------------------------- the blocked AVX-512 NCHWc restatement

NCHWC_FAST_CASES = [  # (C, H, W, M, stride, bias)
    (64, 40, 40, 64, 1, True),      # C2's layer at a quarter of the map
    (128, 40, 40, 256, 2, True),    # C3b's layer at half the map
    (32, 18, 22, 64, 1, True),      # a row tail (22 = 2 x 8 + 6)
    (16, 40, 36, 32, 2, False),     # stride 2, tail, no bias
    (48, 7, 9, 96, 1, True),        # a map narrower than one 8-pixel group on the last row part
]


@pytest.mark.parametrize("case", NCHWC_FAST_CASES, ids=[str(c) for c in NCHWC_FAST_CASES])
@pytest.mark.parametrize("threads", [1, 3])
def test_nchwc_avx512_is_the_nchwc_chain(oracle, case, threads):
    # orc_nchwc_conv_avx512 (blocked input and weights, 2 output blocks x 8
    # pixels a step, the reference's NchwcConv.Row structure) against the scalar
    # loop in the same ib -> ky -> kx -> lane order: the same bits
    if not oracle.nchwc_avx512_ok():
        pytest.skip("no AVX-512 on this host")
    cin, h, w_, m, s, with_bias = case
    x = synth.uniform(31 + cin, (1, cin, h, w_))
    w = synth.normal(32 + m, (m, cin, 3, 3), 0, 0.05)
    b = synth.normal(33, (m,), 0, 0.01) if with_bias else None
    oh, ow = (h, w_) if s == 1 else (h // 2, w_ // 2)
    old = oracle.lib().orc_get_threads()
    oracle.set_threads(threads)
    try:
        fast = oracle.conv_nchwc_avx512(x, w, b, s, (oh, ow))
        ref = oracle.conv2d_f32(x, w, b, (s, s), (1, 1), (1, 1), 1, (oh, ow), order=oracle.ORDER_NCHWC)
        via = oracle.conv_reference(x, w, b, (s, s), (1, 1), (1, 1), 1, (oh, ow))
    finally:
        oracle.set_threads(old)
    assert np.array_equal(fast.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(via.view(np.uint32), ref.view(np.uint32))  # conv_reference takes the fast path


@pytest.mark.parametrize("case", range(len(PLANTED)))
def test_nchwc_avx512_order_pinned_by_planted_magnitudes(oracle, case):
    # the planted terms on a 3x3 map with pad 1 (the gate's padding): the
    # centre output pixel of channel 0 sees every tap, so it must give the
    # hand-derived NCHWc value, not one of the wrong orders'
    if not oracle.nchwc_avx512_ok():
        pytest.skip("no AVX-512 on this host")
    terms, want = PLANTED[case]
    x, w1 = _planted(terms)
    w = np.zeros((32, 32, 3, 3), np.float32)
    w[0] = w1[0]
    y = oracle.conv_nchwc_avx512(x, w, np.zeros(32, np.float32), 1, (3, 3))
    assert y[0, 0, 1, 1] == np.float32(want["nchwc"])


# ----------------------------------------------------------- the oracle's vector paths equal its scalar loops

@pytest.mark.parametrize("m,k,n,bias", [(1024, 768, 768, "col"), (37, 100, 53, "row"), (128, 256, 6400, "row"),
                                        (5, 3, 17, None), (9, 40, 33, "col")])
def test_blocked_gemm_is_the_gemm_chain(oracle, m, k, n, bias):
    # the register-blocked AVX-512 GEMM (packed 32-column panels, 8 x 32 blocks)
    # computes every element's k-ascending fmaf chain from the bias: the same
    # bits as the row loop
    a = synth.uniform(m + 1, (m, k), -1, 1)
    b = synth.uniform(n + 2, (k, n), -1, 1)
    kw = {} if bias is None else {f"{bias}_bias": synth.uniform(3, (n if bias == "col" else m,), -1, 1)}
    assert np.array_equal(oracle.gemm_f32(a, b, **kw).view(np.uint32), oracle.gemm_f32_rows(a, b, **kw).view(np.uint32))


def test_pointwise_conv_through_the_gemm_is_the_im2col_chain(oracle):
    x = synth.uniform(41, (2, 48, 9, 13))
    w = synth.normal(42, (40, 48, 1, 1), 0, 0.05)
    b = synth.normal(43, (40,), 0, 0.01)
    args = ((1, 1), (0, 0), (1, 1), 1, (9, 13))
    fast = oracle.conv_reference(x, w, b, *args)
    slow = oracle.conv2d_f32(x, w, b, *args, order=oracle.ORDER_IM2COL)
    assert np.array_equal(fast.view(np.uint32), slow.view(np.uint32))


@pytest.mark.parametrize("op", [0, 1, 2])
def test_vector_activations_are_the_scalar_loop(oracle, op):
    x = np.concatenate([synth.normal(50 + op, (70001,), 0, 12),
                        np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 88.7, -87.3, 89, -88, 1e30, -1e30],
                                 np.float32)]).astype(np.float32)
    fast = {0: oracle.exp_ref, 1: oracle.silu_ref, 2: oracle.sigmoid_ref}[op](x)
    slow = oracle.unary_scalar(op, x)
    assert np.array_equal(fast.view(np.uint32), slow.view(np.uint32))


@pytest.mark.parametrize("m,k,n,wdt,zp", [(512, 512, 2048, np.int8, None), (33, 100, 70, np.uint8, "column"),
                                          (17, 64, 40, np.uint8, "tensor")])
def test_dqmm_through_the_widened_gemm_is_the_dqmm_chain(oracle, m, k, n, wdt, zp):
    # QuantizeAndWiden + the blocked F32 GEMM with the fused column-scale
    # epilogue (the reference's own CPU route, and the cpu_baseline's) gives
    # dqmm's output bit for bit; the blocked GEMM with a column scale equals
    # the row loop, fused and unfused
    a = synth.normal(m + k, (m, k))
    lo, hi = (-127, 127) if wdt == np.int8 else (0, 255)
    w = synth.randint(m + n, (k, n), lo, hi, wdt)
    wzp = None if zp is None else (np.array([131], np.int32) if zp == "tensor"
                                   else synth.randint(n, (n,), -20, 20, np.int32) + 128)
    ws = synth.uniform(k + n, (n,), 0.001, 0.02)
    b = synth.normal(m + k + n, (n,), 0, 0.01)
    got = oracle.dqmm_widened_gemm(a, w, wzp, ws, b)
    assert np.array_equal(got.view(np.uint32), oracle.dqmm(a, w, wzp, ws, b, fused=True)[0].view(np.uint32))
    af = synth.uniform(3, (m, k), -4, 4)
    wf = synth.uniform(4, (k, n), -4, 4)
    for fused in (True, False):
        for cb in (b, None):
            x = oracle.gemm_f32(af, wf, col_bias=cb, col_scale=ws, fused=fused)
            y = oracle.gemm_f32_rows(af, wf, col_bias=cb, col_scale=ws, fused=fused)
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
