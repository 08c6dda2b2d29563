"""GPU parity: Conv (+ bias + fused Relu/SiLU) through osh_conv2d_f32 against
the oracle's restatements of the reference kernels, in both accumulation
orders the reference uses (NCHWc on AVX-512 hosts, im2col/panel on AVX2)."""
import ctypes as C
import json
import os

import numpy as np
import pytest

from conftest import assert_fp32_close, fp32_violations
from onnxsharp_amd import synth

pytestmark = pytest.mark.gpu


def _t(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def run_conv(cuda, x, w, b, act=None, **attrs):
    from onnxsharp_amd.layers import ConvLayer
    layer = ConvLayer(fused_activation=act, **attrs)
    y = layer.forward(_t(x, cuda), _t(w, cuda), None if b is None else _t(b, cuda))
    return y.cpu().numpy(), layer.resolve(x.shape, w.shape)


def oracle_conv(oracle, x, w, b, p, act, order=None, winograd=1, nchwc=1):
    """The oracle's conv: with order None the kernel the reference's dispatch
    picks for the shape (depthwise, NCHWc, Winograd or im2col chain; nchwc = 0
    on a host without NchwcConv), else the given accumulation order."""
    args = (x, w, b, (p.sh, p.sw), (p.pt, p.pl), (p.dh, p.dw), p.group, (p.oh, p.ow))
    if order is None:
        y = oracle.conv_reference(*args, winograd=winograd, nchwc=nchwc)
    else:
        y = oracle.conv2d_f32(*args, order=order)
    if act == "Silu":
        y = oracle.silu_ref(y)
    elif act == "Relu":
        y = oracle.relu(y)
    return y


# (name, x shape, w shape, attrs, act)
CASES = [
    ("c2_3x3s1_64to64_160", (1, 64, 160, 160), (64, 64, 3, 3), dict(pads=[1, 1, 1, 1]), "Silu"),
    ("c3a_1x1_256to128_80", (1, 256, 80, 80), (128, 256, 1, 1), dict(), "Silu"),
    ("c3b_3x3s2_128to256_80", (1, 128, 80, 80), (256, 128, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1]), "Silu"),
    ("yolo_stem_3to16_s2", (1, 3, 64, 64), (16, 3, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1]), "Silu"),
    ("3x3s1_small_spatial_20", (1, 64, 20, 20), (64, 64, 3, 3), dict(pads=[1, 1, 1, 1]), "Silu"),
    ("3x3s1_c32_m40_partial_tiles", (1, 32, 18, 24), (40, 32, 3, 3), dict(pads=[1, 1, 1, 1]), "Silu"),
    ("3x3s1_c16_batch2", (2, 16, 12, 16), (16, 16, 3, 3), dict(pads=[1, 1, 1, 1]), "Relu"),
    ("3x3s1_c64_m96_80", (1, 64, 40, 80), (96, 64, 3, 3), dict(pads=[1, 1, 1, 1]), None),
    ("3x3s2_c64_m64_40", (1, 64, 80, 80), (64, 64, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1]), "Silu"),
    ("3x3s1_odd_33x45", (1, 24, 33, 45), (40, 24, 3, 3), dict(pads=[1, 1, 1, 1]), "Relu"),
    ("3x3s2_odd_41x37", (1, 16, 41, 37), (72, 16, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1]), None),
    ("1x1_no_bias_batch2", (2, 40, 17, 19), (24, 40, 1, 1), dict(), None),
    ("grouped_2", (2, 8, 9, 7), (6, 4, 3, 3), dict(group=2, strides=[1, 2], pads=[0, 1, 0, 1]), "Silu"),
    ("dilated_5x5", (1, 5, 23, 21), (7, 5, 5, 5), dict(pads=[4, 4, 4, 4], dilations=[2, 2]), None),
    ("depthwise_3x3", (1, 32, 20, 20), (32, 1, 3, 3), dict(group=32, pads=[1, 1, 1, 1]), None),
    ("depthwise_3x3_s2", (1, 24, 19, 18), (24, 1, 3, 3), dict(group=24, strides=[2, 2], pads=[1, 1, 1, 1]), "Silu"),
    ("depthwise_3x3_batch2_pad0", (2, 16, 11, 13), (16, 1, 3, 3), dict(group=16), "Relu"),
    ("depthwise_5x5_generic", (1, 12, 15, 17), (12, 1, 5, 5), dict(group=12, pads=[2, 2, 2, 2]), "Silu"),
    ("depthwise_3x3_dilated_generic", (1, 8, 14, 16), (8, 1, 3, 3), dict(group=8, pads=[2, 2, 2, 2], dilations=[2, 2]),
     None),
    ("same_upper_s2", (1, 1, 9, 11), (1, 1, 3, 3), dict(auto_pad="SAME_UPPER", strides=[2, 2]), None),
    ("valid_1x3", (1, 6, 10, 12), (4, 6, 1, 3), dict(auto_pad="VALID"), None),
]


@pytest.mark.parametrize("name,xs,ws,attrs,act", CASES, ids=[c[0] for c in CASES])
def test_conv_parity(cuda, oracle, name, xs, ws, attrs, act):
    # Every default kernel sums in the order of the reference's kernel for the
    # shape on an AVX-512 host: the depthwise chain, the NCHWc chain where
    # NchwcConv's gate holds, Winograd where Winograd's gate holds, else the
    # im2col / GEMM chain.  With the exact SiLU the output is the oracle's, bit
    # for bit; with the default SiLU it is within the FP32 bar (and within it
    # of the plain im2col order too).
    from onnxsharp_amd import native as N
    print(f"conv {name} x={xs} w={ws} {attrs} act={act}", flush=True)
    seed = sum(xs) * 7 + sum(ws)
    x = synth.uniform(seed, xs)
    w = synth.normal(seed + 1, ws, 0, 0.05)
    b = None if "no_bias" in name else synth.normal(seed + 2, (ws[0],), 0, 0.01)
    y, p = run_conv(cuda, x, w, b, act, **attrs)
    ref = oracle_conv(oracle, x, w, b, p, act)
    nbad, dmax = fp32_violations(y, ref)
    print(f"  max|d|={dmax:.3e} violations={nbad}", flush=True)
    assert_fp32_close(y, ref, name)
    alt = oracle_conv(oracle, x, w, b, p, act, order=oracle.ORDER_IM2COL)
    assert_fp32_close(y, alt, name + " (im2col order)")
    N.call("osh_config_set", b"exact_silu", 1)
    try:
        ye, _ = run_conv(cuda, x, w, b, act, **attrs)
    finally:
        N.call("osh_config_set", b"exact_silu", 0)
    ref = oracle_conv(oracle, x, w, b, p, act)
    assert np.array_equal(ye, ref), f"{name}: max |d| {np.abs(ye - ref).max():.3e}"


def test_conv_known_answer_same_upper(cuda):
    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))["conv_same_upper_s2"]
    x = np.arange(1, 100, dtype=np.float32).reshape(1, 1, 9, 11)
    w = np.ones((1, 1, 3, 3), np.float32)
    ya, _ = run_conv(cuda, x, w, None, auto_pad="SAME_UPPER", strides=[2, 2])
    yb, _ = run_conv(cuda, x, w, None, pads=[1, 1, 1, 1], strides=[2, 2])
    assert ya.shape == tuple(g["out_shape"])
    assert (ya[0, 0] == np.array(g["y"], np.float32)).all()
    assert (ya == yb).all()


def test_conv_silu_epilogue_on_bias_only_input(cuda, oracle):
    # zero input: the conv output is exactly the bias, so the fused SiLU can be
    # compared on its own.  exact_silu=1 must reproduce VectorMath.Silu bit for
    # bit; the default exp2/rcp epilogue must stay within 2e-6 of it.
    from onnxsharp_amd import native as N
    x = np.zeros((1, 64, 40, 40), np.float32)
    w = synth.normal(5, (64, 64, 3, 3), 0, 0.05)
    b = synth.normal(6, (64,), 0, 3.0)
    expect = oracle.silu_ref(b)[:, None, None]
    old = C.c_int()
    N.call("osh_config_get", b"exact_silu", C.byref(old))
    try:
        N.call("osh_config_set", b"exact_silu", 1)
        y, _ = run_conv(cuda, x, w, b, "Silu", pads=[1, 1, 1, 1])
        assert (y[0] == expect).all()
        N.call("osh_config_set", b"exact_silu", 0)
        y, _ = run_conv(cuda, x, w, b, "Silu", pads=[1, 1, 1, 1])
        rel = np.abs(y[0] - expect) / np.maximum(np.abs(expect), 1e-30)
        assert rel.max() < 2e-6
    finally:
        N.call("osh_config_set", b"exact_silu", old.value)


@pytest.mark.parametrize("xs,ws,attrs", [
    ((1, 3, 640, 640), (16, 3, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1])),  # the YOLO11n stem
    ((1, 3, 37, 41), (8, 3, 3, 3), dict(pads=[1, 1, 1, 1])),
    ((2, 4, 20, 18), (32, 4, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1])),
    ((1, 1, 9, 11), (8, 1, 3, 3), dict(auto_pad="SAME_UPPER", strides=[2, 2])),
    ((1, 8, 160, 160), (16, 8, 3, 3), dict(pads=[1, 1, 1, 1])),  # YOLO11n's 8 -> 16 bottleneck conv
    ((2, 8, 21, 19), (32, 8, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1])),
    ((1, 16, 40, 40), (8, 16, 3, 3), dict(strides=[3, 3], pads=[1, 1, 1, 1])),
    ((1, 32, 30, 31), (16, 32, 3, 3), dict(strides=[1, 2], pads=[1, 1, 1, 1])),
], ids=["stem_640", "c3_m8_s1", "c4_m32_s2_batch2", "c1_m8_same_upper", "c8_m16_160", "c8_m32_s2_batch2",
        "c16_m8_s3", "c32_m16_s1x2"])
def test_first_layer_conv_is_the_fma_chain(cuda, oracle, xs, ws, attrs):
    # C <= 4, and 3x3 layers with C = 8 (or 16/32 at strides the LDS-patch
    # tiles do not take) that neither the NCHWc nor the Winograd gate takes,
    # run the direct per-pixel kernel: per output channel the bias, then fmaf
    # over ic -> ky -> kx, the im2col chain -- bit for bit.
    from onnxsharp_amd import native as N
    seed = sum(xs) + sum(ws)
    x = synth.uniform(seed, xs)
    w = synth.normal(seed + 1, ws, 0, 0.05)
    b = synth.normal(seed + 2, (ws[0],), 0, 0.01)
    N.call("osh_config_set", b"exact_silu", 1)
    try:
        y, p = run_conv(cuda, x, w, b, "Silu", **attrs)
    finally:
        N.call("osh_config_set", b"exact_silu", 0)
    ref = oracle_conv(oracle, x, w, b, p, "Silu", order=oracle.ORDER_IM2COL)
    assert np.array_equal(y, ref), f"max |d| {np.abs(y - ref).max():.3e}"


CONV16_CASES = [
    ("c2_3x3s1_64to64_160", (1, 64, 160, 160), (64, 64, 3, 3), dict(pads=[1, 1, 1, 1])),
    ("c3b_3x3s2_128to256_80", (1, 128, 80, 80), (256, 128, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1])),
    ("deep_256to64_20", (1, 256, 20, 20), (64, 256, 3, 3), dict(pads=[1, 1, 1, 1])),
    ("odd_16to40_s1_33x45", (1, 16, 33, 45), (40, 16, 3, 3), dict(pads=[1, 1, 1, 1])),
    ("odd_32to72_s2_41x37", (2, 32, 41, 37), (72, 32, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1])),
    ("pads_0_2_valid_like", (1, 48, 17, 23), (24, 48, 3, 3), dict(pads=[0, 2, 2, 0])),
    ("stride3_16to16_20", (1, 16, 20, 20), (16, 16, 3, 3), dict(strides=[3, 3], pads=[1, 1, 1, 1])),
    ("tall_narrow_32to16_70x9", (1, 32, 70, 9), (16, 32, 3, 3), dict(pads=[1, 1, 1, 1])),
    ("s2_64to48_batch2_23x29", (2, 64, 23, 29), (48, 64, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1])),
    ("deep_256to80_s1_13x11", (1, 256, 13, 11), (80, 256, 3, 3), dict(pads=[1, 1, 1, 1])),
]


@pytest.mark.parametrize("name,xs,ws,attrs", CONV16_CASES, ids=[c[0] for c in CONV16_CASES])
def test_conv16_is_the_nchwc_chain(cuda, oracle, name, xs, ws, attrs):
    # A forced tile runs the in-order 16x16x4 kernels on any 3x3 shape with
    # C % 16 == 0: bit for bit the reference's NCHWc chain (bias, then icb ->
    # ky -> kx -> lane16), whatever tile -- weights streamed or in LDS, or the
    # input patch staged in LDS (stride 1 and 2; other strides fall back to the
    # cost model).  The default dispatch takes them where NchwcConv's gate holds.
    from onnxsharp_amd import native as N
    seed = sum(xs) * 3 + sum(ws)
    x = synth.uniform(seed, xs)
    w = synth.normal(seed + 1, ws, 0, 0.05)
    b = synth.normal(seed + 2, (ws[0],), 0, 0.01)
    nv = C.c_int()
    N.call("osh_config_get", b"conv16_variants", C.byref(nv))
    assert nv.value >= 21
    N.call("osh_config_set", b"exact_silu", 1)
    try:
        ref = None
        for v in range(nv.value):
            print(f"conv16 {name} variant {v}", flush=True)
            N.call("osh_config_set", b"conv16_variant", v)
            y, p = run_conv(cuda, x, w, b, "Silu", **attrs)
            if ref is None:
                ref = oracle_conv(oracle, x, w, b, p, "Silu", order=oracle.ORDER_NCHWC)
            assert np.array_equal(y, ref), f"variant {v}: max |d| {np.abs(y - ref).max():.3e}"
    finally:
        N.call("osh_config_set", b"exact_silu", 0)
        N.call("osh_config_set", b"conv16_variant", -1)


RESIDUAL_CASES = [
    # (name, x, w, attrs, conv16_variant) -- one per kernel family of the dispatch
    ("conv16_3x3_64to64_40", (1, 64, 40, 40), (64, 64, 3, 3), dict(pads=[1, 1, 1, 1]), 4),
    ("conv16l_3x3_32to32_20_batch2", (2, 32, 20, 20), (32, 32, 3, 3), dict(pads=[1, 1, 1, 1]), 10),
    ("conv16s_3x3_32to48_s2_batch2", (2, 32, 21, 19), (48, 32, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1]), 17),
    ("conv16s_3x3_64to64_40", (1, 64, 40, 40), (64, 64, 3, 3), dict(pads=[1, 1, 1, 1]), 13),
    ("conv16_tuned_16to32_80", (1, 16, 80, 80), (32, 16, 3, 3), dict(pads=[1, 1, 1, 1]), -1),
    ("gemm16_1x1_128to64_20", (1, 128, 20, 20), (64, 128, 1, 1), dict(), -1),
    ("pw_gemm_tile_1x1_64to48_40", (1, 64, 40, 40), (48, 64, 1, 1), dict(), 0),
    ("pw_lds_tile_1x1_80to64_20x24", (2, 80, 20, 24), (64, 80, 1, 1), dict(), 5),
    ("pw_lds_tile_1x1_48to32_odd", (1, 48, 17, 19), (32, 48, 1, 1), dict(), 3),
    ("igemm_1x1_c6_odd", (2, 6, 13, 11), (10, 6, 1, 1), dict(), -1),
    ("direct3x3_c8_160", (1, 8, 160, 160), (16, 8, 3, 3), dict(pads=[1, 1, 1, 1]), -1),
    ("depthwise_64_20", (1, 64, 20, 20), (64, 1, 3, 3), dict(group=64, pads=[1, 1, 1, 1]), -1),
    ("first_conv_c3", (1, 3, 64, 64), (16, 3, 3, 3), dict(pads=[1, 1, 1, 1]), -1),
    ("direct_c8_m16_160", (1, 8, 160, 160), (16, 8, 3, 3), dict(pads=[1, 1, 1, 1]), -1),
    ("im2col_tiles_32to16_80", (1, 32, 80, 80), (16, 32, 3, 3), dict(pads=[1, 1, 1, 1]), -1),
    ("direct_c32_m16_s1x2", (1, 32, 30, 31), (16, 32, 3, 3), dict(strides=[1, 2], pads=[1, 1, 1, 1]), -1),
    ("winograd_32to40_18x24", (1, 32, 18, 24), (40, 32, 3, 3), dict(pads=[1, 1, 1, 1]), -1),
    ("winograd_c24_batch2_odd", (2, 24, 13, 11), (16, 24, 3, 3), dict(pads=[1, 1, 1, 1]), -1),
    ("im2col_dilated_5x5", (1, 5, 23, 21), (7, 5, 5, 5), dict(pads=[4, 4, 4, 4], dilations=[2, 2]), -1),
]


@pytest.mark.parametrize("name,xs,ws,attrs,variant", RESIDUAL_CASES, ids=[c[0] for c in RESIDUAL_CASES])
def test_conv_residual_add_is_conv_then_add(cuda, name, xs, ws, attrs, variant):
    # osh_conv2d_add_f32 = osh_conv2d_f32 followed by the Add, bit for bit:
    # the epilogue rounds the activation output, then adds the residual once.
    import torch
    from onnxsharp_amd import native as N
    from onnxsharp_amd.layers import ConvLayer
    print(f"conv+add {name} x={xs} w={ws} variant={variant}", flush=True)
    seed = sum(xs) * 11 + sum(ws)
    x = _t(synth.uniform(seed, xs), cuda)
    w = _t(synth.normal(seed + 1, ws, 0, 0.05), cuda)
    b = _t(synth.normal(seed + 2, (ws[0],), 0, 0.01), cuda)
    key = b"pointwise_variant" if name.startswith("pw_") else b"conv16_variant"
    N.call("osh_config_set", key, variant)
    try:
        layer = ConvLayer(fused_activation="Silu", **attrs)
        plain = layer.forward(x, w, b)
        res = torch.from_numpy(synth.normal(seed + 3, tuple(plain.shape), 0, 1)).to(cuda)
        fused = layer.forward(x, w, b, residual=res)
        torch.cuda.synchronize()
    finally:
        N.call("osh_config_set", key, -1)
    expect = plain.cpu().numpy() + res.cpu().numpy()
    got = fused.cpu().numpy()
    assert np.array_equal(got, expect), f"max |d| {np.abs(got - expect).max():.3e}"


POINTWISE_CASES = [
    ("c3a_1x1_256to128_80", (1, 256, 80, 80), (128, 256, 1, 1)),
    ("1x1_64to64_20", (1, 64, 20, 20), (64, 64, 1, 1)),
    ("1x1_80to80_40_two_chunks", (1, 80, 40, 40), (80, 80, 1, 1)),
    ("1x1_48to40_odd_17x19", (1, 48, 17, 19), (40, 48, 1, 1)),
    ("1x1_32to24_batch2", (2, 32, 12, 16), (24, 32, 1, 1)),
    ("1x1_512to256_20", (1, 512, 20, 20), (256, 512, 1, 1)),
]


@pytest.mark.parametrize("name,xs,ws", POINTWISE_CASES, ids=[c[0] for c in POINTWISE_CASES])
def test_pointwise_tiles_are_the_gemm_chain(cuda, oracle, name, xs, ws):
    # 1x1 stride-1 convolutions with C % 16 == 0 choose between the GEMM tile
    # (variant 0) and the LDS-tile kernel (1..): every choice is the GEMM chain
    # (bias, then input channels ascending), bit for bit, including partial
    # channel chunks and maps whose width is not a multiple of four
    from onnxsharp_amd import native as N
    seed = sum(xs) * 13 + sum(ws)
    x = synth.uniform(seed, xs)
    w = synth.normal(seed + 1, ws, 0, 0.05)
    b = synth.normal(seed + 2, (ws[0],), 0, 0.01)
    nv = C.c_int()
    N.call("osh_config_get", b"pointwise_variants", C.byref(nv))
    assert nv.value >= 9
    N.call("osh_config_set", b"exact_silu", 1)
    try:
        ref = None
        for v in [-1] + list(range(nv.value)):
            print(f"pointwise {name} variant {v}", flush=True)
            N.call("osh_config_set", b"pointwise_variant", v)
            y, p = run_conv(cuda, x, w, b, "Silu")
            if ref is None:
                ref = oracle_conv(oracle, x, w, b, p, "Silu", order=oracle.ORDER_IM2COL)
            assert np.array_equal(y, ref), f"variant {v}: max |d| {np.abs(y - ref).max():.3e}"
    finally:
        N.call("osh_config_set", b"exact_silu", 0)
        N.call("osh_config_set", b"pointwise_variant", -1)


WINOGRAD_CASES = [
    # (name, x, w, act, residual)
    ("yolo_64to64_20", (1, 64, 20, 20), (64, 64, 3, 3), "Silu", False),
    ("yolo_deep_256to64_20", (1, 256, 20, 20), (64, 256, 3, 3), "Silu", False),
    ("yolo_32to32_40", (1, 32, 40, 40), (32, 32, 3, 3), "Silu", True),
    ("max_map_128to64_64x64", (1, 128, 64, 64), (64, 128, 3, 3), None, False),
    ("batch2_16to16", (2, 16, 12, 16), (16, 16, 3, 3), "Relu", False),
    ("odd_24to40_33x45", (1, 24, 33, 45), (40, 24, 3, 3), "Silu", True),
    ("min_8to8_6x6", (1, 8, 6, 6), (8, 8, 3, 3), None, False),
    ("partial_40to24_7x9_no_bias", (1, 40, 7, 9), (24, 40, 3, 3), "Silu", False),
]


@pytest.mark.parametrize("name,xs,ws,act,residual", WINOGRAD_CASES, ids=[c[0] for c in WINOGRAD_CASES])
def test_winograd_is_the_reference_winograd(cuda, oracle, name, xs, ws, act, residual):
    # winograd = 2 runs every Winograd-eligible shape through wino_f23_kernel:
    # Winograd.cs's weight, input and output transforms and its k-ascending
    # component GEMMs, bit for bit against the oracle's restatement (exact SiLU),
    # within the FP32 bar of the direct conv, and the residual epilogue is the
    # conv then the Add.
    import torch
    from onnxsharp_amd import native as N
    from onnxsharp_amd.layers import ConvLayer
    print(f"winograd {name} x={xs} w={ws} act={act} residual={residual}", flush=True)
    seed = sum(xs) * 17 + sum(ws)
    x = synth.uniform(seed, xs)
    w = synth.normal(seed + 1, ws, 0, 0.05)
    b = None if "no_bias" in name else synth.normal(seed + 2, (ws[0],), 0, 0.01)
    attrs = dict(pads=[1, 1, 1, 1])
    old = C.c_int()
    N.call("osh_config_get", b"winograd", C.byref(old))
    N.call("osh_config_set", b"winograd", 2)
    N.call("osh_config_set", b"exact_silu", 1)
    try:
        layer = ConvLayer(fused_activation=act, **attrs)
        xt, wt, bt = _t(x, cuda), _t(w, cuda), None if b is None else _t(b, cuda)
        y = layer.forward(xt, wt, bt)
        p = layer.resolve(x.shape, w.shape)
        if residual:
            r = torch.from_numpy(synth.normal(seed + 3, tuple(y.shape), 0, 1)).to(cuda)
            yr = layer.forward(xt, wt, bt, residual=r)
            torch.cuda.synchronize()
            assert np.array_equal(yr.cpu().numpy(), y.cpu().numpy() + r.cpu().numpy())
        y = y.cpu().numpy()
    finally:
        N.call("osh_config_set", b"winograd", old.value)
        N.call("osh_config_set", b"exact_silu", 0)
    assert oracle.conv_reference_kernel(x.shape, w.shape, (1, 1), (1, 1), (1, 1), 1, (p.oh, p.ow),
                                        winograd=2) == oracle.KERNEL_WINOGRAD
    ref = oracle_conv(oracle, x, w, b, p, act, winograd=2)
    assert np.array_equal(y, ref), f"max |d| {np.abs(y - ref).max():.3e} at {np.argwhere(y != ref)[:3]}"
    direct = oracle_conv(oracle, x, w, b, p, act, order=oracle.ORDER_IM2COL)
    assert_fp32_close(y, direct, name + " (direct conv)")


IM2COL3X3_CASES = [
    # 3x3 shapes with C % 16 == 0 that the reference runs on its im2col chain
    ("yolo_32to16_80", (1, 32, 80, 80), (16, 32, 3, 3), dict(pads=[1, 1, 1, 1])),
    ("yolo_16to8_160", (1, 16, 160, 160), (8, 16, 3, 3), dict(pads=[1, 1, 1, 1])),
    ("s2_odd_32to72_41x37", (1, 32, 41, 37), (72, 32, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1])),
    ("s2_batch2_48to40", (2, 48, 20, 22), (40, 48, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1])),
    ("s1_wide_64to48_70x90", (1, 64, 70, 90), (48, 64, 3, 3), dict(pads=[1, 1, 1, 1])),
    ("pads_0_2_48to24", (1, 48, 17, 23), (24, 48, 3, 3), dict(pads=[0, 2, 2, 0])),
]


@pytest.mark.parametrize("name,xs,ws,attrs", IM2COL3X3_CASES, ids=[c[0] for c in IM2COL3X3_CASES])
def test_im2col_order_tiles_are_the_im2col_chain(cuda, oracle, name, xs, ws, attrs):
    # The LDS-patch tiles with each 16-channel block's terms in the im2col
    # order: bit for bit the reference's im2col chain (bias, then ic -> ky ->
    # kx), for every tile, with the default dispatch choosing them.
    from onnxsharp_amd import native as N
    seed = sum(xs) * 19 + sum(ws)
    x = synth.uniform(seed, xs)
    w = synth.normal(seed + 1, ws, 0, 0.05)
    b = synth.normal(seed + 2, (ws[0],), 0, 0.01)
    nv = C.c_int()
    N.call("osh_config_get", b"im2col3x3_variants", C.byref(nv))
    assert nv.value >= 9
    N.call("osh_config_set", b"exact_silu", 1)
    try:
        ref = None
        for v in [-1] + list(range(nv.value)):
            print(f"im2col3x3 {name} variant {v}", flush=True)
            N.call("osh_config_set", b"im2col3x3_variant", v)
            y, p = run_conv(cuda, x, w, b, "Silu", **attrs)
            if ref is None:
                k = oracle.conv_reference_kernel(x.shape, w.shape, (p.sh, p.sw), (p.pt, p.pl), (p.dh, p.dw),
                                                 p.group, (p.oh, p.ow))
                assert k == oracle.KERNEL_IM2COL, k
                ref = oracle_conv(oracle, x, w, b, p, "Silu", order=oracle.ORDER_IM2COL)
            assert np.array_equal(y, ref), f"variant {v}: max |d| {np.abs(y - ref).max():.3e}"
    finally:
        N.call("osh_config_set", b"exact_silu", 0)
        N.call("osh_config_set", b"im2col3x3_variant", -1)


def test_launch_refuses_weights_packed_for_another_kernel(cuda):
    # Packed layouts depend on the kernel choice; changing "winograd" between
    # packing and launch must be refused, not read as the other layout.
    from onnxsharp_amd import native as N
    from onnxsharp_amd.layers import ConvLayer
    x = _t(synth.uniform(5, (1, 64, 20, 20)), cuda)
    w = _t(synth.normal(6, (64, 64, 3, 3), 0, 0.05), cuda)
    layer = ConvLayer(pads=[1, 1, 1, 1])
    layer.forward(x, w)  # packed for the NCHWc tiles
    N.call("osh_config_set", b"winograd", 2)
    try:
        with pytest.raises(N.OshError, match="packed for another kernel"):
            layer.forward(x, w)  # same key: no repack, the launch sees the Winograd choice
    finally:
        N.call("osh_config_set", b"winograd", 1)
    y = layer.forward(x, w)  # the original choice again
    assert y.shape == (1, 64, 20, 20)


def test_pack_record_follows_the_memory(cuda):
    """Packing into memory drops the records of whatever it overlaps, and
    osh_conv_forget_pack drops a released range: a buffer reused for another
    shape's weights is not refused for its old layout."""
    import torch
    from onnxsharp_amd import native as N
    from onnxsharp_amd.layers import ConvLayer
    x1 = _t(synth.uniform(51, (1, 64, 20, 20)), cuda)
    w1 = _t(synth.normal(52, (64, 64, 3, 3), 0, 0.05), cuda)
    x2 = _t(synth.uniform(53, (1, 32, 16, 16)), cuda)
    w2 = _t(synth.normal(54, (48, 32, 1, 1), 0, 0.05), cuda)
    l1, l2 = ConvLayer(pads=[1, 1, 1, 1]), ConvLayer()
    p1 = l1.resolve(tuple(x1.shape), tuple(w1.shape))
    p2 = l2.resolve(tuple(x2.shape), tuple(w2.shape))
    n1, n2 = C.c_size_t(), C.c_size_t()
    N.call("osh_conv_packed_weight_bytes", C.byref(p1), C.byref(n1))
    N.call("osh_conv_packed_weight_bytes", C.byref(p2), C.byref(n2))
    arena = torch.empty(max(n1.value, n2.value) + 4096, dtype=torch.uint8, device=cuda)
    ptr = C.c_void_p(arena.data_ptr())
    y1 = torch.empty((1, 64, 20, 20), device=cuda)
    y2 = torch.empty((1, 48, 16, 16), device=cuda)
    N.call("osh_conv_pack_weights", C.byref(p1), C.c_void_p(w1.data_ptr()), ptr, None)
    N.call("osh_conv2d_f32", C.byref(p1), C.c_void_p(x1.data_ptr()), ptr, None, N.ACT_NONE,
           C.c_void_p(y1.data_ptr()), None)
    with pytest.raises(N.OshError, match="packed for another kernel"):  # still conv 1's layout
        N.call("osh_conv2d_f32", C.byref(p2), C.c_void_p(x2.data_ptr()), ptr, None, N.ACT_NONE,
               C.c_void_p(y2.data_ptr()), None)
    # packing conv 2 into the same memory replaces the record
    N.call("osh_conv_pack_weights", C.byref(p2), C.c_void_p(w2.data_ptr()), ptr, None)
    N.call("osh_conv2d_f32", C.byref(p2), C.c_void_p(x2.data_ptr()), ptr, None, N.ACT_NONE,
           C.c_void_p(y2.data_ptr()), None)
    ref2 = l2.forward(x2, w2)
    torch.cuda.synchronize()
    assert torch.equal(y2, ref2)
    # a forgotten range is unchecked memory again (the caller owns its contents)
    N.call("osh_conv_pack_weights", C.byref(p1), C.c_void_p(w1.data_ptr()), ptr, None)
    N.call("osh_conv_forget_pack", ptr, arena.numel())
    N.call("osh_conv_pack_weights", C.byref(p2), C.c_void_p(w2.data_ptr()), ptr, None)
    N.call("osh_conv2d_f32", C.byref(p2), C.c_void_p(x2.data_ptr()), ptr, None, N.ACT_NONE,
           C.c_void_p(y2.data_ptr()), None)
    torch.cuda.synchronize()
    assert torch.equal(y2, ref2)


def test_conv_refuses_overlapping_outputs(cuda):
    """A conv writing over its own input, and a group whose member's output
    overlaps another member's input, residual or output, are refused (the
    tiles of one launch run side by side); disjoint slices of one buffer are
    accepted and equal separate launches."""
    import torch
    from onnxsharp_amd import native as N
    from onnxsharp_amd.layers import ConvLayer
    x = _t(synth.uniform(61, (1, 64, 20, 20)), cuda)
    w = _t(synth.normal(62, (64, 64, 1, 1), 0, 0.05), cuda)
    layer = ConvLayer()
    y = layer.forward(x, w)
    _, p, buf = layer._packed
    big = torch.zeros((1, 256, 20, 20), device=cuda)
    sl = lambda c0: C.c_void_p(big[:, c0:c0 + 64].data_ptr())
    with pytest.raises(N.OshError, match="overlaps the input"):  # in place
        N.call("osh_conv2d_f32", C.byref(p), sl(0), C.c_void_p(buf.data_ptr()), None, N.ACT_NONE, sl(32), None)
    pa = (N.ConvParams * 2)(p, p)
    arr = lambda *ps: (C.c_void_p * 2)(*[v.value if isinstance(v, C.c_void_p) else v for v in ps])
    wb = C.c_void_p(buf.data_ptr())
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    cases = [  # channel ranges: x0, x1 -> y0, y1 (64 channels each)
        ("output 0 over input 1", arr(sl(0), sl(128)), arr(sl(96), sl(192)), None),
        ("output 0 is input 1", arr(sl(0), sl(128)), arr(sl(128), sl(192)), None),
        ("outputs overlap", arr(sl(0), sl(64)), arr(sl(128), sl(160)), None),
        ("output 1 over residual 0", arr(sl(0), sl(64)), arr(sl(128), sl(192)), arr(sl(192), None)),
    ]
    for what, xs, ys, rs in cases:
        with pytest.raises(N.OshError, match="overlaps"):
            N.check(N.lib().osh_conv2d_group_f32(2, pa, xs, arr(wb, wb), None, N.ACT_NONE, rs, ys, st))
    big[:, 0:64] = x
    big[:, 64:128] = x
    N.check(N.lib().osh_conv2d_group_f32(2, pa, arr(sl(0), sl(64)), arr(wb, wb), None, N.ACT_NONE, None,
                                         arr(sl(128), sl(192)), st))
    torch.cuda.synchronize()
    assert torch.equal(big[:, 128:192], y) and torch.equal(big[:, 192:256], y)


GROUP_CASES = [
    # (name, [(x shape, w shape, group)], act, residual) -- the head's layer kinds
    ("head_3x3_nchwc", [((1, 64, 80, 80), (64, 64, 3, 3), 1), ((1, 128, 40, 40), (64, 128, 3, 3), 1),
                        ((1, 256, 20, 20), (64, 256, 3, 3), 1)], "Silu", False),
    ("head_depthwise", [((1, 64, 80, 80), (64, 1, 3, 3), 64), ((1, 128, 40, 40), (128, 1, 3, 3), 128),
                        ((1, 256, 20, 20), (256, 1, 3, 3), 256)], "Silu", False),
    ("head_pointwise_res", [((1, 64, 80, 80), (80, 64, 1, 1), 1), ((1, 80, 40, 40), (80, 80, 1, 1), 1),
                            ((1, 80, 20, 20), (80, 80, 1, 1), 1), ((1, 48, 9, 6), (32, 48, 1, 1), 1)], None, True),
    ("mixed_fallback", [((1, 64, 20, 20), (64, 64, 3, 3), 1), ((1, 32, 20, 20), (32, 1, 3, 3), 32)], "Relu", True),
    # six members: the head's final box and class 1x1 layers as one launch
    ("head_final_six", [((1, 64, 80, 80), (64, 64, 1, 1), 1), ((1, 64, 40, 40), (64, 64, 1, 1), 1),
                        ((1, 64, 20, 20), (64, 64, 1, 1), 1), ((1, 80, 80, 80), (80, 80, 1, 1), 1),
                        ((1, 80, 40, 40), (80, 80, 1, 1), 1), ((1, 80, 20, 20), (80, 80, 1, 1), 1)], None, False),
    # stride 2, odd maps, a deep member first (the streamed one-wave member of the mixed tiles)
    ("strided_3x3", [((1, 32, 41, 39), (48, 32, 3, 3), 1, 2), ((1, 128, 11, 13), (32, 128, 3, 3), 1, 2)],
     "Silu", True),
]


def _group_tiles(key):
    from onnxsharp_amd import native as N
    nt = C.c_int()
    N.call("osh_config_get", key + b"s", C.byref(nt))
    return nt.value


@pytest.mark.parametrize("name,convs,act,residual", GROUP_CASES, ids=[c[0] for c in GROUP_CASES])
def test_conv_group_equals_separate_launches(cuda, name, convs, act, residual):
    # osh_conv2d_group_f32 runs independent convs as one launch (or one per
    # conv when they do not share a kernel family): the outputs are those of
    # separate launches, bit for bit.
    import torch
    from onnxsharp_amd import native as N
    from onnxsharp_amd.layers import ConvLayer
    print(f"conv group {name}", flush=True)
    n = len(convs)
    layers, xs, ws, bs, rs, ys, ref, ps, packs = [], [], [], [], [], [], [], [], []
    for k, conv in enumerate(convs):
        xsh, wsh, g = conv[:3]
        stride = conv[3] if len(conv) > 3 else 1
        seed = 23 * k + sum(xsh) + sum(wsh)
        x = _t(synth.uniform(seed, xsh), cuda)
        w = _t(synth.normal(seed + 1, wsh, 0, 0.05), cuda)
        b = _t(synth.normal(seed + 2, (wsh[0],), 0, 0.01), cuda)
        layer = ConvLayer(fused_activation=act, group=g, pads=[1, 1, 1, 1] if wsh[2] == 3 else [0, 0, 0, 0],
                          strides=[stride, stride])
        y0 = layer.forward(x, w, b)
        r = torch.from_numpy(synth.normal(seed + 3, tuple(y0.shape), 0, 1)).to(cuda) if residual else None
        if r is not None:
            y0 = layer.forward(x, w, b, residual=r)
        torch.cuda.synchronize()
        ref.append(y0.cpu().numpy())
        _, p, buf = layer._packed
        layers.append(layer); xs.append(x); ws.append(buf); bs.append(b); rs.append(r); ps.append(p)
        ys.append(torch.full(tuple(y0.shape), float("nan"), device=cuda))
    arr = lambda ts: (C.c_void_p * n)(*[None if t is None else t.data_ptr() for t in ts])
    pa = (N.ConvParams * n)(*ps)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    # the 3x3 and pointwise groups: every tile forced in turn (the first-use
    # timing would keep only the last tile's output), then the automatic choice
    key = {"head_3x3_nchwc": b"group3x3_tile", "strided_3x3": b"group3x3_tile",
           "head_pointwise_res": b"group_pointwise_tile", "head_final_six": b"group_pointwise_tile"}.get(name)
    tiles = list(range(_group_tiles(key))) if key else []
    try:
        for tile in tiles + [-1]:
            if key:
                N.call("osh_config_set", key, tile)
            for y in ys:
                y.fill_(float("nan"))
            N.check(N.lib().osh_conv2d_group_f32(n, pa, arr(xs), arr(ws), arr(bs), N.ACTIVATIONS[act], arr(rs),
                                                 arr(ys), st))
            torch.cuda.synchronize()
            for k in range(n):
                got = ys[k].cpu().numpy()
                assert np.array_equal(got, ref[k]), \
                    f"tile {tile} conv {k}: max |d| {np.nanmax(np.abs(got - ref[k])):.3e}"
    finally:
        if key:
            N.call("osh_config_set", key, -1)


@pytest.mark.parametrize("case", [0, 1, 2])
@pytest.mark.parametrize("m,chain", [(32, "nchwc"), (16, "im2col"), (64, "nchwc")])
def test_device_chain_order_pinned_by_planted_magnitudes(cuda, oracle, case, m, chain):
    """The planted-magnitude inputs of the oracle's order tests (tests/test_oracle.py)
    through the device dispatch: 32 input channels on a 3x3 map with pad 1, so
    the centre output pixel sees every planted tap.  M % 32 == 0 passes the
    reference's NCHWc gate (NchwcConv.cs:100-126) and must give the NCHWc
    chain's hand-derived value; M = 16 fails it and must give the im2col
    chain's (ConvKernels.cs:554-563).  Every output channel carries the same
    planted weights; every output pixel equals the oracle's bit for bit."""
    from test_oracle import PLANTED, _planted
    terms, want = PLANTED[case]
    x, w1 = _planted(terms)
    w = np.repeat(w1, m, axis=0)
    b = np.zeros(m, np.float32)
    print(f"planted case {case}, m={m}: expect the {chain} chain", flush=True)
    y, p = run_conv(cuda, x, w, b, None, pads=[1, 1, 1, 1])
    assert (y[0, :, 1, 1] == np.float32(want[chain])).all(), y[0, :, 1, 1]
    ref = oracle_conv(oracle, x, w, b, p, None)
    assert np.array_equal(y, ref)


PAIR_CASES = [
    # (name, x shape, c1, c2, residual, options) -- a bottleneck's cv1 -> cv2
    ("c3k2_80", (1, 32, 80, 80), 16, 32, True, {}),          # im2col chain, then NCHWc
    ("c3k_40", (1, 32, 40, 40), 32, 32, True, {}),
    ("c3k2_neck_40", (1, 64, 40, 40), 32, 64, False, {}),
    ("c3k_20", (1, 64, 20, 20), 64, 64, True, {}),
    ("odd_map", (1, 32, 13, 11), 16, 32, True, {"winograd": 0}),
    ("deep_ragged", (1, 48, 7, 9), 64, 16, True, {"winograd": 0}),  # 3 input chunks, im2col second conv
    ("exact_silu", (1, 64, 20, 20), 32, 32, False, {"exact_silu": 1}),
    # an 8-channel intermediate: im2col chain, then the first-layer chain
    ("c3k2_160_eight", (1, 16, 160, 160), 8, 16, True, {}),
    ("eight_ragged", (1, 16, 13, 37), 8, 16, False, {"winograd": 0}),
    ("eight_exact_silu", (1, 16, 40, 24), 8, 16, True, {"winograd": 0, "exact_silu": 1}),
]


@pytest.mark.parametrize("name,xs,c1,c2,residual,opts", PAIR_CASES, ids=[c[0] for c in PAIR_CASES])
def test_conv_pair_equals_two_launches(cuda, name, xs, c1, c2, residual, opts):
    # osh_conv2d_pair_f32 runs a bottleneck's two 3x3 convs in one launch with
    # the intermediate on chip: its outputs (and the intermediate it still
    # stores) are those of the two separate launches, bit for bit, under every
    # tile and under the first-use choice.
    import torch
    from onnxsharp_amd import native as N
    from onnxsharp_amd.layers import ConvLayer
    print(f"conv pair {name}", flush=True)
    saved = {}
    for k, v in opts.items():
        cur = C.c_int(); N.call("osh_config_get", k.encode(), C.byref(cur)); saved[k] = cur.value
        N.call("osh_config_set", k.encode(), v)
    try:
        seed = sum(xs) + 7 * c1 + c2
        x = _t(synth.uniform(seed, xs), cuda)
        wa = _t(synth.normal(seed + 1, (c1, xs[1], 3, 3), 0, 0.05), cuda)
        ba = _t(synth.normal(seed + 2, (c1,), 0, 0.01), cuda)
        wb = _t(synth.normal(seed + 3, (c2, c1, 3, 3), 0, 0.05), cuda)
        bb = _t(synth.normal(seed + 4, (c2,), 0, 0.01), cuda)
        la = ConvLayer(pads=[1, 1, 1, 1], fused_activation="Silu")
        lb = ConvLayer(pads=[1, 1, 1, 1], fused_activation="Silu")
        t_ref = la.forward(x, wa, ba)
        r = _t(synth.normal(seed + 5, (1, c2, xs[2], xs[3]), 0, 1), cuda) if residual else None
        y_ref = lb.forward(t_ref, wb, bb, residual=r)
        torch.cuda.synchronize()
        t_ref, y_ref = t_ref.cpu().numpy(), y_ref.cpu().numpy()
        _, pa, bufa = la._packed
        _, pb, bufb = lb._packed
        st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        N.call("osh_conv2d_pair_check", C.byref(pa), C.byref(pb), N.ACT_SILU)
        nt = C.c_int(); N.call("osh_config_get", b"pair_tiles", C.byref(nt))
        ptr = lambda t: C.c_void_p(t.data_ptr()) if t is not None else None
        try:
            for tile in list(range(nt.value)) + [-1]:
                N.call("osh_config_set", b"pair_tile", tile)
                ya = torch.full((1, c1, xs[2], xs[3]), float("nan"), device=cuda)
                y = torch.full((1, c2, xs[2], xs[3]), float("nan"), device=cuda)
                N.call("osh_conv2d_pair_f32", C.byref(pa), C.byref(pb), ptr(x), ptr(bufa), ptr(ba), ptr(bufb),
                       ptr(bb), N.ACT_SILU, ptr(r), ptr(ya), ptr(y), st)
                torch.cuda.synchronize()
                assert np.array_equal(ya.cpu().numpy(), t_ref), f"{name}: intermediate differs under tile {tile}"
                assert np.array_equal(y.cpu().numpy(), y_ref), f"{name}: output differs under tile {tile}"
        finally:
            N.call("osh_config_set", b"pair_tile", -1)
        # the intermediate may be left unstored (first-use timing then only
        # chooses among the fused tiles)
        y2 = torch.full((1, c2, xs[2], xs[3]), float("nan"), device=cuda)
        N.call("osh_conv2d_pair_f32", C.byref(pa), C.byref(pb), ptr(x), ptr(bufa), ptr(ba), ptr(bufb), ptr(bb),
               N.ACT_SILU, ptr(r), None, ptr(y2), st)
        torch.cuda.synchronize()
        assert np.array_equal(y2.cpu().numpy(), y_ref)
        if residual:  # a residual inside the output is refused
            with pytest.raises(N.OshError, match="residual overlaps"):
                N.call("osh_conv2d_pair_f32", C.byref(pa), C.byref(pb), ptr(x), ptr(bufa), ptr(ba), ptr(bufb),
                       ptr(bb), N.ACT_SILU, ptr(y2), None, ptr(y2), st)
    finally:
        for k, v in saved.items():
            N.call("osh_config_set", k.encode(), v)


FIRST_PAIR_CASES = [
    # (name, x shape, first stride, c2, second stride, residual, options): a
    # first-layer conv (16 outputs) -> a 3x3 NCHWc conv over its output
    ("yolo11n_stem_640", (1, 3, 640, 640), 2, 32, 2, False, {}),
    ("ragged_tiles", (1, 3, 68, 92), 2, 32, 2, True, {}),            # 17 x 23 outputs
    ("four_planes_64_out", (1, 4, 40, 50), 1, 64, 2, True, {}),
    ("one_plane_stride_1", (1, 1, 30, 34), 1, 32, 1, True, {}),
    ("two_planes_exact_silu", (1, 2, 64, 48), 2, 32, 1, False, {"exact_silu": 1}),
]


@pytest.mark.parametrize("name,xs,sa,c2,sb,residual,opts", FIRST_PAIR_CASES, ids=[c[0] for c in FIRST_PAIR_CASES])
def test_first_layer_pair_equals_two_launches(cuda, name, xs, sa, c2, sb, residual, opts):
    # The first-layer pair keeps both chains (first_conv_kernel's ic -> ky ->
    # kx, then the NCHWc chain) with the 16-channel map on chip: outputs and
    # the stored intermediate equal the two separate launches bit for bit
    # under every tile, the first-use choice and without the intermediate.
    import torch
    from onnxsharp_amd import native as N
    from onnxsharp_amd.layers import ConvLayer
    print(f"first-layer pair {name}", flush=True)
    saved = {}
    for k, v in opts.items():
        cur = C.c_int(); N.call("osh_config_get", k.encode(), C.byref(cur)); saved[k] = cur.value
        N.call("osh_config_set", k.encode(), v)
    try:
        seed = sum(xs) + 5 * sa + c2 + sb
        x = _t(synth.uniform(seed, xs), cuda)
        wa = _t(synth.normal(seed + 1, (16, xs[1], 3, 3), 0, 0.3), cuda)
        ba = _t(synth.normal(seed + 2, (16,), 0, 0.01), cuda)
        wb = _t(synth.normal(seed + 3, (c2, 16, 3, 3), 0, 0.05), cuda)
        bb = _t(synth.normal(seed + 4, (c2,), 0, 0.01), cuda)
        la = ConvLayer(pads=[1, 1, 1, 1], strides=[sa, sa], fused_activation="Silu")
        lb = ConvLayer(pads=[1, 1, 1, 1], strides=[sb, sb], fused_activation="Silu")
        t_ref = la.forward(x, wa, ba)
        ys = (1, c2, (t_ref.shape[2] - 1) // sb + 1, (t_ref.shape[3] - 1) // sb + 1)
        r = _t(synth.normal(seed + 5, ys, 0, 1), cuda) if residual else None
        y_ref = lb.forward(t_ref, wb, bb, residual=r)
        torch.cuda.synchronize()
        ts = tuple(t_ref.shape)
        t_ref, y_ref = t_ref.cpu().numpy(), y_ref.cpu().numpy()
        _, pa, bufa = la._packed
        _, pb, bufb = lb._packed
        st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        N.call("osh_conv2d_pair_check", C.byref(pa), C.byref(pb), N.ACT_SILU)
        nt = C.c_int(); N.call("osh_config_get", b"pair_tiles", C.byref(nt))
        ptr = lambda t: C.c_void_p(t.data_ptr()) if t is not None else None
        try:
            for tile in list(range(nt.value)) + [-1]:
                N.call("osh_config_set", b"pair_tile", tile)
                ya = torch.full(ts, float("nan"), device=cuda)
                y = torch.full(ys, float("nan"), device=cuda)
                N.call("osh_conv2d_pair_f32", C.byref(pa), C.byref(pb), ptr(x), ptr(bufa), ptr(ba), ptr(bufb),
                       ptr(bb), N.ACT_SILU, ptr(r), ptr(ya), ptr(y), st)
                torch.cuda.synchronize()
                assert np.array_equal(ya.cpu().numpy(), t_ref), f"{name}: intermediate differs under tile {tile}"
                assert np.array_equal(y.cpu().numpy(), y_ref), f"{name}: output differs under tile {tile}"
        finally:
            N.call("osh_config_set", b"pair_tile", -1)
        y2 = torch.full(ys, float("nan"), device=cuda)
        N.call("osh_conv2d_pair_f32", C.byref(pa), C.byref(pb), ptr(x), ptr(bufa), ptr(ba), ptr(bufb), ptr(bb),
               N.ACT_SILU, ptr(r), None, ptr(y2), st)
        torch.cuda.synchronize()
        assert np.array_equal(y2.cpu().numpy(), y_ref)
    finally:
        for k, v in saved.items():
            N.call("osh_config_set", k.encode(), v)


def test_conv_pair_refusals(cuda):
    import torch
    from onnxsharp_amd import native as N
    from onnxsharp_amd.layers import ConvLayer

    def params(xs, m, k=3, s=1, pads=(1, 1, 1, 1)):
        return ConvLayer(pads=list(pads), strides=[s, s]).resolve(xs, (m, xs[1], k, k))

    ok = (params((1, 32, 40, 40), 32), params((1, 32, 40, 40), 64))
    N.call("osh_conv2d_pair_check", C.byref(ok[0]), C.byref(ok[1]), N.ACT_SILU)
    bad = [
        ("stride 2", params((1, 32, 40, 40), 32, s=2), ok[1], N.ACT_SILU),
        ("1x1", params((1, 32, 40, 40), 32, k=1, pads=(0, 0, 0, 0)), ok[1], N.ACT_SILU),
        ("48 outputs", params((1, 32, 40, 40), 48), params((1, 48, 40, 40), 32), N.ACT_SILU),
        ("8 input channels", params((1, 8, 40, 40), 32), ok[1], N.ACT_SILU),
        ("not chained", ok[0], params((1, 16, 40, 40), 32), N.ACT_SILU),
        ("relu", ok[0], ok[1], N.ACT_RELU),
        ("winograd chain", params((1, 32, 40, 40), 16), params((1, 16, 40, 40), 32), N.ACT_SILU),
        # first-layer pairs
        ("first-layer 8 outputs", params((1, 3, 64, 64), 8, s=2), params((1, 8, 32, 32), 32, s=2), N.ACT_SILU),
        ("first-layer then 16 outputs (im2col chain)", params((1, 3, 64, 64), 16, s=2),
         params((1, 16, 32, 32), 16, s=2), N.ACT_SILU),
        ("first-layer then 1x1", params((1, 3, 64, 64), 16, s=2),
         params((1, 16, 32, 32), 32, k=1, pads=(0, 0, 0, 0)), N.ACT_SILU),
        ("first-layer stride 3", params((1, 3, 64, 64), 16, s=3), params((1, 16, 22, 22), 32), N.ACT_SILU),
        ("first-layer relu", params((1, 3, 64, 64), 16, s=2), params((1, 16, 32, 32), 32, s=2), N.ACT_RELU),
        ("first-layer odd map under stride 2", params((1, 3, 66, 66), 16, s=2),
         params((1, 16, 33, 33), 32, s=2), N.ACT_SILU),
    ]
    for what, pa, pb, act in bad:
        with pytest.raises(N.OshError) as e:
            N.call("osh_conv2d_pair_check", C.byref(pa), C.byref(pb), act)
        assert e.value.status == N.OSH_E_UNSUPPORTED, what
    # outputs may not overlap the input
    la, lb = ConvLayer(pads=[1, 1, 1, 1]), ConvLayer(pads=[1, 1, 1, 1])
    buf = torch.zeros((1, 128, 40, 40), device=cuda)
    wa, wb = torch.zeros((32, 32, 3, 3), device=cuda), torch.zeros((64, 32, 3, 3), device=cuda)
    pa, bufa = la.prepack_weights((1, 32, 40, 40), wa)
    pb, bufb = lb.prepack_weights((1, 32, 40, 40), wb)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    sl = lambda c0: C.c_void_p(buf.data_ptr() + 4 * c0 * 1600)
    with pytest.raises(N.OshError, match="overlaps"):
        N.call("osh_conv2d_pair_f32", C.byref(pa), C.byref(pb), sl(0), C.c_void_p(bufa.data_ptr()), None,
               C.c_void_p(bufb.data_ptr()), None, N.ACT_SILU, None, None, sl(16), st)


# (name, x shape [N, C, L], w shape [M, C/g, K], attrs, act)
CONV1D_CASES = [
    ("k3_pad1_batch2", (2, 16, 100), (32, 16, 3), dict(pads=[1, 1]), "Silu"),
    ("k5_s2_dil2_uneven_pads", (1, 8, 77), (12, 8, 5), dict(strides=[2], pads=[4, 2], dilations=[2]), None),
    ("grouped_k3", (1, 16, 50), (16, 4, 3), dict(group=4, pads=[1, 1]), "Relu"),
    ("same_upper_k4_s3", (1, 6, 33), (5, 6, 4), dict(auto_pad="SAME_UPPER", strides=[3]), None),
    ("k1_residual", (1, 32, 40), (64, 32, 1), dict(), "Silu"),
]


def _conv1d_ref(x, w, b, stride, dilation, pad_begin, out_len, group):
    """Forward1D (src/OnnxSharp/Ops/DnnOps.cs:235-300) in float64: output t of
    channel m sums w[m][j][k] * x[j][t*stride - pad_begin + k*dilation] over
    the group's channels j and taps k, positions outside the input skipped."""
    n, c, length = x.shape
    m, cpg, kernel = w.shape
    opg = m // group
    y = np.zeros((n, m, out_len))
    for mm in range(m):
        base = mm // opg * cpg
        for k in range(kernel):
            pos = np.arange(out_len) * stride - pad_begin + k * dilation
            ok = (pos >= 0) & (pos < length)
            y[:, mm, ok] += np.einsum("j,njt->nt", w[mm, :, k].astype(np.float64),
                                      x[:, base:base + cpg, pos[ok]].astype(np.float64))
    return y + (0 if b is None else b.astype(np.float64)[None, :, None])


@pytest.mark.parametrize("name,xs,ws,attrs,act", CONV1D_CASES, ids=[c[0] for c in CONV1D_CASES])
def test_conv1d_rank3_within_fp32_bar(cuda, oracle, name, xs, ws, attrs, act):
    # A rank-3 Conv runs as the 2-D conv of [N, C, 1, L] (its im2col chain:
    # channel -> tap); the reference's Forward1D sums the same terms (channel
    # -> tap with a multiply and an add each, or per tap with FMAs on its
    # stride-1 AVX path), so the bar is the FP32 tolerance against the float64
    # sum, and the output length is Conv1DShape's (the end pad counts).
    import torch
    from onnxsharp_amd.layers import ConvLayer
    print(f"conv1d {name} x={xs} w={ws} {attrs} act={act}", flush=True)
    seed = sum(xs) * 3 + sum(ws)
    x = synth.uniform(seed, xs)
    w = synth.normal(seed + 1, ws, 0, 0.1)
    b = synth.normal(seed + 2, (ws[0],), 0, 0.01)
    layer = ConvLayer(fused_activation=act, **attrs)
    ys = layer.get_memory_shapes(xs, ws)
    p = layer.resolve(xs, ws)
    r = synth.normal(seed + 3, ys, 0, 1) if "residual" in name else None
    y = layer.forward(_t(x, cuda), _t(w, cuda), _t(b, cuda), residual=None if r is None else _t(r, cuda))
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert y.shape == ys
    ref = _conv1d_ref(x, w, b, p.sw, p.dw, p.pl, ys[2], attrs.get("group", 1))
    if act == "Silu":
        ref = ref / (1 + np.exp(-ref))
    elif act == "Relu":
        ref = np.maximum(ref, 0)
    if r is not None:
        ref = ref + r
    assert_fp32_close(y, ref, name)


NCHWC_OFF_CASES = [
    ("c2_3x3s1_64to64_160", (1, 64, 160, 160), (64, 64, 3, 3), 1, "im2col"),
    ("c3b_3x3s2_128to256_80", (1, 128, 80, 80), (256, 128, 3, 3), 2, "im2col"),
    ("3x3s1_64to64_20", (1, 64, 20, 20), (64, 64, 3, 3), 1, "winograd"),
    ("3x3s1_128to128_40", (1, 128, 40, 40), (128, 128, 3, 3), 1, "winograd"),
]


@pytest.mark.parametrize("name,xs,ws,stride,kind", NCHWC_OFF_CASES, ids=[c[0] for c in NCHWC_OFF_CASES])
def test_conv_without_nchwc_follows_the_avx2_dispatch(cuda, oracle, name, xs, ws, stride, kind):
    # nchwc = 0 (ONNXSHARP_NCHWC=0, or a host without AVX-512): the shapes
    # NchwcConv would take go where ConvLayer.Forward then sends them
    # (DnnOps.cs:475-482) -- Winograd where its gate holds, else PackedConv /
    # Im2Col, both the ic -> ky -> kx chain -- bit for bit (exact SiLU)
    from onnxsharp_amd import native as N
    from onnxsharp_amd.layers import ConvLayer
    print(f"nchwc=0 {name} x={xs} w={ws} s={stride}", flush=True)
    seed = sum(xs) * 7 + sum(ws) + stride
    x = synth.uniform(seed, xs)
    w = synth.normal(seed + 1, ws, 0, 0.05)
    b = synth.normal(seed + 2, (ws[0],), 0, 0.01)
    attrs = dict(strides=[stride, stride], pads=[1, 1, 1, 1])
    old = C.c_int()
    N.call("osh_config_get", b"nchwc", C.byref(old))
    N.call("osh_config_set", b"nchwc", 0)
    N.call("osh_config_set", b"exact_silu", 1)
    try:
        layer = ConvLayer(fused_activation="Silu", **attrs)
        y = layer.forward(_t(x, cuda), _t(w, cuda), _t(b, cuda)).cpu().numpy()
        p = layer.resolve(x.shape, w.shape)
        names = N.kernel_log(reset=True)
    finally:
        N.call("osh_config_set", b"nchwc", old.value)
        N.call("osh_config_set", b"exact_silu", 0)
    args = (x.shape, w.shape, (p.sh, p.sw), (p.pt, p.pl), (p.dh, p.dw), p.group, (p.oh, p.ow))
    assert oracle.conv_reference_kernel(*args, nchwc=0) == kind
    assert oracle.conv_reference_kernel(*args, nchwc=1) == oracle.KERNEL_NCHWC
    assert any(n.startswith("wino_f23" if kind == "winograd" else "conv16") for n in names), names
    ref = oracle_conv(oracle, x, w, b, p, "Silu", nchwc=0)
    assert np.array_equal(y, ref), f"max |d| {np.abs(y - ref).max():.3e} at {np.argwhere(y != ref)[:3]}"
    # and not the NCHWc chain's bits (the two orders round differently here)
    assert not np.array_equal(y, oracle_conv(oracle, x, w, b, p, "Silu", nchwc=1))
