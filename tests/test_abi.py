"""CPU tests of the C ABI: the library loads, exports every declared symbol,
and its host-side operator logic (shape inference, pad resolution, errors)
follows the reference.  No kernel is launched here."""
import ctypes as C
import os
import re

import pytest

from onnxsharp_amd import native as N
from onnxsharp_amd.layers import ConvLayer, MatMulLayer, DynamicQuantizeMatMulLayer

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "osh_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"OSH_API\s+[\w\s\*]+?\b(osh_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for must in ("osh_init", "osh_malloc", "osh_memcpy_h2d", "osh_conv2d_f32", "osh_gemm_f32", "osh_dqmm_u8s8",
                 "osh_last_error"):
        assert must in syms


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    for s in declared_symbols():
        assert hasattr(lib, s), s
    assert set(declared_symbols()) == set(N.EXPORTED)


def test_last_error_reports_invalid_arguments():
    st = N.lib().osh_gemm_f32(-1, 1, 1, None, 1, None, 1, None, None, None, 0, None, 1, None)
    assert st == N.OSH_E_INVALID
    assert "negative" in N.last_error()


# ------------------------------------------------------------ Conv shape logic

@pytest.mark.parametrize("attrs,x,w,y", [
    (dict(pads=[1, 1, 1, 1]), (1, 64, 160, 160), (64, 64, 3, 3), (1, 64, 160, 160)),
    (dict(strides=[2, 2], pads=[1, 1, 1, 1]), (1, 128, 80, 80), (256, 128, 3, 3), (1, 256, 40, 40)),
    (dict(), (1, 256, 80, 80), (128, 256, 1, 1), (1, 128, 80, 80)),
    (dict(auto_pad="SAME_UPPER", strides=[2, 2]), (1, 1, 9, 11), (1, 1, 3, 3), (1, 1, 5, 6)),
    (dict(auto_pad="VALID"), (2, 4, 9, 9), (8, 4, 3, 3), (2, 8, 7, 7)),
    (dict(dilations=[2, 2], pads=[2, 2, 2, 2]), (1, 4, 11, 11), (5, 4, 3, 3), (1, 5, 11, 11)),
    (dict(group=2, strides=[1, 2], pads=[0, 1, 0, 1]), (2, 8, 9, 7), (6, 4, 3, 3), (2, 6, 7, 4)),
    (dict(kernel_shape=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1]), (1, 3, 640, 640), (16, 3, 3, 3), (1, 16, 320, 320)),
])
def test_conv_get_memory_shapes(attrs, x, w, y):
    assert ConvLayer(**attrs).get_memory_shapes(x, w) == y


def test_conv_end_pads_follow_the_reference_shape_rule():
    # DnnOps.cs:174-175 reads the end pad only when more than 2*spatial pads are given, so
    # [0, 0, 1, 1] infers the shape as if the pads were [0, 0, 0, 0].
    assert ConvLayer(pads=[0, 0, 1, 1]).get_memory_shapes((1, 1, 8, 8), (1, 1, 3, 3)) == (1, 1, 6, 6)
    p = ConvLayer(pads=[0, 0, 1, 1]).resolve((1, 1, 8, 8), (1, 1, 3, 3))
    assert (p.pt, p.pl, p.pb, p.pr, p.oh, p.ow) == (0, 0, 1, 1, 6, 6)


def test_conv_same_upper_equals_explicit_pads():
    # PadConv1DTests.Conv2DSameUpperWithoutKernelShape
    a = ConvLayer(auto_pad="SAME_UPPER", strides=[2, 2]).resolve((1, 1, 9, 11), (1, 1, 3, 3))
    b = ConvLayer(pads=[1, 1, 1, 1], strides=[2, 2]).resolve((1, 1, 9, 11), (1, 1, 3, 3))
    assert (a.pt, a.pl, a.oh, a.ow) == (b.pt, b.pl, b.oh, b.ow) == (1, 1, 5, 6)


def test_conv_same_lower_puts_the_odd_pad_first():
    p = ConvLayer(auto_pad="SAME_LOWER", strides=[2, 2]).resolve((1, 1, 10, 10), (1, 1, 4, 4))
    assert (p.pt, p.pb) == (1, 1) and (p.oh, p.ow) == (5, 5)
    p = ConvLayer(auto_pad="SAME_LOWER").resolve((1, 1, 10, 10), (1, 1, 4, 4))
    assert (p.pt, p.pb) == (2, 1)
    p = ConvLayer(auto_pad="SAME_UPPER").resolve((1, 1, 10, 10), (1, 1, 4, 4))
    assert (p.pt, p.pb) == (1, 2)


@pytest.mark.parametrize("attrs,x,w,msg", [
    (dict(group=3), (1, 8, 5, 5), (8, 8, 3, 3), "divisible"),
    (dict(), (1, 8, 5, 5), (8, 4, 3, 3), "in-channels"),
    (dict(), (1, 8, 2, 2), (8, 8, 5, 5), "not positive"),
])
def test_conv_shape_errors(attrs, x, w, msg):
    with pytest.raises(N.OshError, match=msg):
        ConvLayer(**attrs).get_memory_shapes(x, w)


def test_conv_rejects_3d():
    # 1-D (rank-3) and 2-D convs are taken (the rank-3 shapes are pinned by
    # test_conv1d_shapes_follow_conv1dshape); volumetric ones are refused
    with pytest.raises(N.OshUnsupported):
        ConvLayer().get_memory_shapes((1, 8, 5, 5, 5), (8, 8, 3, 3, 3))
    with pytest.raises(N.OshUnsupported):
        ConvLayer(strides=[1, 1, 1])


# ------------------------------------------------------------ MatMul shape logic

@pytest.mark.parametrize("a,b,y", [
    ((1024, 768), (768, 768), (1024, 768)),
    ((2, 3, 4), (4, 5), (2, 3, 5)),
    ((4,), (4, 5), (5,)),
    ((3, 4), (4,), (3,)),
    ((4,), (4,), ()),
    ((2, 1, 3, 4), (5, 4, 6), (2, 5, 3, 6)),
])
def test_matmul_get_memory_shapes(a, b, y):
    assert MatMulLayer().get_memory_shapes(a, b) == y


def test_matmul_shape_errors():
    with pytest.raises(N.OshError, match="K mismatch"):
        MatMulLayer().get_memory_shapes((3, 4), (5, 6))
    with pytest.raises(N.OshError, match="broadcast"):
        MatMulLayer().get_memory_shapes((2, 3, 4), (3, 4, 5))


def test_dqmm_shapes():
    assert DynamicQuantizeMatMulLayer.get_memory_shapes((4, 512, 512), (512, 2048)) == (4, 512, 2048)
    with pytest.raises(N.OshError):
        DynamicQuantizeMatMulLayer.get_memory_shapes((4, 512), (256, 2048))


def test_size_queries():
    s = C.c_size_t()
    N.call("osh_dqmm_packed_weight_bytes", 512, 2048, C.byref(s))
    assert s.value == 512 * 2048 + 2048 * 8
    N.call("osh_dqmm_scratch_bytes", 512, 512, C.byref(s))
    assert s.value >= 512 * 512
    p = ConvLayer(pads=[1, 1, 1, 1]).resolve((1, 64, 160, 160), (64, 64, 3, 3))
    N.call("osh_conv_packed_weight_bytes", C.byref(p), C.byref(s))
    assert s.value == 64 * 64 * 9 * 4


def test_conv_add_rejects_a_residual_overlapping_the_output():
    # checked before anything touches memory: the pointers are never dereferenced
    p = ConvLayer(pads=[1, 1, 1, 1]).resolve((1, 16, 8, 8), (16, 16, 3, 3))
    lib = N.lib()
    base = 1 << 40
    nbytes = 16 * 8 * 8 * 4
    for res in (base, base + nbytes - 4, base - nbytes + 4):
        st = lib.osh_conv2d_add_f32(C.byref(p), C.c_void_p(1 << 41), C.c_void_p(1 << 42), None, 0,
                                    C.c_void_p(res), C.c_void_p(base), None)
        assert st == N.OSH_E_INVALID and "overlaps" in N.last_error(), hex(res)
    st = lib.osh_conv2d_add_f32(C.byref(p), C.c_void_p(1 << 41), C.c_void_p(1 << 42), None, 0, None,
                                C.c_void_p(base), None)
    assert st == N.OSH_E_INVALID and "NULL" in N.last_error()


def test_dfl_softmax_shapes():
    from onnxsharp_amd.layers import DflSoftmaxLayer
    assert DflSoftmaxLayer(16).get_memory_shapes((1, 64, 8400)) == (1, 4, 8400)
    with pytest.raises(N.OshError, match="not divisible by bins"):
        DflSoftmaxLayer(16).get_memory_shapes((1, 60, 10))
    with pytest.raises(N.OshError, match="must be"):
        DflSoftmaxLayer(16).get_memory_shapes((64, 10))
    st = N.lib().osh_dfl_f32(1, 4, 1, 10, C.c_void_p(1 << 40), 40, C.c_void_p(1 << 41), 40, None)
    assert st == N.OSH_E_INVALID and "bins" in N.last_error()


def test_attention_shape_rules_match_the_frame_planner():
    # y == qkv: every shape the kernel takes stops at the overlap check
    # (OSH_E_INVALID) before a launch; the rest are OSH_E_UNSUPPORTED, which
    # the frame planner must predict so that it runs the five-launch sequence
    from onnxsharp_amd.yolo11n import attention_fits
    lib = N.lib()
    base = C.c_void_p(1 << 40)
    for kd in (4, 28, 30, 32, 64, 68):
        for hd in (16, 40, 64, 128):
            for n in (16, 100, 400, 408, 480, 496):
                st = lib.osh_attention_f32(2, kd, hd, n, C.c_float(0.5), base, (2 * kd + hd) * n, base, None)
                want = N.OSH_E_INVALID if attention_fits(kd, hd, n) else N.OSH_E_UNSUPPORTED
                assert st == want, (kd, hd, n, N.last_error())
    st = lib.osh_attention_f32(1, 32, 64, 400, C.c_float(1.0), base, 128 * 400 - 1, C.c_void_p(1 << 41), None)
    assert st == N.OSH_E_INVALID and "stride" in N.last_error()


def test_noalloc_dqmm_refuses_sizes_beyond_its_scratch_on_the_host():
    # m = k = 2048 needs more than the 4 MiB static scratch of
    # osh_dqmm_u8s8_noalloc: refused before any HIP call (this runs without a
    # GPU), so no pointer is ever read
    import ctypes as C
    from onnxsharp_amd import native as N
    fake = C.c_void_p(16)
    st = N.lib().osh_dqmm_u8s8_noalloc(2048, 2048, 64, fake, fake, fake, 64, None, fake, None, None, None)
    assert st == N.OSH_E_UNSUPPORTED
    assert "scratch" in N.last_error()
    assert N.lib().osh_dqmm_u8s8_noalloc(0, 512, 64, None, None, None, 64, None, None, None, None, None) == N.OSH_OK


@pytest.mark.parametrize("signed,zp", [(0, -1), (0, 256), (1, -129), (1, 128)])
def test_dqmm_pack_refuses_zero_points_outside_the_weight_type(signed, zp):
    # checked before any HIP call (this runs without a GPU)
    import ctypes as C
    from onnxsharp_amd import native as N
    z = (C.c_int32 * 1)(zp)
    fake = C.c_void_p(16)
    assert N.lib().osh_dqmm_pack_weights(8, 8, fake, signed, z, 1, fake, None) == N.OSH_E_INVALID
    assert "zero point" in N.last_error()


def test_ctypes_structs_match_the_c_header(tmp_path):
    """The ctypes mirrors of the header's structs have the C layout (sizes and
    field offsets as gcc lays them out from include/osh_hip.h)."""
    import ctypes as C
    import os
    import shutil
    import subprocess
    from onnxsharp_amd import native as N
    if not shutil.which("gcc"):
        pytest.skip("no gcc")
    structs = {"osh_conv_params": N.ConvParams, "osh_conv_attrs": N.ConvAttrs, "osh_pw_stage": N.PwStage,
               "osh_pw_chain": N.PwChain}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "osh_hip.h"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'  printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    inc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", inc, str(src), "-o", str(exe)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n") if l)
    for cname, py in structs.items():
        assert int(got[cname]) == C.sizeof(py), cname
        for f, _ in py._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(py, f).offset, f"{cname}.{f}"


def test_conv1d_shapes_follow_conv1dshape():
    # ConvLayer.Conv1DShape / Resolve1D (src/OnnxSharp/Ops/DnnOps.cs:204-227):
    # pads [begin, end], the end pad read when given; auto_pad on the one axis
    from onnxsharp_amd.layers import ConvLayer
    assert ConvLayer(pads=[1, 1]).get_memory_shapes((2, 16, 100), (32, 16, 3)) == (2, 32, 100)
    # (77 + 4 + 2 - 9) // 2 + 1 = 38 (the 2-D rule, begin pad twice, would give 39)
    layer = ConvLayer(strides=[2], pads=[4, 2], dilations=[2])
    assert layer.get_memory_shapes((1, 8, 77), (12, 8, 5)) == (1, 12, 38)
    p = layer.resolve((1, 8, 77), (12, 8, 5))
    assert (p.h, p.w, p.kh, p.kw, p.sh, p.sw, p.dh, p.dw, p.pt, p.pl, p.oh, p.ow) == (1, 77, 1, 5, 1, 2, 1, 2, 0, 4, 1, 38)
    assert ConvLayer(auto_pad="SAME_UPPER", strides=[3]).get_memory_shapes((1, 6, 33), (5, 6, 4)) == (1, 5, 11)
    assert ConvLayer(group=4).get_memory_shapes((1, 16, 50), (16, 4, 3)) == (1, 16, 48)
    with pytest.raises(Exception):
        ConvLayer().get_memory_shapes((1, 16, 50), (16, 4, 3, 3))  # ranks differ


def test_emitter_registry_and_noemit_switch(monkeypatch):
    # the host side of the emitter registry (VkOpRegistry.CanEmit,
    # src/OnnxSharp.Vulkan/VkOpRegistry.cs:168-180): fused activations the
    # launch does not apply are refused, a MatMul's fused bias is taken, and
    # ONNXSHARP_HIP_NOEMIT drops emitters by name (ONNXSHARP_VK_NOEMIT, :154-161)
    from onnxsharp_amd import registry as R
    monkeypatch.delenv("ONNXSHARP_HIP_NOEMIT", raising=False)
    assert R.can_emit("Conv") and R.can_emit("Conv", "Silu") and R.can_emit("Conv", "Relu")
    assert not R.can_emit("Conv", "Sigmoid")
    assert R.can_emit("MatMul", fused_bias=True) and not R.can_emit("MatMul", "Silu")
    assert not R.can_emit("Gemm", fused_bias=True)
    assert R.can_emit("DynamicQuantizeMatMul") and not R.can_emit("Resize")
    monkeypatch.setenv("ONNXSHARP_HIP_NOEMIT", " conv, DQMM ,,")
    assert R.disabled() == {"conv", "dqmm"}
    assert not R.can_emit("Conv") and not R.can_emit("DynamicQuantizeMatMul")
    assert R.can_emit("MatMul") and R.can_emit("MatMulInteger")
    assert not R.can_emit("MatMul", env="matmul")
