"""The YOLO11n network definition against the reference's node/shape fixture
(tests/data/yolo11n.shapes.tsv of the reference, copied as data to
tests/golden/): every Conv, MaxPool, Resize, Add and attention tensor the
device graph produces has the fixture's name and shape at 640 x 640, and the
graph has the fixture's 87 device convolutions (its 88th, the DFL conv, stays
on the host).  CPU only: shape inference, no kernels."""
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _fixture():
    shapes, nodes = {}, []
    with open(os.path.join(HERE, "golden", "yolo11n.shapes.tsv")) as f:
        for line in f:
            cols = line.rstrip("\n").split("\t")
            if len(cols) < 6:
                continue
            if cols[1] == "NODE":
                nodes.append((cols[2], cols[3]))
            elif cols[1] == "TENSOR":
                shapes[cols[3]] = tuple(int(v) for v in cols[5].split(","))
    return shapes, nodes


@pytest.fixture(scope="module")
def model():
    from onnxsharp_amd import yolo11n
    return yolo11n.build(640)


def test_conv_names_and_shapes_match_fixture(model):
    from onnxsharp_amd import yolo11n
    shapes, nodes = _fixture()
    fixture_convs = [n for t, n in nodes if t == "Conv" and "/dfl/" not in n]
    assert len(fixture_convs) == 87
    seen = {}
    for op in model.ops:
        if isinstance(op, yolo11n.ConvOp):
            base = op.name.split("#")[0]
            if base in seen:  # the per-head parts of one depthwise conv
                continue
            seen[base] = op
    assert sorted(seen) == sorted(fixture_convs)
    for name, op in seen.items():
        buf_shape = (1, op.y.buf.c, op.y.h, op.y.w) if "#head" in op.name else op.y.shape
        assert buf_shape == shapes[name + "_output_0"], name


def test_glue_ops_match_fixture(model):
    from onnxsharp_amd import yolo11n
    shapes, nodes = _fixture()
    kinds = {"MaxPool": yolo11n.MaxPoolOp, "Resize": yolo11n.UpsampleOp, "Add": yolo11n.AddOp}
    for kind, cls in kinds.items():
        fixture = [n for t, n in nodes if t == kind and n.startswith("/model.") and not n.startswith("/model.23/")]
        ours = [op for op in model.ops if isinstance(op, cls)]
        assert sorted(op.name for op in ours) == sorted(fixture), kind
        for op in ours:
            assert op.y.shape == shapes[op.name + "_output_0"], op.name
    att = [op for op in model.ops if isinstance(op, yolo11n.AttentionOp)]
    assert len(att) == 1
    a = att[0]
    assert (1, a.heads, a.attn.h, a.attn.w) == shapes[a.name + "/Softmax_output_0"]
    assert (1, a.heads, a.y.c // a.heads, a.y.h * a.y.w) == shapes[a.name + "/MatMul_1_output_0"]
    assert a.qkv.shape == shapes[a.name + "/qkv/conv/Conv_output_0"]


def test_outputs_and_flops(model):
    assert [(b.c, b.h, b.w) for b in model.outputs] == [(144, 80, 80), (144, 40, 40), (144, 20, 20)]
    # the convolutions alone are the published 6.5 GFLOPs of YOLO11n at 640
    # (multiply-add counted as 2); attention adds 2 * 2 * 400^2 * (32 + 64)
    conv = sum(op.flops for op in model.convs)
    assert abs(conv / 1e9 - 6.48) < 0.01, conv / 1e9
    assert model.flops - conv == 2 * 2 * 400 ** 2 * (32 + 64)


@pytest.mark.parametrize("nstreams", [1, 2, 4])
def test_stream_plan_orders_every_dependency(model, nstreams):
    # Vector clocks over the planned streams: for each op, the latest op of
    # each stream known complete when it starts (stream order plus the event
    # waits).  Every read-after-write, write-after-write and write-after-read
    # pair of ops must be ordered.
    from onnxsharp_amd import yolo11n as Y
    plan, waits, recorded = Y.plan_streams(model.ops, nstreams)
    acc = [Y.op_access(o) for o in model.ops]
    clock = [[-1] * nstreams for _ in range(nstreams)]  # per stream: clock before its next op
    after = []
    for i, s in enumerate(plan):
        c = clock[s]
        for j in waits[i]:
            assert j in recorded and plan[j] != s
            c = [max(a, b) for a, b in zip(c, after[j])]
        ri, wi = acc[i]
        for j in range(i):
            rj, wj = acc[j]
            dep = (any(Y._overlap(a, b) for a in wj for b in ri + wi) or
                   any(Y._overlap(a, b) for a in rj for b in wi))
            if dep:
                assert plan[j] == s or c[plan[j]] >= j, f"op {i} {model.ops[i].name} not ordered after op {j}"
        c = list(c)
        c[s] = i
        clock[s] = c
        after.append(c)
    if nstreams > 1:
        assert len(set(plan)) > 1  # the head and the P3 branch do fork
