"""The device frame's wiring against an independent restatement of YOLO11n.

oracle/yolo11n_net.py writes the network from the Ultralytics module
definitions (concat orders, split halves, residual sources, the attention's
q/k/v rows), with the node names of the reference's fixture
(tests/golden/yolo11n.shapes.tsv, the reference's tests/data file) and
without onnxsharp_amd.yolo11n.  These CPU tests check:
* the independent network against the reference fixture: every conv, Add,
  Concat, MaxPool and Resize it produces is a node of the fixture with the
  fixture's output shape, and it has the fixture's Conv nodes (all 88 but
  the DFL's fixed 1x1 conv, which the head's decode stands for);
* the device model's layer list against it: the same convs (input and
  output shapes, kernel, stride, groups, activation, weights bit for bit);
* the device model's op list (before and after its launch fusions) executed
  with the oracle's arithmetic against it: every named tensor and the three
  heads equal bit for bit;
* that a shape-preserving wiring mistake planted in the independent network
  (a swapped concat, swapped split halves) is caught.
The GPU tests run the device frame against the same network at 320 and 640."""
import os

import numpy as np
import pytest

from onnxsharp_amd import synth

HERE = os.path.dirname(os.path.abspath(__file__))


def fixture():
    """{node name: (op type, output shape)} from the reference's shape fixture."""
    nodes = {}
    for line in open(os.path.join(HERE, "golden", "yolo11n.shapes.tsv")):
        f = line.rstrip("\n").split("\t")
        if len(f) >= 6 and f[1] == "TENSOR" and f[3].endswith("_output_0"):
            nodes[f[3][: -len("_output_0")]] = (f[2], tuple(int(v) for v in f[5].split(",")))
    return nodes


def test_independent_network_matches_the_reference_fixture(oracle):
    from oracle.yolo11n_net import Net
    net = Net(oracle, dry=True)
    heads = net.forward(np.zeros((1, 3, 640, 640), np.float32))
    fx = fixture()
    fx_convs = {n for n, (t, _) in fx.items() if t == "Conv"}
    # the export's 88th Conv is the DFL's fixed arange(16) 1x1 conv, which
    # the decode (DflSoftmax) stands for
    assert len(fx_convs) == 88 and "/model.23/dfl/conv/Conv" in fx_convs
    assert {c["name"] for c in net.convs} == fx_convs - {"/model.23/dfl/conv/Conv"}
    checked = 0
    for name, y in net.tensors.items():
        if name in fx:
            assert tuple(y.shape) == fx[name][1], (name, y.shape, fx[name])
            checked += 1
        else:  # only the attention's reshaped output has another name in the export
            assert name.endswith("/attn/Reshape_1"), name
    glue = {n for n, (t, _) in fx.items() if t in ("Add", "MaxPool", "Resize") and not n.startswith("/model.23/")}
    assert glue <= set(net.tensors), sorted(glue - set(net.tensors))
    assert checked >= 87 + len(glue)
    assert [h.shape for h in heads] == [(1, 144, 80, 80), (1, 144, 40, 40), (1, 144, 20, 20)]
    assert [fx[f"/model.23/Concat{s}"][1] for s in ("", "_1", "_2")] == [h.shape for h in heads]


def _device_convs(model):
    """{node name: (x channels, y shape, k, s, group, act, w, b)} of the device
    model's convs, the per-head parts of a conv joined back into one."""
    from onnxsharp_amd import yolo11n as Y
    out = {}
    for op in model.ops:
        if not isinstance(op, Y.ConvOp):
            continue
        name, _, head = op.name.partition("#head")
        e = (op.x.c, (op.y.c, op.y.h, op.y.w), op.k, op.s, op.group, op.act, op.w, op.b)
        if head and name in out:
            p = out[name]
            e = (p[0] + e[0], (p[1][0] + e[1][0],) + e[1][1:], op.k, op.s, p[4] + op.group, op.act,
                 np.concatenate([p[6], op.w]), np.concatenate([p[7], op.b]))
        out[name] = e
    return out


def test_device_model_has_the_independent_networks_layers(oracle):
    from onnxsharp_amd import yolo11n as Y
    from oracle.yolo11n_net import Net
    net = Net(oracle, dry=True)
    net.forward(np.zeros((1, 3, 640, 640), np.float32))
    dev = _device_convs(Y.build(640))
    assert set(dev) == {c["name"] for c in net.convs}
    for c in net.convs:
        xc, yshape, k, s, g, act, w, b = dev[c["name"]]
        ew, eb = net.weights(c["name"], c["w"])
        assert (xc, k, s, g, act) == (c["x"][1], c["w"][2], c["s"], c["g"], c["act"]), c["name"]
        assert yshape[0] == c["w"][0], c["name"]
        assert np.array_equal(w, ew) and np.array_equal(b, eb), c["name"]


def _run_device_model(oracle, model, x):
    """Run the device model's op list with the oracle's arithmetic; returns
    {node name: output} as each op wrote it, and the model's outputs."""
    from onnxsharp_amd import yolo11n as Y
    from oracle import yolo_frame as YO
    fr = YO.Frame(model)
    fr.put(Y.whole(model.input), x)
    seen = {}
    for grouped in model.ops:
        members = grouped.ops if isinstance(grouped, (Y.GroupConvOp, Y.ChainOp, Y.PairOp)) else [grouped]
        for op in members:
            ins = [np.ascontiguousarray(fr.get(s)) for s in YO.op_inputs(op)]
            y = YO.run_op(oracle, op, ins)
            fr.put(op.y, y)
            if isinstance(op, Y.PoolChainOp):
                c = op.y.c // 3
                names = [op.x.buf.name.replace("/Concat", f"/{nm}/MaxPool") for nm in ("m", "m_1", "m_2")]
                for j, nm in enumerate(names):
                    seen[nm] = y[:, j * c:(j + 1) * c]
                continue
            name = op.name
            if isinstance(op, Y.AttentionOp):
                name += "/Reshape_1"
            head = "#head" in name.split("+", 1)[0]  # one head's channels of a conv
            if "+" in name:  # a conv with its residual Add: the Add's output
                name = name.split("+", 1)[1]
            base = name.partition("#head")[0]
            if head:
                prev = seen.get(base)
                seen[base] = y if prev is None else np.concatenate([prev, y], axis=1)
            else:
                seen[name] = y
    return seen, [fr.arrays[id(b)] for b in model.outputs]


@pytest.mark.parametrize("size,fused", [(64, False), (64, True), (128, True)])
def test_device_wiring_gives_the_independent_networks_tensors(oracle, size, fused):
    from onnxsharp_amd import yolo11n as Y
    from oracle.yolo11n_net import Net
    model = Y.build(size)
    if fused:
        model = Y.fuse_launches(model)
    x = synth.uniform(4300 + size, (1, 3, size, size))
    seen, heads = _run_device_model(oracle, model, x)
    net = Net(oracle)
    ref = net.forward(x)
    for i, (g, r) in enumerate(zip(heads, ref)):
        assert np.array_equal(g, r), f"head {i}"
    compared = 0
    for name, y in seen.items():
        assert name in net.tensors, name
        assert np.array_equal(y, net.tensors[name]), name
        compared += 1
    assert compared >= (87 if not fused else 70)


def test_planted_wiring_mistakes_are_caught(oracle):
    """Shape-preserving mistakes in the independent network: the upsampled
    map and the skip swapped in model.12's concat, and the two halves of a
    C3k2's split swapped; each must change the heads."""
    from onnxsharp_amd import yolo11n as Y
    from oracle.yolo11n_net import Net

    class SwappedConcat(Net):
        def cat(self, name, parts):
            if name == "/model.12/Concat":
                parts = parts[::-1]
            return super().cat(name, parts)

    class SwappedSplit(Net):
        def c3k2(self, p, x, c2, c3k, e=0.5, n=1, shortcut=True):
            if p != "/model.13":
                return super().c3k2(p, x, c2, c3k, e, n, shortcut)
            c = int(c2 * e)
            y = self.conv(f"{p}/cv1/conv/Conv", x, 2 * c)
            parts = [y[:, c:], y[:, :c]]
            parts.append(self.bottleneck(f"{p}/m.0", parts[-1], c, shortcut, 0.5))
            return self.conv(f"{p}/cv2/conv/Conv", self.cat(f"{p}/Concat", parts), c2)

    size = 64
    x = synth.uniform(4400, (1, 3, size, size))
    _, heads = _run_device_model(oracle, Y.build(size), x)
    assert all(np.array_equal(g, r) for g, r in zip(heads, Net(oracle).forward(x)))
    for bad in (SwappedConcat, SwappedSplit):
        ref = bad(oracle).forward(x)
        assert not all(np.array_equal(g, r) for g, r in zip(heads, ref)), bad.__name__
