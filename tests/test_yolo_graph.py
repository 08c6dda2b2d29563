"""The YOLO11n network definition against the reference's node/shape fixture
(tests/data/yolo11n.shapes.tsv of the reference, copied as data to
tests/golden/): every Conv, MaxPool, Resize, Add and attention tensor the
device graph produces has the fixture's name and shape at 640 x 640, and the
graph has the fixture's 87 device convolutions (its 88th, the DFL conv, stays
on the host).  CPU only: shape inference, no kernels."""
import os

import numpy as np
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


def test_residual_fusion_folds_every_add(model):
    # every Add of the frame follows the conv that feeds it and is that conv's
    # only reader: all 14 fold into their convs (the attention Add into both
    # per-head parts of the positional depthwise conv)
    from onnxsharp_amd import yolo11n as Y
    f = Y.fuse_residual_adds(model)
    adds = [op for op in model.ops if isinstance(op, Y.AddOp)]
    assert len(adds) == 14
    assert not any(isinstance(op, Y.AddOp) for op in f.ops)
    fused = [op for op in f.ops if isinstance(op, Y.ConvOp) and op.res is not None]
    assert len(fused) == 15
    assert len(f.ops) == len(model.ops) - 14
    for op in fused:
        assert not Y._overlap(op.res, op.y) and not Y._overlap(op.x, op.y)
    # the outputs the adds produced are now written by the convs
    assert {id(op.y.buf) for op in adds} <= {id(op.y.buf) for op in fused}
    # buffers of the folded conv outputs are gone
    assert len(f.bufs) < len(model.bufs)


def test_residual_fusion_keeps_a_shared_conv_output():
    # a conv output that another op also reads must stay a tensor of its own
    from onnxsharp_amd import yolo11n as Y
    bd = Y._Builder(32, 1)
    x = Y.whole(bd.buf("x", 16, 8, 8))
    bd.m.input = x.buf
    t = bd.conv("c1", x, 16, 3, 1)
    a = bd.add("a1", x, t)
    u = bd.conv("c2", t, 16, 1, 1)  # second reader of t
    bd.m.outputs = [a.buf, u.buf]
    f = Y.fuse_residual_adds(bd.m)
    assert [type(o).__name__ for o in f.ops] == ["ConvOp", "AddOp", "ConvOp"]


def test_sppf_pools_become_one_chain(model):
    from onnxsharp_amd import yolo11n as Y
    f = Y.fuse_pool_chains(Y.fuse_residual_adds(model))
    chains = [op for op in f.ops if isinstance(op, Y.PoolChainOp)]
    assert len(chains) == 1 and not any(isinstance(op, Y.MaxPoolOp) for op in f.ops)
    ch = chains[0]
    assert (ch.x.c, ch.y.c, ch.y.c0, ch.k, ch.x.h) == (128, 384, 128, 5, 20)
    assert len(f.ops) == len(model.ops) - 14 - 2


def test_fused_frame_equals_unfused_frame_on_the_oracle(model, oracle):
    # the fused op list computes the same bits as the ONNX node order
    from onnxsharp_amd import synth, yolo11n as Y
    from oracle import yolo_frame as YO
    small = Y.build(64)
    x = synth.uniform(4245, (1, 3, 64, 64))
    ref = YO.Frame(small).run(oracle, x)
    got = YO.Frame(Y.fuse_launches(small)).run(oracle, x)
    for g, r in zip(got, ref):
        assert np.array_equal(g, r)


@pytest.mark.parametrize("fused", [False, True], ids=["onnx_order", "fused"])
@pytest.mark.parametrize("nstreams", [1, 2, 4])
def test_stream_plan_orders_every_dependency(model, nstreams, fused):
    # Vector clocks over the planned streams: for each op, the latest op of
    # each stream known complete when it starts (stream order plus the event
    # waits).  Every read-after-write, write-after-write and write-after-read
    # pair of ops must be ordered.
    from onnxsharp_amd import yolo11n as Y
    if fused:
        model = Y.fuse_launches(model)
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


def test_c2f_block_structure():
    # C2f(128 -> 128, n=1, shortcut) at 80 x 80: cv1 1x1 into the concat, the
    # bottleneck's two 3x3 convs and the shortcut Add on the second half, cv2
    # 1x1 over the 192-channel concat; the Add folds into the second 3x3 conv
    from onnxsharp_amd import yolo11n as Y
    m = Y.build_c2f(80, 128, 128, 1, True)
    convs = [(o.k, o.x.c, o.y.c) for o in m.convs]
    assert convs == [(1, 128, 128), (3, 64, 64), (3, 64, 64), (1, 192, 128)]
    add = [o for o in m.ops if isinstance(o, Y.AddOp)]
    assert len(add) == 1 and (add[0].y.c0, add[0].y.c, add[0].y.buf.c) == (128, 64, 192)
    assert add[0].a.buf is add[0].y.buf and add[0].a.c0 == 64  # the shortcut is the split's second half
    assert abs(sum(o.flops for o in m.convs) / 1e9 - 1.4680064) < 1e-9
    f = Y.fuse_launches(m, pairs=False)
    assert len(f.ops) == 4 and f.ops[2].res is not None and f.ops[2].res.c0 == 64
    # by default the bottleneck's two 3x3 convs run as one pair launch
    f = Y.fuse_launches(m)
    assert len(f.ops) == 3 and isinstance(f.ops[1], Y.PairOp)
    pair = f.ops[1]
    assert pair.b.x.buf is pair.a.y.buf and pair.b.res.c0 == 64 and pair.a.x.c0 == 64
    assert [(b.c, b.h, b.w) for b in m.outputs] == [(128, 80, 80)]


def test_head_branch_ends_share_a_launch():
    # the head's final box and class 1x1 layers end independent branches:
    # the box group moves down to the class group's place and the six convs
    # run as one launch (72 -> 71 launches before the bottleneck pairs)
    from onnxsharp_amd import yolo11n as Y
    m = Y.build(640)
    f = Y.fuse_launches(m, pairs=False)
    assert len(f.ops) == 71
    six = [o for o in f.ops if isinstance(o, Y.GroupConvOp) and len(o.ops) == 6]
    assert len(six) == 1
    g = six[0]
    assert [o.name for o in g.ops] == [f"/model.23/cv{b}.{i}/cv{b}.{i}.2/Conv" for b in (2, 3) for i in range(3)]
    assert len({Y._conv_kind(o) for o in g.ops}) == 1 and all(o.act is None for o in g.ops)
    # every op still reads only what was written before it, and every conv runs once
    assert len(f.convs) == len(m.convs)
    head = lambda mm: sorted(o.name for o in mm.convs if o.name.startswith("/model.23/"))
    assert head(f) == head(m)
    written = {id(m.input)}
    for op in f.ops:
        reads, writes = Y.op_access(op)
        assert all(id(r.buf) in written for r in reads), op.name
        written.update(id(w.buf) for w in writes)
    # a group never moves past an op that reads its output
    a = next(o for o in f.ops if isinstance(o, Y.GroupConvOp) and o.name.startswith("/model.23/cv2.#/cv2.#.0"))
    b = next(o for o in f.ops if isinstance(o, Y.GroupConvOp) and o.name.startswith("/model.23/cv2.#/cv2.#.1"))
    assert not Y._independent(a, b)


def test_pairs_of_the_640_frame():
    # every bottleneck pair the library takes becomes one PairOp (which then
    # times the fused kernel against two launches on first use): all eleven
    # of the frame's, the 160x160 one with its 8-channel intermediate
    # included; and the stem (3 -> 16, stride 2) with the stride-2 16 -> 32
    # conv after it, whose 16 x 320 x 320 intermediate is not stored
    from onnxsharp_amd import yolo11n as Y
    m = Y.build(640)
    f = Y.fuse_launches(m)
    pairs = [o for o in f.ops if isinstance(o, Y.PairOp)]
    stem = [p for p in pairs if p.a.x.c == 3]
    assert len(stem) == 1 and f.ops[0] is stem[0] and not stem[0].store_mid
    assert (stem[0].a.s, stem[0].b.s, stem[0].a.y.c, stem[0].b.y.c, stem[0].b.y.h) == (2, 2, 16, 32, 160)
    pairs = [p for p in pairs if p.a.x.c != 3]
    assert sorted((p.a.x.c, p.a.y.c, p.b.y.c, p.a.x.h) for p in pairs) == sorted(
        [(16, 8, 16, 160)] + [(32, 16, 32, 80)] * 2 + [(32, 32, 32, 40)] * 2 + [(64, 32, 64, 40)] * 2 +
        [(64, 64, 64, 20)] * 4)
    assert all(p.b.res is not None and p.b.res.buf is p.a.x.buf and p.store_mid for p in pairs)
    assert len(f.ops) == len(Y.fuse_launches(m, pairs=False).ops) - 12
    # a map-size floor keeps the smaller maps' convs apart
    g = Y.pair_bottleneck_convs(Y.fuse_launches(m, pairs=False), min_pixels=6400)
    assert len([o for o in g.ops if isinstance(o, Y.PairOp)]) == 4
    # a refusal from the library keeps the convs separate
    h = Y.pair_bottleneck_convs(Y.fuse_launches(m, pairs=False), takes=lambda a, b: False)
    assert not any(isinstance(o, Y.PairOp) for o in h.ops)
    # the stem's map is stored after all when a caller reads it as an output
    mo = Y.build(640)
    stem_map = mo.ops[0].y.buf
    mo.outputs = mo.outputs + [stem_map]
    fo = Y.fuse_launches(mo)
    so = [o for o in fo.ops if isinstance(o, Y.PairOp) and o.a.x.c == 3]
    assert len(so) == 1 and so[0].store_mid and so[0].a.y.buf is stem_map


def test_decode_appends_dfl_and_sigmoid_per_scale():
    from onnxsharp_amd import yolo11n as Y
    m = Y.build(640, decode=True)
    dfl = [o for o in m.ops if isinstance(o, Y.DflOp)]
    sig = [o for o in m.ops if isinstance(o, Y.SigmoidOp)]
    assert len(dfl) == len(sig) == 3
    assert [(b.c, b.h, b.w) for b in m.outputs] == [(84, 80, 80), (84, 40, 40), (84, 20, 20)]
    for d, s_ in zip(dfl, sig):
        assert (d.x.c0, d.x.c, d.y.c0, d.y.c) == (0, 64, 0, 4)
        assert (s_.x.c0, s_.x.c, s_.y.c0, s_.y.c) == (64, 80, 4, 80)
        assert d.y.buf is s_.y.buf


def test_head_convs_group_by_layer(model):
    # The Detect head's 24 convs become 8 groups (one per layer, the three
    # scales in order), placed where the head was; with the C3k blocks' paired
    # 1x1 convs and the positional conv's two heads grouped too, the frame
    # drops from 92 launches to 72 (before the bottleneck pairs and the
    # pointwise chains).
    from onnxsharp_amd import yolo11n as Y
    fused = Y.fuse_launches(model, chains=False, pairs=False, merge=False)
    head = [o for o in fused.ops if isinstance(o, Y.GroupConvOp) and o.name.startswith("/model.23/cv")]
    other = [o for o in fused.ops if isinstance(o, Y.GroupConvOp) and o not in head]
    assert len(head) == 8 and len(other) == 4 and len(fused.ops) == 72
    for g in other:
        assert len({Y._conv_kind(o) for o in g.ops}) == 1
        assert all(Y._independent(a, b) for a in g.ops for b in g.ops if a is not b)
    for g in head:
        assert [o.name for o in g.ops] == [g.name.replace("#", str(i)) for i in range(3)]
        assert len({(o.k, o.s, o.group > 1, o.act) for o in g.ops}) == 1
    assert len(fused.convs) == len(model.convs)
    head = lambda m: sorted(o.name for o in m.convs if o.name.startswith("/model.23/"))
    assert head(fused) == head(model)
    # every op still reads only slices written before it (or the input)
    written = {id(model.input)}
    for op in fused.ops:
        reads, writes = Y.op_access(op)
        for r in reads:
            assert id(r.buf) in written, (op.name, r.buf.name)
        written.update(id(w.buf) for w in writes)


def test_pointwise_chains_of_the_640_frame(model):
    # With chains on, runs of pointwise convs whose weights fit in LDS become
    # chain launches where the cost model says they pay: C3k2's cv1 with the
    # C3k's paired 1x1 convs and C3k's cv3 with C3k2's cv2 (model.6 at 40x40),
    # and the head's class branch in two launches of three scales: 72
    # launches become 67.  (The C2PSA tail's 576 KB of weights do not fit.)
    from onnxsharp_amd import yolo11n as Y
    fused = Y.fuse_launches(model, chains=True, pairs=False, merge=False)
    chains = [o for o in fused.ops if isinstance(o, Y.ChainOp)]
    assert len(fused.ops) == 67 and len(chains) == 4
    assert len(Y.fuse_launches(model, pairs=False, merge=False).ops) == 72  # off by default
    unchained = Y.fuse_launches(model, chains=False, pairs=False, merge=False)
    assert sorted(o.name for o in fused.convs) == sorted(o.name for o in unchained.convs)
    shapes = [[[(o.x.c, o.y.c, o.y.h) for o in ch] for ch in c.chains] for c in chains]
    assert [[(128, 128, 40), (64, 32, 40), (64, 32, 40)]] in shapes  # model.6 cv1 -> C3k cv1, cv2
    head = [c for c in chains if c.name.startswith("/model.23/")]
    assert len(head) == 2 and all(len(c.chains) == 3 for c in head)
    assert all(Y._is_depthwise3x3(ch[0]) for c in head for ch in c.chains)
    # the C2PSA tail: ffn.1 would add proj's output from chip, proj the shortcut from memory
    ops = [o for o in unchained.ops if isinstance(o, Y.ConvOp) and "/model.10/m/m.0/" in o.name and o.k == 1][1:]
    assert Y.chain_res_stage(ops[2], ops[:2]) == 0 and Y.chain_res_stage(ops[0], []) == -1
    assert Y._chain_launch(ops + [next(o for o in unchained.ops if o.name == "/model.10/cv2/conv/Conv")]) is None
    for c in chains:
        assert Y._chain_launch(c.ops) is not None
        for ch in c.chains:
            assert len({(o.y.h, o.y.w) for o in ch}) == 1
            for k, op in enumerate(ch):
                parts = Y.chain_parts(op.x, ch[:k])
                assert [p.c0 for _, p in parts] == [op.x.c0] + [op.x.c0 + sum(q.c for _, q in parts[:i])
                                                               for i in range(1, len(parts))]
                assert sum(p.c for _, p in parts) == op.x.c
                for st, p in parts:
                    if st >= 0:  # inside the stage's output
                        y = ch[st].y
                        assert p.buf is y.buf and y.c0 <= p.c0 and p.c0 + p.c <= y.c0 + y.c
                    else:  # written by no earlier stage
                        assert not any(Y._overlap(p, e.y) for e in ch[:k])
    # C3k's cv3 -> C3k2's cv2 over [C3k2's cv1 output, cv3's output]
    c6 = next(c for c in chains if c.name.startswith("/model.6/m.0/cv3")).chains[0]
    assert [(s, p.c0, p.c) for s, p in Y.chain_parts(c6[1].x, c6[:1])] == [(-1, 0, 128), (0, 128, 64)]


def test_chain_launch_refusals(model):
    from onnxsharp_amd import yolo11n as Y
    fused = Y.fuse_launches(model, chains=False)
    ops = {o.name: o for o in fused.convs}
    g = lambda n: ops[n]
    dw = g("/model.23/cv3.0/cv3.0.1/cv3.0.1.0/conv/Conv")
    pw = g("/model.23/cv3.0/cv3.0.0/cv3.0.0.1/conv/Conv")
    assert Y._chain_launch([pw, dw]) is None  # a depthwise conv only as stage 0
    assert Y._chain_launch([g("/model.6/m.0/m/m.0/cv1/conv/Conv")]) is None  # a dense 3x3 conv
    # four independent chains: one more than a launch takes
    four = [g(f"/model.23/cv3.{i}/cv3.{i}.0/cv3.{i}.0.0/conv/Conv") for i in range(3)] + [dw]
    assert Y._chain_launch(four) is None
    # maps of different sizes in one chain
    a = g("/model.13/cv2/conv/Conv")  # 1x1 at 40x40
    b = g("/model.16/cv1/conv/Conv")  # 1x1 at 80x80
    assert Y._chain_launch([a, b]) is not None  # independent: two chains
    import dataclasses
    b2 = dataclasses.replace(b, x=a.y)
    assert Y._chain_launch([a, b2]) is None  # b2 reads a's output on another map
