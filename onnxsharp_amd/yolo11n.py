"""YOLO11n backbone + neck + head (batch 1, NCHW FP32) on the device.

The network is the one the reference benchmarks as a whole frame: 87 Conv
(+SiLU) layers, the C2PSA attention, SPPF max pools, nearest upsampling and
the channel Concat/Split/Add glue between them (node list in the reference's
tests/data/yolo11n.shapes.tsv; the CPU path per layer is the dispatch of
ConvLayer.Forward, src/OnnxSharp/Ops/DnnOps.cs:411-500).  The Detect head's
DFL/NMS stay on the host: a frame ends with the three per-scale head tensors
[1, 64 + 80, H, W] (box distribution logits, class logits).

Layout: every activation lives in a device buffer; Concat and Split along
channels cost nothing because producers write into, and consumers read from,
channel slices of one buffer (batch 1, so a slice is a pointer offset).  The
op list is in execution order; `Frame` issues it on one stream and can record
it once as a HIP graph and replay it per frame.

Weights are random (no checkpoint is available): conv weights N(0, 0.05) and
biases N(0, 0.01) standing for BatchNorm folded into the conv, from the
counter-based generator in `synth`, seeded by the model seed and the layer's
node name (`synth.layer_seed`).
"""
from __future__ import annotations

import ctypes as C
import re
from dataclasses import dataclass, field

import numpy as np

from . import native as N
from . import synth


@dataclass(eq=False)
class Buf:
    name: str
    c: int
    h: int
    w: int
    tensor: object = None  # torch tensor once allocated

    @property
    def numel(self):
        return self.c * self.h * self.w


@dataclass(eq=False)
class Slice:
    buf: Buf
    c0: int
    c: int

    @property
    def h(self):
        return self.buf.h

    @property
    def w(self):
        return self.buf.w

    @property
    def shape(self):
        return (1, self.c, self.buf.h, self.buf.w)

    def ptr(self):
        return C.c_void_p(self.buf.tensor.data_ptr() + 4 * self.c0 * self.buf.h * self.buf.w)

    def sub(self, c0, c):
        assert 0 <= c0 and c0 + c <= self.c
        return Slice(self.buf, self.c0 + c0, c)


def whole(buf: Buf) -> Slice:
    return Slice(buf, 0, buf.c)


@dataclass(eq=False)
class ConvOp:
    name: str
    x: Slice
    y: Slice
    k: int
    s: int
    group: int
    act: str | None
    w: np.ndarray
    b: np.ndarray
    res: Slice = None  # residual added after the activation (a fused Add)

    @property
    def flops(self):
        return 2.0 * self.y.c * (self.x.c // self.group) * self.k * self.k * self.y.h * self.y.w


@dataclass(eq=False)
class GroupConvOp:
    """Independent convs run as one launch (osh_conv2d_group_f32): the same
    layer of the detection head's three scales."""
    name: str
    ops: list

    @property
    def flops(self):
        return sum(o.flops for o in self.ops)


@dataclass(eq=False)
class ChainOp:
    """Up to three independent chains of convs over one map each -- 1x1 convs,
    the first one may be a 3x3 depthwise -- run as one launch
    (osh_pw_chain_f32): a stage reads earlier stages' outputs on chip, and
    every stage still writes its whole output, so readers outside the chain
    see what the convs one by one would have written."""
    name: str
    chains: list  # per chain: its ConvOps in stage order

    @property
    def ops(self):
        return [o for ch in self.chains for o in ch]

    @property
    def flops(self):
        return sum(o.flops for o in self.ops)


@dataclass(eq=False)
class PairOp:
    """Two chained 3x3 SiLU convs, b reading exactly a's output, run as one
    launch (osh_conv2d_pair_f32): a bottleneck's cv1 -> cv2 over one map, or
    the network's first conv and the stride-2 conv after it.  a's output
    stays on chip for b; it is also written to a.y when store_mid is set
    (which lets first-use timing try the two convs as separate launches)."""
    name: str
    a: ConvOp
    b: ConvOp
    store_mid: bool = True

    @property
    def ops(self):
        return [self.a, self.b]

    @property
    def flops(self):
        return self.a.flops + self.b.flops


@dataclass(eq=False)
class AddOp:
    name: str
    a: Slice
    b: Slice
    y: Slice


@dataclass(eq=False)
class MaxPoolOp:
    name: str
    x: Slice
    y: Slice
    k: int = 5
    s: int = 1
    p: int = 2


@dataclass(eq=False)
class PoolChainOp:
    """Three chained k x k, stride 1, pad k/2 MaxPools whose outputs are the
    three adjacent channel slices of y (y1, y2, y3), as in SPPF."""
    name: str
    x: Slice
    y: Slice
    k: int = 5


@dataclass(eq=False)
class DflOp:
    """DflSoftmax over a head tensor's box channels (sides*bins of them):
    y[side] = sum over b of softmax_b(x[side*bins + b]) * b."""
    name: str
    x: Slice
    y: Slice
    bins: int = 16


@dataclass(eq=False)
class SigmoidOp:
    name: str
    x: Slice
    y: Slice


@dataclass(eq=False)
class UpsampleOp:
    name: str
    x: Slice
    y: Slice
    f: int = 2


@dataclass(eq=False)
class AttentionOp:
    """Attention core of C2PSA (ultralytics Attention.forward, exported as the
    Reshape/Split/Transpose/MatMul/Mul/Softmax/MatMul nodes of /model.10/m/m.0/attn):
    per head h, q = qkv[h, :kd], k = qkv[h, kd:2kd], v = qkv[h, 2kd:] (each
    [rows, N], N = H*W); attn = softmax(scale * q^T k); y[h] = v attn^T."""
    name: str
    qkv: Slice
    y: Slice
    heads: int
    key_dim: int
    head_dim: int
    scale: float
    qt: Buf = None     # [heads, N, key_dim]
    attn: Buf = None   # [heads, N, N] scores, then probabilities
    attn_t: Buf = None  # [heads, N, N] probabilities transposed


@dataclass
class Model:
    size: int
    bufs: list = field(default_factory=list)
    ops: list = field(default_factory=list)
    input: Buf = None
    outputs: list = field(default_factory=list)

    @property
    def convs(self):
        out = []
        for o in self.ops:
            if isinstance(o, ConvOp):
                out.append(o)
            elif isinstance(o, (GroupConvOp, ChainOp, PairOp)):
                out.extend(o.ops)
        return out

    @property
    def flops(self):
        att = sum(2.0 * o.heads * (o.y.h * o.y.w) ** 2 * (o.key_dim + o.head_dim)
                  for o in self.ops if isinstance(o, AttentionOp))
        return sum(o.flops for o in self.convs) + att


class _Builder:
    def __init__(self, size, seed):
        self.m = Model(size)
        self.seed = seed
        self.nconv = 0

    def buf(self, name, c, h, w):
        b = Buf(name, c, h, w)
        self.m.bufs.append(b)
        return b

    def conv(self, name, x: Slice, cout, k, s, act="Silu", group=1, y: Slice = None):
        pad = k // 2
        oh = (x.h + 2 * pad - k) // s + 1
        ow = (x.w + 2 * pad - k) // s + 1
        if y is None:
            y = whole(self.buf(name + "_out", cout, oh, ow))
        assert (y.c, y.h, y.w) == (cout, oh, ow), (name, y.c, y.h, y.w, cout, oh, ow)
        self.nconv += 1
        w = synth.normal(synth.layer_seed(self.seed, name, 0), (cout, x.c // group, k, k), 0.0, 0.05)
        b = synth.normal(synth.layer_seed(self.seed, name, 1), (cout,), 0.0, 0.01)
        self.m.ops.append(ConvOp(name, x, y, k, s, group, act, w, b))
        return y

    def add(self, name, a, b, y=None):
        if y is None:
            y = whole(self.buf(name + "_out", a.c, a.h, a.w))
        self.m.ops.append(AddOp(name, a, b, y))
        return y

    # ---- ultralytics modules (names follow the exported ONNX node names)
    def bottleneck(self, p, x: Slice, c_out, k, e, shortcut, y: Slice = None):
        c_ = int(c_out * e)
        t = self.conv(f"{p}/cv1/conv/Conv", x, c_, k, 1)
        if shortcut and x.c == c_out:
            u = self.conv(f"{p}/cv2/conv/Conv", t, c_out, k, 1)
            return self.add(f"{p}/Add", x, u, y)
        return self.conv(f"{p}/cv2/conv/Conv", t, c_out, k, 1, y=y)

    def c3k(self, p, x: Slice, c_out, n, shortcut, y: Slice):
        c_ = c_out // 2
        cat = self.buf(f"{p}/Concat", 2 * c_, x.h, x.w)
        h = self.conv(f"{p}/cv1/conv/Conv", x, c_, 1, 1)
        for i in range(n):
            last = i == n - 1
            h = self.bottleneck(f"{p}/m/m.{i}", h, c_, 3, 1.0, shortcut,
                                y=Slice(cat, 0, c_) if last else None)
        self.conv(f"{p}/cv2/conv/Conv", x, c_, 1, 1, y=Slice(cat, c_, c_))
        return self.conv(f"{p}/cv3/conv/Conv", whole(cat), c_out, 1, 1, y=y)

    def c3k2(self, p, x: Slice, c_out, c3k, e, shortcut=True, y: Slice = None):
        c = int(c_out * e)
        cat = self.buf(f"{p}/Concat", 3 * c, x.h, x.w)
        self.conv(f"{p}/cv1/conv/Conv", x, 2 * c, 1, 1, y=Slice(cat, 0, 2 * c))
        b = Slice(cat, c, c)
        if c3k:
            self.c3k(f"{p}/m.0", b, c, 2, shortcut, y=Slice(cat, 2 * c, c))
        else:
            self.bottleneck(f"{p}/m.0", b, c, 3, 0.5, shortcut, y=Slice(cat, 2 * c, c))
        return self.conv(f"{p}/cv2/conv/Conv", whole(cat), c_out, 1, 1, y=y)

    def c2f(self, p, x: Slice, c_out, n=1, shortcut=False, e=0.5, y: Slice = None):
        """YOLOv8 C2f: cv1 (1x1) into two halves, n bottlenecks (two 3x3 convs,
        e = 1.0, shortcut Add) on the second half, each appended to the
        concat, then cv2 (1x1) over all (2 + n) parts."""
        c = int(c_out * e)
        cat = self.buf(f"{p}/Concat", (2 + n) * c, x.h, x.w)
        self.conv(f"{p}/cv1/conv/Conv", x, 2 * c, 1, 1, y=Slice(cat, 0, 2 * c))
        prev = Slice(cat, c, c)
        for i in range(n):
            prev = self.bottleneck(f"{p}/m.{i}", prev, c, 3, 1.0, shortcut, y=Slice(cat, (2 + i) * c, c))
        return self.conv(f"{p}/cv2/conv/Conv", whole(cat), c_out, 1, 1, y=y)

    def sppf(self, p, x: Slice, c_out, y: Slice = None):
        c_ = x.c // 2
        cat = self.buf(f"{p}/Concat", 4 * c_, x.h, x.w)
        prev = self.conv(f"{p}/cv1/conv/Conv", x, c_, 1, 1, y=Slice(cat, 0, c_))
        for i, nm in enumerate(["m", "m_1", "m_2"]):
            nxt = Slice(cat, (i + 1) * c_, c_)
            self.m.ops.append(MaxPoolOp(f"{p}/{nm}/MaxPool", prev, nxt))
            prev = nxt
        return self.conv(f"{p}/cv2/conv/Conv", whole(cat), c_out, 1, 1, y=y)

    def c2psa(self, p, x: Slice, c_out, y: Slice = None):
        c = c_out // 2
        heads = c // 64
        head_dim = c // heads
        key_dim = head_dim // 2
        hw = x.h * x.w
        cat = self.buf(f"{p}/Concat", 2 * c, x.h, x.w)
        self.conv(f"{p}/cv1/conv/Conv", x, 2 * c, 1, 1, y=Slice(cat, 0, 2 * c))
        b = Slice(cat, c, c)
        q = f"{p}/m/m.0"
        qkv = self.conv(f"{q}/attn/qkv/conv/Conv", b, c + 2 * key_dim * heads, 1, 1, act=None)
        att = whole(self.buf(f"{q}/attn/Reshape_1", c, x.h, x.w))
        op = AttentionOp(f"{q}/attn", qkv, att, heads, key_dim, head_dim, float(key_dim) ** -0.5,
                         qt=self.buf(f"{q}/attn/Transpose", heads, hw, key_dim),
                         attn=self.buf(f"{q}/attn/Softmax", heads, hw, hw),
                         attn_t=self.buf(f"{q}/attn/Transpose_1", heads, hw, hw))
        self.m.ops.append(op)
        # positional term: depthwise 3x3 over v seen as [1, c, H, W]; the heads'
        # v blocks are not adjacent inside qkv, so the conv runs per head
        pe_name = f"{q}/attn/pe/conv/Conv"
        pe = self.buf(pe_name, c, x.h, x.w)
        rows = 2 * key_dim + head_dim
        w = synth.normal(synth.layer_seed(self.seed, pe_name, 0), (c, 1, 3, 3), 0.0, 0.05)
        bias = synth.normal(synth.layer_seed(self.seed, pe_name, 1), (c,), 0.0, 0.01)
        self.nconv += 1
        for h in range(heads):
            v = qkv.sub(h * rows + 2 * key_dim, head_dim)
            sl = slice(h * head_dim, (h + 1) * head_dim)
            self.m.ops.append(ConvOp(pe_name + (f"#head{h}" if heads > 1 else ""), v,
                                     Slice(pe, h * head_dim, head_dim), 3, 1, head_dim, None, w[sl], bias[sl]))
        s1 = self.add(f"{q}/attn/Add", att, whole(pe))
        pr = self.conv(f"{q}/attn/proj/conv/Conv", s1, c, 1, 1, act=None)
        b1 = self.add(f"{q}/Add", b, pr)
        f0 = self.conv(f"{q}/ffn/ffn.0/conv/Conv", b1, 2 * c, 1, 1)
        f1 = self.conv(f"{q}/ffn/ffn.1/conv/Conv", f0, c, 1, 1, act=None)
        # Concat(split output 0, block output): the block output replaces the
        # split's second half (b is not read after the ffn's residual Add), so
        # the concat is cv1's own buffer and needs no copy
        self.m.ops.append(AddOp(f"{q}/Add_1", b1, f1, Slice(cat, c, c)))
        return self.conv(f"{p}/cv2/conv/Conv", whole(cat), c_out, 1, 1, y=y)

    def detect(self, p, xs, nc=80, reg_max=16):
        c2 = max(16, xs[0].c // 4, reg_max * 4)
        c3 = max(xs[0].c, min(nc, 100))
        outs = []
        for i, x in enumerate(xs):
            out = self.buf(f"{p}/out{i}", 4 * reg_max + nc, x.h, x.w)
            t = self.conv(f"{p}/cv2.{i}/cv2.{i}.0/conv/Conv", x, c2, 3, 1)
            t = self.conv(f"{p}/cv2.{i}/cv2.{i}.1/conv/Conv", t, c2, 3, 1)
            self.conv(f"{p}/cv2.{i}/cv2.{i}.2/Conv", t, 4 * reg_max, 1, 1, act=None, y=Slice(out, 0, 4 * reg_max))
            u = self.conv(f"{p}/cv3.{i}/cv3.{i}.0/cv3.{i}.0.0/conv/Conv", x, x.c, 3, 1, group=x.c)
            u = self.conv(f"{p}/cv3.{i}/cv3.{i}.0/cv3.{i}.0.1/conv/Conv", u, c3, 1, 1)
            u = self.conv(f"{p}/cv3.{i}/cv3.{i}.1/cv3.{i}.1.0/conv/Conv", u, c3, 3, 1, group=c3)
            u = self.conv(f"{p}/cv3.{i}/cv3.{i}.1/cv3.{i}.1.1/conv/Conv", u, c3, 1, 1)
            self.conv(f"{p}/cv3.{i}/cv3.{i}.2/Conv", u, nc, 1, 1, act=None, y=Slice(out, 4 * reg_max, nc))
            outs.append(out)
        return outs


@dataclass(eq=False)
class CopyOp:
    name: str
    x: Slice
    y: Slice


def build(size: int = 640, seed: int = 7000, decode: bool = False) -> Model:
    """YOLO11n at an input of size x size (a multiple of 32).  With decode,
    each head output also goes through the Detect head's DFL (box channels)
    and class Sigmoid into a [4 + 80, H, W] tensor per scale, which become the
    outputs (the anchor/stride box arithmetic and NMS stay with the caller)."""
    if size % 32:
        raise ValueError("YOLO11n input size must be a multiple of 32")
    bd = _Builder(size, seed)
    m = bd.m
    m.input = bd.buf("images", 3, size, size)
    s8, s16, s32 = size // 8, size // 16, size // 32
    # concat buffers of the neck, so that producers write straight into them
    cat12 = bd.buf("/model.12/Concat", 256 + 128, s16, s16)
    cat15 = bd.buf("/model.15/Concat", 128 + 128, s8, s8)
    cat18 = bd.buf("/model.18/Concat", 64 + 128, s16, s16)
    cat21 = bd.buf("/model.21/Concat", 128 + 256, s32, s32)

    x = bd.conv("/model.0/conv/Conv", whole(m.input), 16, 3, 2)
    x = bd.conv("/model.1/conv/Conv", x, 32, 3, 2)
    x = bd.c3k2("/model.2", x, 64, False, 0.25)
    x = bd.conv("/model.3/conv/Conv", x, 64, 3, 2)
    p3 = bd.c3k2("/model.4", x, 128, False, 0.25, y=Slice(cat15, 128, 128))
    x = bd.conv("/model.5/conv/Conv", p3, 128, 3, 2)
    p4 = bd.c3k2("/model.6", x, 128, True, 0.5, y=Slice(cat12, 256, 128))
    x = bd.conv("/model.7/conv/Conv", p4, 256, 3, 2)
    x = bd.c3k2("/model.8", x, 256, True, 0.5)
    x = bd.sppf("/model.9", x, 256)
    p5 = bd.c2psa("/model.10", x, 256, y=Slice(cat21, 128, 256))
    m.ops.append(UpsampleOp("/model.11/Resize", p5, Slice(cat12, 0, 256)))
    h13 = bd.c3k2("/model.13", whole(cat12), 128, False, 0.5, y=Slice(cat18, 64, 128))
    m.ops.append(UpsampleOp("/model.14/Resize", h13, Slice(cat15, 0, 128)))
    o16 = bd.c3k2("/model.16", whole(cat15), 64, False, 0.5)
    bd.conv("/model.17/conv/Conv", o16, 64, 3, 2, y=Slice(cat18, 0, 64))
    o19 = bd.c3k2("/model.19", whole(cat18), 128, False, 0.5)
    bd.conv("/model.20/conv/Conv", o19, 128, 3, 2, y=Slice(cat21, 0, 128))
    o22 = bd.c3k2("/model.22", whole(cat21), 256, True, 0.5)
    m.outputs = bd.detect("/model.23", [o16, o19, o22])
    if decode:
        decoded = []
        for i, out in enumerate(m.outputs):
            dec = bd.buf(f"/model.23/decode{i}", 4 + 80, out.h, out.w)
            m.ops.append(DflOp(f"/model.23/dfl#{i}", Slice(out, 0, 64), Slice(dec, 0, 4)))
            m.ops.append(SigmoidOp(f"/model.23/Sigmoid#{i}", Slice(out, 64, 80), Slice(dec, 4, 80)))
            decoded.append(dec)
        m.outputs = decoded
    return m


def build_c2f(size: int = 80, c_in: int = 128, c_out: int = 128, n: int = 1, shortcut: bool = True,
              seed: int = 9000) -> Model:
    """One depthwise-free C2f block (batch 1, c_in x size x size in, c_out
    out): cv1 1x1 c_in -> c_out, split in halves, n bottlenecks 3x3 -> 3x3 on
    the second half with the shortcut Add, concat of (2 + n) halves, cv2 1x1.
    Weights N(0, 0.05), biases N(0, 0.01) from `seed`."""
    bd = _Builder(size, seed)
    m = bd.m
    m.input = bd.buf("x", c_in, size, size)
    out = bd.c2f("/c2f", whole(m.input), c_out, n, shortcut)
    m.outputs = [out.buf]
    return m


# ------------------------------------------------------------ stream planning

def fuse_residual_adds(model: Model) -> Model:
    """The model with every Add whose operand is a conv output read by nothing
    else folded into that conv as a residual input (ConvOp.res), so that
    conv + Add run as one launch (osh_conv2d_add_f32).  The operand may also be
    tiled by several convs (the per-head parts of one depthwise conv): each
    part then takes the matching channels of the other operand and of the
    Add's output.  Results are unchanged: the conv's output is rounded as
    before and the sum is the same single addition."""
    ops = list(model.ops)
    readers = {}
    for i, op in enumerate(ops):
        for r in op_access(op)[0]:
            readers.setdefault(id(r.buf), set()).add(i)
    out_bufs = {id(b) for b in model.outputs}
    fused, drop = {}, set()
    for i, op in enumerate(ops):
        if not isinstance(op, AddOp):
            continue
        for opnd, other in ((op.b, op.a), (op.a, op.b)):
            buf = opnd.buf
            if opnd.c0 != 0 or opnd.c != buf.c or id(buf) in out_bufs or readers.get(id(buf)) != {i}:
                continue
            prod = [j for j in range(i) if any(w.buf is buf for w in op_access(ops[j])[1])]
            if not prod or any(not isinstance(ops[j], ConvOp) or ops[j].res is not None or j in fused
                               for j in prod):
                continue
            if sorted((ops[j].y.c0, ops[j].y.c) for j in prod) != _tiling(buf.c, [ops[j].y for j in prod]):
                continue
            # the convs move their write of the Add's output back to their own
            # position: nothing in between may touch it or rewrite the other operand
            first = min(prod)
            between = [k for k in range(first + 1, i) if k not in prod]
            if any(_overlap(a, op.y) for k in between for a in op_access(ops[k])[0] + op_access(ops[k])[1]):
                continue
            if any(_overlap(w, other) for k in between for w in op_access(ops[k])[1]):
                continue
            if _overlap(other, op.y) or any(_overlap(ops[j].x, op.y) for j in prod):
                continue
            for j in prod:
                cv = ops[j]
                fused[j] = ConvOp(cv.name + "+" + op.name, cv.x, op.y.sub(cv.y.c0, cv.y.c), cv.k, cv.s, cv.group,
                                  cv.act, cv.w, cv.b, res=other.sub(cv.y.c0, cv.y.c))
            drop.add(i)
            break
    new_ops = [fused.get(j, o) for j, o in enumerate(ops) if j not in drop]
    used = {id(model.input)} | out_bufs
    for o in new_ops:
        r, w = op_access(o)
        used.update(id(t.buf) for t in r + w)
    m = Model(model.size, [b for b in model.bufs if id(b) in used], new_ops, model.input, list(model.outputs))
    return m


def fuse_pool_chains(model: Model) -> Model:
    """Every run of three MaxPools (k x k, stride 1, pad k/2) that pool each
    other's output into three adjacent slices of one buffer becomes one
    PoolChainOp (osh_maxpool_chain3_f32: one launch, same results)."""
    ops = list(model.ops)
    out, i = [], 0
    while i < len(ops):
        t = ops[i:i + 3]
        if (len(t) == 3 and all(isinstance(o, MaxPoolOp) for o in t)
                and all(o.k == t[0].k and o.s == 1 and o.p == o.k // 2 for o in t)
                and t[1].x == t[0].y and t[2].x == t[1].y
                and t[0].y.buf is t[1].y.buf is t[2].y.buf
                and t[1].y.c0 == t[0].y.c0 + t[0].y.c and t[2].y.c0 == t[1].y.c0 + t[1].y.c
                and t[0].y.c == t[0].x.c == t[1].y.c == t[2].y.c
                and not _overlap(t[0].x, Slice(t[0].y.buf, t[0].y.c0, 3 * t[0].y.c))):
            out.append(PoolChainOp(t[0].name.rsplit("/", 2)[0] + "/MaxPool#chain3", t[0].x,
                                   Slice(t[0].y.buf, t[0].y.c0, 3 * t[0].y.c), t[0].k))
            i += 3
        else:
            out.append(ops[i])
            i += 1
    return Model(model.size, list(model.bufs), out, model.input, list(model.outputs))


def group_head_convs(model: Model) -> Model:
    """The Detect head runs two conv chains per scale (box: cv2.i.*, class:
    cv3.i.*), and the three scales' chains are independent of each other.  The
    same layer of the three scales becomes one GroupConvOp, the groups in
    layer order where the head's ops were (24 launches -> 8).  Results are
    unchanged: each conv keeps its own chain."""
    ops = list(model.ops)
    idx = [i for i, o in enumerate(ops) if isinstance(o, ConvOp) and o.name.startswith("/model.23/cv")]
    if not idx or idx != list(range(idx[0], idx[0] + len(idx))):
        return model
    layers = {}
    for i in idx:
        key = re.sub(r"cv([23])\.(\d)", r"cv\1.#", ops[i].name)
        layers.setdefault(key, []).append(ops[i])
    if any(len(v) != 3 or len({o.res is None for o in v}) != 1 or len({o.act for o in v}) != 1
           for v in layers.values()):
        return model
    groups = [GroupConvOp(k, v) for k, v in layers.items()]
    out = ops[:idx[0]] + groups + ops[idx[-1] + 1:]
    return Model(model.size, list(model.bufs), out, model.input, list(model.outputs))


def _conv_kind(op):
    dw = op.group > 1 and op.group == op.x.c == op.y.c
    return (op.k, op.s, dw, op.group if not dw else 0, op.act, op.res is None)


def _independent(a, b) -> bool:
    """Whether op b neither reads what a writes nor writes what a reads or writes."""
    ra, wa = op_access(a)
    rb, wb = op_access(b)
    return not any(_overlap(x, y) for x in rb for y in wa) and not any(
        _overlap(x, y) for x in wb for y in ra + wa)


def group_independent_convs(model: Model, window: int = 12) -> Model:
    """A conv and up to three later convs of the same kind (kernel, stride,
    depthwise or not, activation, residual or not) that depend on nothing
    between them, and nothing between them on them, run as one GroupConvOp at
    the first one's place -- e.g. a C3k block's two 1x1 convs of the same
    input, or the C2PSA positional conv's two heads.  Results are unchanged."""
    ops = list(model.ops)
    out, taken = [], set()
    for i, a in enumerate(ops):
        if i in taken:
            continue
        if not isinstance(a, ConvOp):
            out.append(a)
            continue
        members, between = [a], []
        for j in range(i + 1, min(len(ops), i + 1 + window)):
            if len(members) == 4:
                break
            b = ops[j]
            if j in taken:
                continue
            if (isinstance(b, ConvOp) and _conv_kind(b) == _conv_kind(a)
                    and all(_independent(m, b) and _independent(b, m) for m in members + between)):
                members.append(b)
                taken.add(j)
            else:
                between.append(b)
        out.append(a if len(members) == 1 else GroupConvOp("&".join(m.name for m in members), members))
    return Model(model.size, list(model.bufs), out, model.input, list(model.outputs))


def merge_independent_groups(model: Model, window: int = 8, max_members: int = 6) -> Model:
    """A GroupConvOp and a later one of the same kind that it can move down
    to -- nothing between them, nor the later group, reads what it writes or
    writes what it reads or writes, and it reads nothing they write -- run as
    one group at the later one's place (up to six convs): e.g. the detection
    head's final box and class 1x1 layers, which end independent branches.
    Results are unchanged."""
    ops = list(model.ops)
    kind = lambda g: {_conv_kind(o) for o in g.ops}
    i = 0
    while i < len(ops):
        a = ops[i]
        if isinstance(a, GroupConvOp) and len(kind(a)) == 1:
            for j in range(i + 1, min(len(ops), i + 1 + window)):
                b = ops[j]
                if not (_independent(a, b) and _independent(b, a)):
                    break
                if (isinstance(b, GroupConvOp) and kind(b) == kind(a) and
                        len(a.ops) + len(b.ops) <= max_members):
                    ops[j] = GroupConvOp(a.name + "&" + b.name, a.ops + b.ops)
                    del ops[i]
                    i -= 1
                    break
        i += 1
    return Model(model.size, list(model.bufs), ops, model.input, list(model.outputs))


def _is_depthwise3x3(op) -> bool:
    return op.k == 3 and op.s == 1 and op.group > 1 and op.group == op.x.c == op.y.c


def chain_parts(x: Slice, stages) -> list:
    """The channels of x as the concat parts of a chain stage: (k, slice) where
    earlier stage k wrote them, (-1, slice) where they come from memory."""
    parts, c, end = [], x.c0, x.c0 + x.c
    while c < end:
        hit = [k for k, s in enumerate(stages) if s.y.buf is x.buf and s.y.c0 <= c < s.y.c0 + s.y.c]
        if hit:
            k = hit[-1]
            n = min(end, stages[k].y.c0 + stages[k].y.c) - c
        else:
            k = -1
            n = min([s.y.c0 for s in stages if s.y.buf is x.buf and c < s.y.c0 < end] + [end]) - c
        parts.append((k, Slice(x.buf, c, n)))
        c += n
    return parts


def chain_res_stage(op, stages) -> int:
    """The earlier stage whose output is exactly op's residual, -1 if the
    residual (or its absence) is in memory, -2 if it overlaps a stage's output
    only in part."""
    if op.res is None:
        return -1
    for k, s in enumerate(stages):
        if _overlap(op.res, s.y):
            return k if (op.res.buf, op.res.c0, op.res.c) == (s.y.buf, s.y.c0, s.y.c) else -2
    return -1


def _chain_launch(convs):
    """The chains one osh_pw_chain_f32 launch runs for `convs` (the convs of
    consecutive ops, in program order), or None if the launch cannot take
    them: a conv joins the chain whose outputs it reads (it may read only
    one chain's), otherwise it starts a chain.  The checks are the launch's
    own (include/osh_hip.h): 1x1 convs over multiples of 16 channels, a 3x3
    depthwise only as stage 0, parts and residuals the stages can take, no
    output over another or over a depthwise stage's input, independent
    chains, and the LDS the launch needs."""
    chains = []
    for op in convs:
        reads = [op.x] + ([op.res] if op.res is not None else [])
        owners = {ci for ci, ch in enumerate(chains) for s in ch if any(_overlap(r, s.y) for r in reads)}
        if len(owners) > 1 or op.act not in N.ACTIVATIONS:
            return None
        ci = owners.pop() if owners else len(chains)
        if ci == len(chains):
            chains.append([])
        ch = chains[ci]
        if _is_depthwise3x3(op):
            if ch or op.y.c > 256:
                return None
        elif not (op.k == 1 and op.s == 1 and op.group == 1 and op.x.c % 16 == 0 and op.y.c % 16 == 0):
            return None
        if ch and (op.y.h, op.y.w) != (ch[0].y.h, ch[0].y.w):
            return None
        ch.append(op)
    if len(chains) > N.PW_MAX_CHAINS or any(len(ch) > N.PW_MAX_STAGES for ch in chains):
        return None
    outs = [o.y for o in convs]
    if any(_overlap(a, b) for i, a in enumerate(outs) for b in outs[:i]):
        return None
    for a, ca in enumerate(chains):
        for cb in chains[a + 1:]:
            if not all(_independent(x, y) and _independent(y, x) for x in ca for y in cb):
                return None
    for ch in chains:
        if (ch[0].y.h * ch[0].y.w) % 4:
            return None
        if _is_depthwise3x3(ch[0]) and any(_overlap(ch[0].x, y) for y in outs):
            return None
        floats, kept, segs = 0, set(), 0
        for k, op in enumerate(ch):
            parts = chain_parts(op.x, ch[:k])
            rs = chain_res_stage(op, ch[:k])
            if rs == -2 or (rs >= 0 and ch[rs].y.c != op.y.c):
                return None
            if rs >= 0:
                kept.add(rs)
            kept.update(s for s, _ in parts if s >= 0)
            if k == 0 and _is_depthwise3x3(op):
                continue
            if len(parts) > N.PW_MAX_SRC or any(p.c % 16 for _, p in parts) or op.y.c > 512:
                return None
            if any(p.c > 512 for s, p in parts if s < 0):
                return None
            # LDS: the packed weights, the bias, the parts and residual in memory
            mem = [p.c for s, p in parts if s < 0] + ([op.y.c] if op.res is not None and rs < 0 else [])
            segs += len(mem)
            floats += op.y.c * op.x.c + (op.y.c + 3) // 4 * 4 + 16 * sum(mem)
        floats += 16 * sum(ch[k].y.c for k in kept)
        if segs > 8 or 4 * floats > 160 * 1024:
            return None
    return chains


# Launch floor of one kernel in a serial graph on one MI355X (dispatch, cold
# first loads), and the issue interval of a dependent 16x16x4 FP32 MFMA chain
# (13.7 ns: 32.8 cycles at the ~2.4 GHz clock).
_LAUNCH_US = 3.5
_MFMA_STEP_US = 0.0137


def _chain_gain_us(chains, nops) -> float:
    """Modelled time a chain launch saves over its `nops` launches: the launch
    floors it drops, less the serialisation it adds -- a chain workgroup runs
    all M/16 output blocks of a stage on its CU's four SIMDs, C/4 dependent
    MFMAs each, where the stage alone would spread them over the chip."""
    def extra(op):
        if op.k != 1:
            return 0.0
        return ((op.y.c // 16 + 3) // 4 - 1) * (op.x.c / 4) * _MFMA_STEP_US
    return _LAUNCH_US * (nops - 1) - max(sum(extra(o) for o in ch) for ch in chains)


def chain_pointwise_convs(model: Model, max_ops: int = 6, min_gain_us: float = 0.5) -> Model:
    """Runs of consecutive conv ops that one osh_pw_chain_f32 launch can take
    (see _chain_launch) become one ChainOp where the cost model says the
    launch pays: C3k2's cv1 with the paired 1x1 convs after it, C3k's cv3
    with the block's cv2, C2PSA's proj / ffn / cv2 tail, the class branch of
    the head (depthwise -> 1x1 [-> 1x1]) at its three scales.  Each start
    takes the window of highest modelled gain.  Results are unchanged."""
    ops = list(model.ops)
    out, i = [], 0
    while i < len(ops):
        best, convs = None, []
        for j in range(i, min(len(ops), i + max_ops)):
            o = ops[j]
            if isinstance(o, ConvOp):
                convs.append(o)
            elif isinstance(o, GroupConvOp):
                convs.extend(o.ops)
            else:
                break
            if j == i:
                continue
            chains = _chain_launch(convs)
            if chains is None:
                continue
            gain = _chain_gain_us(chains, j - i + 1)
            if gain >= min_gain_us and (best is None or gain > best[0]):
                best = (gain, j, chains)
        if best is None:
            out.append(ops[i])
            i += 1
            continue
        _, j, chains = best
        name = " | ".join(" > ".join(o.name for o in ch) for ch in chains)
        out.append(ChainOp(name, chains))
        i = j + 1
    return Model(model.size, list(model.bufs), out, model.input, list(model.outputs))


def pair_bottleneck_convs(model: Model, takes=None, min_pixels: int = 0) -> Model:
    """Adjacent 3x3 SiLU convs where the second reads exactly the first's
    output and nothing else touches that buffer (a bottleneck's cv1 -> cv2;
    the first conv and the stride-2 conv after it) become one PairOp, on
    maps of at least `min_pixels`, where `takes(a, b)` (default: the
    library's osh_conv2d_pair_check on the resolved params) accepts them.

    A fused pair saves a launch and the intermediate's round trip, but each
    workgroup also computes the first conv over a one-pixel ring around its
    tile, on its own CU's four MFMA pipes: one 16x16x4 FP32 MFMA keeps a
    pipe busy for its full 32 cycles, so the ring's extra blocks cost time
    one for one.  On the 640 frame's 80x80 pairs (32 -> 16 -> 32) the fused
    kernel ran 7.2 us against 8.9 us as two launches; on the 40x40 and 20x20
    pairs 8.0-15.1 us against 8.1-10.6 us.  osh_conv2d_pair_f32 times both
    forms on first use and keeps the faster one."""
    takes = takes or pair_supported
    ops = list(model.ops)
    users = {}
    for o in ops:
        r, w = op_access(o)
        for sl in r + w:
            users.setdefault(id(sl.buf), set()).add(id(o))
    out, i = [], 0
    while i < len(ops):
        a = ops[i]
        b = ops[i + 1] if i + 1 < len(ops) else None
        if (isinstance(a, ConvOp) and isinstance(b, ConvOp) and a.res is None and
                all(c.k == 3 and c.group == 1 and c.act == "Silu" for c in (a, b)) and
                a.y.h * a.y.w >= min_pixels and
                b.x.buf is a.y.buf and b.x.c0 == a.y.c0 and b.x.c == a.y.c == a.y.buf.c and
                users.get(id(a.y.buf)) == {id(a), id(b)} and takes(a, b)):
            # a first-layer pair leaves its 16-channel map unstored (the
            # fused kernel beats two launches there by far), unless the map is
            # also a model output
            is_output = any(a.y.buf is o for o in model.outputs)
            out.append(PairOp(a.name.rsplit("/", 3)[0] + "#pair", a, b, store_mid=a.x.c > 4 or is_output))
            i += 2
            continue
        out.append(a)
        i += 1
    m = Model(model.size, model.bufs, out, model.input, model.outputs)
    return m


def _conv_params(op: ConvOp) -> N.ConvParams:
    attrs = N.ConvAttrs()
    attrs.group = op.group
    attrs.n_kernel_shape, attrs.kernel_shape[0], attrs.kernel_shape[1] = 2, op.k, op.k
    attrs.n_strides, attrs.strides[0], attrs.strides[1] = 2, op.s, op.s
    attrs.n_pads = 4
    for i in range(4):
        attrs.pads[i] = op.k // 2
    p = N.ConvParams()
    N.call("osh_conv_resolve", C.byref(attrs), N.dims64(op.x.shape), N.dims64(op.w.shape), C.byref(p))
    return p


def pair_supported(a: ConvOp, b: ConvOp) -> bool:
    """Whether osh_conv2d_pair_f32 takes conv a followed by conv b (a host-side check)."""
    pa, pb = _conv_params(a), _conv_params(b)
    return N.lib().osh_conv2d_pair_check(C.byref(pa), C.byref(pb), N.ACTIVATIONS[a.act]) == 0


def fuse_launches(model: Model, chains: bool = False, pairs: bool = True, merge: bool = True) -> Model:
    """The launch-saving rewrites of the op list (residual Adds into their
    convs, SPPF's pool chain into one op, the head's three scales per layer
    into one op, other independent convs of one kind into one op, and with
    chains=True runs of pointwise convs into chain launches); results are
    unchanged.  Chains are off by default: on one MI355X every chain the
    pass picks in the 640 frame ran slower than its separate launches (a
    chain workgroup runs its stages one after another with one dependent
    MFMA accumulator per wave, while separate launches spread each stage over
    the chip), 0.493 against 0.465 ms per frame."""
    m = group_independent_convs(group_head_convs(fuse_pool_chains(fuse_residual_adds(model))))
    if merge:
        m = merge_independent_groups(m)
    if pairs:
        m = pair_bottleneck_convs(m)
    return chain_pointwise_convs(m) if chains else m


def _tiling(c, slices):
    """[(c0, c)] of slices that tile channels [0, c) exactly, in order, else None."""
    parts = sorted((s.c0, s.c) for s in slices)
    at = 0
    for c0, n in parts:
        if c0 != at:
            return None
        at += n
    return parts if at == c else None


def op_access(op):
    """(reads, writes) of an op as lists of channel slices."""
    if isinstance(op, (GroupConvOp, ChainOp, PairOp)):
        acc = [op_access(o) for o in op.ops]
        return [r for a in acc for r in a[0]], [w for a in acc for w in a[1]]
    if isinstance(op, AddOp):
        return [op.a, op.b], [op.y]
    if isinstance(op, ConvOp) and op.res is not None:
        return [op.x, op.res], [op.y]
    if isinstance(op, AttentionOp):
        return [op.qkv], [op.y, whole(op.qt), whole(op.attn), whole(op.attn_t)]
    return [op.x], [op.y]


def _overlap(a: Slice, b: Slice) -> bool:
    return a.buf is b.buf and a.c0 < b.c0 + b.c and b.c0 < a.c0 + a.c


def plan_streams(ops, nstreams=4):
    """Spread the op list over `nstreams` streams along its data dependencies.

    An op depends on every earlier op it reads after (RAW), writes after (WAW)
    or overwrites the input of (WAR).  It continues the stream whose last op
    is its latest dependency; an op that starts a new branch takes the least
    recently used stream.  Returns (stream per op, waits per op: indices of
    earlier ops on other streams to wait for, ops whose completion some other
    stream waits for)."""
    acc = [op_access(o) for o in ops]
    deps = []
    for i, (ri, wi) in enumerate(acc):
        d = []
        for j in range(i):
            rj, wj = acc[j]
            if (any(_overlap(a, b) for a in wj for b in ri + wi) or any(_overlap(a, b) for a in rj for b in wi)):
                d.append(j)
        deps.append(d)
    stream_of, waits = [], []
    last = [-1] * nstreams
    seen = [[-1] * nstreams for _ in range(nstreams)]  # seen[s][t]: latest op of t that s has waited for
    recorded = set()
    for i, d in enumerate(deps):
        d = list(d)
        cands = [stream_of[j] for j in d if last[stream_of[j]] == j]
        if cands:
            s = max(cands, key=lambda t: last[t])
        else:
            s = min(range(nstreams), key=lambda t: last[t])
        w = []
        for j in sorted(d, reverse=True):
            t = stream_of[j]
            if t != s and seen[s][t] < j:
                w.append(j)
                seen[s][t] = j
                recorded.add(j)
        stream_of.append(s)
        waits.append(sorted(w))
        last[s] = i
    return stream_of, waits, recorded


def op_dependencies(ops):
    """For each op, the earlier ops it must follow (RAW, WAW and WAR on channel slices)."""
    acc = [op_access(o) for o in ops]
    out = []
    for i, (ri, wi) in enumerate(acc):
        d = []
        for j in range(i):
            rj, wj = acc[j]
            if (any(_overlap(a, b) for a in wj for b in ri + wi) or any(_overlap(a, b) for a in rj for b in wi)):
                d.append(j)
        out.append(d)
    return out


# --------------------------------------------------------------- device side

def attention_fits(key_dim: int, head_dim: int, n: int) -> bool:
    """The shapes osh_attention_f32 takes: 16-row query tiles, key_dim / 4 <= 16
    k-steps in registers, 16-channel output blocks, and 16 score rows of n <= 480
    beside the staged v chunks in 64 KiB of LDS."""
    return key_dim % 4 == 0 and key_dim <= 64 and head_dim % 16 == 0 and n % 16 == 0 and n <= 480


class Frame:
    """Device buffers, packed weights and the launch list of one model, spread
    over `nstreams` streams (fork/join through events) so that independent
    branches -- the detection head's six chains, the P3 head beside the rest
    of the neck -- run side by side."""

    def __init__(self, model: Model, device, nstreams: int = 4, fuse: bool = True, fused_attention: bool = True,
                 chains: bool = False, pairs: bool = True):
        import torch
        self.fused_attention = fused_attention
        if fuse:  # conv -> residual Add pairs, SPPF's pools, grouped, paired and chained convs as single launches
            model = fuse_launches(model, chains=chains, pairs=pairs)
        self.model = model
        self.device = device
        for b in model.bufs:
            b.tensor = torch.empty((1, b.c, b.h, b.w), dtype=torch.float32, device=device)
        self.streams = []
        for _ in range(max(1, nstreams)):
            st = C.c_void_p()
            N.call("osh_stream_create", C.byref(st))
            self.streams.append(st)
        self.stream = self.streams[0]  # the frame's stream: joins every branch
        self.plan, self.waits, rec = plan_streams(model.ops, len(self.streams))
        self.events = {}
        for i in sorted(rec) + ["fork"] + ["join%d" % k for k in range(1, len(self.streams))]:
            ev = C.c_void_p()
            N.call("osh_event_create", C.byref(ev))
            self.events[i] = ev
        self.graph = None
        self._calls = []
        self._keep = []
        self._packs = []  # packed conv weights: their records are dropped in close()
        for op in model.ops:
            self._calls.append(self._prepare(op))
        torch.cuda.synchronize()

    def _prepare(self, op):
        import torch
        lib = N.lib()
        if isinstance(op, GroupConvOp):
            parts = [self._prepare_conv(o) for o in op.ops]
            n = len(parts)
            ps = (N.ConvParams * n)(*[pp for pp, _, _ in parts])
            arr = lambda vals: (C.c_void_p * n)(*vals)
            xs, ws = arr([o.x.ptr() for o in op.ops]), arr([pk.data_ptr() for _, pk, _ in parts])
            bs, ys = arr([b.data_ptr() for _, _, b in parts]), arr([o.y.ptr() for o in op.ops])
            rs = arr([o.res.ptr() if o.res is not None else None for o in op.ops])
            self._keep += [ps, xs, ws, bs, ys, rs]
            act = N.ACTIVATIONS[op.ops[0].act]
            return lambda st: N.check(lib.osh_conv2d_group_f32(n, ps, xs, ws, bs, act, rs, ys, st))
        if isinstance(op, ChainOp):
            return self._prepare_chain(op)
        if isinstance(op, PairOp):
            pa, wa, ba = self._prepare_conv(op.a)
            pb, wb, bb = self._prepare_conv(op.b)
            act = N.ACTIVATIONS[op.a.act]
            res = op.b.res.ptr() if op.b.res is not None else None
            return lambda st: N.check(lib.osh_conv2d_pair_f32(
                C.byref(pa), C.byref(pb), op.a.x.ptr(), C.c_void_p(wa.data_ptr()), C.c_void_p(ba.data_ptr()),
                C.c_void_p(wb.data_ptr()), C.c_void_p(bb.data_ptr()), act, res,
                op.a.y.ptr() if op.store_mid else None, op.b.y.ptr(), st))
        if isinstance(op, ConvOp):
            p, packed, b = self._prepare_conv(op)
            act = N.ACTIVATIONS[op.act]
            if op.res is not None:
                return lambda st: N.check(lib.osh_conv2d_add_f32(C.byref(p), op.x.ptr(), C.c_void_p(packed.data_ptr()),
                                                                 C.c_void_p(b.data_ptr()), act, op.res.ptr(),
                                                                 op.y.ptr(), st))
            return lambda st: N.check(lib.osh_conv2d_f32(C.byref(p), op.x.ptr(), C.c_void_p(packed.data_ptr()),
                                                         C.c_void_p(b.data_ptr()), act, op.y.ptr(), st))
        return self._prepare_other(op)

    def _prepare_conv(self, op):
        """Resolved params, packed weights and bias of a conv (packed once)."""
        import torch
        p = _conv_params(op)
        assert (p.m, p.oh, p.ow) == (op.y.c, op.y.h, op.y.w), op.name
        nbytes = C.c_size_t()
        N.call("osh_conv_packed_weight_bytes", C.byref(p), C.byref(nbytes))
        w = torch.from_numpy(np.ascontiguousarray(op.w)).to(self.device)
        b = torch.from_numpy(np.ascontiguousarray(op.b)).to(self.device)
        packed = torch.empty(max(1, nbytes.value // 4), dtype=torch.float32, device=self.device)
        torch.cuda.synchronize()  # the uploads ran on torch's stream; packing runs on the frame's
        N.call("osh_conv_pack_weights", C.byref(p), C.c_void_p(w.data_ptr()), C.c_void_p(packed.data_ptr()),
               self.stream)
        self._keep += [p, w, b, packed]
        self._packs.append(packed)
        return p, packed, b

    def _prepare_chain(self, op: ChainOp):
        """osh_pw_chain_f32 descriptors of a ChainOp: stage parts that an
        earlier stage wrote point into that stage's output, the rest into
        memory; a residual that is an earlier stage's output comes from chip."""
        lib = N.lib()
        arr = (N.PwChain * len(op.chains))()
        for ci, ch in enumerate(op.chains):
            d = arr[ci]
            d.h, d.w, d.nstages = ch[0].y.h, ch[0].y.w, len(ch)
            for k, cv in enumerate(ch):
                _, packed, b = self._prepare_conv(cv)
                st = d.stage[k]
                st.kind = N.PW_DW3X3 if _is_depthwise3x3(cv) else N.PW_1X1
                st.m, st.act = cv.y.c, N.ACTIVATIONS[cv.act]
                parts = chain_parts(cv.x, ch[:k])
                st.nsrc = len(parts)
                for i, (s, sl) in enumerate(parts):
                    st.src_stage[i], st.src[i], st.src_c[i] = s, sl.ptr().value, sl.c
                st.w, st.bias = packed.data_ptr(), b.data_ptr()
                rs = chain_res_stage(cv, ch[:k])
                assert rs >= -1, cv.name
                st.res_stage = rs
                st.res = cv.res.ptr().value if cv.res is not None and rs < 0 else None
                st.y = cv.y.ptr().value
        self._keep.append(arr)
        n = len(op.chains)
        return lambda s: N.check(lib.osh_pw_chain_f32(n, arr, s))

    def _prepare_other(self, op):
        lib = N.lib()
        if isinstance(op, AddOp):
            n = op.y.c * op.y.h * op.y.w
            return lambda st: N.check(lib.osh_add_f32(n, op.a.ptr(), op.b.ptr(), op.y.ptr(), st))
        if isinstance(op, CopyOp):
            nb = 4 * op.y.c * op.y.h * op.y.w
            return lambda st: N.check(lib.osh_memcpy_d2d(op.y.ptr(), op.x.ptr(), nb, st))
        if isinstance(op, MaxPoolOp):
            pp = N.PoolParams(1, op.x.c, op.x.h, op.x.w, op.k, op.k, op.s, op.s, op.p, op.p, op.y.h, op.y.w)
            self._keep.append(pp)
            return lambda st: N.check(lib.osh_maxpool2d_f32(C.byref(pp), op.x.ptr(), op.y.ptr(), st))
        if isinstance(op, PoolChainOp):
            c, hw = op.x.c, op.x.h * op.x.w
            y1 = op.y.sub(0, c)
            y2, y3 = op.y.sub(c, c), op.y.sub(2 * c, c)
            xs, ys = op.x.buf.c * hw, op.y.buf.c * hw
            return lambda st: N.check(lib.osh_maxpool_chain3_f32(1, c, op.x.h, op.x.w, op.k, op.x.ptr(), xs, y1.ptr(),
                                                                 y2.ptr(), y3.ptr(), ys, st))
        if isinstance(op, DflOp):
            hw = op.x.h * op.x.w
            sides = op.x.c // op.bins
            return lambda st: N.check(lib.osh_dfl_f32(1, sides, op.bins, hw, op.x.ptr(), op.x.buf.c * hw, op.y.ptr(),
                                                      op.y.buf.c * hw, st))
        if isinstance(op, SigmoidOp):
            n = op.x.c * op.x.h * op.x.w
            return lambda st: N.check(lib.osh_activation_f32(n, op.x.ptr(), N.ACT_SIGMOID, op.y.ptr(), st))
        if isinstance(op, UpsampleOp):
            return lambda st: N.check(lib.osh_resize_nearest_f32(1, op.x.c, op.x.h, op.x.w, op.f, op.f, op.x.ptr(),
                                                                 op.y.ptr(), op.y.c * op.y.h * op.y.w, st))
        if isinstance(op, AttentionOp):
            return self._prepare_attention(op)
        raise TypeError(op)

    def _prepare_attention(self, op: AttentionOp):
        lib = N.lib()
        n = op.qkv.h * op.qkv.w
        rows = 2 * op.key_dim + op.head_dim
        hs = rows * n  # head stride inside qkv
        base = op.qkv.ptr().value
        q = C.c_void_p(base)
        k = C.c_void_p(base + 4 * op.key_dim * n)
        v = C.c_void_p(base + 4 * 2 * op.key_dim * n)
        qt, sc, st = (C.c_void_p(b.tensor.data_ptr()) for b in (op.qt, op.attn, op.attn_t))
        y = op.y.ptr()

        if self.fused_attention and attention_fits(op.key_dim, op.head_dim, n):
            def run_fused(stream):
                N.check(lib.osh_attention_f32(op.heads, op.key_dim, op.head_dim, n, C.c_float(op.scale), q, hs, y,
                                              stream))
            return run_fused

        def run(stream):
            # q^T per head: [kd, N] -> [N, kd]
            N.check(lib.osh_transpose_f32(op.heads, op.key_dim, n, q, hs, qt, n * op.key_dim, stream))
            # scores[h] = q^T k: [N, kd] x [kd, N]
            N.check(lib.osh_gemm_f32_batched(op.heads, n, n, op.key_dim, qt, op.key_dim, n * op.key_dim, k, n, hs,
                                             None, N.ACT_NONE, sc, n, n * n, stream))
            N.check(lib.osh_softmax_f32(op.heads * n, n, C.c_float(op.scale), sc, st, stream))
            # probabilities transposed back into the scores buffer
            N.check(lib.osh_transpose_f32(op.heads, n, n, st, n * n, sc, n * n, stream))
            # y[h] = v attn^T: [hd, N] x [N, N]
            N.check(lib.osh_gemm_f32_batched(op.heads, op.head_dim, n, n, v, n, hs, sc, n, n * n, None, N.ACT_NONE,
                                             y, n, op.head_dim * n, stream))
        return run

    def run_op(self, i):
        """Issue op i on its planned stream, after the events it waits for."""
        st = self.streams[self.plan[i]]
        for j in self.waits[i]:
            N.call("osh_stream_wait_event", st, self.events[j])
        self._calls[i](st)
        if i in self.events:
            N.call("osh_event_record", self.events[i], st)

    def run(self):
        """Issue every op of one frame (no sync); every branch joins the
        frame's stream at the end."""
        # the side streams start after the frame stream's earlier work (the input)
        start = self.events["fork"] if len(self.streams) > 1 else None
        if start is not None:
            N.call("osh_event_record", start, self.stream)
            for st in self.streams[1:]:
                N.call("osh_stream_wait_event", st, start)
        for i in range(len(self._calls)):
            self.run_op(i)
        for k, st in enumerate(self.streams[1:], start=1):
            ev = self.events["join%d" % k]
            N.call("osh_event_record", ev, st)
            N.call("osh_stream_wait_event", self.stream, ev)

    def segments(self):
        """Runs of ops of one planned stream between cross-stream waits:
        [(first op index, op indices, dependency segment indices)]."""
        segs, open_seg, seg_of = [], {}, {}
        for i, st in enumerate(self.plan):
            k = open_seg.get(st)
            if k is None or self.waits[i]:
                deps = set()
                if k is not None:
                    deps.add(k)
                deps.update(seg_of[j] for j in self.waits[i])
                k = len(segs)
                segs.append((i, [], sorted(deps)))
                open_seg[st] = k
            segs[k][1].append(i)
            seg_of[i] = k
        return segs

    def capture(self, parallel=False, flat=False):
        """Record one frame as a HIP graph (replayed by `launch`).

        parallel=False: the ops in program order on the frame's stream (one
        chain of kernels).  parallel=True: each stream segment of the plan is
        captured alone and becomes one child-graph node that depends on the
        segments it waits for, so independent branches may overlap at replay;
        with flat=True the segment's kernel launches become kernel nodes of
        one flat DAG instead (no child graphs).  On one MI355X the chain
        replays faster than the child-graph DAG (0.51 vs 0.72 ms per 640 x 640
        frame), so it is the default."""
        if self.graph is not None:
            return self.graph
        if parallel and flat:
            return self._capture_flat()
        if not parallel:
            g = C.c_void_p()
            N.call("osh_graph_begin", self.stream)
            try:
                for c in self._calls:
                    c(self.stream)
            finally:
                N.call("osh_graph_end", self.stream, C.byref(g))
            self.graph = g
            return g
        b = C.c_void_p()
        N.call("osh_graph_builder_create", C.byref(b))
        try:
            nodes = []
            for first, ops, deps in self.segments():
                arr = (C.c_void_p * max(1, len(deps)))(*[nodes[k] for k in deps])
                node = C.c_void_p()
                N.call("osh_graph_begin", self.stream)
                try:
                    for i in ops:
                        self._calls[i](self.stream)
                finally:
                    N.call("osh_graph_add_captured", b, self.stream, arr, len(deps), C.byref(node))
                nodes.append(node.value)
            g = C.c_void_p()
            N.call("osh_graph_instantiate", b, C.byref(g))
            self.graph = g
        finally:
            N.call("osh_graph_builder_destroy", b)
        return self.graph

    def _capture_flat(self):
        b = C.c_void_p()
        N.call("osh_graph_builder_create", C.byref(b))
        try:
            exits = []  # per segment: the nodes a dependent segment waits for
            for first, ops, deps in self.segments():
                dep_nodes = list(dict.fromkeys(n for k in deps for n in exits[k]))
                arr = (C.c_void_p * max(1, len(dep_nodes)))(*dep_nodes)
                f, l = C.c_void_p(), C.c_void_p()
                N.call("osh_graph_begin", self.stream)
                try:
                    for i in ops:
                        self._calls[i](self.stream)
                finally:
                    N.call("osh_graph_add_captured_flat", b, self.stream, arr, len(dep_nodes), C.byref(f),
                           C.byref(l))
                exits.append([l.value] if l.value else dep_nodes)
            g = C.c_void_p()
            N.call("osh_graph_instantiate", b, C.byref(g))
            self.graph = g
        finally:
            N.call("osh_graph_builder_destroy", b)
        return self.graph

    def launch(self):
        if self.graph is not None:
            N.call("osh_graph_launch", self.graph, self.stream)
        else:
            self.run()

    def sync(self):
        N.call("osh_stream_sync", self.stream)

    def set_input(self, x):
        """Copy an input image into the frame (synchronous: the frame's stream
        does not order itself after torch's)."""
        import torch
        t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(x, np.float32))
        self.model.input.tensor.copy_(t.reshape(self.model.input.tensor.shape))
        torch.cuda.synchronize()

    def outputs(self):
        return [b.tensor for b in self.model.outputs]

    def close(self):
        if self.graph is not None:
            N.call("osh_graph_destroy", self.graph)
            self.graph = None
        for buf in self._packs:
            N.call("osh_conv_forget_pack", C.c_void_p(buf.data_ptr()), buf.numel() * buf.element_size())
        self._packs = []
        for ev in self.events.values():
            N.call("osh_event_destroy", ev)
        self.events = {}
        for st in self.streams:
            N.call("osh_stream_destroy", st)
        self.streams = []
        self.stream = C.c_void_p()
