"""YOLO11n forward pass restated on its own, for checking the device frame.

TEST INFRASTRUCTURE ONLY: used by tests/ as the checker of the device frame's
topology (which tensor feeds which layer, concat orders, residual sources).

The network is written here from the Ultralytics module definitions the
reference's model was exported from (yolo11.yaml at scale n: depth 0.50,
width 0.25; modules Conv, C3k2, C3k, Bottleneck, SPPF, C2PSA / PSABlock /
Attention, Detect), with the ONNX node names that the reference's fixture
tests/data/yolo11n.shapes.tsv lists, and without the device package's
network builder: a wiring mistake in either one shows as a difference
between the two.  Tensors are plain numpy arrays; concat and split are
np.concatenate and slicing.

Arithmetic is the oracle's restatement of the reference's CPU kernels
(oracle.conv_reference: the kernel ConvLayer.Forward picks per shape on the
host that `nchwc` describes, src/OnnxSharp/Ops/DnnOps.cs:437-482;
silu_ref: VectorMath.Silu; gemm_f32, softmax, maxpool2d, resize_nearest,
dfl, sigmoid_ref).  Weights come from
the seeded generator keyed by node name (synth.layer_seed), as the device
model's do: conv weights N(0, 0.05), biases N(0, 0.01).
"""
from __future__ import annotations

import numpy as np

from onnxsharp_amd import synth  # the seeded data generator (not the network builder)

NC = 80       # classes
REG_MAX = 16  # DFL bins


class Net:
    """One forward pass; `tensors` maps each node name to its output (a conv's
    output after its SiLU, an Add's sum, a Concat, a MaxPool), `convs` lists
    every conv as it ran (name, input shape, weight shape, stride, group,
    activation).  With dry=True no arithmetic runs: outputs are zeros of the
    right shapes (wiring and shape checks)."""

    def __init__(self, oracle, seed: int = 7000, winograd: int = 1, dry: bool = False, nchwc: int = 1):
        self.o = oracle
        self.seed = seed
        self.winograd = winograd
        self.nchwc = nchwc
        self.dry = dry
        self.tensors = {}
        self.convs = []

    # ------------------------------------------------------------ primitives
    def weights(self, name, shape):
        w = synth.normal(synth.layer_seed(self.seed, name, 0), shape, 0.0, 0.05)
        b = synth.normal(synth.layer_seed(self.seed, name, 1), (shape[0],), 0.0, 0.01)
        return w, b

    def conv(self, name, x, c2, k=1, s=1, g=1, act=True):
        """Conv2d(k, s, pad k // 2, groups g) with bias, then SiLU when act
        (ultralytics Conv with BatchNorm folded; act=False is a plain Conv2d
        or Conv(act=False))."""
        _, c1, h, w_ = x.shape
        w, b = self.weights(name, (c2, c1 // g, k, k))
        p = k // 2
        oh, ow = (h + 2 * p - k) // s + 1, (w_ + 2 * p - k) // s + 1
        self.convs.append({"name": name, "x": tuple(x.shape), "w": tuple(w.shape), "s": s, "g": g,
                           "act": "Silu" if act else None})
        if self.dry:
            y = np.zeros((1, c2, oh, ow), np.float32)
        else:
            y = self.o.conv_reference(np.ascontiguousarray(x), w, b, (s, s), (p, p), (1, 1), g, (oh, ow),
                                      winograd=self.winograd, nchwc=self.nchwc)
            if act:
                y = self.o.silu_ref(y)
        return self.keep(name, y)

    def keep(self, name, y):
        self.tensors[name] = y
        return y

    def add(self, name, a, b):
        return self.keep(name, (a + b).astype(np.float32))

    def cat(self, name, parts):
        return self.keep(name, np.concatenate(parts, axis=1))

    def maxpool(self, name, x, k=5):
        y = np.zeros_like(x) if self.dry else self.o.maxpool2d(np.ascontiguousarray(x), k, 1, k // 2)
        return self.keep(name, y)

    def upsample(self, name, x):
        if self.dry:
            return self.keep(name, np.zeros((1, x.shape[1], 2 * x.shape[2], 2 * x.shape[3]), np.float32))
        return self.keep(name, self.o.resize_nearest(np.ascontiguousarray(x), 2))

    # --------------------------------------------------------------- modules
    def bottleneck(self, p, x, c2, shortcut, e):
        """Bottleneck(c1, c2, shortcut, k=(3, 3), e): cv1 3x3 to int(c2*e),
        cv2 3x3 to c2, plus x when shortcut and c1 == c2."""
        t = self.conv(f"{p}/cv1/conv/Conv", x, int(c2 * e), 3)
        y = self.conv(f"{p}/cv2/conv/Conv", t, c2, 3)
        return self.add(f"{p}/Add", x, y) if shortcut and x.shape[1] == c2 else y

    def c3k(self, p, x, c2, n=2, shortcut=True):
        """C3k(c1, c2, n=2): cv3(cat(m(cv1(x)), cv2(x))), m = n bottlenecks with e = 1."""
        c_ = c2 // 2
        a = self.conv(f"{p}/cv1/conv/Conv", x, c_)
        for i in range(n):
            a = self.bottleneck(f"{p}/m/m.{i}", a, c_, shortcut, 1.0)
        b = self.conv(f"{p}/cv2/conv/Conv", x, c_)
        return self.conv(f"{p}/cv3/conv/Conv", self.cat(f"{p}/Concat", [a, b]), c2)

    def c3k2(self, p, x, c2, c3k, e=0.5, n=1, shortcut=True):
        """C3k2 (C2f with C3k or Bottleneck(e=0.5) blocks): cv1 1x1 to 2c,
        chunk into halves y0, y1, each block appended reading the last part,
        cv2 1x1 over cat(y0, y1, blocks...)."""
        c = int(c2 * e)
        y = self.conv(f"{p}/cv1/conv/Conv", x, 2 * c)
        parts = [y[:, :c], y[:, c:]]
        for i in range(n):
            if c3k:
                parts.append(self.c3k(f"{p}/m.{i}", parts[-1], c, 2, shortcut))
            else:
                parts.append(self.bottleneck(f"{p}/m.{i}", parts[-1], c, shortcut, 0.5))
        return self.conv(f"{p}/cv2/conv/Conv", self.cat(f"{p}/Concat", parts), c2)

    def sppf(self, p, x, c2, k=5):
        """SPPF: cv1 1x1 to c1/2, three chained k x k max pools, cv2 1x1 over
        cat(cv1, pool1, pool2, pool3)."""
        y = [self.conv(f"{p}/cv1/conv/Conv", x, x.shape[1] // 2)]
        for nm in ("m", "m_1", "m_2"):
            y.append(self.maxpool(f"{p}/{nm}/MaxPool", y[-1], k))
        return self.conv(f"{p}/cv2/conv/Conv", self.cat(f"{p}/Concat", y), c2)

    def attention(self, p, x, heads, attn_ratio=0.5):
        """Attention(dim, heads, attn_ratio): qkv 1x1 (no act) viewed as
        [heads, 2*key_dim + head_dim, N] rows (q, k, v); per head
        softmax(scale * q^T k) and v attn^T; plus pe (3x3 depthwise, no act)
        over v as [C, H, W]; then proj 1x1 (no act)."""
        _, c, h, w = x.shape
        n = h * w
        head_dim = c // heads
        key_dim = int(head_dim * attn_ratio)
        scale = float(key_dim) ** -0.5
        qkv = self.conv(f"{p}/qkv/conv/Conv", x, c + 2 * key_dim * heads, act=False)
        rows = qkv.reshape(heads, 2 * key_dim + head_dim, n)
        q, k, v = rows[:, :key_dim], rows[:, key_dim:2 * key_dim], rows[:, 2 * key_dim:]
        outs = []
        for hh in range(heads):
            if self.dry:
                outs.append(np.zeros((head_dim, n), np.float32))
                continue
            scores = self.o.gemm_f32(np.ascontiguousarray(q[hh].T), np.ascontiguousarray(k[hh]))
            probs = self.o.softmax(scores, scale)
            outs.append(self.o.gemm_f32(np.ascontiguousarray(v[hh]), np.ascontiguousarray(probs.T)))
        att = self.keep(f"{p}/Reshape_1", np.stack(outs).reshape(1, c, h, w))
        pe = self.conv(f"{p}/pe/conv/Conv", np.ascontiguousarray(v.reshape(1, c, h, w)), c, 3, g=c, act=False)
        return self.conv(f"{p}/proj/conv/Conv", self.add(f"{p}/Add", att, pe), c, act=False)

    def psa_block(self, p, x, heads):
        """PSABlock: x + attn(x), then that + ffn (1x1 to 2c SiLU, 1x1 back, no act)."""
        c = x.shape[1]
        x = self.add(f"{p}/Add", x, self.attention(f"{p}/attn", x, heads))
        f = self.conv(f"{p}/ffn/ffn.0/conv/Conv", x, 2 * c)
        f = self.conv(f"{p}/ffn/ffn.1/conv/Conv", f, c, act=False)
        return self.add(f"{p}/Add_1", x, f)

    def c2psa(self, p, x, c2, e=0.5):
        """C2PSA: cv1 1x1 to 2c split (a, b), b through one PSABlock
        (heads = c // 64), cv2 1x1 over cat(a, b)."""
        c = int(x.shape[1] * e)
        y = self.conv(f"{p}/cv1/conv/Conv", x, 2 * c)
        a, b = y[:, :c], y[:, c:]
        b = self.psa_block(f"{p}/m/m.0", b, c // 64)
        return self.conv(f"{p}/cv2/conv/Conv", self.cat(f"{p}/Concat", [a, b]), c2)

    def detect(self, p, xs):
        """Detect (non-legacy head): per scale i, box branch cv2.i = 3x3, 3x3,
        1x1 plain to 4*REG_MAX; class branch cv3.i = (DW 3x3, 1x1 to c3),
        (DW 3x3, 1x1), 1x1 plain to NC; output cat(box, class)."""
        c2 = max(16, xs[0].shape[1] // 4, REG_MAX * 4)
        c3 = max(xs[0].shape[1], min(NC, 100))
        outs = []
        for i, x in enumerate(xs):
            b = self.conv(f"{p}/cv2.{i}/cv2.{i}.0/conv/Conv", x, c2, 3)
            b = self.conv(f"{p}/cv2.{i}/cv2.{i}.1/conv/Conv", b, c2, 3)
            b = self.conv(f"{p}/cv2.{i}/cv2.{i}.2/Conv", b, 4 * REG_MAX, act=False)
            u = self.conv(f"{p}/cv3.{i}/cv3.{i}.0/cv3.{i}.0.0/conv/Conv", x, x.shape[1], 3, g=x.shape[1])
            u = self.conv(f"{p}/cv3.{i}/cv3.{i}.0/cv3.{i}.0.1/conv/Conv", u, c3)
            u = self.conv(f"{p}/cv3.{i}/cv3.{i}.1/cv3.{i}.1.0/conv/Conv", u, c3, 3, g=c3)
            u = self.conv(f"{p}/cv3.{i}/cv3.{i}.1/cv3.{i}.1.1/conv/Conv", u, c3)
            u = self.conv(f"{p}/cv3.{i}/cv3.{i}.2/Conv", u, NC, act=False)
            outs.append(self.cat(f"{p}/Concat_{i}" if i else f"{p}/Concat", [b, u]))
        return outs

    def decode(self, heads):
        """The head's DFL over the box channels and Sigmoid over the class
        channels, per scale: [1, 4 + NC, H, W]."""
        out = []
        for y in heads:
            _, _, h, w = y.shape
            if self.dry:
                out.append(np.zeros((1, 4 + NC, h, w), np.float32))
                continue
            box = self.o.dfl(np.ascontiguousarray(y[:, :4 * REG_MAX]).reshape(1, 4 * REG_MAX, h * w), REG_MAX)
            cls = self.o.sigmoid_ref(np.ascontiguousarray(y[:, 4 * REG_MAX:]))
            out.append(np.concatenate([box.reshape(1, 4, h, w), cls], axis=1))
        return out

    # --------------------------------------------------------------- network
    def forward(self, x, decode=False):
        """yolo11.yaml at scale n; returns the three head tensors
        [1, 4*REG_MAX + NC, H, W] at strides 8, 16, 32 (decoded with decode)."""
        x0 = self.conv("/model.0/conv/Conv", x, 16, 3, 2)
        x1 = self.conv("/model.1/conv/Conv", x0, 32, 3, 2)
        x2 = self.c3k2("/model.2", x1, 64, False, 0.25)
        x3 = self.conv("/model.3/conv/Conv", x2, 64, 3, 2)
        x4 = self.c3k2("/model.4", x3, 128, False, 0.25)
        x5 = self.conv("/model.5/conv/Conv", x4, 128, 3, 2)
        x6 = self.c3k2("/model.6", x5, 128, True)
        x7 = self.conv("/model.7/conv/Conv", x6, 256, 3, 2)
        x8 = self.c3k2("/model.8", x7, 256, True)
        x9 = self.sppf("/model.9", x8, 256)
        x10 = self.c2psa("/model.10", x9, 256)
        x11 = self.upsample("/model.11/Resize", x10)
        x12 = self.cat("/model.12/Concat", [x11, x6])
        x13 = self.c3k2("/model.13", x12, 128, False)
        x14 = self.upsample("/model.14/Resize", x13)
        x15 = self.cat("/model.15/Concat", [x14, x4])
        x16 = self.c3k2("/model.16", x15, 64, False)
        x17 = self.conv("/model.17/conv/Conv", x16, 64, 3, 2)
        x18 = self.cat("/model.18/Concat", [x17, x13])
        x19 = self.c3k2("/model.19", x18, 128, False)
        x20 = self.conv("/model.20/conv/Conv", x19, 128, 3, 2)
        x21 = self.cat("/model.21/Concat", [x20, x10])
        x22 = self.c3k2("/model.22", x21, 256, True)
        heads = self.detect("/model.23", [x16, x19, x22])
        return self.decode(heads) if decode else heads


def forward(oracle, x, seed=7000, decode=False, winograd=1, nchwc=1):
    """The three head tensors of YOLO11n for input x [1, 3, S, S]; nchwc = 0
    for a reference host that does not run NchwcConv."""
    return Net(oracle, seed, winograd, nchwc=nchwc).forward(np.ascontiguousarray(x, np.float32), decode=decode)
