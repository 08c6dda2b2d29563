"""CPU execution of a yolo11n.Model with the oracle.

TEST INFRASTRUCTURE ONLY: used by tests/ and by bench.py's cpu_baseline leg.

Each op is restated with the oracle's functions in the order the reference's
AVX-512 dispatch uses for that layer (ConvLayer.Forward,
src/OnnxSharp/Ops/DnnOps.cs:437-482, restated by
oracle.conv_reference_kernel): depthwise for g == C == M, the NCHWc chain
where NchwcConv's gate holds, Winograd F(2x2,3x3) where Winograd's gate holds,
the im2col/pointwise FMA chain otherwise; SiLU is the reference polynomial.  The
attention core uses the GEMM chain for both MatMuls and the oracle softmax.
"""
import numpy as np


def conv(oracle, op, x, res=None, winograd=1, nchwc=1):
    k, s, pad = op.k, op.s, op.k // 2
    out_hw = (op.y.h, op.y.w)
    y = oracle.conv_reference(x, op.w, op.b, (s, s), (pad, pad), (1, 1), op.group, out_hw, winograd=winograd,
                              nchwc=nchwc)
    if op.act == "Silu":
        y = oracle.silu_ref(y)
    if res is not None:  # a fused residual Add: one float addition per element
        y = (y + res).astype(np.float32)
    return y


def attention(oracle, op, qkv):
    n = op.qkv.h * op.qkv.w
    rows = 2 * op.key_dim + op.head_dim
    q3 = qkv.reshape(op.heads, rows, n)
    ys = []
    for h in range(op.heads):
        q = q3[h, :op.key_dim]
        k = q3[h, op.key_dim:2 * op.key_dim]
        v = q3[h, 2 * op.key_dim:]
        scores = oracle.gemm_f32(np.ascontiguousarray(q.T), k)
        probs = oracle.softmax(scores, op.scale)
        ys.append(oracle.gemm_f32(v, np.ascontiguousarray(probs.T)))
    return np.concatenate(ys, axis=0).reshape(1, op.y.c, op.y.h, op.y.w)


def run_op(oracle, op, inputs, nchwc=1):
    """Output of one op from its input arrays (in the op's own input order);
    nchwc = 0 for a reference host that does not run NchwcConv."""
    from onnxsharp_amd import yolo11n as Y
    if isinstance(op, Y.ConvOp):
        return conv(oracle, op, inputs[0], inputs[1] if op.res is not None else None, nchwc=nchwc)
    if isinstance(op, Y.AddOp):
        return (inputs[0] + inputs[1]).astype(np.float32)
    if isinstance(op, Y.CopyOp):
        return inputs[0].copy()
    if isinstance(op, Y.MaxPoolOp):
        return oracle.maxpool2d(inputs[0], op.k, op.s, op.p)
    if isinstance(op, Y.PoolChainOp):  # three pools in turn, outputs side by side
        y1 = oracle.maxpool2d(inputs[0], op.k, 1, op.k // 2)
        y2 = oracle.maxpool2d(y1, op.k, 1, op.k // 2)
        y3 = oracle.maxpool2d(y2, op.k, 1, op.k // 2)
        return np.concatenate([y1, y2, y3], axis=1)
    if isinstance(op, Y.UpsampleOp):
        return oracle.resize_nearest(inputs[0], op.f)
    if isinstance(op, Y.DflOp):
        x = inputs[0]
        return oracle.dfl(x.reshape(1, x.shape[1], -1), op.bins).reshape(1, x.shape[1] // op.bins, *x.shape[2:])
    if isinstance(op, Y.SigmoidOp):
        return oracle.sigmoid_ref(inputs[0])
    if isinstance(op, Y.AttentionOp):
        return attention(oracle, op, inputs[0])
    raise TypeError(op)


def op_inputs(op):
    """The slices an op reads, in run_op order."""
    from onnxsharp_amd import yolo11n as Y
    if isinstance(op, Y.AddOp):
        return [op.a, op.b]
    if isinstance(op, Y.AttentionOp):
        return [op.qkv]
    if isinstance(op, Y.ConvOp) and op.res is not None:
        return [op.x, op.res]
    return [op.x]


class Frame:
    """The whole model on numpy buffers (one array per device buffer).
    `oracle` is the oracle.oracle module."""

    def __init__(self, model):
        self.model = model
        self.arrays = {id(b): np.zeros((1, b.c, b.h, b.w), np.float32) for b in model.bufs}

    def get(self, sl):
        return self.arrays[id(sl.buf)][:, sl.c0:sl.c0 + sl.c]

    def put(self, sl, val):
        self.arrays[id(sl.buf)][:, sl.c0:sl.c0 + sl.c] = val

    def run(self, oracle, x):
        from onnxsharp_amd import yolo11n as Y
        self.put(Y.whole(self.model.input), x)
        for grouped in self.model.ops:
            # a GroupConvOp's convs are independent, a ChainOp's chains are
            # (stages in order) and a PairOp is two convs in order: run the
            # convs one by one
            for op in grouped.ops if isinstance(grouped, (Y.GroupConvOp, Y.ChainOp, Y.PairOp)) else [grouped]:
                ins = [np.ascontiguousarray(self.get(s)) for s in op_inputs(op)]
                self.put(op.y, run_op(oracle, op, ins))
        return [self.arrays[id(b)] for b in self.model.outputs]
