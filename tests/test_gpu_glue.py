"""GPU parity of the frame's continuity ops through the C ABI: Add, MaxPool,
the SPPF pool chain, nearest Resize, Transpose and Softmax against the
oracle's restatements, bit for bit, including odd sizes and batch strides.  MaxPool inputs carry NaNs: the
device follows the reference's scalar comparison (start at -inf, take v when
v > max: NaNs are skipped).  The reference's 8-wide path (Vector256.Max)
treats a NaN by operand order instead, so NaN results are pinned to the
scalar path only; inputs without NaN give the same bits on both paths."""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_fp32_close
from onnxsharp_amd import synth

pytestmark = pytest.mark.gpu


def _dev(a, cuda):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(cuda)


def _p(t):
    return C.c_void_p(t.data_ptr())


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("n,aligned", [(1 << 20, True), (1001, True), (4096, False)])
def test_add_exact_and_in_place(cuda, n, aligned):
    import torch
    from onnxsharp_amd import native as N
    a = synth.normal(900 + n, (n + 1,), 0, 1)
    b = synth.normal(901 + n, (n + 1,), 0, 1)
    off = 0 if aligned else 1  # a 4-byte offset takes the scalar kernel
    da, db = _dev(a, cuda), _dev(b, cuda)
    y = torch.empty(n + 1, device=cuda)
    N.call("osh_add_f32", n, C.c_void_p(da.data_ptr() + 4 * off), C.c_void_p(db.data_ptr() + 4 * off),
           C.c_void_p(y.data_ptr() + 4 * off), None)
    # in place: y aliases a
    N.call("osh_add_f32", n, C.c_void_p(da.data_ptr() + 4 * off), C.c_void_p(db.data_ptr() + 4 * off),
           C.c_void_p(da.data_ptr() + 4 * off), None)
    torch.cuda.synchronize()
    expect = (a[off:off + n] + b[off:off + n]).astype(np.float32)
    assert np.array_equal(y.cpu().numpy()[off:off + n], expect)
    assert np.array_equal(da.cpu().numpy()[off:off + n], expect)


POOLS = [((1, 128, 20, 20), 5, 1, 2), ((2, 3, 33, 47), 3, 2, 1), ((1, 4, 16, 16), 2, 2, 0), ((1, 2, 9, 7), 7, 1, 3)]


@pytest.mark.parametrize("shape,k,s,p", POOLS, ids=[f"{s}_k{k}s{st}p{p}" for s, k, st, p in POOLS])
def test_maxpool_matches_oracle_with_nans(cuda, oracle, shape, k, s, p):
    import torch
    from onnxsharp_amd import native as N
    x = synth.normal(910 + k, shape, 0, 1)
    x.reshape(-1)[::37] = np.nan  # skipped by the comparison
    n, c, h, w = shape
    oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    pp = N.PoolParams(n, c, h, w, k, k, s, s, p, p, oh, ow)
    dx = _dev(x, cuda)
    y = torch.empty((n, c, oh, ow), device=cuda)
    N.call("osh_maxpool2d_f32", C.byref(pp), _p(dx), _p(y), None)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y.cpu().numpy()), _bits(oracle.maxpool2d(x, k, s, p)))


CHAINS = [((1, 128, 20, 20), 5), ((2, 5, 70, 45), 5), ((1, 3, 40, 33), 3), ((1, 2, 37, 64), 7), ((1, 1, 1, 1), 5)]


@pytest.mark.parametrize("shape,k", CHAINS, ids=[f"{s}_k{k}" for s, k in CHAINS])
def test_pool_chain_is_three_pools(cuda, oracle, shape, k):
    # one launch = three osh_maxpool2d_f32 launches in turn, bit for bit (NaNs
    # included), with the outputs written as channel slices of one buffer
    import torch
    from onnxsharp_amd import native as N
    n, c, h, w = shape
    print(f"pool chain {shape} k={k}", flush=True)
    x = synth.normal(920 + k + h, shape, 0, 1)
    x.reshape(-1)[::29] = np.nan
    cat = torch.full((n, 4 * c, h, w), float("inf"), device=cuda)
    cat[:, :c] = _dev(x, cuda)
    hw = h * w
    base = cat.data_ptr()
    ys = [C.c_void_p(base + 4 * (i + 1) * c * hw) for i in range(3)]
    N.call("osh_maxpool_chain3_f32", n, c, h, w, k, C.c_void_p(base), 4 * c * hw, ys[0], ys[1], ys[2], 4 * c * hw,
           None)
    # the same through three single pools
    pp = N.PoolParams(n, c, h, w, k, k, 1, 1, k // 2, k // 2, h, w)
    prev = _dev(x, cuda)
    singles = []
    for _ in range(3):
        nxt = torch.empty((n, c, h, w), device=cuda)
        N.call("osh_maxpool2d_f32", C.byref(pp), _p(prev), _p(nxt), None)
        singles.append(nxt)
        prev = nxt
    torch.cuda.synchronize()
    got = cat.cpu().numpy()
    assert np.array_equal(_bits(got[:, :c]), _bits(x))  # input untouched
    ref = x
    for i in range(3):
        ref = oracle.maxpool2d(ref, k, 1, k // 2)
        part = got[:, (i + 1) * c:(i + 2) * c]
        assert np.array_equal(_bits(part), _bits(singles[i].cpu().numpy())), f"pool {i + 1} vs single launch"
        assert np.array_equal(_bits(part), _bits(ref)), f"pool {i + 1} vs oracle"


@pytest.mark.parametrize("shape,f", [((1, 256, 20, 20), 2), ((2, 3, 7, 5), 3), ((2, 5, 6, 8), 2), ((1, 4, 5, 7), 2)],
                         ids=["yolo_2x", "3x", "batch2_2x", "odd_width_2x"])
def test_resize_nearest_into_a_channel_slice(cuda, oracle, shape, f):
    # 2x with an even width takes the paired kernel (16-byte stores), other
    # shapes the per-element one; both into a channel slice of a wider buffer
    import torch
    from onnxsharp_amd import native as N
    n, c, h, w = shape
    x = synth.normal(930 + f, shape, 0, 1)
    out = torch.zeros((n, c + 5, h * f, w * f), device=cuda)
    dx = _dev(x, cuda)
    N.call("osh_resize_nearest_f32", n, c, h, w, f, f, _p(dx), _p(out), (c + 5) * h * f * w * f, None)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got[:, :c], oracle.resize_nearest(x, f))
    assert not got[:, c:].any()


@pytest.mark.parametrize("batch,rows,cols", [(2, 400, 32), (1, 33, 65), (3, 1, 17)])
def test_transpose_last_two_axes(cuda, batch, rows, cols):
    import torch
    from onnxsharp_amd import native as N
    x = synth.normal(940 + rows, (batch, rows, cols), 0, 1)
    dx = _dev(x, cuda)
    y = torch.empty((batch, cols, rows), device=cuda)
    N.call("osh_transpose_f32", batch, rows, cols, _p(dx), rows * cols, _p(y), rows * cols, None)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), x.transpose(0, 2, 1))


@pytest.mark.parametrize("rows,cols,scale", [(800, 400, 32 ** -0.5), (7, 1000, 1.0), (3, 5, 10.0), (9, 13, 0.5),
                                              (33, 8, 1.0)])
def test_softmax_is_the_reference_row_order(cuda, oracle, rows, cols, scale):
    # eight lane sums combined in lane order, the tail after them, as
    # VectorMath.SoftmaxRow adds them: the oracle's bits exactly
    import torch
    from onnxsharp_amd import native as N
    x = synth.normal(950 + cols, (rows, cols), 0, 4)
    dx = _dev(x, cuda)
    y = torch.empty_like(dx)
    N.call("osh_softmax_f32", rows, cols, C.c_float(scale), _p(dx), _p(y), None)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.array_equal(got, oracle.softmax(x, scale)), f"softmax {rows}x{cols}"
    assert np.allclose(got.sum(axis=1), 1.0, atol=1e-5)


DFL_CASES = [((1, 64, 8400), 16), ((1, 64, 6400), 16), ((2, 64, 400), 16), ((1, 64, 300), 16),
             ((1, 32, 13), 16), ((3, 24, 77), 8)]


@pytest.mark.parametrize("shape,bins", DFL_CASES, ids=[f"{s}_b{b}" for s, b in DFL_CASES])
def test_dfl_matches_oracle(cuda, oracle, shape, bins):
    # the vector-path columns and the scalar-line columns (the last width % 8
    # of a 256-column block) both restate the reference; the scalar lines call
    # MathF.Exp in the reference, whose bits are not pinned (exp_ref here)
    from onnxsharp_amd.layers import DflSoftmaxLayer
    x = synth.normal(960 + shape[2], shape, 0, 3)
    if shape[2] == 300:
        # a NaN bin: Avx.Max(max, row) drops it at the next bin and the exp
        # clamp (maxps against -87.3) sends it to e^-87.3, so it weighs ~0
        x[0, 5, 17] = np.nan
    y = DflSoftmaxLayer(bins).forward(_dev(x, cuda)).cpu().numpy()
    ref = oracle.dfl(x, bins)
    assert np.array_equal(_bits(y), _bits(ref))
    if shape[2] == 300:
        assert np.isfinite(y).all()


def test_dfl_reads_a_head_tensor_slice(cuda, oracle):
    # the box channels of a [1, 144, H, W] head output, in place: batch stride
    # of the whole head tensor, output into a wider buffer
    import torch
    from onnxsharp_amd import native as N
    head = synth.normal(970, (2, 144, 20, 20), 0, 2)
    dh = _dev(head, cuda)
    out = torch.zeros((2, 6, 400), device=cuda)
    N.call("osh_dfl_f32", 2, 4, 16, 400, _p(dh), 144 * 400, _p(out), 6 * 400, None)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = oracle.dfl(np.ascontiguousarray(head[:, :64].reshape(2, 64, 400)))
    assert np.array_equal(got[:, :4], ref) and not got[:, 4:].any()


def test_sigmoid_matches_oracle(cuda, oracle):
    from onnxsharp_amd.layers import ActivationLayer
    x = synth.normal(980, (1, 80, 40, 40), 0, 6)
    y = ActivationLayer("Sigmoid").forward(_dev(x, cuda)).cpu().numpy()
    assert np.array_equal(y, oracle.sigmoid_ref(x))


ATTENTION = [(2, 32, 64, 400), (1, 4, 16, 16), (3, 8, 32, 480), (2, 16, 48, 80), (1, 32, 64, 32), (1, 64, 16, 48),
             (2, 28, 32, 272), (1, 32, 128, 208)]


@pytest.mark.parametrize("heads,kd,hd,n", ATTENTION, ids=[f"h{h}_kd{k}_hd{d}_n{n}" for h, k, d, n in ATTENTION])
def test_fused_attention_is_the_node_sequence(cuda, oracle, heads, kd, hd, n):
    # one launch against MatMul(q^T, k) -> Mul -> Softmax -> MatMul(v, P^T) as
    # the oracle restates the nodes, and against the five-launch device path
    import types
    import torch
    from onnxsharp_amd import native as N
    from oracle import yolo_frame as YO
    rows = 2 * kd + hd
    pad = 7 * n  # a head stride above the dense one
    hs = rows * n + pad
    qkv = synth.normal(960 + n, (heads, hs), 0, 1)
    scale = kd ** -0.5
    dq = _dev(qkv, cuda)
    y = torch.full((heads * hd * n,), float("nan"), device=cuda)
    N.call("osh_attention_f32", heads, kd, hd, n, C.c_float(scale), _p(dq), hs, _p(y), None)
    # five launches: q^T, scores, softmax, P^T, v P^T
    qt = torch.empty(heads * n * kd, device=cuda)
    sc = torch.empty(heads * n * n, device=cuda)
    st = torch.empty_like(sc)
    y5 = torch.empty_like(y)
    base = dq.data_ptr()
    N.call("osh_transpose_f32", heads, kd, n, C.c_void_p(base), hs, _p(qt), n * kd, None)
    N.call("osh_gemm_f32_batched", heads, n, n, kd, _p(qt), kd, n * kd, C.c_void_p(base + 4 * kd * n), n, hs,
           None, N.ACT_NONE, _p(sc), n, n * n, None)
    N.call("osh_softmax_f32", heads * n, n, C.c_float(scale), _p(sc), _p(st), None)
    N.call("osh_transpose_f32", heads, n, n, _p(st), n * n, _p(sc), n * n, None)
    N.call("osh_gemm_f32_batched", heads, hd, n, n, C.c_void_p(base + 8 * kd * n), n, hs, _p(sc), n, n * n, None,
           N.ACT_NONE, _p(y5), n, hd * n, None)
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(heads, hd, n)
    dense = np.ascontiguousarray(qkv[:, :rows * n])
    op = types.SimpleNamespace(qkv=types.SimpleNamespace(h=1, w=n), key_dim=kd, head_dim=hd, heads=heads,
                               scale=scale, y=types.SimpleNamespace(c=heads * hd, h=1, w=n))
    expect = YO.attention(oracle, op, dense).reshape(heads, hd, n)
    assert np.array_equal(_bits(got), _bits(expect)), f"attention h{heads} kd{kd} hd{hd} n{n} vs oracle"
    assert np.array_equal(_bits(got), _bits(y5.cpu().numpy().reshape(heads, hd, n))), "fused vs five launches"


def test_fused_attention_rejects_what_it_cannot_take(cuda):
    import torch
    from onnxsharp_amd import native as N
    q = torch.zeros(2 * 128 * 1008, device=cuda)
    y = torch.zeros(64 * 1008, device=cuda)
    for heads, kd, hd, n in [(1, 32, 64, 1008), (1, 32, 64, 496), (1, 30, 64, 400), (1, 32, 40, 400),
                             (1, 32, 64, 408), (1, 68, 64, 400)]:
        rc = N.lib().osh_attention_f32(heads, kd, hd, n, C.c_float(1.0), _p(q), (2 * kd + hd) * n, _p(y), None)
        assert rc == N.OSH_E_UNSUPPORTED, (heads, kd, hd, n)
    # y inside qkv
    rc = N.lib().osh_attention_f32(1, 32, 64, 400, C.c_float(1.0), _p(q), 128 * 400, C.c_void_p(q.data_ptr() + 4),
                                   None)
    assert rc == N.OSH_E_INVALID
