"""GPU parity: MatMul + fused column bias (osh_gemm_f32) against the oracle's
FMA-chain restatement of GemmKernel (tolerance in conftest: relative 1e-4,
absolute 1e-5)."""
import numpy as np
import pytest

from conftest import assert_fp32_close, fp32_violations
from onnxsharp_amd import synth

pytestmark = pytest.mark.gpu


def _t(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


# GemmKernelTests shapes (tests/OnnxSharp.Tests/GemmKernelTests.cs:27-36,126-136) plus the 1024x768x768 workload
SHAPES = [(257, 64, 257), (257, 257, 64), (64, 64, 64), (257, 384, 1536), (300, 256, 256), (1, 257, 64),
          (5, 17, 33), (17, 1, 257), (3, 1, 7), (9, 64, 17), (96, 320, 1280)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_gemm_column_bias(cuda, oracle, m, k, n):
    from onnxsharp_amd.layers import MatMulLayer
    print(f"gemm m={m} k={k} n={n}", flush=True)
    a = synth.uniform(m * 17 + k * 5 + n * 3, (m, k), -1, 1)
    b = synth.uniform(m * 13 + k * 29 + n * 11, (k, n), -1, 1)
    bias = synth.uniform(m + k + n, (n,), -1, 1)
    y = MatMulLayer(fused_bias=_t(bias, cuda)).forward(_t(a, cuda), _t(b, cuda)).cpu().numpy()
    ref = oracle.gemm_f32(a, b, col_bias=bias)
    # the reference test's own bar (|d| / max(1, |x|) <= 1e-4 vs float64) ...
    exact = oracle.gemm_f64(a, b, col_bias=bias)
    assert (np.abs(y - exact) / np.maximum(1.0, np.abs(exact))).max() <= 1e-4
    # ... and the parity bar against the FMA chain: the MFMA kernels add the
    # products in k order with one rounding per step, so the match is exact
    assert_fp32_close(y, ref, f"gemm {m}x{k}x{n}")
    assert np.array_equal(y, ref), f"gemm {m}x{k}x{n}: not bit-identical to the FMA chain"


def test_gemm_workload_1024x768x768(cuda, oracle):
    from onnxsharp_amd.layers import MatMulLayer
    print("gemm 1024x768x768 + bias", flush=True)
    a = synth.uniform(101, (1024, 768), -1, 1)
    b = synth.uniform(102, (768, 768), -1, 1)
    bias = synth.uniform(103, (768,), -1, 1)
    y = MatMulLayer(fused_bias=_t(bias, cuda)).forward(_t(a, cuda), _t(b, cuda)).cpu().numpy()
    ref = oracle.gemm_f32(a, b, col_bias=bias)
    nbad, dmax = fp32_violations(y, ref)
    print(f"  violations={nbad} max|d|={dmax:.3e}", flush=True)
    assert_fp32_close(y, ref, "gemm 1024x768x768")
    assert np.array_equal(y, ref), "gemm 1024x768x768: not bit-identical to the FMA chain"


def test_gemm_row_bias_scale_and_activation(cuda, oracle):
    import ctypes as C
    import torch
    from onnxsharp_amd import native as N
    m, k, n = 70, 96, 45
    a = synth.uniform(111, (m, k), -1, 1)
    b = synth.uniform(112, (k, n), -1, 1)
    rb = synth.uniform(113, (m,), -1, 1)
    cs = synth.uniform(114, (n,), 1e-4, 1e-2)
    cb = synth.uniform(115, (n,), -1, 1)
    ta, tb, trb, tcs, tcb = (_t(v, cuda) for v in (a, b, rb, cs, cb))
    out = torch.empty((m, n), dtype=torch.float32, device=cuda)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: C.c_void_p(t.data_ptr())
    N.call("osh_gemm_f32", m, n, k, p(ta), k, p(tb), n, None, p(trb), None, N.ACT_SILU, p(out), n, st)
    pre = oracle.gemm_f32(a, b, row_bias=rb)
    assert_fp32_close(out.cpu().numpy(), oracle.silu_ref(pre), "row bias + silu")
    N.call("osh_gemm_f32", m, n, k, p(ta), k, p(tb), n, p(tcb), None, p(tcs), N.ACT_RELU, p(out), n, st)
    ref = oracle.relu(oracle.gemm_f32(a, b, col_bias=cb, col_scale=cs))
    assert_fp32_close(out.cpu().numpy(), ref, "column scale + bias + relu")


def test_gemm_ldc_and_unaligned(cuda, oracle):
    import ctypes as C
    import torch
    from onnxsharp_amd import native as N
    # GemmKernelTests.MatchesNaiveWithLdcAndBias: ldc wider than n; operands at odd offsets
    m, k, n, ldc = 64, 63, 5, 9
    a = synth.uniform(121, (m, k), -1, 1)
    b = synth.uniform(122, (k, n), -1, 1)
    ta = _t(np.concatenate([[0.0], a.ravel()]).astype(np.float32), cuda)
    tb = _t(np.concatenate([[0.0], b.ravel()]).astype(np.float32), cuda)
    out = torch.full((m * ldc,), -7.0, dtype=torch.float32, device=cuda)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    N.call("osh_gemm_f32", m, n, k, C.c_void_p(ta.data_ptr() + 4), k, C.c_void_p(tb.data_ptr() + 4), n, None, None,
           None, 0, C.c_void_p(out.data_ptr()), ldc, st)
    o = out.cpu().numpy().reshape(m, ldc)
    assert_fp32_close(o[:, :n], oracle.gemm_f32(a, b), "ldc")
    assert (o[:, n:] == -7.0).all(), "wrote outside the ldc row"


def test_matmul_batched_broadcast(cuda, oracle):
    from onnxsharp_amd.layers import MatMulLayer
    a = synth.uniform(131, (2, 1, 33, 20), -1, 1)
    b = synth.uniform(132, (3, 20, 17), -1, 1)
    bias = synth.uniform(133, (17,), -1, 1)
    y = MatMulLayer(fused_bias=_t(bias, cuda)).forward(_t(a, cuda), _t(b, cuda)).cpu().numpy()
    assert y.shape == (2, 3, 33, 17)
    for i in range(2):
        for j in range(3):
            assert_fp32_close(y[i, j], oracle.gemm_f32(a[i, 0], b[j], col_bias=bias), f"batch {i},{j}")
    # rank-3 A times a constant rank-2 B merges batch rows into one GEMM
    a3 = synth.uniform(134, (4, 25, 20), -1, 1)
    b2 = synth.uniform(135, (20, 17), -1, 1)
    y = MatMulLayer(fused_bias=_t(bias, cuda)).forward(_t(a3, cuda), _t(b2, cuda)).cpu().numpy()
    assert_fp32_close(y.reshape(100, 17), oracle.gemm_f32(a3.reshape(100, 20), b2, col_bias=bias), "merged rows")
