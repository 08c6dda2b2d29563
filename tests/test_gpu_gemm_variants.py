"""GPU parity of every gemm16 wave tile (osh_config_set("gemm_variant", v)) and
of the LDS-staged tile (v = -2) against the oracle's FMA-chain GEMM, on shapes
that exercise partial row/column tiles, K tails shorter than one chunk, padded
leading dimensions, row bias, column scale and fused activations.  Every tile
sums k in order with one rounding per product, so outputs must be
bit-identical to the chain (and within the conftest tolerance, relative 1e-4,
absolute 1e-5, in any case)."""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_fp32_close
from onnxsharp_amd import synth

pytestmark = pytest.mark.gpu


def _t(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _variants():
    from onnxsharp_amd import native as N
    n = C.c_int()
    N.call("osh_config_get", b"gemm_variants", C.byref(n))
    return [-2] + list(range(n.value))


@pytest.fixture()
def variant_reset():
    yield
    from onnxsharp_amd import native as N
    N.call("osh_config_set", b"gemm_variant", -1)


# (m, k, n, lda_pad, ldc_pad): K tails shorter than a chunk, K < 4, partial tiles in both directions
CASES = [(1024, 768, 768, 0, 0), (70, 36, 96, 0, 0), (33, 4, 8, 0, 0), (5, 13, 132, 3, 4),
         (200, 100, 260, 4, 8), (97, 64, 36, 0, 0)]


def _gemm(cuda, m, k, n, lda, ldc, a, b, col_bias=None, row_bias=None, col_scale=None, act=0):
    import torch
    from onnxsharp_amd import native as N
    a_pad = np.zeros((m, lda), np.float32)
    a_pad[:, :k] = a
    da, db = _t(a_pad, cuda), _t(b, cuda)
    dc = torch.full((m, ldc), 7.0, dtype=torch.float32, device=cuda)
    ptr = lambda t: C.c_void_p(t.data_ptr()) if t is not None else None
    keep = [_t(x, cuda) if x is not None else None for x in (col_bias, row_bias, col_scale)]
    N.call("osh_gemm_f32", m, n, k, ptr(da), lda, ptr(db), n, ptr(keep[0]), ptr(keep[1]), ptr(keep[2]), act,
           ptr(dc), ldc, C.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    out = dc.cpu().numpy()
    assert (out[:, n:] == 7.0).all(), "wrote past n into the padding of C"
    return out[:, :n]


@pytest.mark.parametrize("m,k,n,lpad,cpad", CASES)
def test_gemm_variants_column_bias(cuda, oracle, variant_reset, m, k, n, lpad, cpad):
    from onnxsharp_amd import native as N
    a = synth.uniform(m * 7 + k, (m, k), -1, 1)
    b = synth.uniform(n * 5 + k, (k, n), -1, 1)
    bias = synth.uniform(m + n, (n,), -1, 1)
    ref = oracle.gemm_f32(a, b, col_bias=bias)
    for v in _variants():
        print(f"gemm variant {v}: m={m} k={k} n={n} lda=k+{lpad} ldc=n+{cpad}", flush=True)
        N.call("osh_config_set", b"gemm_variant", v)
        y = _gemm(cuda, m, k, n, k + lpad, n + cpad, a, b, col_bias=bias)
        assert_fp32_close(y, ref, f"variant {v} gemm {m}x{k}x{n}")
        assert np.array_equal(y, ref), f"variant {v} gemm {m}x{k}x{n}: not bit-identical"


def test_gemm_variants_row_bias_silu_and_column_scale(cuda, oracle, variant_reset):
    from onnxsharp_amd import native as N
    m, k, n = 128, 256, 640
    a = synth.uniform(301, (m, k), -1, 1)
    b = synth.uniform(302, (k, n), 0, 1)
    rb = synth.normal(303, (m,), 0, 0.1)
    cs = synth.uniform(304, (n,), 1e-3, 1e-1)
    cb = synth.uniform(305, (n,), -1, 1)
    ref_silu = oracle.silu_ref(oracle.gemm_f32(a, b, row_bias=rb))
    ref_scale = oracle.relu(oracle.gemm_f32(a, b, col_bias=cb, col_scale=cs))
    N.call("osh_config_set", b"exact_silu", 1)
    try:
        for v in _variants():
            print(f"gemm variant {v}: row bias + SiLU, column scale + Relu", flush=True)
            N.call("osh_config_set", b"gemm_variant", v)
            y = _gemm(cuda, m, k, n, k, n, a, b, row_bias=rb, act=N.ACT_SILU)
            assert_fp32_close(y, ref_silu, f"variant {v} row bias + silu")
            assert np.array_equal(y, ref_silu), f"variant {v} row bias + silu: not bit-identical"
            y = _gemm(cuda, m, k, n, k, n, a, b, col_bias=cb, col_scale=cs, act=N.ACT_RELU)
            assert_fp32_close(y, ref_scale, f"variant {v} column scale + relu")
            assert np.array_equal(y, ref_scale), f"variant {v} column scale + relu: not bit-identical"
    finally:
        N.call("osh_config_set", b"exact_silu", 0)


def test_gemm_variants_batched_broadcast(cuda, oracle, variant_reset):
    import torch
    from onnxsharp_amd import native as N
    batch, m, k, n = 3, 40, 72, 64
    a = synth.uniform(311, (batch, m, k), -1, 1)
    b = synth.uniform(312, (k, n), -1, 1)  # broadcast over the batch (stride 0)
    bias = synth.uniform(313, (n,), -1, 1)
    ref = np.stack([oracle.gemm_f32(a[i], b, col_bias=bias) for i in range(batch)])
    da, db, dbias = _t(a, cuda), _t(b, cuda), _t(bias, cuda)
    for v in _variants():
        print(f"gemm variant {v}: batched {batch}x{m}x{k}x{n}", flush=True)
        N.call("osh_config_set", b"gemm_variant", v)
        dc = torch.empty((batch, m, n), dtype=torch.float32, device=cuda)
        N.call("osh_gemm_f32_batched", batch, m, n, k, C.c_void_p(da.data_ptr()), k, m * k,
               C.c_void_p(db.data_ptr()), n, 0, C.c_void_p(dbias.data_ptr()), 0, C.c_void_p(dc.data_ptr()), n,
               m * n, C.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert_fp32_close(dc.cpu().numpy(), ref, f"variant {v} batched")
        assert np.array_equal(dc.cpu().numpy(), ref), f"variant {v} batched: not bit-identical"


def test_gemm_variant_option_range():
    from onnxsharp_amd import native as N
    with pytest.raises(N.OshError):
        N.call("osh_config_set", b"gemm_variant", 1000)
