"""GPU parity: DynamicQuantizeMatMul / DynamicQuantizeLinear.  int32
accumulators and quantization parameters are bit-exact; the FP32 output is
bit-exact against the fused epilogue fmaf(acc, scale * w_scale, bias)."""
import json
import os

import numpy as np
import pytest

from onnxsharp_amd import synth

pytestmark = pytest.mark.gpu


def _t(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def run_dqmm(cuda, a, w, wzp, ws, bias):
    import torch
    from onnxsharp_amd.layers import DynamicQuantizeMatMulLayer
    m = a.size // a.shape[-1]
    n = w.shape[1]
    acc = torch.empty((m, n), dtype=torch.int32, device=cuda)
    qp = torch.empty(2, dtype=torch.int32, device=cuda)
    layer = DynamicQuantizeMatMulLayer()
    out = layer.forward(_t(a, cuda), _t(w, cuda), wzp, None if ws is None else _t(np.atleast_1d(ws), cuda),
                        None if bias is None else _t(bias, cuda), acc_out=acc, qparams_out=qp)
    q = qp.cpu().numpy()
    return out.cpu().numpy(), acc.cpu().numpy(), np.float32(q[0:1].view(np.float32)[0]), int(q[1])


@pytest.mark.parametrize("m,k,n,wdt,zp_kind", [
    (512, 512, 2048, np.int8, None),       # encoder-FFN workload
    (4, 13, 11, np.int8, None),
    (33, 100, 70, np.uint8, "tensor"),
    (17, 64, 40, np.uint8, "column"),
    (5, 1280, 32, np.int8, "column"),      # Int8Tests.F32SubstituteExactAtLongK shape
    (1, 7, 3, np.int8, "tensor"),
    (3, 2100, 17, np.int8, None),          # K with a partial load chunk
    (70, 96, 300, np.uint8, "column"),     # row and column tiles both partial
])
def test_dqmm_parity(cuda, oracle, m, k, n, wdt, zp_kind):
    print(f"dqmm m={m} k={k} n={n} w={wdt.__name__} zp={zp_kind}", flush=True)
    a = synth.normal(m + k, (m, k))
    lo, hi = (-127, 127) if wdt == np.int8 else (0, 255)
    w = synth.randint(m + n, (k, n), lo, hi, wdt)
    base = 0 if wdt == np.int8 else 128
    wzp = None if zp_kind is None else (
        np.array([base + 3], np.int32) if zp_kind == "tensor" else synth.randint(n, (n,), -20, 20, np.int32) + base)
    ws = synth.uniform(k + n, (n,), 0.001, 0.02)
    bias = synth.normal(m + k + n, (n,), 0, 0.01)
    out, acc, s, z = run_dqmm(cuda, a, w, wzp, ws, bias)
    eo, eacc, eaccf, es, ez = oracle.dqmm(a, w, wzp, ws, bias, fused=True)
    assert (s, z) == (es, ez), "quantization parameters"
    assert np.array_equal(acc, eacc), f"int32 accumulators differ at {np.argwhere(acc != eacc)[:5]}"
    assert np.array_equal(eaccf, eacc.astype(np.float32))  # the reference's FP32 chain is exact here
    assert np.array_equal(out, eo), "fused dequant epilogue"
    # the reference's unfused tail rows (acc*s + b) are within one rounding
    eu = oracle.dqmm(a, w, wzp, ws, bias, fused=False)[0]
    assert np.abs(out - eu).max() <= 1e-6 * max(1.0, np.abs(eu).max())


def test_dqmm_scalar_scale_no_bias_and_edge_values(cuda, oracle):
    a = np.concatenate([synth.normal(1, (6, 40)), np.zeros((1, 40), np.float32)]).astype(np.float32)
    a[2, 5] = 0.0
    a[3, :] = 7.25  # a constant positive row
    w = synth.randint(2, (40, 9), -128, 127, np.int8)
    out, acc, s, z = run_dqmm(cuda, a, w, None, np.float32(0.05), None)
    eo, eacc, _, es, ez = oracle.dqmm(a, w, None, np.float32(0.05), None)
    assert (s, z) == (es, ez)
    assert np.array_equal(acc, eacc)
    assert np.array_equal(out, eo)


def test_dqmm_all_zero_input_uses_unit_scale(cuda, oracle):
    a = np.zeros((3, 16), np.float32)
    w = synth.randint(3, (16, 5), -127, 127, np.int8)
    out, acc, s, z = run_dqmm(cuda, a, w, None, np.float32(1.0), None)
    assert (s, z) == (np.float32(1.0), 0)
    assert (acc == 0).all() and (out == 0).all()


def test_dqmm_nan_row_propagates(cuda, oracle):
    a = synth.normal(4, (4, 32))
    a[1, 3] = np.nan
    w = synth.randint(5, (32, 6), -127, 127, np.int8)
    out, acc, s, z = run_dqmm(cuda, a, w, None, np.float32(0.5), None)
    # Quantizer.MinMax skips NaN, so the parameters come from the other values
    es, ez = oracle.dql_params(*oracle.minmax(a))
    assert (s, z) == (es, ez)
    assert np.isnan(out[1]).all() and np.isfinite(np.delete(out, 1, axis=0)).all()
    good = np.delete(np.arange(4), 1)
    _, eacc, _, _, _ = oracle.dqmm(a[good], w, None, np.float32(0.5), None)
    # rows without NaN quantize with the same global parameters
    q = oracle.quantize_u8(a[good], es, ez)
    assert np.array_equal(acc[good], (q.astype(np.int64) - ez) @ w.astype(np.int64))


def test_dynamic_quantize_linear_known_answer(cuda):
    from onnxsharp_amd.layers import DynamicQuantizeLinearLayer
    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))["dynamic_quantize_linear"]
    q, s, z = DynamicQuantizeLinearLayer().forward(_t(np.array(g["x"], np.float32), cuda))
    assert np.float32(s) == np.float32(3) / np.float32(255)
    assert z == g["zero_point"]
    assert q.cpu().numpy().tolist() == g["q"]


def test_dynamic_quantize_linear_matches_oracle(cuda, oracle):
    from onnxsharp_amd.layers import DynamicQuantizeLinearLayer
    x = synth.normal(9, (1000003,), 0.3, 2.0)
    q, s, z = DynamicQuantizeLinearLayer().forward(_t(x, cuda))
    eq, es, ez = oracle.dynamic_quantize_linear(x)
    assert (np.float32(s), z) == (es, ez)
    assert np.array_equal(q.cpu().numpy(), eq)


@pytest.mark.parametrize("m,k,n", [(512, 512, 2048), (3, 2100, 17), (70, 96, 300), (33, 1040, 130), (1, 7, 3),
                                   (64, 1024, 256), (128, 512, 512), (256, 1024, 1024)])
def test_dqmm_fused_and_three_launch_pipelines_identical(cuda, oracle, m, k, n):
    """dqmm_variant 0 (min/max launch, then quantize inside the GEMM launch, K
    in chunks of 512; where every tile is full, the 16 x 16 tile kernel whose
    epilogue overlaps its MFMAs), 1 (min/max, quantize and GEMM launches) and
    2 (as 0, with the 32 x 32 tile kernel for full tiles) give the same bits,
    all equal to the oracle."""
    import ctypes as C
    from onnxsharp_amd import native as N
    print(f"dqmm pipelines m={m} k={k} n={n}", flush=True)
    a = synth.normal(3 * m + k, (m, k))
    a[m // 2, k // 3] = np.nan  # one NaN row on both pipelines
    w = synth.randint(m + 2 * n, (k, n), -127, 127, np.int8)
    ws = synth.uniform(k + 3 * n, (n,), 0.001, 0.02)
    bias = synth.normal(m + n, (n,), 0, 0.01)
    old = C.c_int()
    N.call("osh_config_get", b"dqmm_variant", C.byref(old))
    got, launches = [], []
    try:
        for v in (0, 1, 2):
            N.call("osh_config_set", b"dqmm_variant", v)
            got.append(run_dqmm(cuda, a, w, None, ws, bias))
            nl = C.c_int()
            N.call("osh_config_get", b"dqmm_launches", C.byref(nl))
            launches.append(nl.value)
    finally:
        N.call("osh_config_set", b"dqmm_variant", old.value)
    assert launches == [2, 3, 2], launches
    (o0, a0, s0, z0), (o1, a1, s1, z1), (o2, a2, s2, z2) = got
    assert (s0, z0) == (s1, z1) == (s2, z2)
    assert np.array_equal(a0, a1) and np.array_equal(a0, a2)
    assert np.array_equal(o0.view(np.uint32), o1.view(np.uint32))
    assert np.array_equal(o0.view(np.uint32), o2.view(np.uint32))
    eo, eacc, _, es, ez = oracle.dqmm(a, w, None, ws, bias)
    assert (s0, z0) == (es, ez)
    good = np.ones(m, bool)
    good[m // 2] = False
    assert np.isnan(o0[m // 2]).all()
    q = oracle.quantize_u8(a[good], es, ez)
    assert np.array_equal(a0[good], (q.astype(np.int64) - ez) @ w.astype(np.int64))
    assert np.array_equal(o0[good], eo[good])


@pytest.mark.parametrize("m,k,n", [(512, 512, 2048), (33, 100, 70)])
def test_fused_dqmm_equals_the_node_chain_it_replaces(cuda, oracle, m, k, n):
    """GraphFusion.FuseQuantizedMatMul (src/OnnxSharp/Core/GraphFusion.cs:635-782)
    replaces DynamicQuantizeLinear -> MatMulInteger -> Cast -> Mul(a_scale *
    w_scale) -> Add(bias) by one DynamicQuantizeMatMul [A, W, w_zp, w_scale,
    bias] (:739-744).  On the device the unfused chain (osh_dynamic_quantize_linear,
    osh_matmul_integer, then the Cast/Mul/Add node outputs) must give the
    fused op's int32 accumulators bit for bit, and outputs within the one
    rounding the fused fmaf(acc, s, b) saves over round(round(acc*s) + b)."""
    import torch
    from onnxsharp_amd.layers import DynamicQuantizeLinearLayer, MatMulIntegerLayer
    print(f"DQL -> MatMulInteger -> Cast -> Mul -> Add vs DQM, m={m} k={k} n={n}", flush=True)
    a = synth.normal(300 + m, (m, k))
    w = synth.randint(301 + n, (k, n), -127, 127, np.int8)
    ws = synth.uniform(302 + k, (n,), 0.001, 0.02)
    bias = synth.normal(303, (n,), 0, 0.01)
    # the node chain
    q, a_scale, a_zp = DynamicQuantizeLinearLayer().forward(_t(a, cuda))
    acc_chain = MatMulIntegerLayer().forward(q, _t(w, cuda), [a_zp], None)
    comb = torch.tensor([a_scale], dtype=torch.float32, device=cuda) * _t(ws, cuda)  # Mul(a_scale, w_scale)
    cast = acc_chain.to(torch.float32)                                              # Cast(int32 -> f32)
    mul = cast * comb                                                               # Mul
    out_chain = (mul + _t(bias, cuda)).cpu().numpy()                                # Add(bias)
    # the fused op
    out, acc, s, z = run_dqmm(cuda, a, w, None, ws, bias)
    assert (s, z) == (np.float32(a_scale), a_zp)
    assert np.array_equal(acc, acc_chain.cpu().numpy()), "int32 accumulators"
    # the fused epilogue differs from the chain by at most the rounding of acc*s
    comb_h = (np.float32(a_scale) * ws).astype(np.float32)
    prod = acc.astype(np.float32) * comb_h
    # |fused - chain| <= ulp(fused)/2 + ulp(acc*s)/2 + ulp(chain)/2
    bound = 0.5 * (np.abs(np.spacing(out)) + np.abs(np.spacing(prod)) + np.abs(np.spacing(out_chain)))
    d = np.abs(out.astype(np.float64) - out_chain)
    assert (d <= bound).all(), f"max |d| {d.max():.3e}"
    # the chain's own nodes on the host: the oracle's unfused form, bit for bit
    eo_unfused = (acc.astype(np.float32) * comb_h).astype(np.float32) + bias
    assert np.array_equal(out_chain, eo_unfused.astype(np.float32))
    eo, eacc, _, _, _ = oracle.dqmm(a, w, None, ws, bias)
    assert np.array_equal(out, eo) and np.array_equal(acc, eacc)


def _packed(cuda, w):
    import ctypes as C
    import torch
    from onnxsharp_amd import native as N
    k, n = w.shape
    nb = C.c_size_t()
    N.call("osh_dqmm_packed_weight_bytes", k, n, C.byref(nb))
    packed = torch.empty(nb.value, dtype=torch.uint8, device=cuda)
    dw = _t(w, cuda)
    N.call("osh_dqmm_pack_weights", k, n, C.c_void_p(dw.data_ptr()), 1, None, 0, C.c_void_p(packed.data_ptr()),
           None)
    return packed


def test_dqmm_calls_in_a_row_over_changing_inputs_and_dirty_scratch(cuda, oracle):
    """Calls in a row on one scratch buffer whose A ranges differ (a stale
    min/max partial would change the scale), starting from a scratch full of
    arbitrary bytes, each equal the oracle bit for bit."""
    import ctypes as C
    import torch
    from onnxsharp_amd import native as N
    m, k, n = 512, 512, 2048
    w = synth.randint(900, (k, n), -127, 127, np.int8)
    ws = synth.uniform(901, (n,), 0.001, 0.02)
    bias = synth.normal(902, (n,), 0, 0.01)
    packed = _packed(cuda, w)
    sb = C.c_size_t()
    N.call("osh_dqmm_scratch_bytes", m, k, C.byref(sb))
    for fill in (0xFF, None):
        scratch = torch.empty(sb.value, dtype=torch.uint8, device=cuda)
        if fill is None:
            scratch.copy_(torch.from_numpy(synth.randint(903, (sb.value,), 0, 255, np.uint8)))
        else:
            scratch.fill_(fill)
        for call, (seed, scale_a) in enumerate(((910, 1.0), (911, 7.5), (910, 1.0), (912, 0.01))):
            print(f"DQM calls in a row: scratch fill {fill}, call {call}, A seed {seed} x {scale_a}", flush=True)
            a = (synth.normal(seed, (m, k)) * np.float32(scale_a)).astype(np.float32)
            da, dws, db = _t(a, cuda), _t(ws, cuda), _t(bias, cuda)
            out = torch.empty((m, n), dtype=torch.float32, device=cuda)
            acc = torch.empty((m, n), dtype=torch.int32, device=cuda)
            qp = torch.empty(2, dtype=torch.int32, device=cuda)
            p = lambda x: C.c_void_p(x.data_ptr())
            N.call("osh_dqmm_u8s8", m, k, n, p(da), p(packed), p(dws), n, p(db), p(out), p(acc), p(qp), p(scratch),
                   None)
            torch.cuda.synchronize()
            eo, eacc, _, es, ez = oracle.dqmm(a, w, None, ws, bias)
            q = qp.cpu().numpy()
            assert (np.float32(q[0:1].view(np.float32)[0]), int(q[1])) == (es, ez)
            assert np.array_equal(acc.cpu().numpy(), eacc)
            assert np.array_equal(out.cpu().numpy(), eo)


def test_dqmm_graph_replays_see_new_inputs(cuda, oracle):
    """A HIP graph holding one DynamicQuantizeMatMul (min/max launch, then the
    fused launch) replays with frozen kernel arguments; each replay after new
    data is copied into A quantizes with that data's own min/max."""
    import ctypes as C
    import torch
    from onnxsharp_amd import native as N
    m, k, n = 512, 512, 2048
    w = synth.randint(920, (k, n), -127, 127, np.int8)
    ws = synth.uniform(921, (n,), 0.001, 0.02)
    bias = synth.normal(922, (n,), 0, 0.01)
    packed = _packed(cuda, w)
    sb = C.c_size_t()
    N.call("osh_dqmm_scratch_bytes", m, k, C.byref(sb))
    scratch = torch.empty(sb.value, dtype=torch.uint8, device=cuda)
    da = torch.empty((m, k), dtype=torch.float32, device=cuda)
    dws, db = _t(ws, cuda), _t(bias, cuda)
    out = torch.empty((m, n), dtype=torch.float32, device=cuda)
    acc = torch.empty((m, n), dtype=torch.int32, device=cuda)
    st = C.c_void_p()
    N.call("osh_stream_create", C.byref(st))
    g = C.c_void_p()
    p = lambda x: C.c_void_p(x.data_ptr())
    try:
        da.copy_(_t(synth.normal(930, (m, k)), cuda))
        torch.cuda.synchronize()
        N.call("osh_graph_begin", st)
        try:
            N.call("osh_dqmm_u8s8", m, k, n, p(da), p(packed), p(dws), n, p(db), p(out), p(acc), None, p(scratch),
                   st)
        finally:
            N.call("osh_graph_end", st, C.byref(g))
        for rep, (seed, scale_a) in enumerate(((931, 1.0), (932, 20.0), (931, 1.0), (933, 0.05))):
            print(f"DQM graph replay {rep}: A seed {seed} x {scale_a}", flush=True)
            a = (synth.normal(seed, (m, k)) * np.float32(scale_a)).astype(np.float32)
            da.copy_(_t(a, cuda))
            torch.cuda.synchronize()
            N.call("osh_graph_launch", g, st)
            N.call("osh_stream_sync", st)
            eo, eacc, _, _, _ = oracle.dqmm(a, w, None, ws, bias)
            assert np.array_equal(acc.cpu().numpy(), eacc), f"replay {rep}: accumulators"
            assert np.array_equal(out.cpu().numpy(), eo), f"replay {rep}: outputs"
    finally:
        if g.value:
            N.call("osh_graph_destroy", g)
        N.call("osh_stream_destroy", st)


@pytest.mark.parametrize("m,k,n", [(512, 512, 2048), (70, 96, 300)])
@pytest.mark.parametrize("noalloc", [False, True])
@pytest.mark.parametrize("offset", [0, 4])
@pytest.mark.parametrize("variant", [0, 2])
def test_dqmm_output_without_accumulators(cuda, oracle, m, k, n, noalloc, offset, variant):
    """With no int32 accumulator output (d_acc NULL, as the benchmark and the
    C# emitter call it) the full-tile kernel writes its output tiles through
    LDS as 16-byte vectors when `out` is 16-byte aligned, and element by
    element otherwise (offset 4).  Both must give the oracle's bits, a NaN row
    included, from osh_dqmm_u8s8 and from osh_dqmm_u8s8_noalloc, with the
    16 x 16 tile kernel (variant 0) and the 32 x 32 one (variant 2)."""
    import ctypes as C
    import torch
    from onnxsharp_amd import native as N
    print(f"dqmm no-acc m={m} k={k} n={n} noalloc={noalloc} offset={offset} variant={variant}", flush=True)
    old = C.c_int()
    N.call("osh_config_get", b"dqmm_variant", C.byref(old))
    N.call("osh_config_set", b"dqmm_variant", variant)
    try:
        _no_acc_case(cuda, oracle, m, k, n, noalloc, offset)
    finally:
        N.call("osh_config_set", b"dqmm_variant", old.value)


def _no_acc_case(cuda, oracle, m, k, n, noalloc, offset):
    import ctypes as C
    import torch
    from onnxsharp_amd import native as N
    a = synth.normal(7 * m + k, (m, k))
    a[m // 3, k // 2] = np.nan
    w = synth.randint(7 * n + k, (k, n), -127, 127, np.int8)
    ws = synth.uniform(7 * k + n, (n,), 0.001, 0.02)
    bias = synth.normal(7 * m + n, (n,), 0, 0.01)
    nb = C.c_size_t()
    N.call("osh_dqmm_packed_weight_bytes", k, n, C.byref(nb))
    packed = torch.empty(nb.value, dtype=torch.uint8, device=cuda)
    dw = _t(w, cuda)
    N.call("osh_dqmm_pack_weights", k, n, C.c_void_p(dw.data_ptr()), 1, None, 0, C.c_void_p(packed.data_ptr()),
           None)
    da, dws, db = _t(a, cuda), _t(ws, cuda), _t(bias, cuda)
    raw = torch.full((m * n + 4,), float("inf"), dtype=torch.float32, device=cuda)
    out_ptr = C.c_void_p(raw.data_ptr() + offset)
    ptr = lambda t: C.c_void_p(t.data_ptr())
    if noalloc:
        N.call("osh_dqmm_u8s8_noalloc", m, k, n, ptr(da), ptr(packed), ptr(dws), n, ptr(db), out_ptr, None, None,
               None)
    else:
        sb = C.c_size_t()
        N.call("osh_dqmm_scratch_bytes", m, k, C.byref(sb))
        scratch = torch.empty(sb.value, dtype=torch.uint8, device=cuda)
        N.call("osh_dqmm_u8s8", m, k, n, ptr(da), ptr(packed), ptr(dws), n, ptr(db), out_ptr, None, None,
               ptr(scratch), None)
    torch.cuda.synchronize()
    flat = raw.cpu().numpy()
    got = flat[offset // 4: offset // 4 + m * n].reshape(m, n)
    # nothing written outside [out, out + m*n)
    assert np.isinf(np.delete(flat, np.arange(offset // 4, offset // 4 + m * n))).all()
    eo, _, _, _, _ = oracle.dqmm(a, w, None, ws, bias)
    good = np.ones(m, bool)
    good[m // 3] = False
    assert np.isnan(got[m // 3]).all()
    assert np.array_equal(got[good].view(np.uint32), eo[good].view(np.uint32))
