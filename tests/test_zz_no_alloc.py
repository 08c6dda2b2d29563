"""GPU: osh_dqmm_u8s8_noalloc, the DynamicQuantizeMatMul entry point that
allocates nothing (its scratch is a static per-GPU array in the library),
against osh_dqmm_u8s8 with a caller scratch buffer: same int32 accumulators,
quantization parameters and outputs, bit for bit, on two calls in a row (the
second smaller, so it runs over what the first left in the shared array), on
both pipelines (two launches; three launches with the quantized A in scratch)."""
import ctypes as C

import numpy as np
import pytest

from onnxsharp_amd import synth

pytestmark = pytest.mark.gpu


def _t(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _case(cuda, m, k, n, seed):
    import torch
    from onnxsharp_amd import native as N
    a = synth.normal(seed, (m, k))
    a[m // 3, k // 2] = np.nan  # one NaN row
    w = synth.randint(seed + 1, (k, n), -127, 127, np.int8)
    ws = synth.uniform(seed + 2, (n,), 0.001, 0.02)
    bias = synth.normal(seed + 3, (n,), 0, 0.01)
    nb = C.c_size_t()
    N.call("osh_dqmm_packed_weight_bytes", k, n, C.byref(nb))
    packed = torch.empty(nb.value, dtype=torch.uint8, device=cuda)
    dw = _t(w, cuda)
    N.call("osh_dqmm_pack_weights", k, n, C.c_void_p(dw.data_ptr()), 1, None, 0, C.c_void_p(packed.data_ptr()),
           None)
    return dict(a=_t(a, cuda), packed=packed, ws=_t(ws, cuda), bias=_t(bias, cuda))


def _run(cuda, m, k, n, t, noalloc):
    import torch
    from onnxsharp_amd import native as N
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device=cuda)
    acc = torch.full((m, n), -7, dtype=torch.int32, device=cuda)
    qp = torch.zeros(2, dtype=torch.int32, device=cuda)
    p = lambda x: C.c_void_p(x.data_ptr())
    if noalloc:
        N.call("osh_dqmm_u8s8_noalloc", m, k, n, p(t["a"]), p(t["packed"]), p(t["ws"]), n, p(t["bias"]), p(out),
               p(acc), p(qp), None)
    else:
        sb = C.c_size_t()
        N.call("osh_dqmm_scratch_bytes", m, k, C.byref(sb))
        scratch = torch.empty(sb.value, dtype=torch.uint8, device=cuda)
        N.call("osh_dqmm_u8s8", m, k, n, p(t["a"]), p(t["packed"]), p(t["ws"]), n, p(t["bias"]), p(out), p(acc),
               p(qp), p(scratch), None)
    torch.cuda.synchronize()
    return out.cpu().numpy(), acc.cpu().numpy(), qp.cpu().numpy()


@pytest.mark.parametrize("variant", [0, 1, 2])
def test_noalloc_dqmm_matches_the_scratch_entry_point(cuda, variant):
    from onnxsharp_amd import native as N
    old = C.c_int()
    N.call("osh_config_get", b"dqmm_variant", C.byref(old))
    N.call("osh_config_set", b"dqmm_variant", variant)
    try:
        for (m, k, n), seed in (((512, 512, 2048), 600), ((70, 96, 300), 610)):
            print(f"no-alloc DQM variant {variant}: m={m} k={k} n={n}", flush=True)
            t = _case(cuda, m, k, n, seed)
            o0, a0, q0 = _run(cuda, m, k, n, t, noalloc=False)
            o1, a1, q1 = _run(cuda, m, k, n, t, noalloc=True)
            assert np.array_equal(q0, q1), "quantization parameters"
            assert np.array_equal(a0, a1), "int32 accumulators"
            assert np.array_equal(o0.view(np.uint32), o1.view(np.uint32)), "outputs"
            assert np.isnan(o1[m // 3]).all() and np.isfinite(np.delete(o1, m // 3, axis=0)).all()
    finally:
        N.call("osh_config_set", b"dqmm_variant", old.value)
