"""GPU parity of ONNX Gemm (GemmLayer, src/OnnxSharp/Ops/AttnOps.cs:31-135):
transA/transB, alpha, beta and the C forms the reference accepts (full
[M,N], scalar, a row indexed by column j % len).  The reference's steps --
materialized transposes, the FMA chain from 0, alpha * y then + beta * c --
are each exact or single-rounded, so the device result is bit-identical to
the oracle's restatement."""
import numpy as np
import pytest

from onnxsharp_amd import synth

pytestmark = pytest.mark.gpu


def _t(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


CASES = [
    (64, 48, 32, False, False, 1.0, 1.0, "row"),
    (64, 48, 32, True, False, 0.5, 1.0, "full"),
    (33, 70, 17, False, True, 1.0, 0.25, "row"),
    (33, 70, 17, True, True, 2.0, 1.0, "scalar"),
    (100, 128, 96, False, True, 1.0, 1.0, "short"),   # len 5: j % 5
    (8, 8, 8, True, True, 1.0, 0.0, "full"),          # beta 0: C ignored
    (300, 256, 768, False, True, 1.0, 1.0, "row"),    # a Linear layer (transB weights)
    (5, 3, 2, False, False, 1.5, 1.0, None),
]


@pytest.mark.parametrize("m,k,n,ta,tb,alpha,beta,ckind", CASES)
def test_gemm_ex(cuda, oracle, m, k, n, ta, tb, alpha, beta, ckind):
    from onnxsharp_amd.layers import GemmLayer
    print(f"gemm_ex m={m} k={k} n={n} transA={ta} transB={tb} alpha={alpha} beta={beta} C={ckind}", flush=True)
    seed = m * 3 + k * 5 + n * 7 + ta + 2 * tb
    a = synth.uniform(seed, (k, m) if ta else (m, k), -1, 1)
    b = synth.uniform(seed + 1, (n, k) if tb else (k, n), -1, 1)
    c = {None: None, "row": synth.uniform(seed + 2, (n,), -1, 1), "full": synth.uniform(seed + 2, (m, n), -1, 1),
         "scalar": np.float32([0.75]), "short": synth.uniform(seed + 2, (5,), -1, 1)}[ckind]
    layer = GemmLayer(alpha=alpha, beta=beta, transA=ta, transB=tb)
    y = layer.forward(_t(a, cuda), _t(b, cuda), None if c is None else _t(c, cuda)).cpu().numpy()
    ref = oracle.gemm_ex(a, b, c, alpha, beta, ta, tb)
    assert y.shape == (m, n)
    assert np.array_equal(y, ref), f"max |d| {np.abs(y - ref).max():.3e}"


def test_gemm_ex_shape_errors(cuda):
    import torch
    from onnxsharp_amd import native as N
    from onnxsharp_amd.layers import GemmLayer
    a = torch.zeros((4, 3), device=cuda)
    b = torch.zeros((4, 5), device=cuda)
    with pytest.raises(N.OshError, match="K mismatch"):
        GemmLayer().forward(a, b)
    with pytest.raises(N.OshError, match="only 2-D"):
        GemmLayer().forward(torch.zeros((2, 4, 3), device=cuda), b)
