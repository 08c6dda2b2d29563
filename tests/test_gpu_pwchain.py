"""GPU: osh_pw_chain_f32 -- runs of pointwise convs (and a leading 3x3
depthwise) as one launch -- against the same convs launched one by one
through ConvLayer: every stage's output bit for bit, with the fast and the
exact SiLU epilogue, on full and partial 16-pixel tiles, several chains per
launch; and the launch's refusals."""
import ctypes as C

import numpy as np
import pytest

from onnxsharp_amd import synth

pytestmark = pytest.mark.gpu


def _t(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


class _Conv:
    """One conv of a chain: weights, bias and its standalone layer."""

    def __init__(self, cuda, seed, c, m, k, act, group=1):
        from onnxsharp_amd.layers import ConvLayer
        self.w = _t(synth.normal(seed, (m, c // group, k, k), 0, 0.05), cuda)
        self.b = _t(synth.normal(seed + 1, (m,), 0, 0.01), cuda)
        self.layer = ConvLayer(fused_activation=act, group=group, pads=[1, 1, 1, 1] if k == 3 else [0, 0, 0, 0])
        self.m, self.act = m, act

    def run(self, x, res=None):
        return self.layer.forward(x, self.w, self.b, residual=res)

    def packed(self, x_shape):
        if self.layer._packed is None or self.layer._packed[0][2] != tuple(x_shape):
            self.layer.prepack_weights(tuple(x_shape), self.w)
        return self.layer._packed[2]


def _stage(conv, x_shape, kind, parts, res_stage=-1, res=None, y=None):
    from onnxsharp_amd import native as N
    st = N.PwStage()
    st.kind, st.m, st.act, st.nsrc = kind, conv.m, N.ACTIVATIONS[conv.act], len(parts)
    for i, (src_stage, tensor, c) in enumerate(parts):
        st.src_stage[i] = src_stage
        st.src[i] = tensor.data_ptr() if tensor is not None else None
        st.src_c[i] = c
    st.w = conv.packed(x_shape).data_ptr()
    st.bias = conv.b.data_ptr()
    st.res_stage = res_stage
    st.res = res.data_ptr() if res is not None else None
    st.y = y.data_ptr()
    return st


def _psa_chain(cuda, hw, seed, c=32):
    """C2PSA's tail with c channels (128 in YOLO11n; its weights do not fit
    in LDS at 128, so the frame keeps those convs apart): proj (+ shortcut)
    -> ffn.0 -> ffn.1 (+ proj's output) -> cv2 over the concat of cv1's first
    half and ffn.1's output."""
    import torch
    from onnxsharp_amd import native as N
    h, w = hw
    s1 = _t(synth.uniform(seed, (1, c, h, w), -1, 1), cuda)
    b = _t(synth.uniform(seed + 1, (1, c, h, w), -1, 1), cuda)
    cat = torch.empty((1, 2 * c, h, w), device=cuda)
    cat[:, :c] = _t(synth.uniform(seed + 2, (1, c, h, w), -1, 1), cuda)
    proj = _Conv(cuda, seed + 10, c, c, 1, None)
    f0 = _Conv(cuda, seed + 20, c, 2 * c, 1, "Silu")
    f1 = _Conv(cuda, seed + 30, 2 * c, c, 1, None)
    cv2 = _Conv(cuda, seed + 40, 2 * c, 2 * c, 1, "Silu")
    # one by one
    r_b1 = proj.run(s1, res=b)
    r_f0 = f0.run(r_b1)
    r_f1 = f1.run(r_f0, res=r_b1)
    cat_ref = cat.clone()
    cat_ref[:, c:] = r_f1
    r_y = cv2.run(cat_ref)
    # as one chain
    y_b1 = torch.full_like(r_b1, float("nan"))
    y_f0 = torch.full_like(r_f0, float("nan"))
    y_y = torch.full_like(r_y, float("nan"))
    cat_out = cat[:, c:]  # ffn.1 writes the concat's second half
    ch = N.PwChain()
    ch.h, ch.w, ch.nstages = h, w, 4
    ch.stage[0] = _stage(proj, (1, c, h, w), N.PW_1X1, [(-1, s1, c)], res=b, y=y_b1)
    ch.stage[1] = _stage(f0, (1, c, h, w), N.PW_1X1, [(0, None, c)], y=y_f0)
    ch.stage[2] = _stage(f1, (1, 2 * c, h, w), N.PW_1X1, [(1, None, 2 * c)], res_stage=0, y=cat_out)
    ch.stage[3] = _stage(cv2, (1, 2 * c, h, w), N.PW_1X1, [(-1, cat[:, :c], c), (2, None, c)], y=y_y)
    refs = [(y_b1, r_b1), (y_f0, r_f0), (cat_out, r_f1), (y_y, r_y)]
    return ch, refs, [s1, b, cat, proj, f0, f1, cv2]


def _head_chain(cuda, c, hw, seed):
    """The detection head's class branch tail at one scale: depthwise 3x3 ->
    1x1 (SiLU) -> 1x1 (no activation)."""
    import torch
    from onnxsharp_amd import native as N
    h, w = hw
    x = _t(synth.uniform(seed, (1, c, h, w), -1, 1), cuda)
    dw = _Conv(cuda, seed + 10, c, c, 3, "Silu", group=c)
    pw1 = _Conv(cuda, seed + 20, c, c, 1, "Silu")
    pw2 = _Conv(cuda, seed + 30, c, c, 1, None)
    r0 = dw.run(x)
    r1 = pw1.run(r0)
    r2 = pw2.run(r1)
    ys = [torch.full_like(r, float("nan")) for r in (r0, r1, r2)]
    ch = N.PwChain()
    ch.h, ch.w, ch.nstages = h, w, 3
    ch.stage[0] = _stage(dw, (1, c, h, w), N.PW_DW3X3, [(-1, x, c)], y=ys[0])
    ch.stage[1] = _stage(pw1, (1, c, h, w), N.PW_1X1, [(0, None, c)], y=ys[1])
    ch.stage[2] = _stage(pw2, (1, c, h, w), N.PW_1X1, [(1, None, c)], y=ys[2])
    return ch, list(zip(ys, (r0, r1, r2))), [x, dw, pw1, pw2]


def _run(chains):
    import torch
    from onnxsharp_amd import native as N
    arr = (N.PwChain * len(chains))(*chains)
    N.check(N.lib().osh_pw_chain_f32(len(chains), arr, C.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()


@pytest.mark.parametrize("exact", [0, 1])
@pytest.mark.parametrize("hw", [(20, 20), (10, 10), (4, 4)])
def test_psa_tail_chain_equals_separate_convs(cuda, exact, hw):
    from onnxsharp_amd import native as N
    print(f"pointwise chain: C2PSA tail at {hw}, exact_silu={exact}", flush=True)
    N.call("osh_config_set", b"exact_silu", exact)
    try:
        ch, refs, keep = _psa_chain(cuda, hw, 100 + hw[0])
        _run([ch])
    finally:
        N.call("osh_config_set", b"exact_silu", 0)
    for k, (got, ref) in enumerate(refs):
        assert np.array_equal(got.cpu().numpy(), ref.cpu().numpy()), f"stage {k}"


def test_chain_stage_may_overwrite_what_it_read_earlier(cuda):
    """C2PSA's ffn.1 writes the concat half whose old contents (the block's
    shortcut) proj added as its residual two stages earlier: a tile reads
    everything first, so the chain equals the convs one by one; and a stage
    part may take some channels of an earlier stage's output (C3k's two 1x1
    convs over the second half of cv1's output)."""
    import torch
    from onnxsharp_amd import native as N
    h = w = 20
    c = 32
    cat = torch.empty((1, 2 * c, h, w), device=cuda)
    cat[:] = _t(synth.uniform(77, (1, 2 * c, h, w), -1, 1), cuda)
    s1 = _t(synth.uniform(78, (1, c, h, w), -1, 1), cuda)
    proj = _Conv(cuda, 80, c, c, 1, None)
    f0 = _Conv(cuda, 90, c, 2 * c, 1, "Silu")
    f1 = _Conv(cuda, 100, 2 * c, c, 1, None)
    cv2 = _Conv(cuda, 110, 2 * c, 2 * c, 1, "Silu")
    half = _Conv(cuda, 120, c, 16, 1, "Silu")
    ref_cat = cat.clone()
    r_b1 = proj.run(s1, res=ref_cat[:, c:].contiguous())
    r_f0 = f0.run(r_b1)
    ref_cat[:, c:] = f1.run(r_f0, res=r_b1)
    r_y = cv2.run(ref_cat)
    r_h = half.run(r_f0[:, c:].contiguous())
    y_b1, y_f0, y_y, y_h = (torch.empty_like(t) for t in (r_b1, r_f0, r_y, r_h))
    ch = N.PwChain()
    ch.h, ch.w, ch.nstages = h, w, 5
    ch.stage[0] = _stage(proj, (1, c, h, w), N.PW_1X1, [(-1, s1, c)], res=cat[:, c:], y=y_b1)
    ch.stage[1] = _stage(f0, (1, c, h, w), N.PW_1X1, [(0, None, c)], y=y_f0)
    ch.stage[2] = _stage(f1, (1, 2 * c, h, w), N.PW_1X1, [(1, None, 2 * c)], res_stage=0, y=cat[:, c:])
    ch.stage[3] = _stage(cv2, (1, 2 * c, h, w), N.PW_1X1, [(-1, cat[:, :c], c), (2, None, c)], y=y_y)
    ch.stage[4] = _stage(half, (1, c, h, w), N.PW_1X1, [(1, y_f0[:, c:], c)], y=y_h)
    _run([ch])
    for name, got, ref in (("proj", y_b1, r_b1), ("ffn.0", y_f0, r_f0), ("ffn.1", cat[:, c:], ref_cat[:, c:]),
                           ("cv2", y_y, r_y), ("half", y_h, r_h)):
        assert np.array_equal(got.cpu().numpy(), ref.cpu().numpy()), name


def test_chain_with_three_parts_and_a_wide_stage(cuda):
    """A stage over three parts (memory, an earlier stage, memory) and a
    stage of 512 channels: parts start inside an unrolled group of input
    blocks, and the wide stage takes two bias values a thread and eight
    output blocks a wave."""
    import torch
    from onnxsharp_amd import native as N
    h, w = 8, 12
    a = _t(synth.uniform(501, (1, 48, h, w), -1, 1), cuda)
    m = _t(synth.uniform(502, (1, 80, h, w), -1, 1), cuda)
    c0 = _Conv(cuda, 510, 48, 64, 1, "Silu")
    c1 = _Conv(cuda, 520, 48 + 64 + 80, 32, 1, None)
    c2 = _Conv(cuda, 530, 32, 512, 1, "Silu")
    r0 = c0.run(a)
    r1 = c1.run(torch.cat([a, r0, m], dim=1))
    r2 = c2.run(r1)
    y0, y1, y2 = (torch.full_like(t, float("nan")) for t in (r0, r1, r2))
    ch = N.PwChain()
    ch.h, ch.w, ch.nstages = h, w, 3
    ch.stage[0] = _stage(c0, (1, 48, h, w), N.PW_1X1, [(-1, a, 48)], y=y0)
    ch.stage[1] = _stage(c1, (1, 192, h, w), N.PW_1X1, [(-1, a, 48), (0, None, 64), (-1, m, 80)], y=y1)
    ch.stage[2] = _stage(c2, (1, 32, h, w), N.PW_1X1, [(1, None, 32)], y=y2)
    _run([ch])
    for k, (got, ref) in enumerate(((y0, r0), (y1, r1), (y2, r2))):
        assert np.array_equal(got.cpu().numpy(), ref.cpu().numpy()), f"stage {k}"


@pytest.mark.parametrize("exact", [0, 1])
def test_head_tails_of_three_scales_in_one_launch(cuda, exact):
    from onnxsharp_amd import native as N
    print(f"pointwise chain: head tails at 80/40/20 in one launch, exact_silu={exact}", flush=True)
    N.call("osh_config_set", b"exact_silu", exact)
    try:
        built = [_head_chain(cuda, 80, (s, s), 300 + s) for s in (80, 40, 20)]
        _run([b[0] for b in built])
    finally:
        N.call("osh_config_set", b"exact_silu", 0)
    for s, (_, refs, _) in zip((80, 40, 20), built):
        for k, (got, ref) in enumerate(refs):
            assert np.array_equal(got.cpu().numpy(), ref.cpu().numpy()), f"scale {s} stage {k}"


def test_chain_refusals(cuda):
    """An output over a tensor a later stage reads from memory, an output over
    a depthwise stage's input, weights not packed for the stage, a depthwise
    stage after stage 0, a depthwise output that overlaps its residual other
    than exactly, and a chain whose weights do not fit in LDS are refused."""
    import torch
    from onnxsharp_amd import native as N
    ch, refs, keep = _psa_chain(cuda, (20, 20), 7)
    cat = keep[2]
    bad = N.PwChain.from_buffer_copy(ch)
    bad.stage[0].y = cat[:, :32].data_ptr()  # proj over the part cv2 reads later
    with pytest.raises(N.OshError, match="overlaps"):
        _run([bad])
    hch0, _, hkeep0 = _head_chain(cuda, 80, (20, 20), 8)
    bad = N.PwChain.from_buffer_copy(hch0)
    bad.stage[2].y = hkeep0[0].data_ptr()  # the last 1x1 over the depthwise input
    with pytest.raises(N.OshError, match="overlaps"):
        _run([bad])
    bad = N.PwChain.from_buffer_copy(ch)
    bad.stage[3].w = keep[5].w.data_ptr()  # raw weights, never packed
    with pytest.raises(N.OshError, match="not packed"):
        _run([bad])
    hch, _, hkeep = _head_chain(cuda, 80, (20, 20), 9)
    bad = N.PwChain.from_buffer_copy(hch)
    bad.stage[1], bad.stage[0] = hch.stage[0], hch.stage[1]
    with pytest.raises(N.OshError):
        _run([bad])
    # a depthwise stage whose output overlaps its own residual a plane away
    hch1, _, hkeep1 = _head_chain(cuda, 80, (20, 20), 11)
    planes = torch.zeros((1, 81, 20, 20), dtype=torch.float32, device=cuda)
    bad = N.PwChain.from_buffer_copy(hch1)
    bad.stage[0].res = planes.data_ptr()
    bad.stage[0].y = planes[:, 1:].data_ptr()
    with pytest.raises(N.OshError, match="overlaps"):
        _run([bad])
    big, _, _ = _psa_chain(cuda, (20, 20), 10, c=128)  # 576 KB of weights
    with pytest.raises(N.OshError, match="LDS"):
        _run([big])
    torch.cuda.synchronize()
