"""GPU: a segment driven through the C ABI alone, the way the C# HIP
partition layer drives it (VkPartitionLayer.Forward,
src/OnnxSharp.Vulkan/VkPartitionLayer.cs:221-263; VkSegment.Execute,
src/OnnxSharp.Vulkan/VkSegment.cs:324-600; pooled device buffers,
src/OnnxSharp.Vulkan/VkBufferPool.cs:20-190).

No torch tensor is involved: device memory comes from osh_malloc, host
staging from osh_host_alloc (pinned), inputs go in with osh_memcpy_h2d, the
weights are packed once on the device, the op launches, the outputs come back
with osh_memcpy_d2h, the stream is synchronised once, and everything is freed
with osh_free / osh_host_free.  Results are checked against the oracle:
bit-exact for the FP32 chains (exact SiLU) and the int32 accumulators."""
import ctypes as C

import numpy as np
import pytest

from onnxsharp_amd import synth

pytestmark = pytest.mark.gpu


class Segment:
    """Device buffers, pinned staging buffers and one stream, all owned
    through the C ABI; freed on close()."""

    def __init__(self):
        from onnxsharp_amd import native as N
        self.N = N
        self.dev, self.host = [], []
        self.stream = C.c_void_p()
        N.call("osh_stream_create", C.byref(self.stream))

    def dmalloc(self, nbytes):
        p = C.c_void_p()
        self.N.call("osh_malloc", C.byref(p), max(1, int(nbytes)))
        self.dev.append(p)
        return p

    def hstage(self, arr=None, nbytes=None):
        nbytes = arr.nbytes if arr is not None else int(nbytes)
        p = C.c_void_p()
        self.N.call("osh_host_alloc", C.byref(p), max(1, nbytes))
        self.host.append(p)
        if arr is not None:
            C.memmove(p, np.ascontiguousarray(arr).ctypes.data, nbytes)
        return p

    def upload(self, arr):
        """Stage a host array in pinned memory and copy it to a new device buffer."""
        h = self.hstage(arr)
        d = self.dmalloc(arr.nbytes)
        self.N.call("osh_memcpy_h2d", d, h, arr.nbytes, self.stream)
        return d

    def download_to(self, d, shape, dtype):
        """Queue a copy of device buffer d into a new pinned buffer; returns a
        reader that is valid after sync()."""
        nbytes = int(np.prod(shape)) * np.dtype(dtype).itemsize
        h = self.hstage(nbytes=nbytes)
        self.N.call("osh_memcpy_d2h", h, d, nbytes, self.stream)

        def read():
            out = np.empty(shape, dtype)
            C.memmove(out.ctypes.data, h, nbytes)
            return out
        return read

    def sync(self):
        self.N.call("osh_stream_sync", self.stream)

    def close(self):
        for p in self.dev:
            self.N.call("osh_free", p)
        for p in self.host:
            self.N.call("osh_host_free", p)
        self.N.call("osh_stream_destroy", self.stream)
        self.dev, self.host = [], []


@pytest.fixture()
def exact_silu(cuda):
    from onnxsharp_amd import native as N
    N.call("osh_config_set", b"exact_silu", 1)
    yield
    N.call("osh_config_set", b"exact_silu", 0)


def test_segment_gemm_bias_c1(cuda, oracle):
    from onnxsharp_amd import native as N
    m, k, n = 1024, 768, 768
    print(f"segment gemm {m}x{k}x{n} + bias through the C ABI", flush=True)
    a = synth.uniform(101, (m, k), -1, 1)
    b = synth.uniform(102, (k, n), -1, 1)
    bias = synth.uniform(103, (n,), -1, 1)
    seg = Segment()
    try:
        da, db, dbias = seg.upload(a), seg.upload(b), seg.upload(bias)
        dc = seg.dmalloc(m * n * 4)
        N.call("osh_gemm_f32", m, n, k, da, k, db, n, dbias, None, None, N.ACT_NONE, dc, n, seg.stream)
        read = seg.download_to(dc, (m, n), np.float32)
        seg.sync()
        got = read()
    finally:
        seg.close()
    assert np.array_equal(got, oracle.gemm_f32(a, b, col_bias=bias))


@pytest.mark.parametrize("xs,ws,stride", [((1, 64, 160, 160), (64, 64, 3, 3), 1),
                                           ((1, 256, 80, 80), (128, 256, 1, 1), 1),
                                           ((1, 128, 80, 80), (256, 128, 3, 3), 2)],
                         ids=["c2", "c3a", "c3b"])
def test_segment_conv_silu(cuda, oracle, exact_silu, xs, ws, stride):
    from onnxsharp_amd import native as N
    print(f"segment conv {xs} * {ws} s{stride} + bias + SiLU through the C ABI", flush=True)
    x = synth.uniform(1, xs)
    w = synth.normal(2, ws, 0.0, 0.05)
    b = synth.normal(3, (ws[0],), 0.0, 0.01)
    pad = ws[2] // 2
    attrs = N.ConvAttrs()
    attrs.group = 1
    attrs.n_strides, attrs.strides[0], attrs.strides[1] = 2, stride, stride
    attrs.n_pads = 4
    for i in range(4):
        attrs.pads[i] = pad
    p = N.ConvParams()
    N.call("osh_conv_resolve", C.byref(attrs), N.dims64(xs), N.dims64(ws), C.byref(p))
    nbytes = C.c_size_t()
    N.call("osh_conv_packed_weight_bytes", C.byref(p), C.byref(nbytes))
    seg = Segment()
    try:
        dx, dw, db = seg.upload(x), seg.upload(w), seg.upload(b)
        dpk = seg.dmalloc(nbytes.value)
        N.call("osh_conv_pack_weights", C.byref(p), dw, dpk, seg.stream)  # once per model
        dy = seg.dmalloc(p.n * p.m * p.oh * p.ow * 4)
        N.call("osh_memset_d8", dy, 0xFF, p.n * p.m * p.oh * p.ow * 4, seg.stream)  # NaN: the conv must overwrite
        N.call("osh_conv2d_f32", C.byref(p), dx, dpk, db, N.ACT_SILU, dy, seg.stream)
        read = seg.download_to(dy, (p.n, p.m, p.oh, p.ow), np.float32)
        seg.sync()
        got = read()
    finally:
        seg.close()
    ref = oracle.silu_ref(oracle.conv_reference(x, w, b, (stride, stride), (pad, pad), (1, 1), 1, (p.oh, p.ow)))
    assert np.array_equal(got, ref), f"max |d| {np.abs(got - ref).max():.3e}"


def test_segment_dqmm_c5(cuda, oracle):
    from onnxsharp_amd import native as N
    m, k, n = 512, 512, 2048
    print(f"segment DynamicQuantizeMatMul {m}x{k}x{n} through the C ABI", flush=True)
    a = synth.normal(201, (m, k))
    w = synth.randint(202, (k, n), -127, 127, np.int8)
    ws = synth.uniform(203, (n,), 0.001, 0.02)
    bias = synth.normal(204, (n,), 0, 0.01)
    pbytes, sbytes = C.c_size_t(), C.c_size_t()
    N.call("osh_dqmm_packed_weight_bytes", k, n, C.byref(pbytes))
    N.call("osh_dqmm_scratch_bytes", m, k, C.byref(sbytes))
    seg = Segment()
    try:
        da, dw, dws, dbias = seg.upload(a), seg.upload(w), seg.upload(ws), seg.upload(bias)
        dpk = seg.dmalloc(pbytes.value)
        N.call("osh_dqmm_pack_weights", k, n, dw, 1, None, 0, dpk, seg.stream)
        dscr = seg.dmalloc(sbytes.value)
        dout, dacc, dqp = seg.dmalloc(m * n * 4), seg.dmalloc(m * n * 4), seg.dmalloc(8)
        N.call("osh_dqmm_u8s8", m, k, n, da, dpk, dws, n, dbias, dout, dacc, dqp, dscr, seg.stream)
        r_out = seg.download_to(dout, (m, n), np.float32)
        r_acc = seg.download_to(dacc, (m, n), np.int32)
        r_qp = seg.download_to(dqp, (2,), np.int32)
        seg.sync()
        out, acc, qp = r_out(), r_acc(), r_qp()
    finally:
        seg.close()
    eo, eacc, _, es, ez = oracle.dqmm(a, w, None, ws, bias)
    assert (qp[0:1].view(np.float32)[0], int(qp[1])) == (es, ez)
    assert np.array_equal(acc, eacc)
    assert np.array_equal(out, eo)


def test_segment_memset_and_d2d(cuda):
    from onnxsharp_amd import native as N
    seg = Segment()
    try:
        nb = (1 << 20) + 13  # odd length: the fill kernel's byte tail
        d1, d2 = seg.dmalloc(nb), seg.dmalloc(nb)
        N.call("osh_memset_d8", d1, 0x5A, nb, seg.stream)
        N.call("osh_memcpy_d2d", d2, d1, nb, seg.stream)
        N.call("osh_memset_d8", d1, 0x00, 7, seg.stream)
        r1 = seg.download_to(d1, (nb,), np.uint8)
        r2 = seg.download_to(d2, (nb,), np.uint8)
        seg.sync()
        g1, g2 = r1(), r2()
    finally:
        seg.close()
    assert (g2 == 0x5A).all()
    assert (g1[:7] == 0).all() and (g1[7:] == 0x5A).all()


def test_segment_errors_are_status_codes(cuda):
    from onnxsharp_amd import native as N
    p = C.c_void_p()
    st = N.lib().osh_malloc(C.byref(p), 1 << 48)  # 256 TiB: far beyond the 288 GB of HBM
    assert st == N.OSH_E_NOMEM and N.last_error() and not p.value
    # the failure stays inside the status code: the next allocation works
    import torch
    t = torch.empty(1 << 20, device=cuda)
    t.fill_(1.0)
    torch.cuda.synchronize()
    assert N.lib().osh_gemm_f32(4, 4, 4, None, 4, None, 4, None, None, None, 0, None, 4, None) == N.OSH_E_INVALID
    assert "NULL" in N.last_error()
