"""Operator layers over the HIP backend, mirroring OnnxSharp's own layers.

Names, attribute meaning and errors follow the reference operators (paths
relative to the OnnxSharp source tree):

  ConvLayer                    src/OnnxSharp/Ops/DnnOps.cs:101-501
  MatMulLayer (+ FusedBias)    src/OnnxSharp/Ops/DnnOps.cs:2789-3103
  GemmLayer                    src/OnnxSharp/Ops/AttnOps.cs:31-135
  DynamicQuantizeMatMulLayer   src/OnnxSharp/Ops/QuantizedMatMulOps.cs:28-376
  DynamicQuantizeLinearLayer   src/OnnxSharp/Ops/QuantOps.cs:166-227
  MatMulIntegerLayer           src/OnnxSharp/Ops/QuantOps.cs:235-428

Shape inference, pad resolution and kernel choice run inside libosh_hip.so
(C++); this module only moves torch device pointers across the C ABI.  Tensors
are device tensors (torch on ROCm is used for device memory and streams).
Shape errors raise OshError (the reference raises OnnxSharpException); shapes
the backend does not take raise OshUnsupported (an emitter refusing an op).
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import torch

from . import native as N


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else C.c_void_p(t.data_ptr())


def _need_f32(name: str, t: torch.Tensor) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {t.dtype}")
    return t.contiguous()


class ConvLayer:
    """2-D Conv with an optional fused activation ("Relu" / "Silu").

    Attributes follow ONNX Conv as ConvLayer reads them: an attribute that is
    not given stays empty (kernel_shape then comes from the weights)."""

    def __init__(self, group: int = 1, kernel_shape: Sequence[int] = (), strides: Sequence[int] = (),
                 pads: Sequence[int] = (), dilations: Sequence[int] = (), auto_pad: str = "NOTSET",
                 fused_activation: Optional[str] = None, name: str = "conv"):
        if auto_pad not in N.AUTO_PAD:
            raise ValueError(f"Conv '{name}': unknown auto_pad {auto_pad!r}")
        if fused_activation not in N.ACTIVATIONS:
            raise ValueError(f"Conv '{name}': activation {fused_activation!r} cannot be fused")
        self.name = name
        self.fused_activation = fused_activation
        lists = [list(kernel_shape), list(strides), list(pads), list(dilations)]
        for vals, cap in zip(lists, (2, 2, 4, 2)):
            if len(vals) > cap:
                raise N.OshUnsupported(N.OSH_E_UNSUPPORTED, f"Conv '{name}': only 1-D and 2-D convolution are implemented")
        self.attrs = self._make_attrs(group, auto_pad, *lists)
        # A rank-3 input (ConvLayer.Forward1D, src/OnnxSharp/Ops/DnnOps.cs:235-300,
        # 422-428) runs as the 2-D conv of [N, C, 1, L] by [M, C/g, 1, K]: the
        # 1-D attributes on the width axis, kernel 1, stride 1, no pads and
        # dilation 1 on the height axis (auto_pad then pads only the width).
        one = lambda v, lead: (lead + v) if len(v) == 1 else v
        pads1 = [0, pads[0], 0, pads[1]] if len(pads) == 2 else list(pads)
        self.attrs1d = self._make_attrs(group, auto_pad, one(list(kernel_shape), [1]), one(list(strides), [1]), pads1,
                                        one(list(dilations), [1]))
        # 1-D attribute lists: the [N, C, 1, L] view of a rank-3 input takes
        # the width-axis form too (with no attributes both forms agree)
        self._attrs_1d = (any(len(v) == 1 for v in (lists[0], lists[1], lists[3])) or len(lists[2]) == 2)
        self._lists, self._auto_pad = lists, auto_pad
        self._packed = None  # (key, params, buffer)

    @staticmethod
    def _make_attrs(group, auto_pad, kernel_shape, strides, pads, dilations) -> N.ConvAttrs:
        a = N.ConvAttrs()
        a.group = int(group)
        a.auto_pad = N.AUTO_PAD[auto_pad]
        for field, count, vals in (("kernel_shape", "n_kernel_shape", kernel_shape), ("strides", "n_strides", strides),
                                   ("pads", "n_pads", pads), ("dilations", "n_dilations", dilations)):
            setattr(a, count, len(vals))
            arr = getattr(a, field)
            for i, v in enumerate(vals):
                arr[i] = int(v)
        return a

    def _shapes2d(self, x_shape: Sequence[int], w_shape: Sequence[int]):
        """(attrs, x shape, w shape) of the 2-D conv that computes this one."""
        if len(x_shape) == 3 and len(w_shape) == 3:
            return self.attrs1d, (x_shape[0], x_shape[1], 1, x_shape[2]), (w_shape[0], w_shape[1], 1, w_shape[2])
        return (self.attrs1d if self._attrs_1d else self.attrs), tuple(x_shape), tuple(w_shape)

    # -- shape logic (C++ side of the library)
    def _length1d(self, length: int, weight_kernel: int) -> Optional[int]:
        """Output length of a rank-3 conv with explicit pads (Conv1DShape /
        Resolve1D, DnnOps.cs:204-227: pads [begin, end], the end pad read when
        given), or None where the width axis of the 2-D form gives it already
        (auto_pad, or equal pads: the 2-D shape takes the begin pad twice)."""
        k, st, pads, dl = self._lists
        if self._auto_pad != "NOTSET" or len(pads) != 2 or pads[0] == pads[1]:
            return None
        kernel = k[0] if k else weight_kernel
        stride = st[0] if st else 1
        dilation = dl[0] if dl else 1
        out = (length + pads[0] + pads[1] - ((kernel - 1) * dilation + 1)) // stride + 1
        if out <= 0:
            raise N.OshError(N.OSH_E_INVALID, f"Conv '{self.name}': output length {out}")
        return out

    def get_memory_shapes(self, x_shape: Sequence[int], w_shape: Sequence[int]) -> tuple:
        if len(x_shape) != len(w_shape) or len(x_shape) not in (3, 4):
            raise N.OshUnsupported(N.OSH_E_UNSUPPORTED,
                                   f"Conv '{self.name}': only 1-D (NCL) and 2-D (NCHW) convolution are implemented")
        attrs, xs, ws = self._shapes2d(x_shape, w_shape)
        y = N.dims64([0, 0, 0, 0])
        N.call("osh_conv_infer_shape", C.byref(attrs), N.dims64(xs), N.dims64(ws), y)
        y = tuple(int(v) for v in y)
        if len(x_shape) == 3:
            n1 = self._length1d(x_shape[2], w_shape[2])
            return (y[0], y[1], y[3] if n1 is None else n1)
        return y

    def resolve(self, x_shape: Sequence[int], w_shape: Sequence[int]) -> N.ConvParams:
        """The launch parameters (for a rank-3 conv: of its 2-D form, h = 1)."""
        self.get_memory_shapes(x_shape, w_shape)
        attrs, xs, ws = self._shapes2d(x_shape, w_shape)
        p = N.ConvParams()
        N.call("osh_conv_resolve", C.byref(attrs), N.dims64(xs), N.dims64(ws), C.byref(p))
        n1 = self._length1d(xs[3], ws[3]) if self._attrs_1d else None
        if n1 is not None:  # every kernel reads the begin pad and bounds-checks the input
            p.ow, p.pr = n1, self._lists[2][1]
        return p

    # -- one-time weight packing (PrepackWeights)
    def prepack_weights(self, x_shape: Sequence[int], w: torch.Tensor):
        w = _need_f32("weight", w)
        p = self.resolve(x_shape, tuple(w.shape))
        nbytes = C.c_size_t()
        N.call("osh_conv_packed_weight_bytes", C.byref(p), C.byref(nbytes))
        buf = torch.empty(max(1, nbytes.value), dtype=torch.uint8, device=w.device)
        N.call("osh_conv_pack_weights", C.byref(p), _ptr(w), _ptr(buf), C.c_void_p(_stream()))
        self._release_pack()
        self._packed = ((w.data_ptr(), tuple(w.shape), tuple(x_shape), w._version), p, buf)
        return p, buf

    def _release_pack(self):
        """Drop the library's record of the packed buffer this layer is about
        to let go (torch may hand its memory to another tensor)."""
        if self._packed is not None:
            buf = self._packed[2]
            N.lib().osh_conv_forget_pack(_ptr(buf), buf.numel())
            self._packed = None

    def __del__(self):
        try:
            self._release_pack()
        except Exception:  # interpreter shutdown: nothing left to keep consistent
            pass

    def forward(self, x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """y = act(conv(x) + bias), plus `residual` (the shortcut operand of a
        following Add, same shape as y) when given: one launch for both.  A
        rank-3 x ([N, C, L], weights [M, C/g, K]) gives a rank-3 y."""
        x = _need_f32("input", x)
        if x.dim() == 3:
            out4 = None if out is None else out.unsqueeze(2)
            res4 = None if residual is None else residual.unsqueeze(2)
            return self.forward(x.unsqueeze(2), w.unsqueeze(2) if w.dim() == 3 else w, bias, out4, res4).squeeze(2)
        key = (w.data_ptr(), tuple(w.shape), tuple(x.shape), w._version)
        if self._packed is None or self._packed[0] != key:
            self.prepack_weights(tuple(x.shape), w)
        _, p, buf = self._packed
        y_shape = (p.n, p.m, p.oh, p.ow)
        if bias is not None:
            bias = _need_f32("bias", bias)
            if bias.numel() < p.m:
                raise N.OshError(N.OSH_E_INVALID, f"Conv '{self.name}': bias has {bias.numel()} values, {p.m} needed")
        if out is None:
            out = torch.empty(y_shape, dtype=torch.float32, device=x.device)
        elif tuple(out.shape) != y_shape or not out.is_contiguous():
            raise ValueError(f"Conv '{self.name}': output must be a contiguous {y_shape} tensor")
        if residual is not None:
            residual = _need_f32("residual", residual)
            if tuple(residual.shape) != y_shape:
                raise ValueError(f"Conv '{self.name}': residual must have the output shape {y_shape}")
            N.call("osh_conv2d_add_f32", C.byref(p), _ptr(x), _ptr(buf), _ptr(bias),
                   N.ACTIVATIONS[self.fused_activation], _ptr(residual), _ptr(out), C.c_void_p(_stream()))
            return out
        N.call("osh_conv2d_f32", C.byref(p), _ptr(x), _ptr(buf), _ptr(bias), N.ACTIVATIONS[self.fused_activation],
               _ptr(out), C.c_void_p(_stream()))
        return out


class MatMulLayer:
    """numpy-broadcast MatMul with an optional fused column bias (FusedBias)."""

    def __init__(self, fused_bias: Optional[torch.Tensor] = None, name: str = "matmul"):
        self.fused_bias = fused_bias
        self.name = name

    def get_memory_shapes(self, a_shape: Sequence[int], b_shape: Sequence[int]) -> tuple:
        y = N.dims64([0] * 8)
        ry = C.c_int()
        N.call("osh_matmul_infer_shape", N.dims64(a_shape), len(a_shape), N.dims64(b_shape), len(b_shape), y,
               C.byref(ry))
        return tuple(int(y[i]) for i in range(ry.value))

    def forward(self, a: torch.Tensor, b: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        a = _need_f32("A", a)
        b = _need_f32("B", b)
        y_shape = self.get_memory_shapes(tuple(a.shape), tuple(b.shape))
        bias = self.fused_bias
        if out is None:
            out = torch.empty(y_shape, dtype=torch.float32, device=a.device)
        a2 = a.reshape(1, -1) if a.dim() == 1 else a
        b2 = b.reshape(-1, 1) if b.dim() == 1 else b
        m, k = a2.shape[-2], a2.shape[-1]
        n = b2.shape[-1]
        if bias is not None:
            bias = _need_f32("bias", bias)
            if bias.numel() != n:
                raise N.OshError(N.OSH_E_INVALID, f"MatMul '{self.name}': fused bias has {bias.numel()} values, {n} needed")
        stream = C.c_void_p(_stream())
        if b2.dim() == 2:
            # all batch rows share B: one GEMM over batch*m rows (DnnOps.cs:2975-3034)
            rows = a2.numel() // k
            N.call("osh_gemm_f32", rows, n, k, _ptr(a2), k, _ptr(b2), n, _ptr(bias), None, None, N.ACT_NONE,
                   _ptr(out), n, stream)
            return out
        # general broadcast: expand batch dims, one strided batched GEMM
        batch_shape = y_shape[:-2] if (a.dim() > 1 and b.dim() > 1) else y_shape[:-1]
        ab = a2.expand(*batch_shape, m, k) if a2.dim() > 2 or batch_shape else a2
        bb = b2.expand(*batch_shape, k, n)
        ab = ab.reshape(-1, m, k)
        bb = bb.reshape(-1, k, n)
        sa = ab.stride(0) if ab.shape[0] > 1 else 0
        sb = bb.stride(0) if bb.shape[0] > 1 else 0
        if ab.stride(1) != k or ab.stride(2) != 1:
            ab = ab.contiguous()
            sa = m * k
        if bb.stride(1) != n or bb.stride(2) != 1:
            bb = bb.contiguous()
            sb = k * n
        batch = max(ab.shape[0], bb.shape[0])
        N.call("osh_gemm_f32_batched", batch, m, n, k, _ptr(ab), k, sa, _ptr(bb), n, sb, _ptr(bias), N.ACT_NONE,
               _ptr(out), n, m * n, stream)
        return out


class GemmLayer:
    """ONNX Gemm: Y = alpha * A' B' + beta * C on 2-D A and B."""

    def __init__(self, alpha: float = 1.0, beta: float = 1.0, transA: int = 0, transB: int = 0,
                 name: str = "gemm"):
        self.alpha = float(alpha)
        self.beta = float(beta)
        self.trans_a = bool(transA)
        self.trans_b = bool(transB)
        self.name = name

    def resolve(self, a_shape: Sequence[int], b_shape: Sequence[int]):
        """(m, k, n) as GemmLayer.Resolve (AttnOps.cs:48-66)."""
        if len(a_shape) != 2 or len(b_shape) != 2:
            raise N.OshError(N.OSH_E_INVALID, f"Gemm '{self.name}': only 2-D A/B are supported")
        m = a_shape[1] if self.trans_a else a_shape[0]
        k = a_shape[0] if self.trans_a else a_shape[1]
        n = b_shape[0] if self.trans_b else b_shape[1]
        bk = b_shape[1] if self.trans_b else b_shape[0]
        if bk != k:
            raise N.OshError(N.OSH_E_INVALID, f"Gemm '{self.name}': K mismatch ({list(a_shape)} / {list(b_shape)})")
        return m, k, n

    def get_memory_shapes(self, a_shape: Sequence[int], b_shape: Sequence[int]) -> tuple:
        m, _, n = self.resolve(a_shape, b_shape)
        return (m, n)

    def forward(self, a: torch.Tensor, b: torch.Tensor, c: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
        a = _need_f32("A", a)
        b = _need_f32("B", b)
        m, k, n = self.resolve(tuple(a.shape), tuple(b.shape))
        if c is not None:
            c = _need_f32("C", c)
            if c.numel() == 0:
                c = None
        if out is None:
            out = torch.empty((m, n), dtype=torch.float32, device=a.device)
        nbytes = C.c_size_t()
        N.call("osh_gemm_ex_workspace_bytes", int(self.trans_a), int(self.trans_b), m, n, k, C.byref(nbytes))
        ws = torch.empty(max(1, nbytes.value // 4), dtype=torch.float32, device=a.device) if nbytes.value else None
        N.call("osh_gemm_ex_f32", int(self.trans_a), int(self.trans_b), m, n, k, C.c_float(self.alpha), _ptr(a),
               _ptr(b), C.c_float(self.beta), _ptr(c), 0 if c is None else c.numel(), _ptr(out), _ptr(ws),
               C.c_void_p(_stream()))
        return out


class DynamicQuantizeMatMulLayer:
    """DynamicQuantizeMatMul with inputs [A, W, w_zero_point, w_scale, bias] (the reference's order)."""

    def __init__(self, name: str = "dqmm"):
        self.name = name
        self._packed = None
        self._scratch = None

    @staticmethod
    def get_memory_shapes(a_shape: Sequence[int], w_shape: Sequence[int]) -> tuple:
        if len(w_shape) != 2:
            raise N.OshError(N.OSH_E_INVALID, f"DynamicQuantizeMatMul: weight must be 2-D, got {tuple(w_shape)}")
        if a_shape[-1] != w_shape[0]:
            raise N.OshError(N.OSH_E_INVALID, f"DynamicQuantizeMatMul: K mismatch ({tuple(a_shape)} x {tuple(w_shape)})")
        return tuple(a_shape[:-1]) + (int(w_shape[1]),)

    def prepack_weights(self, w: torch.Tensor, w_zero_point=None):
        if w.dtype not in (torch.int8, torch.uint8) or w.dim() != 2 or not w.is_cuda:
            raise N.OshError(N.OSH_E_INVALID, "DynamicQuantizeMatMul: W must be a 2-D int8/uint8 device tensor")
        w = w.contiguous()
        k, n = w.shape
        zps = [] if w_zero_point is None else [int(v) for v in torch.as_tensor(w_zero_point).reshape(-1).tolist()]
        zarr = (C.c_int32 * max(1, len(zps)))(*zps)
        nbytes = C.c_size_t()
        N.call("osh_dqmm_packed_weight_bytes", k, n, C.byref(nbytes))
        buf = torch.empty(nbytes.value, dtype=torch.uint8, device=w.device)
        N.call("osh_dqmm_pack_weights", k, n, _ptr(w), 1 if w.dtype == torch.int8 else 0, zarr, len(zps), _ptr(buf),
               C.c_void_p(_stream()))
        self._packed = ((w.data_ptr(), tuple(w.shape), w._version, tuple(zps)), buf)
        return buf

    def forward(self, a: torch.Tensor, w: torch.Tensor, w_zero_point=None, w_scale: Optional[torch.Tensor] = None,
                bias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                acc_out: Optional[torch.Tensor] = None, qparams_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        a = _need_f32("A", a)
        y_shape = self.get_memory_shapes(tuple(a.shape), tuple(w.shape))
        k, n = w.shape
        m = a.numel() // k
        zps = () if w_zero_point is None else tuple(int(v) for v in torch.as_tensor(w_zero_point).reshape(-1).tolist())
        key = (w.data_ptr(), tuple(w.shape), w._version, zps)
        if self._packed is None or self._packed[0] != key:
            self.prepack_weights(w, w_zero_point)
        wbuf = self._packed[1]
        if w_scale is None:
            w_scale = torch.ones(1, dtype=torch.float32, device=a.device)
        w_scale = _need_f32("w_scale", w_scale)
        if bias is not None:
            bias = _need_f32("bias", bias)
        sbytes = C.c_size_t()
        N.call("osh_dqmm_scratch_bytes", m, k, C.byref(sbytes))
        if self._scratch is None or self._scratch.numel() < sbytes.value:
            self._scratch = torch.empty(sbytes.value, dtype=torch.uint8, device=a.device)
        if out is None:
            out = torch.empty(y_shape, dtype=torch.float32, device=a.device)
        N.call("osh_dqmm_u8s8", m, k, n, _ptr(a), _ptr(wbuf), _ptr(w_scale), w_scale.numel(), _ptr(bias), _ptr(out),
               _ptr(acc_out), _ptr(qparams_out), _ptr(self._scratch), C.c_void_p(_stream()))
        return out


class DynamicQuantizeLinearLayer:
    """DynamicQuantizeLinear: (q u8, scale, zero point)."""

    def __init__(self, name: str = "dql"):
        self.name = name
        self._scratch = None

    def forward(self, x: torch.Tensor):
        x = _need_f32("x", x)
        sbytes = C.c_size_t()
        N.call("osh_dqmm_scratch_bytes", 0, 1, C.byref(sbytes))
        if self._scratch is None or self._scratch.numel() < sbytes.value:
            self._scratch = torch.empty(sbytes.value, dtype=torch.uint8, device=x.device)
        q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
        qp = torch.empty(2, dtype=torch.int32, device=x.device)
        N.call("osh_dynamic_quantize_linear", x.numel(), _ptr(x), _ptr(q), _ptr(qp), _ptr(self._scratch),
               C.c_void_p(_stream()))
        qh = qp.cpu()
        scale = qh[0:1].view(torch.float32).item()
        return q, scale, int(qh[1].item())


class MatMulIntegerLayer:
    """MatMulInteger: int32 C = (A - a_zero_point) x (B - b_zero_point[col]),
    A u8/s8 [M,K] (or [1,M,K]), B u8/s8 [K,N] (or [1,K,N]); B is packed once per
    (tensor, zero points) like the reference's constant-weight cache."""

    def __init__(self, name: str = "matmulinteger"):
        self.name = name
        self._packed = None

    def resolve(self, a_shape: Sequence[int], b_shape: Sequence[int]):
        """(m, k, n, batched) as MatMulIntegerLayer.Resolve (QuantOps.cs:255-272)."""
        ar = 2 if (len(a_shape) == 3 and a_shape[0] == 1) else len(a_shape)
        br = 2 if (len(b_shape) == 3 and b_shape[0] == 1) else len(b_shape)
        if ar != 2 or br != 2:
            raise N.OshError(N.OSH_E_INVALID,
                             f"MatMulInteger: only 2-D (or batch=1 3-D) is supported, got {list(a_shape)} x {list(b_shape)}")
        m, k, n = a_shape[-2], a_shape[-1], b_shape[-1]
        if b_shape[-2] != k:
            raise N.OshError(N.OSH_E_INVALID, f"MatMulInteger: K mismatch ({list(a_shape)} x {list(b_shape)})")
        return m, k, n, len(a_shape) == 3 or len(b_shape) == 3

    def forward(self, a: torch.Tensor, b: torch.Tensor, a_zero_point=None, b_zero_point=None) -> torch.Tensor:
        if a.dtype not in (torch.uint8, torch.int8) or b.dtype not in (torch.uint8, torch.int8):
            raise TypeError("MatMulInteger takes uint8/int8 tensors")
        m, k, n, batched = self.resolve(tuple(a.shape), tuple(b.shape))
        a_zp = 0 if a_zero_point is None or len(list(a_zero_point)) == 0 else int(list(a_zero_point)[0])
        zps = [0] if b_zero_point is None or len(list(b_zero_point)) == 0 else [int(v) for v in b_zero_point]
        key = (b.data_ptr(), tuple(b.shape), b.dtype, tuple(zps), getattr(b, "_version", 0))
        if self._packed is None or self._packed[0] != key:
            nbytes = C.c_size_t()
            N.call("osh_dqmm_packed_weight_bytes", k, n, C.byref(nbytes))
            buf = torch.empty(nbytes.value, dtype=torch.uint8, device=b.device)
            z = (C.c_int32 * len(zps))(*zps)
            bb = b.reshape(k, n).contiguous()
            N.call("osh_dqmm_pack_weights", k, n, _ptr(bb), 1 if b.dtype == torch.int8 else 0, z, len(zps),
                   _ptr(buf), C.c_void_p(_stream()))
            self._packed = (key, buf)
        sbytes = C.c_size_t()
        N.call("osh_dqmm_scratch_bytes", m, k, C.byref(sbytes))
        scratch = torch.empty(sbytes.value, dtype=torch.uint8, device=a.device)
        out = torch.empty((1, m, n) if batched else (m, n), dtype=torch.int32, device=a.device)
        aa = a.reshape(m, k).contiguous()
        N.call("osh_matmul_integer", m, k, n, _ptr(aa), 1 if a.dtype == torch.int8 else 0, a_zp,
               _ptr(self._packed[1]), _ptr(out), _ptr(scratch), C.c_void_p(_stream()))
        return out


class ActivationLayer:
    """Standalone Relu / Silu / Sigmoid (ActivationLayer with its UnaryOpKind,
    src/OnnxSharp/Ops/ActivationLayer.cs; vector-path arithmetic of
    VectorMath.Silu / Sigmoid)."""

    KINDS = {"Relu": N.ACT_RELU, "Silu": N.ACT_SILU, "Sigmoid": N.ACT_SIGMOID}

    def __init__(self, kind: str, name: str = "activation"):
        if kind not in self.KINDS:
            raise ValueError(f"activation '{name}': unknown kind {kind!r}")
        self.kind = kind
        self.name = name

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        x = _need_f32("input", x)
        if out is None:
            out = torch.empty_like(x)
        elif out.shape != x.shape or not out.is_contiguous():
            raise ValueError(f"activation '{self.name}': output must be a contiguous {tuple(x.shape)} tensor")
        N.call("osh_activation_f32", x.numel(), _ptr(x), self.KINDS[self.kind], _ptr(out), C.c_void_p(_stream()))
        return out


class DflSoftmaxLayer:
    """The fused DFL decode of a YOLO Detect head (DflLayer, registered as
    "DflSoftmax", src/OnnxSharp/Ops/DflOps.cs:31-240): input [B, sides*bins, N]
    -> output [B, sides, N], the softmax over each side's bins weighted by the
    bin index."""

    def __init__(self, bins: int = 16, name: str = "dfl"):
        self.bins = int(bins)
        self.name = name

    def get_memory_shapes(self, x_shape: Sequence[int]) -> tuple:
        # DflLayer.Resolve (DflOps.cs:48-60)
        if len(x_shape) != 3:
            raise N.OshError(N.OSH_E_INVALID,
                             f"DflSoftmax '{self.name}': input must be [B, sides*bins, N], got {tuple(x_shape)}")
        if self.bins < 2 or x_shape[1] % self.bins != 0:
            raise N.OshError(N.OSH_E_INVALID,
                             f"DflSoftmax '{self.name}': {x_shape[1]} channels not divisible by bins={self.bins}")
        return (int(x_shape[0]), int(x_shape[1]) // self.bins, int(x_shape[2]))

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        x = _need_f32("input", x)
        b, sides, n = self.get_memory_shapes(tuple(x.shape))
        if out is None:
            out = torch.empty((b, sides, n), dtype=torch.float32, device=x.device)
        elif tuple(out.shape) != (b, sides, n) or not out.is_contiguous():
            raise ValueError(f"DflSoftmax '{self.name}': output must be a contiguous {(b, sides, n)} tensor")
        if b and sides and n:
            N.call("osh_dfl_f32", b, sides, self.bins, n, _ptr(x), sides * self.bins * n, _ptr(out), sides * n,
                   C.c_void_p(_stream()))
        return out
