"""onnxsharp_amd -- MI355X (gfx950) backend for OnnxSharp's dense-contraction path.

Conv (+ fused Relu/SiLU), MatMul with a fused column bias and the int8
DynamicQuantizeMatMul run as hand-written HIP kernels in libosh_hip.so behind
the C ABI of include/osh_hip.h; `layers` mirrors the reference operators over
that ABI.
"""
from . import native  # noqa: F401

__all__ = ["native", "layers", "synth"]
