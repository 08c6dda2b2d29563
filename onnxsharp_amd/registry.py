"""Which operators the HIP backend takes: the host side of the emitter
registry, mirroring OnnxSharp's Vulkan registry (VkOpRegistry.Register /
CanEmit, src/OnnxSharp.Vulkan/VkOpRegistry.cs:19-36,120-180).

A partition planner asks `can_emit(op_type, fused_activation, fused_bias)`
before it puts a node in a GPU segment; a False keeps the node on the CPU.
Like the reference registry:
* an operator whose fused activation its emitter does not apply is refused
  (a fused Silu left out computes wrong numbers with the right shapes,
  VkOpRegistry.cs:168-180);
* ONNXSHARP_HIP_NOEMIT=conv,matmul,dqmm (comma-separated emitter keys, the
  counterpart of ONNXSHARP_VK_NOEMIT, VkOpRegistry.cs:154-161) drops the
  named emitters, so a wrong result can be narrowed to one operator by
  turning emitters off one at a time.
A MatMul with a fused bias is taken: the MatMul emitter passes
IBiasAddable.FusedBias as the column bias (src/OnnxSharp/Core/LayerInfo.cs:174-178).
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Optional


@dataclass(frozen=True)
class Emitter:
    key: str                      # the ONNXSHARP_HIP_NOEMIT name
    activations: frozenset        # fused activations the launch applies
    takes_fused_bias: bool = False


# operator type -> its emitter (the layers in layers.py run them)
EMITTERS = {
    "Conv": Emitter("conv", frozenset({"Relu", "Silu"})),
    "MatMul": Emitter("matmul", frozenset(), takes_fused_bias=True),
    "Gemm": Emitter("gemm", frozenset()),
    "DynamicQuantizeMatMul": Emitter("dqmm", frozenset()),
    "DynamicQuantizeLinear": Emitter("dql", frozenset()),
    "MatMulInteger": Emitter("matmulinteger", frozenset()),
}


def disabled(env: Optional[str] = None) -> frozenset:
    """Emitter keys named in ONNXSHARP_HIP_NOEMIT (or in `env` when given)."""
    raw = os.environ.get("ONNXSHARP_HIP_NOEMIT", "") if env is None else env
    return frozenset(p.strip().lower() for p in raw.split(",") if p.strip())


def can_emit(op_type: str, fused_activation: Optional[str] = None, fused_bias: bool = False,
             env: Optional[str] = None) -> bool:
    """Whether the backend takes a node of `op_type` with this fused
    activation (None for none) and, for MatMul, a fused bias."""
    e = EMITTERS.get(op_type)
    if e is None or e.key in disabled(env):
        return False
    if fused_activation is not None and fused_activation not in e.activations:
        return False
    if fused_bias and not e.takes_fused_bias:
        return False
    return True
