"""mem::fused_attention, registered by rldx_amd, under the name the reference module
rldx/inference/memory/engine/ops/op_fused_memory_attention.py
gives it (`fused_memory_attention`)."""

from rldx_amd import ops as _ops

fused_memory_attention = _ops.mem_fused_attention

__all__ = ["fused_memory_attention"]
