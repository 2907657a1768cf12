"""rldx_backbone::fused_attention, registered by rldx_amd, under the name the reference module
rldx/inference/backbone/llm/engine/ops/op_fused_llm_attention.py
gives it (`fused_llm_attention`)."""

from rldx_amd import ops as _ops

fused_llm_attention = _ops.rldx_backbone_fused_attention

__all__ = ["fused_llm_attention"]
