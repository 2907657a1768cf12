"""rldx_backbone::fused_epilogue_add2_rmsnorm, registered by rldx_amd, under the name the reference module
rldx/inference/backbone/llm/engine/ops/op_fused_epilogue_add2_rmsnorm.py
gives it (`fused_epilogue_add2_rmsnorm`)."""

from rldx_amd import ops as _ops

fused_epilogue_add2_rmsnorm = _ops.rldx_backbone_fused_epilogue_add2_rmsnorm

__all__ = ["fused_epilogue_add2_rmsnorm"]
