"""Registers the operators of rldx/inference/backbone/llm/engine/ops/ (importing this package
registers them all, as the reference's does), backed by rldx_amd:
  rldx_backbone::fused_attention
  rldx_backbone::fused_epilogue_add2_rmsnorm
  rldx_backbone::fused_epilogue_add3_rmsnorm
"""

from rldx_amd import ops as _ops  # noqa: F401  (the registrations)
