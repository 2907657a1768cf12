"""Registers the operators of rldx/inference/action_model/single_stream/engine/ops/ (importing this package
registers them all, as the reference's does), backed by rldx_amd:
  ss::fused_attention_2way
  ss::fused_attention_3way
  ss::fused_epilogue_ln
  ss::fused_mlp_swiglu
"""

from rldx_amd import ops as _ops  # noqa: F401  (the registrations)
