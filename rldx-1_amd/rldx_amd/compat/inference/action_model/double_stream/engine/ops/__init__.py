"""Registers the operators of rldx/inference/action_model/double_stream/engine/ops/ (importing this package
registers them all, as the reference's does), backed by rldx_amd:
  ds::fused_attention_2way
  ds::fused_attention_3way
  ds::vl_epilogue_ln
  ds::grouped_swiglu
  ds::grouped_res_ln
"""

from rldx_amd import ops as _ops  # noqa: F401  (the registrations)
