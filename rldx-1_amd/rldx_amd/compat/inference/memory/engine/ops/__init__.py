"""Registers the operators of rldx/inference/memory/engine/ops/ (importing this package
registers them all, as the reference's does), backed by rldx_amd:
  mem::fused_attention
  mem::fused_epilogue_add2_rmsnorm
"""

from rldx_amd import ops as _ops  # noqa: F401  (the registrations)
