"""Registers the operators of rldx/inference/backbone/vision_encoder/engine/ops/ (importing this package
registers them all, as the reference's does), backed by rldx_amd:
  rldx_backbone::vision_attention
"""

from rldx_amd import ops as _ops  # noqa: F401  (the registrations)
