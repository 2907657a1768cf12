"""rldx_backbone::vision_attention, registered by rldx_amd, under the name the reference module
rldx/inference/backbone/vision_encoder/engine/ops/op_fused_vision_attention.py
gives it (`vision_attention`)."""

from rldx_amd import ops as _ops

vision_attention = _ops.rldx_backbone_vision_attention

__all__ = ["vision_attention"]
