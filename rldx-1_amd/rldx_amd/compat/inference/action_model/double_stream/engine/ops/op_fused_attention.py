"""ds::fused_attention_2way, registered by rldx_amd, under the name the reference module
rldx/inference/action_model/double_stream/engine/ops/op_fused_attention.py
gives it (`fused_attention`)."""

from rldx_amd import ops as _ops

fused_attention = _ops.ds_fused_attention_2way

__all__ = ["fused_attention"]
