"""ds::fused_attention_3way, registered by rldx_amd, under the name the reference module
rldx/inference/action_model/double_stream/engine/ops/op_fused_attention_3way.py
gives it (`fused_attention_3way`)."""

from rldx_amd import ops as _ops

fused_attention_3way = _ops.ds_fused_attention_3way

__all__ = ["fused_attention_3way"]
