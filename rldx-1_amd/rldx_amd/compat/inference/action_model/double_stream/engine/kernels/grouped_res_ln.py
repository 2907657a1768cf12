"""fused_grouped_res_ln of rldx/inference/action_model/double_stream/engine/kernels/
grouped_res_ln.py:150-211 (SA and VL residual + proj + bias, then LayerNorm, one
launch), on rldx_grouped_res_ln_bf16."""

from rldx_amd.functional import fused_grouped_res_ln

__all__ = ["fused_grouped_res_ln"]
