"""fused_vl_epilogue_ln of rldx/inference/action_model/double_stream/engine/kernels/
vl_epilogue_ln.py:134-183 (VL residual + both biases + w3 output, then LayerNorm;
static `new_vl_out` / `ln_vl_out` buffers honoured), on rldx_vl_epilogue_ln_bf16."""

from rldx_amd.functional import fused_vl_epilogue_ln

__all__ = ["fused_vl_epilogue_ln"]
