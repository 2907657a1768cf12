"""fused_ss_epilogue_ln of rldx/inference/action_model/single_stream/engine/kernels/
ss_epilogue_ln.py:146-205 (optional residual add, then LayerNorm; static buffers
honoured), on rldx_ss_epilogue_ln_bf16."""

from rldx_amd.functional import fused_ss_epilogue_ln

__all__ = ["fused_ss_epilogue_ln"]
