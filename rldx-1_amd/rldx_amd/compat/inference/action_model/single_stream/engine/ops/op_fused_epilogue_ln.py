"""ss::fused_epilogue_ln, registered by rldx_amd, under the name the reference module
rldx/inference/action_model/single_stream/engine/ops/op_fused_epilogue_ln.py
gives it (`fused_epilogue_ln`)."""

from rldx_amd import ops as _ops

fused_epilogue_ln = _ops.ss_fused_epilogue_ln

__all__ = ["fused_epilogue_ln"]
