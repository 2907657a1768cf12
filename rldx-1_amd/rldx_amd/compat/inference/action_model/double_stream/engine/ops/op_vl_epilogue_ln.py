"""ds::vl_epilogue_ln, registered by rldx_amd, under the name the reference module
rldx/inference/action_model/double_stream/engine/ops/op_vl_epilogue_ln.py
gives it (`vl_epilogue_ln`)."""

from rldx_amd import ops as _ops

vl_epilogue_ln = _ops.ds_vl_epilogue_ln

__all__ = ["vl_epilogue_ln"]
