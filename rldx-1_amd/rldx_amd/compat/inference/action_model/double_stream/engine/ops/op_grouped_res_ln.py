"""ds::grouped_res_ln, registered by rldx_amd, under the name the reference module
rldx/inference/action_model/double_stream/engine/ops/op_grouped_res_ln.py
gives it (`grouped_res_ln`)."""

from rldx_amd import ops as _ops

grouped_res_ln = _ops.ds_grouped_res_ln

__all__ = ["grouped_res_ln"]
