"""ds::grouped_swiglu, registered by rldx_amd, under the name the reference module
rldx/inference/action_model/double_stream/engine/ops/op_grouped_swiglu.py
gives it (`grouped_swiglu`)."""

from rldx_amd import ops as _ops

grouped_swiglu = _ops.ds_grouped_swiglu

__all__ = ["grouped_swiglu"]
