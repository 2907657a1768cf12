"""ss::fused_mlp_swiglu, registered by rldx_amd, under the name the reference module
rldx/inference/action_model/single_stream/engine/ops/op_fused_mlp_swiglu.py
gives it (`fused_mlp_swiglu`)."""

from rldx_amd import ops as _ops

fused_mlp_swiglu = _ops.ss_fused_mlp_swiglu

__all__ = ["fused_mlp_swiglu"]
