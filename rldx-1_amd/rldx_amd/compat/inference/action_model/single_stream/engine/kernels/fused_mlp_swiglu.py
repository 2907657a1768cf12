"""fused_mlp_swiglu of rldx/inference/action_model/single_stream/engine/kernels/
fused_mlp_swiglu.py:199-267 (GEMM + bias + SwiGLU, optional split-K), on the
grouped GEMM's SwiGLU epilogue."""

import torch

from rldx_amd import ops as _ops  # noqa: F401  (registers ss::fused_mlp_swiglu)

__all__ = ["fused_mlp_swiglu"]


def fused_mlp_swiglu(x, weight, bias, split_k=1):
    """silu(x W_gate^T + b_gate) * (x W_up^T + b_up) with weight = [W_gate; W_up]
    (2 N_half, K): (M, N_half) bf16.  The weight is packed once per tensor."""
    return torch.ops.ss.fused_mlp_swiglu(x, weight, bias, split_k)
