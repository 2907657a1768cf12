"""`forward` of rldx/inference/backbone/llm/engine/kernels/fused_add2_rmsnorm.py:85-115
(bf16 residual adds, then the Qwen3-VL RMSNorm; returns (new_hidden, normed)),
on rldx_add_rmsnorm_bf16."""

from rldx_amd import functional as Fn

__all__ = ["forward"]


def forward(hidden, residual, weight):
    return Fn.fused_add2_rmsnorm(hidden, residual, weight)
