"""`forward` of rldx/inference/backbone/llm/engine/kernels/fused_add3_rmsnorm.py:86-117
(bf16 residual adds, then the Qwen3-VL RMSNorm; returns (new_hidden, normed)),
on rldx_add_rmsnorm_bf16."""

from rldx_amd import functional as Fn

__all__ = ["forward"]


def forward(hidden, residual, deepstack, weight):
    return Fn.fused_add3_rmsnorm(hidden, residual, deepstack, weight)
