"""`forward` of rldx/inference/memory/engine/kernels/fused_add2_rmsnorm.py (the
reference re-exports the backbone kernel's launcher), on rldx_add_rmsnorm_bf16."""

from rldx_amd import functional as Fn

__all__ = ["forward"]


def forward(hidden, residual, weight):
    return Fn.fused_add2_rmsnorm(hidden, residual, weight)
