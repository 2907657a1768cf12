"""Mirror of rldx/model/modules/norms.py on the rldx_amd kernels: RMSNorm
(:7-22) through rldx_rms_norm_*, the no-affine LayerNorm of
create_norm_layer / create_qk_norm_layers (:25-63) through the add + LayerNorm
row kernel.  Same constructors, parameters (`weight`, `eps`) and factory
signatures; CUDA tensors only (no CPU path)."""

from __future__ import annotations

import torch
import torch.nn as nn

from rldx_amd import functional as Fn

__all__ = ["RMSNorm", "LayerNorm", "create_norm_layer", "create_qk_norm_layers"]


class RMSNorm(nn.Module):
    """y = (weight * (x * rsqrt(mean(x^2) + eps))).to(x.dtype), fp32 arithmetic,
    one rounding (rldx_rms_norm_bf16 / _f32)."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return Fn.rms_norm(x, self.weight.detach(), self.eps)


class LayerNorm(nn.Module):
    """nn.LayerNorm(dim, elementwise_affine=False, eps) on bf16 rows: mean and
    biased variance in fp32, one rounding (rldx_ss_epilogue_ln_bf16 without a
    residual)."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.normalized_shape = (dim,)
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        Fn._require(x.dtype == torch.bfloat16, "LayerNorm: the rldx_amd kernel takes bfloat16 rows")
        Fn._require(x.shape[-1] == self.normalized_shape[0], "LayerNorm: last dimension mismatch")
        rows = x.reshape(-1, x.shape[-1])
        return Fn.fused_ss_epilogue_ln(rows, eps=self.eps)[1].reshape(x.shape)


def create_norm_layer(norm_type: str, dim: int, eps: float = 1e-6) -> nn.Module:
    """"none", "layer_norm" or "rms_norm" (norms.py:25-41)."""
    if norm_type == "none":
        return nn.Identity()
    if norm_type == "layer_norm":
        return LayerNorm(dim, eps=eps)
    if norm_type == "rms_norm":
        return RMSNorm(dim, eps=eps)
    raise ValueError(f"Unknown norm_type: {norm_type}")


def create_qk_norm_layers(qk_norm: str, head_dim: int, eps: float = 1e-6):
    """(q_norm, k_norm) pair (norms.py:44-63)."""
    if qk_norm == "none":
        return nn.Identity(), nn.Identity()
    if qk_norm in ("layer_norm", "rms_norm"):
        return create_norm_layer(qk_norm, head_dim, eps), create_norm_layer(qk_norm, head_dim, eps)
    raise ValueError(f"Unknown qk_norm: {qk_norm}")
