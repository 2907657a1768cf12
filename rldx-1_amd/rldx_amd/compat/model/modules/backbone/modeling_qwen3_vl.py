"""Mirror of the rotary helpers of rldx/model/modules/backbone/
modeling_qwen3_vl.py on the rldx_amd kernels: rotate_half (:118-122) and
apply_rotary_pos_emb (:377-401, rotate-half RoPE through
rldx_qk_rmsnorm_rope_half_* with RLDX_ROPE_NO_NORM).  CUDA tensors only."""

from __future__ import annotations

import torch

from rldx_amd import functional as Fn

__all__ = ["rotate_half", "apply_rotary_pos_emb"]


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """cat(-x[..., D/2:], x[..., :D/2]) (a tensor view helper, as in the reference)."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin, position_ids=None, unsqueeze_dim=1):
    """q * cos + rotate_half(q) * sin (and k), in the input type with eager
    rounding.  unsqueeze_dim 1: q, k [B, H, S, D] and cos, sin [B, S, D];
    unsqueeze_dim 2: q, k [B, S, H, D].  position_ids is unused (deprecated
    there too)."""
    Fn._require(unsqueeze_dim in (1, 2), "unsqueeze_dim must be 1 ([B, H, S, D]) or 2 ([B, S, H, D])")
    Fn._require(cos.dim() in (2, 3), "cos and sin must be [S, D] or [B, S, D]")
    if unsqueeze_dim == 1:  # the kernel takes [B, S, H, D] strides: transposed views, no copy
        qo, ko = torch.empty_like(q), torch.empty_like(k)
        Fn.rope_half(q.transpose(1, 2), k.transpose(1, 2), cos, sin, q_out=qo.transpose(1, 2),
                     k_out=ko.transpose(1, 2))
        return qo, ko
    return Fn.rope_half(q, k, cos, sin)
