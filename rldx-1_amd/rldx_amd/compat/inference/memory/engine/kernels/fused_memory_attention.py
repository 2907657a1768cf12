"""The launcher module of rldx/inference/memory/engine/kernels/
fused_memory_attention.py on the gfx950 block-causal attention: `forward`
(:228-264) and the set-up helpers (:186-225)."""

import torch

from rldx_amd import functional as Fn
from rldx_amd.compat.inference.backbone.llm.engine.kernels.fused_llm_attention import prepare_signed_sin

__all__ = ["forward", "prepare_fused_qkv_weight", "prepare_signed_sin", "prepare_rope_buffers"]


def prepare_fused_qkv_weight(layer):
    """[q_proj; k_proj; v_proj] weights of a memory layer's self_attn as one matrix."""
    attn = layer.self_attn
    return torch.cat([attn.q_proj.weight.data, attn.k_proj.weight.data, attn.v_proj.weight.data]).contiguous()


def prepare_rope_buffers(rotary_emb, position_ids, device, dtype=torch.bfloat16):
    """cos (M, D) and signed sin (M, D) in `dtype` from a rotary-embedding module
    called as rotary_emb(x, position_ids) with position_ids (1, M)."""
    D = rotary_emb.dim
    probe = torch.empty(1, 1, 1, D, device=device, dtype=dtype)
    cos, sin = rotary_emb(probe, position_ids)
    return cos[0].contiguous(), prepare_signed_sin(sin[0], D)


def forward(qkv, cos, signed_sin, num_heads, head_dim, block_attn_size):
    """bf16 RoPE on Q/K + block-causal attention: qkv (M, 3 H D) bf16 -> (M, H D) bf16."""
    return Fn.memory_attention(qkv, cos, signed_sin, num_heads, head_dim, block_attn_size)
