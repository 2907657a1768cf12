"""The launcher module of rldx/inference/backbone/llm/engine/kernels/
fused_llm_attention.py on the gfx950 GQA prefill kernels: `forward`
(:1005-1057), the set-up helpers `prepare_fused_qkv_weight`,
`prepare_signed_sin`, `prepare_norm_weight_rot` (:778-804) and
`autotune_split_m_threshold` (:928-1002)."""

import torch

from rldx_amd import ops as _ops
from rldx_amd import workloads as _W

__all__ = ["forward", "prepare_fused_qkv_weight", "prepare_signed_sin", "prepare_norm_weight_rot",
           "autotune_split_m_threshold", "SPLIT_M_THRESHOLD", "THRESHOLD_CANDIDATES"]

# The reference switches between a direct and a split-KV kernel at this many
# query rows.  The rldx_amd path has one kernel for every M (no split-KV
# workspace, no reduce launch), so the threshold only exists for callers that
# read or tune it.
SPLIT_M_THRESHOLD = 128
THRESHOLD_CANDIDATES = (64, 128, 256, 512)


def forward(qkv, q_norm_w, q_norm_w_rot, k_norm_w, k_norm_w_rot, cos, signed_sin, num_heads=32, num_kv_heads=8,
            head_dim=128, out=None):
    """QK-RMSNorm + rotate-half RoPE + causal GQA attention: qkv (M, (Hq + 2 Hkv) D)
    bf16 -> (M, Hq D) bf16 (into `out` when given)."""
    return _ops.llm_fused_attention(qkv, q_norm_w, q_norm_w_rot, k_norm_w, k_norm_w_rot, cos, signed_sin,
                                    num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim, out=out)


def prepare_fused_qkv_weight(layer):
    """[q_proj; k_proj; v_proj] weights of a decoder layer (or its self_attn) as one (QKV_DIM, hidden) matrix."""
    attn = getattr(layer, "self_attn", layer)
    return torch.cat([attn.q_proj.weight.data, attn.k_proj.weight.data, attn.v_proj.weight.data]).contiguous()


def prepare_signed_sin(sin, head_dim):
    """sin (M, D) with rotate_half's sign folded in: columns [0, D/2) negated, [D/2, D) kept."""
    if sin.shape[-1] != head_dim:
        raise ValueError(f"sin has {sin.shape[-1]} columns, head_dim is {head_dim}")
    return _W.signed_sin(sin)


def prepare_norm_weight_rot(norm_weight, head_dim):
    """The norm weight with its halves swapped (w_rot[d] = w[(d + D/2) mod D]).  The
    rldx_amd kernels read the rotate-half partner's own weight, so `forward`
    accepts it only for signature compatibility."""
    if norm_weight.shape[0] != head_dim:
        raise ValueError(f"norm weight has {norm_weight.shape[0]} entries, head_dim is {head_dim}")
    return _W.norm_weight_rot(norm_weight)


def autotune_split_m_threshold(workloads, candidates=THRESHOLD_CANDIDATES, warmup=3, iters=10):
    """Nothing to tune: one kernel serves every M.  Returns SPLIT_M_THRESHOLD."""
    return SPLIT_M_THRESHOLD
