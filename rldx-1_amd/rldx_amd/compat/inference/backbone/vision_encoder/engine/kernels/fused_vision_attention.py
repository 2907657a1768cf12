"""The launcher module of rldx/inference/backbone/vision_encoder/engine/kernels/
fused_vision_attention.py on the gfx950 varlen attention: `forward` (:622-645)
and `autotune_split_m_threshold` (:576-618)."""

from rldx_amd import functional as Fn

__all__ = ["forward", "autotune_split_m_threshold", "SPLIT_M_THRESHOLD", "THRESHOLD_CANDIDATES"]

# One kernel serves every M here (see fused_llm_attention); kept for callers that read or tune it.
SPLIT_M_THRESHOLD = 128
THRESHOLD_CANDIDATES = (64, 128, 256, 512)


def forward(qkv, rope_cos, rope_sin, cu_seqlens, scaling, num_heads, head_dim):
    """RoPE on Q/K (fp32 tables, sin's rotate-half sign baked in) + non-causal
    attention within each cu_seqlens segment: qkv (M, 3 H D) bf16 -> (M, H D) bf16."""
    return Fn.vision_attention(qkv, rope_cos.contiguous(), rope_sin.contiguous(), cu_seqlens, scaling, num_heads,
                               head_dim)


def autotune_split_m_threshold(workloads, candidates=THRESHOLD_CANDIDATES, warmup=3, iters=10):
    """Nothing to tune: one kernel serves every M.  Returns SPLIT_M_THRESHOLD."""
    return SPLIT_M_THRESHOLD
