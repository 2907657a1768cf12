"""`torch.library` operators under the reference's own qualified names.

Importing this module registers, backed by the gfx950 kernels of librldx_amd.so:

  ds::fused_attention_2way   ds::fused_attention_3way   ds::grouped_swiglu
  ds::grouped_res_ln         ds::vl_epilogue_ln
  ss::fused_attention_2way   ss::fused_attention_3way   ss::fused_mlp_swiglu
  ss::fused_epilogue_ln
  rldx_backbone::fused_attention   rldx_backbone::vision_attention   mem::fused_attention
  rldx_backbone::fused_epilogue_add2_rmsnorm   rldx_backbone::fused_epilogue_add3_rmsnorm
  mem::fused_epilogue_add2_rmsnorm
  rldx_amd::swiglu           (the eager `F.silu(x1) * x2` the chains inline)

Argument order and defaults follow the reference registrations
(rldx/inference/action_model/{double,single}_stream/engine/ops/*.py,
rldx/inference/backbone/llm/engine/ops/op_fused_llm_attention.py,
rldx/inference/backbone/vision_encoder/engine/ops/op_fused_vision_attention.py,
rldx/inference/memory/engine/ops/op_fused_memory_attention.py,
op_fused_epilogue_add2_rmsnorm.py).  Additive,
optional keyword arguments: `num_heads` / `head_dim` (the reference hard-codes
24 x 64), `num_kv_heads` for the backbone op (reference: 32 / 8 / 128 with a
fixed 4096-wide output), and `kv_mask` on the 3-way ops (1 = visible key,
0 = padded key, the eager encoder/physics mask convention).  Every op has a
`register_fake` so `torch.compile` can trace it.
"""

from __future__ import annotations

import math
import weakref
from typing import Optional

import torch

from . import functional as Fn

# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------


def _attn_from_qkv(q, kvp, key_bias, M, H, D):
    """(H, M, D) Q + packed K/V tiles (H, E) -> (1, M, H*D) bf16, written directly in token-major order."""
    out = torch.empty((1, M, H, D), dtype=torch.bfloat16, device=q.device)
    Fn.attention_packed(q.unsqueeze(0), kvp.unsqueeze(0), M, key_bias=key_bias, layout="bhsd",
                        out=out.permute(0, 2, 1, 3))
    return out.view(1, M, H * D)


def _qkv_cols(t: torch.Tensor) -> torch.Tensor:
    return t if t.dim() == 2 else t.reshape(-1, t.shape[-1])


# ---------------------------------------------------------------------------
# ds::  (DoubleStreamBlock / ExpandedDoubleStreamBlock)
# ---------------------------------------------------------------------------


@torch.library.custom_op("ds::fused_attention_2way", mutates_args=())
def ds_fused_attention_2way(
    sa_qkv: torch.Tensor,
    vl_qkv: torch.Tensor,
    q_norm_sa_weight: torch.Tensor,
    k_norm_sa_weight: torch.Tensor,
    q_norm_vl_weight: torch.Tensor,
    k_norm_vl_weight: torch.Tensor,
    rope_cos: torch.Tensor,
    rope_sin: torch.Tensor,
    n_sa: int,
    n_vl: int,
    num_heads: int = 24,
    head_dim: int = 64,
) -> torch.Tensor:
    """QK-RMSNorm + interleaved RoPE (SA rows) + joint attention over [VL | SA].

    Reference: op_fused_attention.py:12-82 (double_stream)."""
    H, D = num_heads, head_dim
    streams = [
        Fn.StreamSpec(_qkv_cols(vl_qkv)[:n_vl], q_norm_vl_weight, k_norm_vl_weight),
        Fn.StreamSpec(_qkv_cols(sa_qkv)[:n_sa], q_norm_sa_weight, k_norm_sa_weight, rope_cos, rope_sin),
    ]
    q, kvp = Fn.msat_qkv_norm_rope(streams, H, D, kv_packed=True)
    return _attn_from_qkv(q, kvp, None, n_vl + n_sa, H, D)


@ds_fused_attention_2way.register_fake
def _(sa_qkv, vl_qkv, q_norm_sa_weight, k_norm_sa_weight, q_norm_vl_weight, k_norm_vl_weight, rope_cos, rope_sin,
      n_sa, n_vl, num_heads=24, head_dim=64):
    return sa_qkv.new_empty((1, n_sa + n_vl, num_heads * head_dim))


@torch.library.custom_op("ds::fused_attention_3way", mutates_args=())
def ds_fused_attention_3way(
    sa_qkv: torch.Tensor,
    vl_qkv: torch.Tensor,
    p_qkv: torch.Tensor,
    q_norm_sa_weight: torch.Tensor,
    k_norm_sa_weight: torch.Tensor,
    q_norm_vl_weight: torch.Tensor,
    k_norm_vl_weight: torch.Tensor,
    q_norm_p_weight: torch.Tensor,
    k_norm_p_weight: torch.Tensor,
    sa_rope_cos: torch.Tensor,
    sa_rope_sin: torch.Tensor,
    p_rope_cos: torch.Tensor,
    p_rope_sin: torch.Tensor,
    n_sa: int,
    n_vl: int,
    n_p: int,
    num_heads: int = 24,
    head_dim: int = 64,
    kv_mask: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Three-stream [VL | SA | P] version; `kv_mask` [1, M] masks padded keys.

    Reference: op_fused_attention_3way.py:13-116 (double_stream); mask semantics
    of ExpandedDoubleStreamBlock.forward (blocks.py:843-866)."""
    H, D = num_heads, head_dim
    streams = [
        Fn.StreamSpec(_qkv_cols(vl_qkv)[:n_vl], q_norm_vl_weight, k_norm_vl_weight),
        Fn.StreamSpec(_qkv_cols(sa_qkv)[:n_sa], q_norm_sa_weight, k_norm_sa_weight, sa_rope_cos, sa_rope_sin),
        Fn.StreamSpec(_qkv_cols(p_qkv)[:n_p], q_norm_p_weight, k_norm_p_weight, p_rope_cos, p_rope_sin),
    ]
    q, kvp = Fn.msat_qkv_norm_rope(streams, H, D, kv_packed=True)
    bias = Fn.mask_to_key_bias(kv_mask) if kv_mask is not None else None
    return _attn_from_qkv(q, kvp, bias, n_vl + n_sa + n_p, H, D)


@ds_fused_attention_3way.register_fake
def _(sa_qkv, vl_qkv, p_qkv, q_norm_sa_weight, k_norm_sa_weight, q_norm_vl_weight, k_norm_vl_weight,
      q_norm_p_weight, k_norm_p_weight, sa_rope_cos, sa_rope_sin, p_rope_cos, p_rope_sin, n_sa, n_vl, n_p,
      num_heads=24, head_dim=64, kv_mask=None):
    return sa_qkv.new_empty((1, n_sa + n_vl + n_p, num_heads * head_dim))


@torch.library.custom_op("ds::grouped_swiglu", mutates_args=())
def ds_grouped_swiglu(
    sa_w12: torch.Tensor,
    sa_bias: torch.Tensor,
    vl_w12: torch.Tensor,
    vl_bias: torch.Tensor,
    m_sa: int,
    m_vl: int,
    n_half_sa: int,
    n_half_vl: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """SiLU(x[:, :N] + b[:N]) * (x[:, N:] + b[N:]) for the SA and VL groups in one launch.

    Reference: op_grouped_swiglu.py:12-49.  Rounds like eager bf16 tensors
    (bias add, silu and product each rounded to bf16)."""
    return Fn.grouped_swiglu(sa_w12, sa_bias, vl_w12, vl_bias, m_sa, m_vl, n_half_sa, n_half_vl)


@ds_grouped_swiglu.register_fake
def _(sa_w12, sa_bias, vl_w12, vl_bias, m_sa, m_vl, n_half_sa, n_half_vl):
    return sa_w12.new_empty((m_sa, n_half_sa)), vl_w12.new_empty((m_vl, n_half_vl))


# ---------------------------------------------------------------------------
# ss::  (SingleStreamBlock / ExpandedSingleStreamBlock)
# ---------------------------------------------------------------------------


@torch.library.custom_op("ss::fused_attention_2way", mutates_args=())
def ss_fused_attention_2way(
    qkv: torch.Tensor,
    q_norm_weight: torch.Tensor,
    k_norm_weight: torch.Tensor,
    rope_cos: torch.Tensor,
    rope_sin: torch.Tensor,
    n_sa: int,
    num_heads: int = 24,
    head_dim: int = 64,
) -> torch.Tensor:
    """One packed `linear1` buffer [M, >= 3*inner]; RoPE on its last n_sa rows.

    Reference: single_stream/engine/ops/op_fused_attention.py:12-65."""
    H, D = num_heads, head_dim
    x = _qkv_cols(qkv)
    M = x.shape[0]
    streams = []
    if M - n_sa > 0:
        streams.append(Fn.StreamSpec(x[: M - n_sa], q_norm_weight, k_norm_weight))
    if n_sa > 0:
        streams.append(Fn.StreamSpec(x[M - n_sa:], q_norm_weight, k_norm_weight, rope_cos, rope_sin))
    q, kvp = Fn.msat_qkv_norm_rope(streams, H, D, kv_packed=True)
    return _attn_from_qkv(q, kvp, None, M, H, D)


@ss_fused_attention_2way.register_fake
def _(qkv, q_norm_weight, k_norm_weight, rope_cos, rope_sin, n_sa, num_heads=24, head_dim=64):
    # the op flattens every leading dim of qkv into the token count, as _qkv_cols does
    return qkv.new_empty((1, math.prod(qkv.shape[:-1]), num_heads * head_dim))


@torch.library.custom_op("ss::fused_attention_3way", mutates_args=())
def ss_fused_attention_3way(
    x_qkv: torch.Tensor,
    p_qkv: torch.Tensor,
    x_q_norm_weight: torch.Tensor,
    x_k_norm_weight: torch.Tensor,
    p_q_norm_weight: torch.Tensor,
    p_k_norm_weight: torch.Tensor,
    sa_rope_cos: torch.Tensor,
    sa_rope_sin: torch.Tensor,
    p_rope_cos: torch.Tensor,
    p_rope_sin: torch.Tensor,
    n_x: int,
    n_sa: int,
    n_p: int,
    num_heads: int = 24,
    head_dim: int = 64,
    kv_mask: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """[VL+SA | P]: RoPE on the last n_sa rows of x and on all P rows.

    Reference: single_stream/engine/ops/op_fused_attention_3way.py:13-129."""
    H, D = num_heads, head_dim
    x = _qkv_cols(x_qkv)[:n_x]
    p = _qkv_cols(p_qkv)[:n_p]
    streams = []
    if n_x - n_sa > 0:
        streams.append(Fn.StreamSpec(x[: n_x - n_sa], x_q_norm_weight, x_k_norm_weight))
    if n_sa > 0:
        streams.append(Fn.StreamSpec(x[n_x - n_sa:], x_q_norm_weight, x_k_norm_weight, sa_rope_cos, sa_rope_sin))
    if n_p > 0:
        streams.append(Fn.StreamSpec(p, p_q_norm_weight, p_k_norm_weight, p_rope_cos, p_rope_sin))
    q, kvp = Fn.msat_qkv_norm_rope(streams, H, D, kv_packed=True)
    bias = Fn.mask_to_key_bias(kv_mask) if kv_mask is not None else None
    return _attn_from_qkv(q, kvp, bias, n_x + n_p, H, D)


@ss_fused_attention_3way.register_fake
def _(x_qkv, p_qkv, x_q_norm_weight, x_k_norm_weight, p_q_norm_weight, p_k_norm_weight, sa_rope_cos, sa_rope_sin,
      p_rope_cos, p_rope_sin, n_x, n_sa, n_p, num_heads=24, head_dim=64, kv_mask=None):
    return x_qkv.new_empty((1, n_x + n_p, num_heads * head_dim))


# ---------------------------------------------------------------------------
# rldx_backbone::  (Qwen3-VL LLM decoder)
# ---------------------------------------------------------------------------


def llm_fused_attention(qkv, q_norm_w, q_norm_w_rot, k_norm_w, k_norm_w_rot, cos, signed_sin, num_heads=32,
                        num_kv_heads=8, head_dim=128, out=None):
    """QK-RMSNorm + rotate-half RoPE + causal GQA attention on a packed
    (M, (Hq + 2*Hkv) * D) QKV buffer -> (M, Hq*D).

    Same Python signature as fused_llm_attention.forward
    (rldx/inference/backbone/llm/engine/kernels/fused_llm_attention.py:1005-1057).
    `q_norm_w_rot` / `k_norm_w_rot` are accepted for signature compatibility;
    the kernels read the rotate-half partner directly, which gives the same
    values (w_rot[d] * x[d +- D/2] == w[d +- D/2] * x[d +- D/2])."""
    return Fn.llm_fused_attention(qkv, q_norm_w, k_norm_w, cos, signed_sin, num_heads, num_kv_heads, head_dim,
                                  sin_is_signed=True, out=out)


@torch.library.custom_op("rldx_backbone::fused_attention", mutates_args=())
def rldx_backbone_fused_attention(
    qkv: torch.Tensor,
    q_norm_w: torch.Tensor,
    q_norm_w_rot: torch.Tensor,
    k_norm_w: torch.Tensor,
    k_norm_w_rot: torch.Tensor,
    cos: torch.Tensor,
    signed_sin: torch.Tensor,
    num_heads: int = 32,
    num_kv_heads: int = 8,
    head_dim: int = 128,
) -> torch.Tensor:
    """Reference: backbone/llm/engine/ops/op_fused_llm_attention.py:13-45."""
    return llm_fused_attention(qkv, q_norm_w, q_norm_w_rot, k_norm_w, k_norm_w_rot, cos, signed_sin, num_heads,
                               num_kv_heads, head_dim)


@rldx_backbone_fused_attention.register_fake
def _(qkv, q_norm_w, q_norm_w_rot, k_norm_w, k_norm_w_rot, cos, signed_sin, num_heads=32, num_kv_heads=8,
      head_dim=128):
    return qkv.new_empty((qkv.shape[0], num_heads * head_dim))


@torch.library.custom_op("rldx_backbone::vision_attention", mutates_args=())
def rldx_backbone_vision_attention(
    qkv: torch.Tensor,
    rope_cos: torch.Tensor,
    rope_sin: torch.Tensor,
    cu_seqlens: torch.Tensor,
    scaling: float,
    num_heads: int,
    head_dim: int,
) -> torch.Tensor:
    """Fused vision RoPE (baked cos / signed sin) + non-causal attention per
    cu_seqlens segment on a fused (M, 3*H*D) QKV buffer -> (M, H*D).

    Reference: backbone/vision_encoder/engine/ops/op_fused_vision_attention.py:14-42."""
    return Fn.vision_attention(qkv, rope_cos, rope_sin, cu_seqlens, scaling, num_heads, head_dim)


@rldx_backbone_vision_attention.register_fake
def _(qkv, rope_cos, rope_sin, cu_seqlens, scaling, num_heads, head_dim):
    return qkv.new_empty((qkv.shape[0], num_heads * head_dim))


@torch.library.custom_op("mem::fused_attention", mutates_args=())
def mem_fused_attention(
    qkv: torch.Tensor,
    cos: torch.Tensor,
    signed_sin: torch.Tensor,
    num_heads: int,
    head_dim: int,
    block_attn_size: int,
) -> torch.Tensor:
    """bf16 RoPE + block-causal attention of the TransformerMemory layers on a
    fused (M, 3*H*D) QKV buffer -> (M, H*D).

    Reference: memory/engine/ops/op_fused_memory_attention.py:12-36."""
    return Fn.memory_attention(qkv, cos, signed_sin, num_heads, head_dim, block_attn_size)


@mem_fused_attention.register_fake
def _(qkv, cos, signed_sin, num_heads, head_dim, block_attn_size):
    return qkv.new_empty((qkv.shape[0], num_heads * head_dim))


# ---------------------------------------------------------------------------
# rldx_amd::swiglu  (the activation of SwiGLUFFN and the chains' inline SwiGLU)
# ---------------------------------------------------------------------------


@torch.library.custom_op("rldx_amd::swiglu", mutates_args=())
def swiglu_op(x: torch.Tensor) -> torch.Tensor:
    """`F.silu(x1) * x2` with `x1, x2 = x.chunk(2, -1)` (action_model/ops.py:157-161)."""
    return Fn.swiglu(x)


@swiglu_op.register_fake
def _(x):
    return x.new_empty((*x.shape[:-1], x.shape[-1] // 2))


# ---------------------------------------------------------------------------
# ss::fused_mlp_swiglu — GEMM + bias + SwiGLU
# ---------------------------------------------------------------------------
# The grouped GEMM reads weights in its packed operand order.  Weights are
# static, so each one is packed once and the packed copy is kept for as long as
# the weight tensor lives; an in-place update of the weight (version change)
# packs it again.
_packed_weights: dict = {}  # id(weight) -> (weakref to weight, version, swiglu_pairs, PackedWeight)


def _packed_weight(w: torch.Tensor, swiglu_pairs: bool) -> Fn.PackedWeight:
    hit = _packed_weights.get(id(w))
    if hit is not None and hit[0]() is w and hit[1] == w._version and hit[2] == swiglu_pairs:
        return hit[3]
    pw = Fn.pack_weight(w if w.stride(1) == 1 else w.contiguous(), swiglu_pairs=swiglu_pairs)
    if hit is None or hit[0]() is not w:
        weakref.finalize(w, _packed_weights.pop, id(w), None)
    _packed_weights[id(w)] = (weakref.ref(w), w._version, swiglu_pairs, pw)
    return pw


@torch.library.custom_op("ss::fused_mlp_swiglu", mutates_args=())
def ss_fused_mlp_swiglu(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, split_k: int = 1) -> torch.Tensor:
    """silu(x W_gate^T + b_gate) * (x W_up^T + b_up), W = [W_gate; W_up] (2*N_half, K).

    rldx/inference/action_model/single_stream/engine/ops/op_fused_mlp_swiglu.py:13-43
    (kernel fused_mlp_swiglu.py:199-267).  split_k > 1 splits K across
    workgroups (fp32 partials in a workspace allocated per call, as the
    reference's launcher does; the last workgroup of each tile sums them in
    split order and applies the epilogue), the largest power of two <= split_k
    that divides the K stages.  Rounding: the eager chain (GEMM output rounded to
    bf16, then SwiGLU's two roundings).  Needs K % 128 == 0 and N_half % 32 == 0."""
    M, K = x.shape
    nh = weight.shape[0] // 2
    out = torch.empty((M, nh), dtype=torch.bfloat16, device=x.device)
    if M == 0:
        return out
    xx = x if x.stride(1) == 1 else x.contiguous()
    items = [(xx, _packed_weight(weight, True), bias.contiguous(), out, None)]
    ws = None
    if split_k > 1:
        need = Fn.grouped_gemm_workspace_bytes(items, "swiglu", split_k)
        ws = Fn.GemmWorkspace(need, x.device) if need > 0 else None
    Fn.grouped_gemm(items, "swiglu", split_k=split_k if ws is not None else 1, workspace=ws)
    return out


@ss_fused_mlp_swiglu.register_fake
def _(x, weight, bias, split_k=1):
    return x.new_empty((x.shape[0], weight.shape[0] // 2))


# ---------------------------------------------------------------------------
# Residual-add + norm epilogues at block boundaries
# ---------------------------------------------------------------------------


@torch.library.custom_op("ds::grouped_res_ln", mutates_args=())
def ds_grouped_res_ln(
    sa_res: torch.Tensor,
    sa_bias: torch.Tensor,
    sa_proj: torch.Tensor,
    vl_res: torch.Tensor,
    vl_bias: torch.Tensor,
    vl_proj: torch.Tensor,
    m_sa: int,
    m_vl: int,
    sa_dim: int,
    vl_dim: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per stream LayerNorm(residual + proj_output + proj_bias), no affine, fp32 sum.

    Reference: op_grouped_res_ln.py:13-45 (kernel grouped_res_ln.py:40-148)."""
    return Fn.fused_grouped_res_ln(sa_res, sa_bias, sa_proj, vl_res, vl_bias, vl_proj, M_sa=m_sa, M_vl=m_vl,
                                   SA_DIM=sa_dim, VL_DIM=vl_dim)


@ds_grouped_res_ln.register_fake
def _(sa_res, sa_bias, sa_proj, vl_res, vl_bias, vl_proj, m_sa, m_vl, sa_dim, vl_dim):
    return sa_res.new_empty((1, m_sa, sa_dim)), vl_res.new_empty((1, m_vl, vl_dim))


@torch.library.custom_op("ds::vl_epilogue_ln", mutates_args=())
def ds_vl_epilogue_ln(
    vl_res: torch.Tensor,
    proj_bias: torch.Tensor,
    w3_bias: torch.Tensor,
    w3_out: torch.Tensor,
    m: int,
    dim: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """new_vl = ((vl_res + proj_bias) + w3_bias) + w3_out (bf16 adds); ln_vl = LayerNorm(new_vl).

    Reference: op_vl_epilogue_ln.py:13-45 (kernel vl_epilogue_ln.py:31-125)."""
    return Fn.fused_vl_epilogue_ln(vl_res, proj_bias, w3_bias, w3_out, M=m, DIM=dim)


@ds_vl_epilogue_ln.register_fake
def _(vl_res, proj_bias, w3_bias, w3_out, m, dim):
    return vl_res.new_empty((1, m, dim)), vl_res.new_empty((1, m, dim))


@torch.library.custom_op("ss::fused_epilogue_ln", mutates_args=())
def ss_fused_epilogue_ln(hidden: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """new_hidden = hidden + residual (bf16); ln_out = LayerNorm(new_hidden).

    Reference: single_stream/engine/ops/op_fused_epilogue_ln.py:11-35, which fixes
    DIM = 1536; here DIM is hidden.shape[-1] (M = hidden.shape[1] as there)."""
    new_hidden, ln = Fn.fused_ss_epilogue_ln(hidden, M=hidden.shape[1], DIM=hidden.shape[-1], residual=residual)
    return new_hidden.view(hidden.shape), ln.view(hidden.shape)


@ss_fused_epilogue_ln.register_fake
def _(hidden, residual):
    return torch.empty_like(hidden), torch.empty_like(hidden)


@torch.library.custom_op("rldx_backbone::fused_epilogue_add2_rmsnorm", mutates_args=())
def rldx_backbone_fused_epilogue_add2_rmsnorm(
    hidden: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """new_hidden = hidden + residual (bf16); normed = RMSNorm(new_hidden) (Qwen3-VL, eager rounding).

    Reference: backbone/llm/engine/ops/op_fused_epilogue_add2_rmsnorm.py:20-45."""
    return Fn.fused_add2_rmsnorm(hidden, residual, weight)


@rldx_backbone_fused_epilogue_add2_rmsnorm.register_fake
def _(hidden, residual, weight):
    return torch.empty_like(hidden), torch.empty_like(hidden)


@torch.library.custom_op("rldx_backbone::fused_epilogue_add3_rmsnorm", mutates_args=())
def rldx_backbone_fused_epilogue_add3_rmsnorm(
    hidden: torch.Tensor,
    residual: torch.Tensor,
    deepStack: torch.Tensor,
    weight: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """new_hidden = (hidden + residual) + deepStack (bf16 adds); normed = RMSNorm(new_hidden).

    Reference: backbone/llm/engine/ops/op_fused_epilogue_add3_rmsnorm.py:20-47."""
    return Fn.fused_add3_rmsnorm(hidden, residual, deepStack, weight)


@rldx_backbone_fused_epilogue_add3_rmsnorm.register_fake
def _(hidden, residual, deepStack, weight):
    return torch.empty_like(hidden), torch.empty_like(hidden)


@torch.library.custom_op("mem::fused_epilogue_add2_rmsnorm", mutates_args=())
def mem_fused_epilogue_add2_rmsnorm(
    hidden: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The TransformerMemory layers' cross-layer epilogue: the same arithmetic as
    rldx_backbone::fused_epilogue_add2_rmsnorm (the reference reuses that kernel).

    Reference: memory/engine/ops/op_fused_epilogue_add2_rmsnorm.py:16-40."""
    return Fn.fused_add2_rmsnorm(hidden, residual, weight)


@mem_fused_epilogue_add2_rmsnorm.register_fake
def _(hidden, residual, weight):
    return torch.empty_like(hidden), torch.empty_like(hidden)
