"""CPU oracle: a restatement of RLDX-1's eager PyTorch formulas for the hot path.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke() as the
checker, and by bench.py's cpu_baseline leg as the timed CPU path.  No product
code imports it; the HIP kernels never route through it.

Every function follows the cited reference source line by line in its
arithmetic (same ops, same dtypes, same rounding points), written out here in
plain torch so it runs on the CPU without the reference package, diffusers or
transformers.  How each function is pinned independently of itself
(closed forms, invariants, fp64 brute force, exhaustive bf16 sweeps) is listed
in tests/test_oracle.py.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# Qwen3-VL text attention pieces
# ---------------------------------------------------------------------------
def qwen_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Qwen3VLTextRMSNorm.forward — modeling_qwen3_vl.py:366-371."""
    input_dtype = x.dtype
    h = x.to(torch.float32)
    variance = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(variance + eps)
    return w * h.to(input_dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """modeling_qwen3_vl.py:118-122."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim: int = 1):
    """modeling_qwen3_vl.py:377-401."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    q_embed = (q * cos) + (rotate_half(q) * sin)
    k_embed = (k * cos) + (rotate_half(k) * sin)
    return q_embed, k_embed


def qk_rmsnorm_rope_half(q, k, q_w, k_w, cos, sin, eps: float = 1e-6):
    """q_norm/k_norm then RoPE on [B, S, H, D] tensors, cos/sin [S, D] or [B, S, D]
    (Qwen3VLTextAttention.forward, modeling_qwen3_vl.py:449-456, with the head
    axis kept at position 2: unsqueeze_dim=2)."""
    if cos.dim() == 2:
        cos, sin = cos.unsqueeze(0), sin.unsqueeze(0)
    return apply_rotary_pos_emb(qwen_rmsnorm(q, q_w, eps), qwen_rmsnorm(k, k_w, eps), cos, sin, unsqueeze_dim=2)


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """modeling_qwen3_vl.py:139-150 ([B, Hkv, S, D] -> [B, Hkv*n_rep, S, D])."""
    b, h, s, d = x.shape
    if n_rep == 1:
        return x
    return x[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def llm_fused_attention(qkv, q_norm_w, k_norm_w, cos, sin, num_heads, num_kv_heads, head_dim, eps=1e-6):
    """Eager equivalent of rldx_backbone::fused_attention: packed (M, QKV_DIM)
    bf16 -> (M, Hq*D).  q/k norm + rotate-half RoPE (modeling_qwen3_vl.py:449-456),
    causal SDPA with repeated KV (:139-176; flash/sdpa path is_causal)."""
    M = qkv.shape[0]
    Hq, Hkv, D = num_heads, num_kv_heads, head_dim
    q = qkv[:, : Hq * D].reshape(1, M, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(1, M, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].reshape(1, M, Hkv, D)
    q, k = qk_rmsnorm_rope_half(q, k, q_norm_w, k_norm_w, cos, sin, eps)
    q, k, v = (t.transpose(1, 2) for t in (q, k, v))
    o = sdpa(q, repeat_kv(k, Hq // Hkv), repeat_kv(v, Hq // Hkv), causal=True)
    return o.transpose(1, 2).reshape(M, Hq * D)


# ---------------------------------------------------------------------------
# Vision tower (Qwen3-VL ViT) attention
# ---------------------------------------------------------------------------
def vision_rope(x: torch.Tensor, rope_cos: torch.Tensor, rope_sin: torch.Tensor) -> torch.Tensor:
    """Baked rotate-half RoPE of the Qwen3-VL vision tower as the fused op applies it
    (fused_vision_attention.py:47-80, :117-139): x [M, H, D] bf16, rope_cos / rope_sin
    [M, D] fp32 with rotate_half's sign folded into the first half of rope_sin
    (custom_vision_encoder_chain.py:101-108):
        y[d] = bf16(x[d] * cos[d] + x[d +- D/2] * sin_baked[d])   in fp32.
    Equal, product by product, to apply_rotary_pos_emb_vision (modeling_qwen3_vl.py:125-136)
    with the unbaked sin."""
    D = x.shape[-1]
    half = D // 2
    rot = torch.cat([torch.arange(half, D), torch.arange(0, half)])
    xf = x.float()
    c = rope_cos.float()[:, None, :]
    sn = rope_sin.float()[:, None, :]
    return (xf * c + xf[..., rot] * sn).to(torch.bfloat16)


def vision_attention(qkv: torch.Tensor, rope_cos: torch.Tensor, rope_sin: torch.Tensor, cu_seqlens: torch.Tensor,
                     scaling: float, num_heads: int, head_dim: int) -> torch.Tensor:
    """rldx_backbone::vision_attention (op_fused_vision_attention.py:13-45; kernel
    fused_vision_attention.py:83-159, :206-320, :622-645): qkv [M, 3 H D] bf16 with
    columns Q | K | V (head h at h D), baked RoPE on Q and K (vision_rope), then
    non-causal attention inside each sequence [cu_seqlens[s], cu_seqlens[s+1]):
    S = Q K^T (fp32 sums of bf16 products) * scaling, softmax in fp32, P rounded to
    bf16 for the P.V product, fp32 sums, output rounded to bf16.  Returns [M, H D]."""
    M = qkv.shape[0]
    H, D = num_heads, head_dim
    q, k, v = qkv.reshape(M, 3, H, D).unbind(1)
    qr = vision_rope(q, rope_cos, rope_sin)
    kr = vision_rope(k, rope_cos, rope_sin)
    out = torch.zeros(M, H, D, dtype=torch.float32)
    cu = [int(x) for x in cu_seqlens.tolist()]
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        if b <= a:
            continue
        qs = qr[a:b].float().transpose(0, 1)  # [H, L, D]
        ks = kr[a:b].float().transpose(0, 1)
        vs = v[a:b].float().transpose(0, 1)
        sc = torch.matmul(qs, ks.transpose(1, 2)) * scaling
        m = sc.amax(dim=-1, keepdim=True)
        pe = torch.exp(sc - m)
        l = pe.sum(dim=-1, keepdim=True)
        o = torch.matmul(pe.to(torch.bfloat16).float(), vs) / l
        out[a:b] = o.transpose(0, 1)
    return out.to(torch.bfloat16).reshape(M, H * D)


def vision_attention_eager(qkv: torch.Tensor, rope_cos: torch.Tensor, rope_sin: torch.Tensor,
                           cu_seqlens: torch.Tensor, scaling: float, num_heads: int, head_dim: int) -> torch.Tensor:
    """The eager path the fused op replaces: Qwen3VLVisionAttention.forward without
    flash attention (modeling_qwen3_vl.py:193-262) with apply_rotary_pos_emb_vision
    (:125-136) and eager_attention_forward (:153-176): bf16 score matmul, softmax in
    fp32 rounded back to bf16, bf16 P.V.  Used to pin vision_attention (they differ
    by the score and probability roundings)."""
    M = qkv.shape[0]
    H, D = num_heads, head_dim
    q, k, v = qkv.reshape(M, 3, H, D).permute(1, 0, 2, 3).unbind(0)
    half = D // 2
    sin = rope_sin.clone()
    sin[:, :half] = -sin[:, :half]
    cos_, sin_ = rope_cos.unsqueeze(-2).float(), sin.unsqueeze(-2).float()
    qe = (q.float() * cos_ + rotate_half(q.float()) * sin_).to(q.dtype)
    ke = (k.float() * cos_ + rotate_half(k.float()) * sin_).to(k.dtype)
    qe, ke, ve = (t.transpose(0, 1).unsqueeze(0) for t in (qe, ke, v))
    lengths = (cu_seqlens[1:] - cu_seqlens[:-1]).tolist()
    outs = []
    for qs, ks, vs in zip(torch.split(qe, lengths, dim=2), torch.split(ke, lengths, dim=2),
                          torch.split(ve, lengths, dim=2)):
        w = torch.matmul(qs, ks.transpose(2, 3)) * scaling
        w = F.softmax(w, dim=-1, dtype=torch.float32).to(qs.dtype)
        outs.append(torch.matmul(w, vs).transpose(1, 2))
    return torch.cat(outs, dim=1).reshape(M, H * D)


# ---------------------------------------------------------------------------
# TransformerMemory attention (block-causal)
# ---------------------------------------------------------------------------
def memory_rope(x: torch.Tensor, cos: torch.Tensor, signed_sin: torch.Tensor) -> torch.Tensor:
    """bf16 rotate-half RoPE of the memory module, every step rounded to bf16 as the
    eager apply_rotary_pos_emb does on bf16 tensors (memory.py:45-57;
    fused_memory_attention.py:84-108, :124-138): x [M, H, D] bf16, cos / signed_sin
    [M, D] bf16 with rotate_half's sign folded into the first half of signed_sin
    (fused_memory_attention.py:185-195):
        y[d] = bf16(bf16(x[d] * cos[d]) + bf16(x[d +- D/2] * signed_sin[d]))."""
    D = x.shape[-1]
    half = D // 2
    rot = torch.cat([torch.arange(half, D), torch.arange(0, half)])
    c = cos.to(torch.bfloat16)[:, None, :]
    sn = signed_sin.to(torch.bfloat16)[:, None, :]
    return x * c + x[..., rot] * sn


def memory_attention(qkv: torch.Tensor, cos: torch.Tensor, signed_sin: torch.Tensor, num_heads: int, head_dim: int,
                     block_attn_size: int) -> torch.Tensor:
    """mem::fused_attention (op_fused_memory_attention.py:12-36; kernel
    fused_memory_attention.py:35-173): qkv [M, 3 H D] bf16 (Q | K | V, head h at
    h D), bf16 RoPE on Q and K (memory_rope), then softmax(Q K^T / sqrt(D)) V with
    the block-causal mask: query i sees key j iff j // B <= i // B
    (memory.py:214-226).  fp32 scores and softmax, P rounded to bf16 for P.V, fp32
    sums, output rounded to bf16.  Returns [M, H D]."""
    M = qkv.shape[0]
    H, D, B = num_heads, head_dim, block_attn_size
    q, k, v = qkv.reshape(M, 3, H, D).unbind(1)
    qr = memory_rope(q, cos, signed_sin).float().transpose(0, 1)  # [H, M, D]
    kr = memory_rope(k, cos, signed_sin).float().transpose(0, 1)
    vs = v.float().transpose(0, 1)
    idx = torch.arange(M)
    visible = (idx[None, :] // B) <= (idx[:, None] // B)
    sc = torch.matmul(qr, kr.transpose(1, 2)) * (1.0 / math.sqrt(D))
    sc = sc.masked_fill(~visible, float("-inf"))
    m = sc.amax(dim=-1, keepdim=True)
    pe = torch.exp(sc - m)
    l = pe.sum(dim=-1, keepdim=True)
    o = torch.matmul(pe.to(torch.bfloat16).float(), vs) / l
    return o.transpose(0, 1).to(torch.bfloat16).reshape(M, H * D)


def memory_block_mask(M: int, block_attn_size: int) -> torch.Tensor:
    """_make_causal_mask(..., use_causal_attn=False) (memory.py:214-226): [M, M]
    additive bf16 mask, 0 where key j is visible to query i, finfo.min elsewhere."""
    mask = torch.full((M, M), torch.finfo(torch.bfloat16).min)
    for i in range(0, M, block_attn_size):
        end = min(i + block_attn_size, M)
        mask[i:end, :end] = 0
    return mask.to(torch.bfloat16)


# ---------------------------------------------------------------------------
# MSAT pieces
# ---------------------------------------------------------------------------
def msat_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm.forward — rldx/model/modules/norms.py:18-22 (one rounding)."""
    input_dtype = x.dtype
    x_float = x.float()
    x_normed = x_float * torch.rsqrt(x_float.pow(2).mean(-1, keepdim=True) + eps)
    return (w * x_normed).to(input_dtype)


def apply_rotary_emb(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor):
    """Interleaved complex RoPE — rldx/model/modules/action_model/ops.py:48-67.
    xq, xk [B, H, N, D]; freqs_cis complex64 [B, N, D/2]."""
    xq_ = torch.view_as_complex(xq.float().reshape(*xq.shape[:-1], -1, 2))
    xk_ = torch.view_as_complex(xk.float().reshape(*xk.shape[:-1], -1, 2))
    fc = freqs_cis.unsqueeze(1)
    xq_out = torch.view_as_real(xq_ * fc).flatten(3)
    xk_out = torch.view_as_real(xk_ * fc).flatten(3)
    return xq_out.type_as(xq), xk_out.type_as(xk)


def split_heads(x: torch.Tensor, num_heads: int) -> torch.Tensor:
    """ops.py:167-171."""
    B, N, D = x.shape
    return x.view(B, N, num_heads, D // num_heads).permute(0, 2, 1, 3).contiguous()


def merge_heads(x: torch.Tensor) -> torch.Tensor:
    """ops.py:174-177."""
    B, H, N, Dh = x.shape
    return x.permute(0, 2, 1, 3).contiguous().view(B, N, H * Dh)


def msat_qkv_norm_rope(streams, num_heads: int, head_dim: int, eps: float = 1e-6):
    """Per-stream QK RMSNorm then joint interleaved RoPE, eager order of
    ExpandedDoubleStreamBlock.forward (blocks.py:804-833): split heads, norm each
    stream, concat [s0 | s1 | s2], apply_rotary_emb with a per-row table (rows
    without a table get the identity rotation, i.e. position 0).

    streams: list of (qkv [n, >=3*inner] bf16, q_w, k_w, cos or None, sin or None).
    Returns q, k, v (H, M, D) bf16."""
    inner = num_heads * head_dim
    qs, ks, vs, pes = [], [], [], []
    for qkv, q_w, k_w, cos, sin in streams:
        n = qkv.shape[0]
        x = qkv[:, : 3 * inner].unsqueeze(0)
        q, k, v = (split_heads(t, num_heads) for t in x.chunk(3, dim=-1))
        B, H, _, Dh = q.shape
        q = msat_rmsnorm(q.reshape(B * H, n, Dh), q_w, eps).reshape(B, H, n, Dh)
        k = msat_rmsnorm(k.reshape(B * H, n, Dh), k_w, eps).reshape(B, H, n, Dh)
        qs.append(q), ks.append(k), vs.append(v)
        if cos is None:
            pes.append(torch.polar(torch.ones(n, head_dim // 2), torch.zeros(n, head_dim // 2)))
        else:
            pes.append(torch.complex(cos.float(), sin.float()))
    q = torch.cat(qs, dim=2)
    k = torch.cat(ks, dim=2)
    v = torch.cat(vs, dim=2)
    pe = torch.cat(pes, dim=0).unsqueeze(0)
    q, k = apply_rotary_emb(q, k, pe)
    return q[0], k[0], v[0]


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
def swiglu(x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """SwiGLUFFN activation — ops.py:157-161 (`x12.chunk(2, -1)`, `F.silu(x1) * x2`).
    With bias: the bias-added w12 output, rounded like an eager bf16 add."""
    if bias is not None:
        x = x + bias
    x1, x2 = x.chunk(2, dim=-1)
    return F.silu(x1) * x2


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
def sdpa(q, k, v, key_bias: Optional[torch.Tensor] = None, causal: bool = False, scale: Optional[float] = None):
    """F.scaled_dot_product_attention as called on the path (blocks.py:577-579, :866).

    key_bias: [B, Sk] additive mask in the eager dtype convention: cast to
    q.dtype and broadcast as [B, 1, 1, Sk] (blocks.py:843-864)."""
    mask = None
    if key_bias is not None:
        kb = key_bias if key_bias.dim() == 2 else key_bias.unsqueeze(0)
        mask = kb[:, None, None, :].to(q.dtype)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=causal, scale=scale)


def mask_to_bias(kv_mask: torch.Tensor) -> torch.Tensor:
    """1 visible / 0 masked -> 0 / -inf (blocks.py:843-864)."""
    return torch.where(kv_mask == 0, torch.tensor(float("-inf")), torch.tensor(0.0)).float()


# ---------------------------------------------------------------------------
# LayerNorm without affine (pre-norm of the MSAT blocks)
# ---------------------------------------------------------------------------
def layer_norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """nn.LayerNorm(dim, elementwise_affine=False, eps) — norms.py:35-36."""
    return F.layer_norm(x, (x.shape[-1],), eps=eps)


# ---------------------------------------------------------------------------
# Residual-add + norm epilogues at block boundaries
# ---------------------------------------------------------------------------
def _ln_rows_fp32(x: torch.Tensor, eps: float) -> torch.Tensor:
    """LayerNorm without affine on fp32 rows, as the reference epilogue kernels
    write it: mean = sum / D, var = sum((x - mean)^2) / D,
    out = (x - mean) * (1 / sqrt(var + eps)) (grouped_res_ln.py:81-108)."""
    d = x.shape[-1]
    mean = x.sum(-1, keepdim=True) / d
    diff = x - mean
    var = (diff * diff).sum(-1, keepdim=True) / d
    return diff * (1.0 / torch.sqrt(var + eps))


def grouped_res_ln(res: torch.Tensor, proj: torch.Tensor, bias: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """One stream of ds::grouped_res_ln — grouped_res_ln.py:74-113: x = res + proj + bias
    summed in fp32 (no intermediate rounding), LayerNorm, one rounding to bf16."""
    x = res.float() + proj.float() + bias.float()
    return _ln_rows_fp32(x, eps).to(torch.bfloat16)


def vl_epilogue_ln(res: torch.Tensor, proj_bias: torch.Tensor, w3_bias: torch.Tensor, w3_out: torch.Tensor,
                   eps: float = 1e-6):
    """ds::vl_epilogue_ln — vl_epilogue_ln.py:62-85: new = ((res + proj_bias) + w3_bias) + w3_out
    as bf16 tensor adds (each rounded), ln = LayerNorm(new) in fp32, one rounding."""
    new = ((res + proj_bias) + w3_bias) + w3_out
    return new, _ln_rows_fp32(new.float(), eps).to(torch.bfloat16)


def ss_epilogue_ln(hidden: torch.Tensor, residual: Optional[torch.Tensor] = None, eps: float = 1e-6):
    """ss::fused_epilogue_ln — ss_epilogue_ln.py:60-79: new = hidden + residual (bf16 add),
    ln = LayerNorm(new); without residual ln = LayerNorm(hidden)."""
    new = hidden + residual if residual is not None else hidden
    return new, _ln_rows_fp32(new.float(), eps).to(torch.bfloat16)


def add_rmsnorm(hidden: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                deepstack: Optional[torch.Tensor] = None, eps: float = 1e-6):
    """rldx_backbone::fused_epilogue_add{2,3}_rmsnorm in the eager arithmetic the op files
    promise (op_fused_epilogue_add2_rmsnorm.py:7-10): the decoder layer's
    `residual + hidden_states` (bf16), the DeepStack add (bf16,
    Qwen3-VL `_deepstack_process`), then Qwen3VLTextRMSNorm (modeling_qwen3_vl.py:366-371)."""
    new = residual + hidden
    if deepstack is not None:
        new = new + deepstack
    return new, qwen_rmsnorm(new, weight, eps)
