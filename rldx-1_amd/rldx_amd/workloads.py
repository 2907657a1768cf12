"""The five synthetic workloads of the hot path, with their seeded CPU inputs.

Inputs are generated on the CPU (`torch.manual_seed` + `torch.randn`) so the
GPU kernels and the CPU oracle see bit-identical data; callers move them to the
device.  Seeds: RMSNorm+RoPE 0, joint attention 1 (both given by the workload
definitions), SwiGLU 3, GQA prefill 2, MSAT step 5.
"""

from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass

import torch


def sha256_of(*tensors: torch.Tensor) -> str:
    h = hashlib.sha256()
    for t in tensors:
        t = t.detach().contiguous().cpu()
        h.update(str(tuple(t.shape)).encode())
        h.update(str(t.dtype).encode())
        h.update(t.view(torch.uint8).numpy().tobytes() if t.numel() else b"")
    return h.hexdigest()


# ---------------------------------------------------------------------------
# RoPE tables, built on the host with the reference's fp32 recipes
# ---------------------------------------------------------------------------
def qwen_rope_cos_sin(seq: int, head_dim: int, theta: float, dtype=torch.float32, start: int = 0):
    """Rotate-half tables [seq, D]: inv_freq = 1/theta^(2i/D), emb = cat(f, f).

    rldx/model/modules/backbone/modeling_qwen3_vl.py:331-353 (text MRoPE with
    equal t/h/w positions reduces to 1-D RoPE); default rope init of
    transformers (`1 / base**(arange(0, D, 2)/D)`)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    pos = torch.arange(start, start + seq, dtype=torch.float32)
    freqs = (inv_freq[:, None].float() @ pos[None, :].float()).transpose(0, 1)  # [seq, D/2]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def msat_freqs_cis(dim: int, end: int, theta: float = 10000.0) -> torch.Tensor:
    """precompute_freqs_cis (rldx/model/modules/action_model/ops.py:11-25)."""
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2)[: (dim // 2)].float() / dim))
    t = torch.arange(end, device=freqs.device)
    freqs = torch.outer(t, freqs).float()
    return torch.polar(torch.ones_like(freqs), freqs)


def msat_rope_tables(ids: torch.Tensor, head_dim: int, theta: float = 10000.0, max_seq_len: int = 2048):
    """2-axis RoPE (rope_sa_only axes [D/4, 3D/4]) for position ids [N, 2] ->
    fp32 cos, sin [N, D/2] (RoPEEmbedder1D.forward, ops.py:70-119;
    axes from msat.py:883-893)."""
    axes = [head_dim // 4, head_dim - head_dim // 4]
    parts = []
    for i, ad in enumerate(axes):
        fc = msat_freqs_cis(ad, max_seq_len, theta)
        parts.append(fc[ids[:, i]])
    pe = torch.cat(parts, dim=-1)
    return pe.real.contiguous().float(), pe.imag.contiguous().float()


# ---------------------------------------------------------------------------
# workload 1: RMSNorm + rotate-half RoPE, fp32
# ---------------------------------------------------------------------------
@dataclass
class RmsRopeCfg:
    batch: int = 1
    seq: int = 256
    heads: int = 16
    head_dim: int = 64
    eps: float = 1e-6
    theta: float = 10000.0
    seed: int = 0


def rmsnorm_rope_inputs(cfg: RmsRopeCfg = RmsRopeCfg()):
    g = torch.Generator().manual_seed(cfg.seed)
    shape = (cfg.batch, cfg.seq, cfg.heads, cfg.head_dim)
    q = torch.randn(shape, generator=g)
    k = torch.randn(shape, generator=g)
    w = 1.0 + 0.02 * torch.randn(cfg.head_dim, generator=g)
    cos, sin = qwen_rope_cos_sin(cfg.seq, cfg.head_dim, cfg.theta)
    return dict(q=q, k=k, w=w, cos=cos, sin=sin)


def rmsnorm_rope_bytes(cfg: RmsRopeCfg = RmsRopeCfg()) -> int:
    n = cfg.batch * cfg.seq * cfg.heads * cfg.head_dim * 4
    return 4 * n + cfg.head_dim * 4 + 2 * cfg.seq * cfg.head_dim * 4


# ---------------------------------------------------------------------------
# workload 2: SwiGLU, bf16
# ---------------------------------------------------------------------------
@dataclass
class SwigluCfg:
    tokens: int = 2048
    n_half: int = 11008
    seed: int = 3


def swiglu_inputs(cfg: SwigluCfg = SwigluCfg()):
    g = torch.Generator().manual_seed(cfg.seed)
    x = torch.randn(cfg.tokens, 2 * cfg.n_half, generator=g).to(torch.bfloat16)
    return dict(x=x)


def swiglu_bytes(cfg: SwigluCfg = SwigluCfg()) -> int:
    return cfg.tokens * 2 * cfg.n_half * 2 + cfg.tokens * cfg.n_half * 2


# ---------------------------------------------------------------------------
# workload 3: MSAT joint attention, bf16, non-causal, key padding mask
# ---------------------------------------------------------------------------
@dataclass
class JointAttnCfg:
    heads: int = 16
    head_dim: int = 128
    n_cog: int = 512
    n_action: int = 64
    n_phys: int = 32
    n_phys_pad: int = 8
    seed: int = 1

    @property
    def tokens(self) -> int:
        return self.n_cog + self.n_action + self.n_phys


def joint_attn_inputs(cfg: JointAttnCfg = JointAttnCfg()):
    """Sequence order [VL | SA | P] = cognition | action | physics; the last
    n_phys_pad physics keys are padding (mask 0)."""
    g = torch.Generator().manual_seed(cfg.seed)
    shape = (1, cfg.heads, cfg.tokens, cfg.head_dim)
    s = math.sqrt(cfg.head_dim)
    q = (torch.randn(shape, generator=g) / s).to(torch.bfloat16)
    k = (torch.randn(shape, generator=g) / s).to(torch.bfloat16)
    v = (torch.randn(shape, generator=g) / s).to(torch.bfloat16)
    kv_mask = torch.ones(1, cfg.tokens)
    kv_mask[:, cfg.tokens - cfg.n_phys_pad:] = 0
    return dict(q=q, k=k, v=v, kv_mask=kv_mask)


def joint_attn_flops(cfg: JointAttnCfg = JointAttnCfg()) -> int:
    return 4 * cfg.heads * cfg.tokens * cfg.tokens * cfg.head_dim


# ---------------------------------------------------------------------------
# workload 4: GQA causal prefill with QK-RMSNorm + rotate-half RoPE (theta 1e6)
# ---------------------------------------------------------------------------
@dataclass
class GqaCfg:
    q_heads: int = 28
    kv_heads: int = 4
    head_dim: int = 128
    seq: int = 1280
    theta: float = 1e6
    eps: float = 1e-6
    seed: int = 2


def gqa_inputs(cfg: GqaCfg = GqaCfg()):
    """Packed QKV (M, (Hq + 2*Hkv) * D) bf16 as the QKV GEMM would produce it,
    per-layer norm weights and bf16 cos/sin tables."""
    g = torch.Generator().manual_seed(cfg.seed)
    q = torch.randn(cfg.seq, cfg.q_heads, cfg.head_dim, generator=g)
    k = torch.randn(cfg.seq, cfg.kv_heads, cfg.head_dim, generator=g)
    v = torch.randn(cfg.seq, cfg.kv_heads, cfg.head_dim, generator=g)
    qw = 1.0 + 0.02 * torch.randn(cfg.head_dim, generator=g)
    kw = 1.0 + 0.02 * torch.randn(cfg.head_dim, generator=g)
    qkv = torch.cat([q.reshape(cfg.seq, -1), k.reshape(cfg.seq, -1), v.reshape(cfg.seq, -1)], dim=1)
    cos, sin = qwen_rope_cos_sin(cfg.seq, cfg.head_dim, cfg.theta, dtype=torch.bfloat16)
    return dict(qkv=qkv.to(torch.bfloat16), q_norm_w=qw.to(torch.bfloat16), k_norm_w=kw.to(torch.bfloat16),
                cos=cos, sin=sin)


def gqa_flops(cfg: GqaCfg = GqaCfg()) -> int:
    return 4 * cfg.q_heads * cfg.head_dim * cfg.seq * (cfg.seq + 1) // 2


# ---------------------------------------------------------------------------
# ViT attention (Qwen3-VL vision tower): fused QKV of several images, baked
# 2-D rotary tables, one cu_seqlens segment per image
# ---------------------------------------------------------------------------
@dataclass
class VitAttnCfg:
    images: int = 2
    grid_h: int = 14
    grid_w: int = 14
    heads: int = 16
    head_dim: int = 72
    merge: int = 2
    theta: float = 10000.0
    seed: int = 6
    lengths: tuple = ()  # explicit per-sequence lengths (ragged batches); positions row-major in grid_w columns

    @property
    def seq_lengths(self) -> list:
        return list(self.lengths) if self.lengths else [self.grid_h * self.grid_w] * self.images

    @property
    def tokens(self) -> int:
        return sum(self.seq_lengths)


def vit_positions(cfg: VitAttnCfg) -> torch.Tensor:
    """(row, col) patch coordinates per token, Qwen3VLVisionModel.rot_pos_emb order
    (modeling_qwen3_vl.py:787-824): merge x merge blocks row-major, patches
    row-major inside a block.  Explicit lengths use plain row-major coordinates."""
    if cfg.lengths:
        return torch.cat([torch.stack((torch.arange(n) // cfg.grid_w, torch.arange(n) % cfg.grid_w), dim=-1)
                          for n in cfg.lengths])
    m = cfg.merge
    bh, bw = cfg.grid_h // m, cfg.grid_w // m
    rows = (torch.arange(bh)[:, None, None, None] * m + torch.arange(m)[None, None, :, None]).expand(bh, bw, m, m)
    cols = (torch.arange(bw)[None, :, None, None] * m + torch.arange(m)[None, None, None, :]).expand(bh, bw, m, m)
    one = torch.stack((rows.reshape(-1), cols.reshape(-1)), dim=-1)
    return one.repeat(cfg.images, 1)


def vit_rope_tables(cfg: VitAttnCfg):
    """Baked fp32 cos / sin [M, head_dim]: Qwen3VLVisionRotaryEmbedding(head_dim // 2)
    frequencies looked up at the (row, col) coordinates, emb = cat(f, f)
    (modeling_qwen3_vl.py:84-95, :912-918), rotate_half's sign folded into the
    first half of sin (custom_vision_encoder_chain.py:101-108)."""
    dim = cfg.head_dim // 2
    inv_freq = 1.0 / (cfg.theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    pos = vit_positions(cfg)
    table = torch.outer(torch.arange(int(pos.max()) + 1, dtype=torch.float32), inv_freq)
    freqs = table[pos].flatten(1)  # [M, dim]
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos(), emb.sin()
    sin[:, : cfg.head_dim // 2] = -sin[:, : cfg.head_dim // 2]
    return cos.contiguous(), sin.contiguous()


def vit_attention_inputs(cfg: VitAttnCfg = VitAttnCfg()):
    """Fused QKV (M, 3 * H * D) bf16 ~ N(0, 1), baked rope tables, cu_seqlens
    int32 and scaling = D ** -0.5."""
    g = torch.Generator().manual_seed(cfg.seed)
    M = cfg.tokens
    qkv = torch.randn(M, 3 * cfg.heads * cfg.head_dim, generator=g).to(torch.bfloat16)
    cos, sin = vit_rope_tables(cfg)
    cu = torch.tensor([0] + cfg.seq_lengths, dtype=torch.int64).cumsum(0).to(torch.int32)
    return dict(qkv=qkv, rope_cos=cos, rope_sin=sin, cu_seqlens=cu, scaling=cfg.head_dim ** -0.5,
                num_heads=cfg.heads, head_dim=cfg.head_dim)


def vit_attention_flops(cfg: VitAttnCfg = VitAttnCfg()) -> int:
    """Q K^T and P V of every sequence at the true head_dim."""
    return 4 * cfg.heads * cfg.head_dim * sum(n * n for n in cfg.seq_lengths)


# ---------------------------------------------------------------------------
# TransformerMemory block-causal attention: memory_length timesteps x
# n_cog cognition tokens, 16 heads x 256 (Qwen3-VL-8B text width 4096)
# ---------------------------------------------------------------------------
@dataclass
class MemAttnCfg:
    memory_length: int = 4
    n_cog: int = 16  # block_attn_size
    heads: int = 16
    head_dim: int = 256
    theta: float = 10000.0
    seed: int = 7

    @property
    def tokens(self) -> int:
        return self.memory_length * self.n_cog


def memory_rope_tables(cfg: MemAttnCfg):
    """cos / signed_sin [M, D] bf16: RotaryEmbedding(head_dim) at the block-wise
    positions arange(M) // block_attn_size (memory.py:21-42, :327-334), cast to
    bf16, sin's first half negated (prepare_rope_buffers / prepare_signed_sin,
    fused_memory_attention.py:185-217)."""
    D = cfg.head_dim
    inv_freq = 1.0 / (cfg.theta ** (torch.arange(0, D, 2).float() / D))
    pos = (torch.arange(cfg.tokens) // cfg.n_cog).float()
    freqs = torch.outer(pos, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    return cos.contiguous(), signed_sin(sin)


def memory_attention_inputs(cfg: MemAttnCfg = MemAttnCfg()):
    """Fused QKV (M, 3 * H * D) bf16 ~ N(0, 1) and the bf16 rope tables."""
    g = torch.Generator().manual_seed(cfg.seed)
    qkv = torch.randn(cfg.tokens, 3 * cfg.heads * cfg.head_dim, generator=g).to(torch.bfloat16)
    cos, ssin = memory_rope_tables(cfg)
    return dict(qkv=qkv, cos=cos, signed_sin=ssin, num_heads=cfg.heads, head_dim=cfg.head_dim,
                block_attn_size=cfg.n_cog)


def memory_attention_flops(cfg: MemAttnCfg = MemAttnCfg()) -> int:
    """Q K^T and P V over the visible (query, key) pairs of the block-causal mask."""
    M, B = cfg.tokens, cfg.n_cog
    pairs = sum(min(M, (i // B + 1) * B) for i in range(M))
    return 4 * cfg.heads * cfg.head_dim * pairs


def signed_sin(sin: torch.Tensor) -> torch.Tensor:
    """prepare_signed_sin (fused_llm_attention.py:787-796): first half negated."""
    D = sin.shape[-1]
    sign = torch.ones(D, dtype=sin.dtype, device=sin.device)
    sign[: D // 2] = -1
    return (sign * sin).contiguous()


def norm_weight_rot(w: torch.Tensor) -> torch.Tensor:
    """prepare_norm_weight_rot (fused_llm_attention.py:799-804)."""
    half = w.shape[0] // 2
    return torch.cat([w[half:], w[:half]]).contiguous()
