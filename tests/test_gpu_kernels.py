"""GPU parity tests: each HIP kernel, called through the C ABI, against the CPU oracle.

Tolerances: fp32 max-abs <= 1e-5; bf16 max-abs <= 2e-2 and relative L2 <= 1e-2.
SwiGLU is additionally required to be bit-exact.
"""

import math

import numpy as np
import pytest
import torch

from oracle import cpu_reference as ref
from rldx_amd import functional as Fn
from rldx_amd import workloads as W
from tolerances import assert_bf16_close, assert_fp32_close

pytestmark = pytest.mark.gpu


def packed_kv_layout(k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """CPU construction of the packed K/V tiles from their definition: for tile t,
    lane l, element i, K chunk ks holds K[32t + l%32][16 ks + 8 (l//32) + i] and V
    chunk 2 db + s2 holds V[32t + 16 s2 + 8 (i//4) + 4 (l//32) + i%4][32 db + l%32];
    keys past the end are zero.  k, v: [B, H, S, D] bf16 -> [B, H, tiles * 64 * D]."""
    B, H, S, D = k.shape
    T = (S + 31) // 32
    kp = torch.zeros(B, H, T * 32, D, dtype=k.dtype)
    vp = torch.zeros_like(kp)
    kp[:, :, :S], vp[:, :, :S] = k, v
    kp, vp = kp.view(B, H, T, 32, D), vp.view(B, H, T, 32, D)
    lane = torch.arange(64)[None, :, None]
    i = torch.arange(8)[None, None, :]
    c = torch.arange(D // 16)[:, None, None]
    k_key = (lane % 32).expand(D // 16, 64, 8)
    k_d = 16 * c + 8 * (lane // 32) + i
    v_key = 16 * (c % 2) + 8 * (i // 4) + 4 * (lane // 32) + i % 4
    v_d = (32 * (c // 2) + lane % 32).expand(D // 16, 64, 8)
    kpart = kp[:, :, :, k_key, k_d].reshape(B, H, T, -1)
    vpart = vp[:, :, :, v_key, v_d].reshape(B, H, T, -1)
    return torch.cat([kpart, vpart], dim=3).reshape(B, H, -1)


def _all_bf16():
    u = np.arange(65536, dtype=np.uint32) << 16
    return torch.from_numpy(u.view(np.float32).copy()).to(torch.bfloat16)


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows", [1, 64, 1024])
def test_swiglu_exhaustive_gate_bitexact(dev, rows):
    """Every bf16 gate value, several up values (3e-30 gives fp32 denormal
    products): bit-identical to eager CPU.  rows > 1 spreads the gates over a
    [rows, 65536 / rows] layout (row index from the chunk index)."""
    g = _all_bf16().view(rows, -1)
    for up_val in (1.0, -3.0, 0.3125, 3e-30):
        x = torch.cat([g, torch.full_like(g, up_val)], dim=1)
        y = Fn.swiglu(x.to(dev)).cpu()
        r = ref.swiglu(x)
        same = (y.view(torch.int16) == r.view(torch.int16)) | (torch.isnan(y) & torch.isnan(r))
        assert bool(same.all()), f"up={up_val}: {int((~same).sum())} mismatching bf16 words"


@pytest.mark.parametrize("tokens", [2048, 64])
def test_swiglu_workload_bitexact(dev, tokens):
    cfg = W.SwigluCfg(tokens=tokens)
    x = W.swiglu_inputs(cfg)["x"]
    y = Fn.swiglu(x.to(dev)).cpu()
    r = ref.swiglu(x)
    assert_bf16_close(y, r, f"swiglu {tokens}")
    assert torch.equal(y.view(torch.int16), r.view(torch.int16))


@pytest.mark.parametrize("rows,n_half", [(0, 64), (1, 8), (3, 13), (5, 1000), (7, 4096), (333, 1384), (2, 8 * 4099)])
def test_swiglu_ragged(dev, rows, n_half):
    g = torch.Generator().manual_seed(rows * 1000 + n_half)
    x = (3 * torch.randn(rows, 2 * n_half, generator=g)).to(torch.bfloat16)
    y = Fn.swiglu(x.to(dev)).cpu()
    assert torch.equal(y.view(torch.int16), ref.swiglu(x).view(torch.int16))


def test_swiglu_strided_rows_and_bias(dev):
    g = torch.Generator().manual_seed(11)
    big = torch.randn(37, 2 * 512 + 64, generator=g).to(torch.bfloat16)
    x = big[:, : 2 * 512]  # row stride 1088, not the packed width
    bias = (0.5 * torch.randn(1024, generator=g)).to(torch.bfloat16)
    y = Fn.swiglu(x.to(dev), bias=bias.to(dev)).cpu()
    assert torch.equal(y.view(torch.int16), ref.swiglu(x, bias).view(torch.int16))


def test_grouped_swiglu_bias(dev):
    import rldx_amd.ops  # noqa: F401  registers ds::grouped_swiglu

    g = torch.Generator().manual_seed(5)
    sa = torch.randn(18, 2 * 4096, generator=g).to(torch.bfloat16)
    vl = torch.randn(64, 2 * 10922, generator=g).to(torch.bfloat16)
    sb = torch.randn(2 * 4096, generator=g).to(torch.bfloat16)
    vb = torch.randn(2 * 10922, generator=g).to(torch.bfloat16)
    so, vo = torch.ops.ds.grouped_swiglu(sa.to(dev), sb.to(dev), vl.to(dev), vb.to(dev), 18, 64, 4096, 10922)
    assert torch.equal(so.cpu().view(torch.int16), ref.swiglu(sa, sb).view(torch.int16))
    assert torch.equal(vo.cpu().view(torch.int16), ref.swiglu(vl, vb).view(torch.int16))


# ---------------------------------------------------------------------------
# RMSNorm + RoPE
# ---------------------------------------------------------------------------
def test_rmsnorm_rope_half_fp32_workload(dev):
    cfg = W.RmsRopeCfg()
    inp = W.rmsnorm_rope_inputs(cfg)
    q, k, w, cos, sin = (inp[n] for n in ("q", "k", "w", "cos", "sin"))
    qo, ko = Fn.qk_rmsnorm_rope_half(q.to(dev), k.to(dev), w.to(dev), w.to(dev), cos.to(dev), sin.to(dev), cfg.eps)
    rq, rk = ref.qk_rmsnorm_rope_half(q, k, w, w, cos, sin, cfg.eps)
    assert_fp32_close(qo, rq, "q")
    assert_fp32_close(ko, rk, "k")


@pytest.mark.parametrize("D,hq,hk,S", [(128, 28, 4, 1280), (64, 3, 2, 77), (128, 2, 1, 5)])
def test_rmsnorm_rope_half_bf16(dev, D, hq, hk, S):
    g = torch.Generator().manual_seed(D + S)
    q = torch.randn(1, S, hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, S, hk, D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.02 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.02 * torch.randn(D, generator=g)).to(torch.bfloat16)
    cos, sin = W.qwen_rope_cos_sin(S, D, 1e6, dtype=torch.bfloat16)
    qo, ko = Fn.qk_rmsnorm_rope_half(*(t.to(dev) for t in (q, k, qw, kw, cos, sin)))
    rq, rk = ref.qk_rmsnorm_rope_half(q, k, qw, kw, cos, sin)
    assert_bf16_close(qo, rq, "q")
    assert_bf16_close(ko, rk, "k")


@pytest.mark.parametrize("dtype,D,hq,hk,S", [(torch.float32, 64, 16, 16, 4096), (torch.bfloat16, 128, 12, 4, 8192),
                                              (torch.bfloat16, 128, 6, 2, 16384)])
def test_rmsnorm_rope_half_large_launches(dev, dtype, D, hq, hk, S):
    """Launches of >= 2^21 threads' worth of rows take 4 or 2 heads per thread
    (whichever divides both head counts): the cases take 4, 4 and 2.
    Norm weights ~0.5 keep |out| below 4: over millions of rows a normalised
    element reaches 5, where one bf16 ulp (0.031) exceeds the 2e-2 bound and
    the kernel's and the oracle's fp32 row sums (different orders) flip a
    rounding now and then."""
    g = torch.Generator().manual_seed(S + hq)
    q = torch.randn(1, S, hq, D, generator=g).to(dtype)
    k = torch.randn(1, S, hk, D, generator=g).to(dtype)
    qw = (0.5 + 0.01 * torch.randn(D, generator=g)).to(dtype)
    kw = (0.5 + 0.01 * torch.randn(D, generator=g)).to(dtype)
    cos, sin = W.qwen_rope_cos_sin(S, D, 1e6, dtype=dtype)
    qo, ko = Fn.qk_rmsnorm_rope_half(*(t.to(dev) for t in (q, k, qw, kw, cos, sin)))
    rq, rk = ref.qk_rmsnorm_rope_half(q, k, qw, kw, cos, sin)
    close = assert_fp32_close if dtype == torch.float32 else assert_bf16_close
    close(qo, rq, "q")
    close(ko, rk, "k")


def _msat_streams(D, H, sizes, seed):
    g = torch.Generator().manual_seed(seed)
    inner = H * D
    streams = []
    for si, n in enumerate(sizes):
        qkv = torch.randn(n, 3 * inner + 16, generator=g).to(torch.bfloat16)[:, : 3 * inner + 8]
        qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
        kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
        if si == 0:
            cos = sin = None
        else:
            ids = torch.zeros(n, 2, dtype=torch.long)
            ids[:, 0] = 1 if si == 2 else 0
            ids[:, 1] = torch.arange(n)
            cos, sin = W.msat_rope_tables(ids, D)
        streams.append((qkv, qw, kw, cos, sin))
    return streams


@pytest.mark.parametrize("D,H,sizes", [(128, 12, (512, 64, 32)), (64, 24, (64, 18)), (64, 4, (3, 0, 5))])
def test_msat_qkv_norm_rope(dev, D, H, sizes):
    streams = _msat_streams(D, H, sizes, seed=D + H)
    specs = [Fn.StreamSpec(*(t.to(dev) if t is not None else None for t in s)) for s in streams if s[0].shape[0] > 0]
    q, k, v = Fn.msat_qkv_norm_rope(specs, H, D)
    rq, rk, rv = ref.msat_qkv_norm_rope([s for s in streams if s[0].shape[0] > 0], H, D)
    assert torch.equal(v.cpu(), rv)
    assert_bf16_close(q, rq, "q")
    assert_bf16_close(k, rk, "k")
    # packed K/V output mode: same Q, K/V tiles equal to the standalone packing of K and V
    q2, kvp = Fn.msat_qkv_norm_rope(specs, H, D, kv_packed=True)
    assert torch.equal(q2, q)
    assert torch.equal(kvp, Fn.kv_pack(k.unsqueeze(0), v.unsqueeze(0))[0])
    assert torch.equal(kvp.cpu(), packed_kv_layout(k.cpu().unsqueeze(0), v.cpu().unsqueeze(0))[0])


@pytest.mark.parametrize("D,H,sizes,per", [(128, 12, (512, 64, 32), (512, 56, 32)), (64, 24, (96, 32, 17), (96, 18, 17)),
                                          (64, 4, (3, 5), (3, 5))])
def test_msat_qkv_norm_rope_batch(dev, D, H, sizes, per):
    """rldx_msat_qkv_norm_rope_batch_bf16: three batch entries in one launch,
    each stream's rows stacked entry after entry (`per` rows apart; where
    per < sizes, an entry's last rows are the next entry's first, as the
    batched RLDX chain reads its padding rows), equal bit for bit to one
    launch per entry on the same rows, for the (q, k, v) and packed outputs."""
    B = 3
    g = torch.Generator().manual_seed(D + H + 7)
    inner = H * D
    streams = _msat_streams(D, H, sizes, seed=D + H + 1)
    bufs = []
    for (qkv, qw, kw, cos, sin), n, p in zip(streams, sizes, per):
        rows = (B - 1) * p + n
        bufs.append((torch.randn(rows, 3 * inner + 8, generator=g).to(torch.bfloat16).to(dev), qw.to(dev), kw.to(dev),
                     None if cos is None else cos.to(dev), None if sin is None else sin.to(dev)))
    for kv_packed in (False, True):
        specs = [Fn.StreamSpec(buf[:n], qw, kw, cos, sin) for (buf, qw, kw, cos, sin), n in zip(bufs, sizes)]
        got = Fn.msat_qkv_norm_rope(specs, H, D, kv_packed=kv_packed, batch=B, batch_rows=list(per))
        for b in range(B):
            one = [Fn.StreamSpec(buf[b * p:b * p + n], qw, kw, cos, sin)
                   for (buf, qw, kw, cos, sin), n, p in zip(bufs, sizes, per)]
            want = Fn.msat_qkv_norm_rope(one, H, D, kv_packed=kv_packed)
            for x, y in zip(got, want):
                assert torch.equal(x[b].view(torch.int16), y.view(torch.int16)), (kv_packed, b)
    # a stream whose last entry would read past its buffer is refused on the host
    bad = [Fn.StreamSpec(buf[:n], qw, kw, cos, sin) for (buf, qw, kw, cos, sin), n in zip(bufs, sizes)]
    with pytest.raises(RuntimeError):
        Fn.msat_qkv_norm_rope(bad, H, D, kv_packed=True, batch=B + 1, batch_rows=list(per))


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
def test_joint_attention_workload(dev):
    cfg = W.JointAttnCfg()
    inp = W.joint_attn_inputs(cfg)
    bias = ref.mask_to_bias(inp["kv_mask"])
    o = Fn.attention(inp["q"].to(dev), inp["k"].to(dev), inp["v"].to(dev), key_bias=bias.to(dev))
    r = ref.sdpa(inp["q"], inp["k"], inp["v"], key_bias=bias)
    assert_bf16_close(o, r, "joint attention")


def test_gqa_prefill_workload(dev):
    cfg = W.GqaCfg()
    inp = W.gqa_inputs(cfg)
    M, Hq, Hkv, D = cfg.seq, cfg.q_heads, cfg.kv_heads, cfg.head_dim
    qkv = inp["qkv"]
    q = qkv[:, : Hq * D].reshape(1, M, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(1, M, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].reshape(1, M, Hkv, D)
    rq, rk = ref.qk_rmsnorm_rope_half(q, k, inp["q_norm_w"], inp["k_norm_w"], inp["cos"], inp["sin"])
    o = Fn.attention(rq.to(dev), rk.to(dev), v.to(dev), causal=True, layout="bshd")
    r = ref.sdpa(rq.transpose(1, 2), ref.repeat_kv(rk.transpose(1, 2), Hq // Hkv),
                 ref.repeat_kv(v.transpose(1, 2), Hq // Hkv), causal=True).transpose(1, 2)
    assert_bf16_close(o, r, "gqa causal")


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,causal,masked", [
    (2, 3, 3, 77, 77, 64, False, True),
    (1, 4, 2, 130, 130, 128, True, False),
    (1, 2, 1, 1, 1, 128, True, False),
    (1, 2, 2, 200, 65, 128, False, True),
    (2, 7, 1, 64, 64, 64, True, False),
    # large grids (several workgroups per CU)
    (4, 32, 8, 512, 512, 128, True, False),
    (4, 32, 32, 520, 520, 64, False, True),
    # GQA at prefill sizes: 7 query heads per KV head at head_dim 64, 8 per KV head
    # non-causal over two batch entries, 4 per KV head with a ragged end
    (1, 28, 4, 1024, 1024, 64, True, False),
    (2, 16, 2, 1024, 1024, 128, False, False),
    (1, 32, 8, 1000, 1000, 128, True, False),
])
def test_attention_shapes(dev, B, Hq, Hkv, Sq, Sk, D, causal, masked):
    g = torch.Generator().manual_seed(B * 100 + Sq + Sk + D)
    q = torch.randn(B, Hq, Sq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, Sk, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, Sk, D, generator=g).to(torch.bfloat16)
    bias = None
    if masked:
        m = torch.ones(B, Sk)
        m[:, -3:] = 0
        bias = ref.mask_to_bias(m)
    o = Fn.attention(q.to(dev), k.to(dev), v.to(dev), key_bias=None if bias is None else bias.to(dev), causal=causal)
    r = ref.sdpa(q, ref.repeat_kv(k, Hq // Hkv), ref.repeat_kv(v, Hq // Hkv), key_bias=bias, causal=causal)
    assert_bf16_close(o, r, "attention")


@pytest.mark.parametrize("D,causal", [(128, False), (64, False), (128, True)])
def test_attention_bias_patterns(dev, D, causal):
    """Key bias with a different pattern per batch: dense float values (every
    tile carries bias), and a sparse row (masked keys in middle tiles, one
    positive entry in the first tile, zeros elsewhere)."""
    g = torch.Generator().manual_seed(D + 7 * causal)
    B, Hq, Hkv, S = 2, 4, 2, 300
    q = torch.randn(B, Hq, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    bias = torch.zeros(B, S)
    bias[0] = 0.5 * torch.randn(S, generator=g)
    bias[1, 100:141] = float("-inf")
    bias[1, 7] = 1.5
    o = Fn.attention(q.to(dev), k.to(dev), v.to(dev), key_bias=bias.to(dev), causal=causal)
    r = ref.sdpa(q, ref.repeat_kv(k, Hq // Hkv), ref.repeat_kv(v, Hq // Hkv), key_bias=bias, causal=causal)
    assert_bf16_close(o, r, "attention bias patterns")


@pytest.mark.parametrize("S,D,layout", [(608, 128, "bhsd"), (77, 64, "bshd"), (1, 128, "bhsd"), (1280, 128, "bshd")])
def test_kv_pack_layout(dev, S, D, layout):
    """Packed K/V tiles, element for element, against the layout definition."""
    g = torch.Generator().manual_seed(S + D)
    k = torch.randn(2, 3, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 3, S, D, generator=g).to(torch.bfloat16)
    if layout == "bshd":
        kd, vd = k.transpose(1, 2).contiguous().to(dev), v.transpose(1, 2).contiguous().to(dev)
    else:
        kd, vd = k.to(dev), v.to(dev)
    kvp = Fn.kv_pack(kd, vd, layout=layout).cpu()
    assert torch.equal(kvp, packed_kv_layout(k, v))


def test_attention_packed_matches_attention(dev):
    g = torch.Generator().manual_seed(21)
    q = torch.randn(1, 12, 608, 128, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(1, 12, 608, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(1, 12, 608, 128, generator=g).to(torch.bfloat16).to(dev)
    bias = torch.zeros(608, device=dev)
    bias[-8:] = float("-inf")
    a = Fn.attention(q, k, v, key_bias=bias)
    b = Fn.attention_packed(q, Fn.kv_pack(k, v), 608, key_bias=bias)
    assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# operator boundary (reference op names)
# ---------------------------------------------------------------------------
def test_backbone_fused_attention_op(dev):
    import rldx_amd.ops  # noqa: F401

    cfg = W.GqaCfg()
    inp = W.gqa_inputs(cfg)
    ssin = W.signed_sin(inp["sin"])
    args = (inp["qkv"], inp["q_norm_w"], W.norm_weight_rot(inp["q_norm_w"]), inp["k_norm_w"],
            W.norm_weight_rot(inp["k_norm_w"]), inp["cos"], ssin)
    o = torch.ops.rldx_backbone.fused_attention(*(t.to(dev) for t in args), num_heads=cfg.q_heads,
                                                num_kv_heads=cfg.kv_heads, head_dim=cfg.head_dim)
    r = ref.llm_fused_attention(inp["qkv"], inp["q_norm_w"], inp["k_norm_w"], inp["cos"], inp["sin"],
                                cfg.q_heads, cfg.kv_heads, cfg.head_dim)
    assert o.shape == (cfg.seq, cfg.q_heads * cfg.head_dim)
    assert_bf16_close(o, r, "rldx_backbone::fused_attention")


@pytest.mark.parametrize("M,Hq,Hkv,D", [(100, 4, 2, 64), (333, 14, 2, 128), (257, 16, 2, 64), (169, 32, 8, 128),
                                        (70, 12, 2, 128), (150, 10, 2, 128), (1, 8, 2, 128),
                                        (1100, 28, 4, 64), (2048, 16, 2, 128), (1055, 32, 8, 128)])
def test_backbone_fused_attention_op_shapes(dev, M, Hq, Hkv, D):
    """Groups of 2 to 8 query heads per KV head, from one token to prefill sizes
    (1055 - 2048 tokens), ragged sequence ends, head_dim 64 and 128."""
    import rldx_amd.ops  # noqa: F401

    cfg = W.GqaCfg(q_heads=Hq, kv_heads=Hkv, head_dim=D, seq=M, seed=M)
    inp = W.gqa_inputs(cfg)
    args = (inp["qkv"], inp["q_norm_w"], W.norm_weight_rot(inp["q_norm_w"]), inp["k_norm_w"],
            W.norm_weight_rot(inp["k_norm_w"]), inp["cos"], W.signed_sin(inp["sin"]))
    o = torch.ops.rldx_backbone.fused_attention(*(t.to(dev) for t in args), num_heads=Hq, num_kv_heads=Hkv,
                                                head_dim=D)
    r = ref.llm_fused_attention(inp["qkv"], inp["q_norm_w"], inp["k_norm_w"], inp["cos"], inp["sin"], Hq, Hkv, D)
    assert_bf16_close(o, r, "rldx_backbone::fused_attention")


def test_ds_fused_attention_3way_op(dev):
    import rldx_amd.ops  # noqa: F401

    D, H = 128, 12
    streams = _msat_streams(D, H, (512, 64, 32), seed=3)
    (vl, qvl, kvl, _, _), (sa, qsa, ksa, csa, ssa), (p, qp, kp, cp, sp) = streams
    kv_mask = torch.ones(1, 608)
    kv_mask[:, -8:] = 0
    args = [sa, vl, p, qsa, ksa, qvl, kvl, qp, kp, csa, ssa, cp, sp]
    o = torch.ops.ds.fused_attention_3way(*(t.to(dev) for t in args), 64, 512, 32, num_heads=H, head_dim=D,
                                          kv_mask=kv_mask.to(dev))
    q, k, v = ref.msat_qkv_norm_rope(streams, H, D)
    r = ref.sdpa(q[None], k[None], v[None], key_bias=ref.mask_to_bias(kv_mask))[0]
    r = r.permute(1, 0, 2).reshape(1, 608, H * D)
    assert_bf16_close(o, r, "ds::fused_attention_3way")


def test_ss_fused_attention_2way_op(dev):
    import rldx_amd.ops  # noqa: F401

    D, H = 64, 24
    g = torch.Generator().manual_seed(9)
    M, n_sa = 82, 18
    qkv = torch.randn(M, 16896, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    ids = torch.zeros(n_sa, 2, dtype=torch.long)
    ids[:, 1] = torch.arange(n_sa)
    cos, sin = W.msat_rope_tables(ids, D)
    o = torch.ops.ss.fused_attention_2way(qkv.to(dev), qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev), n_sa)
    q, k, v = ref.msat_qkv_norm_rope([(qkv[: M - n_sa], qw, kw, None, None), (qkv[M - n_sa:], qw, kw, cos, sin)], H, D)
    r = ref.sdpa(q[None], k[None], v[None])[0].permute(1, 0, 2).reshape(1, M, H * D)
    assert_bf16_close(o, r, "ss::fused_attention_2way")
