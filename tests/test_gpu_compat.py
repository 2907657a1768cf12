"""GPU parity through the drop-in module mirror: every launcher the reference's
chains import, called by the reference's module and function names after
rldx_amd.compat.install(), against the CPU oracle (or bit-exact where the
oracle's rounding chain is the kernel's: SwiGLU and the residual sums)."""

import sys

import pytest
import torch

from oracle import cpu_reference as ref
from rldx_amd import compat
from rldx_amd import workloads as W
from tolerances import assert_bf16_close, assert_fp32_close

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


@pytest.fixture(scope="module")
def mods():
    compat.install()
    yield sys.modules
    compat.uninstall()


def _r(shape, g, std=1.0, mean=0.0):
    return (mean + std * torch.randn(*shape, generator=g)).to(BF16)


def _eq(a, b):
    return torch.equal(a.cpu().view(torch.int16), b.view(torch.int16))


def test_double_stream_launchers(dev, mods):
    """fused_vl_epilogue_ln (static out buffers), fused_grouped_res_ln and
    fused_grouped_swiglu (row / width defaults) at the release shapes."""
    from double_stream.engine.kernels.grouped_res_ln import fused_grouped_res_ln
    from double_stream.engine.kernels.grouped_swiglu import fused_grouped_swiglu
    from double_stream.engine.kernels.vl_epilogue_ln import fused_vl_epilogue_ln

    g = torch.Generator().manual_seed(301)
    r, w3, pb, wb = _r((1, 64, 4096), g, 2.0), _r((64, 4096), g), _r((4096,), g, 0.3), _r((4096,), g, 0.3)
    nv_buf, ln_buf = torch.empty(1, 64, 4096, dtype=BF16, device=dev), torch.empty(1, 64, 4096, dtype=BF16, device=dev)
    nv, ln = fused_vl_epilogue_ln(r.to(dev), pb.to(dev), wb.to(dev), w3.to(dev), new_vl_out=nv_buf, ln_vl_out=ln_buf)
    rn, rl = ref.vl_epilogue_ln(r[0], pb, wb, w3)
    assert nv.data_ptr() == nv_buf.data_ptr() and ln.data_ptr() == ln_buf.data_ptr()
    assert _eq(nv[0], rn)
    assert_bf16_close(ln[0], rl, "fused_vl_epilogue_ln")

    sr, sp, sb = _r((1, 18, 1536), g, 2.0), _r((18, 1536), g), _r((1536,), g, 0.5)
    vr, vp, vb = _r((1, 64, 4096), g, 2.0), _r((64, 4096), g), _r((4096,), g, 0.5)
    so, vo = fused_grouped_res_ln(sr.to(dev), sb.to(dev), sp.to(dev), vr.to(dev), vb.to(dev), vp.to(dev))
    assert so.shape == (1, 18, 1536) and vo.shape == (1, 64, 4096)
    assert_bf16_close(so[0], ref.grouped_res_ln(sr[0], sp, sb), "fused_grouped_res_ln sa")
    assert_bf16_close(vo[0], ref.grouped_res_ln(vr[0], vp, vb), "fused_grouped_res_ln vl")

    sa, sab = _r((18, 2 * 4096), g), _r((2 * 4096,), g)
    vl, vlb = _r((64, 2 * 10922), g), _r((2 * 10922,), g)
    so, vo = fused_grouped_swiglu(sa.to(dev), sab.to(dev), vl.to(dev), vlb.to(dev))
    assert so.shape == (18, 4096) and vo.shape == (64, 10922)
    assert _eq(so, ref.swiglu(sa, sab)) and _eq(vo, ref.swiglu(vl, vlb))


def test_single_stream_launchers(dev, mods):
    from single_stream.engine.kernels.fused_mlp_swiglu import fused_mlp_swiglu
    from single_stream.engine.kernels.ss_epilogue_ln import fused_ss_epilogue_ln

    g = torch.Generator().manual_seed(302)
    h, res = _r((1, 82, 1536), g), _r((1, 82, 1536), g, 2.0)
    nh, ln = fused_ss_epilogue_ln(h.to(dev), residual=res.to(dev))
    rn, rl = ref.ss_epilogue_ln(h[0], res[0])
    assert _eq(nh[0], rn)
    assert_bf16_close(ln[0], rl, "fused_ss_epilogue_ln")
    nh0, ln0 = fused_ss_epilogue_ln(h.to(dev))
    assert_bf16_close(ln0[0], ref.ss_epilogue_ln(h[0])[1], "fused_ss_epilogue_ln without residual")

    x, w, b = _r((82, 1536), g), _r((2 * 1024, 1536), g, 0.02), _r((2 * 1024,), g, 0.1)
    y = fused_mlp_swiglu(x.to(dev), w.to(dev), b.to(dev))
    lin = (x.float() @ w.float().t() + b.float()).to(BF16)
    assert y.shape == (82, 1024)
    assert_bf16_close(y, ref.swiglu(lin), "fused_mlp_swiglu")
    assert_bf16_close(fused_mlp_swiglu(x.to(dev), w.to(dev), b.to(dev), split_k=2), ref.swiglu(lin),
                      "fused_mlp_swiglu split_k=2")


def test_llm_launchers(dev, mods):
    """fused_llm_attention.forward with the tables and weights from the
    module's own prepare_* helpers, at the reference backbone's shape (32 / 8
    heads x 128, 169 tokens), into a static `out` buffer; add2 / add3 RMSNorm."""
    from backbone.llm.engine.kernels.fused_add2_rmsnorm import forward as add2
    from llm.engine.kernels.fused_add3_rmsnorm import forward as add3
    from llm.engine.kernels.fused_llm_attention import forward, prepare_norm_weight_rot, prepare_signed_sin

    cfg = W.GqaCfg(seq=169, q_heads=32, kv_heads=8, head_dim=128, seed=169)
    inp = W.gqa_inputs(cfg)
    D = cfg.head_dim
    args = [inp["qkv"], inp["q_norm_w"], prepare_norm_weight_rot(inp["q_norm_w"], D), inp["k_norm_w"],
            prepare_norm_weight_rot(inp["k_norm_w"], D), inp["cos"], prepare_signed_sin(inp["sin"], D)]
    out = torch.empty(cfg.seq, cfg.q_heads * D, dtype=BF16, device=dev)
    o = forward(*(t.to(dev) for t in args), num_heads=cfg.q_heads, num_kv_heads=cfg.kv_heads, head_dim=D, out=out)
    assert o.data_ptr() == out.data_ptr()
    r = ref.llm_fused_attention(inp["qkv"], inp["q_norm_w"], inp["k_norm_w"], inp["cos"], inp["sin"], cfg.q_heads,
                                cfg.kv_heads, D)
    assert_bf16_close(o, r, "fused_llm_attention.forward")

    g = torch.Generator().manual_seed(303)
    h, res, ds, wt = _r((169, 2048), g), _r((169, 2048), g, 3.0), _r((169, 2048), g, 0.5), _r((2048,), g, 0.1, 1.0)
    new, normed = add2(h.to(dev), res.to(dev), wt.to(dev))
    rn, rnorm = ref.add_rmsnorm(h, res, wt)
    assert _eq(new, rn)
    assert_bf16_close(normed, rnorm, "fused_add2_rmsnorm.forward")
    new, normed = add3(h.to(dev), res.to(dev), ds.to(dev), wt.to(dev))
    rn, rnorm = ref.add_rmsnorm(h, res, wt, ds)
    assert _eq(new, rn)
    assert_bf16_close(normed, rnorm, "fused_add3_rmsnorm.forward")


def test_vision_and_memory_launchers(dev, mods):
    from memory.engine.kernels.fused_add2_rmsnorm import forward as mem_add2
    from memory.engine.kernels.fused_memory_attention import forward as mem_forward
    from memory.engine.kernels.fused_memory_attention import prepare_rope_buffers
    from vision_encoder.engine.kernels.fused_vision_attention import forward as vit_forward

    inp = W.vit_attention_inputs()
    t = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in inp.items()}
    o = vit_forward(t["qkv"], t["rope_cos"], t["rope_sin"], t["cu_seqlens"], t["scaling"], t["num_heads"],
                    t["head_dim"])
    assert_bf16_close(o, ref.vision_attention(**inp), "fused_vision_attention.forward")

    mc = W.MemAttnCfg()
    mi = W.memory_attention_inputs(mc)
    cos_ref, ssin_ref = mi["cos"], mi["signed_sin"]

    class Rotary:  # rotary-embedding module convention: (x, position_ids (1, M)) -> cos, sin (1, M, D)
        dim = mc.head_dim

        def __call__(self, x, position_ids):
            assert position_ids.shape == (1, mc.tokens)
            sin = torch.cat([-ssin_ref[:, : self.dim // 2], ssin_ref[:, self.dim // 2:]], dim=-1)  # unsigned
            return cos_ref[None].to(x.device), sin[None].to(x.device)

    cos, ssin = prepare_rope_buffers(Rotary(), torch.arange(mc.tokens, device=dev)[None], dev)
    assert _eq(cos, cos_ref) and _eq(ssin, ssin_ref)
    o = mem_forward(mi["qkv"].to(dev), cos, ssin, mc.heads, mc.head_dim, mc.n_cog)
    assert_bf16_close(o, ref.memory_attention(**mi), "fused_memory_attention.forward")

    g = torch.Generator().manual_seed(304)
    h, res, wt = _r((64, 2048), g), _r((64, 2048), g, 3.0), _r((2048,), g, 0.1, 1.0)
    new, normed = mem_add2(h.to(dev), res.to(dev), wt.to(dev))
    rn, rnorm = ref.add_rmsnorm(h, res, wt)
    assert _eq(new, rn)
    assert_bf16_close(normed, rnorm, "memory fused_add2_rmsnorm.forward")
    new2, normed2 = torch.ops.mem.fused_epilogue_add2_rmsnorm(h.to(dev), res.to(dev), wt.to(dev))
    assert torch.equal(new2, new) and torch.equal(normed2, normed)


# ---------------------------------------------------------------------------
# model-level mirrors (rldx.model.modules.*)
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def model():
    compat.install_model()
    yield sys.modules
    compat.uninstall()


@pytest.mark.parametrize("shape,wdtype", [((2, 24, 82, 64), torch.float32), ((1, 12, 608, 128), torch.bfloat16),
                                          ((3, 7, 1536), torch.float32), ((64, 2048), torch.bfloat16),
                                          ((5, 72), torch.float32), ((2, 4, 5, 4096), torch.float32)])
def test_rmsnorm_module(dev, model, shape, wdtype):
    """RMSNorm (norms.py:7-22) against the oracle's one-rounding restatement: bf16
    rows within the bf16 contract, fp32 rows within 1e-5; weight fp32 (the
    parameter) or bf16 (a model cast to bf16)."""
    from rldx.model.modules.norms import RMSNorm

    g = torch.Generator().manual_seed(sum(shape))
    n = RMSNorm(shape[-1], eps=1e-6)
    with torch.no_grad():
        n.weight.copy_(1 + 0.1 * torch.randn(shape[-1], generator=g))
    n = n.to(dev, wdtype)
    x = torch.randn(*shape, generator=g).to(BF16)
    y = n(x.to(dev))
    r = ref.msat_rmsnorm(x, n.weight.detach().cpu(), 1e-6)
    assert y.dtype == BF16 and y.shape == x.shape
    assert_bf16_close(y, r, f"RMSNorm bf16 {shape}")
    xf = torch.randn(*shape, generator=g)
    yf = n(xf.to(dev))
    assert yf.dtype == torch.float32
    assert_fp32_close(yf, ref.msat_rmsnorm(xf, n.weight.detach().cpu(), 1e-6), f"RMSNorm fp32 {shape}")


def test_layernorm_from_create_norm_layer(dev, model):
    from rldx.model.modules.norms import create_norm_layer, create_qk_norm_layers

    g = torch.Generator().manual_seed(7)
    x = (torch.randn(2, 82, 1536, generator=g) * 2 + 0.3).to(BF16)
    y = create_norm_layer("layer_norm", 1536)(x.to(dev))
    assert_bf16_close(y, ref.layer_norm(x), "create_norm_layer('layer_norm')")
    qn, kn = create_qk_norm_layers("rms_norm", 64)
    xq = torch.randn(1, 24, 82, 64, generator=g).to(BF16)
    assert_bf16_close(qn.to(dev)(xq.to(dev)), ref.msat_rmsnorm(xq, torch.ones(64)), "create_qk_norm_layers")


@pytest.mark.parametrize("dtype", [BF16, torch.float32])
@pytest.mark.parametrize("fshape", ["nd", "bnd"])
def test_apply_rotary_emb(dev, model, dtype, fshape):
    """Interleaved RoPE (action_model/ops.py:48-67) against the oracle's complex
    multiplication: a permuted (non-contiguous) q, a separately shaped k, tables
    [N, D/2] or [B, N, D/2] from precompute_freqs_cis."""
    from rldx.model.modules.action_model.ops import apply_rotary_emb, precompute_freqs_cis

    g = torch.Generator().manual_seed(11)
    B, H, N, D = 2, 6, 37, 64
    xq = torch.randn(B, N, H, D, generator=g).to(dtype).permute(0, 2, 1, 3)  # [B, H, N, D] view
    xk = torch.randn(B, 2 * H, N, D, generator=g).to(dtype)
    f = precompute_freqs_cis(D, 64)[:N]
    if fshape == "bnd":
        f = torch.stack([f, precompute_freqs_cis(D, 64, theta=500.0)[5:5 + N]])
    qo, ko = apply_rotary_emb(xq.to(dev), xk.to(dev), f.to(dev))
    fr = f if f.dim() == 3 else f.expand(B, N, D // 2)
    rq = ref.apply_rotary_emb(xq, xq, fr)[0]
    rk = ref.apply_rotary_emb(xk, xk, fr)[0]
    close = assert_bf16_close if dtype == BF16 else assert_fp32_close
    assert qo.dtype == dtype and qo.shape == (B, H, N, D) and ko.shape == (B, 2 * H, N, D)
    close(qo, rq, f"apply_rotary_emb q {dtype} {fshape}")
    close(ko, rk, f"apply_rotary_emb k {dtype} {fshape}")


@pytest.mark.parametrize("dtype", [BF16, torch.float32])
@pytest.mark.parametrize("unsqueeze_dim", [1, 2])
def test_apply_rotary_pos_emb(dev, model, dtype, unsqueeze_dim):
    """Rotate-half RoPE alone (modeling_qwen3_vl.py:377-401): bf16 bit-exact with
    the eager op order (two rounded products, rounded sum), fp32 within 1e-5;
    q [B, H, S, D] (unsqueeze_dim 1) or [B, S, H, D] (2), per-batch tables."""
    from rldx.model.modules.backbone.modeling_qwen3_vl import apply_rotary_pos_emb

    g = torch.Generator().manual_seed(13 + unsqueeze_dim)
    B, H, Hk, S, D = 2, 8, 2, 45, 128
    qs, ks = ((B, H, S, D), (B, Hk, S, D)) if unsqueeze_dim == 1 else ((B, S, H, D), (B, S, Hk, D))
    q, k = torch.randn(*qs, generator=g).to(dtype), torch.randn(*ks, generator=g).to(dtype)
    cos, sin = W.qwen_rope_cos_sin(S + 3, D, 1e6, dtype=dtype)
    cos = torch.stack([cos[:S], cos[3:]])
    sin = torch.stack([sin[:S], sin[3:]])
    qo, ko = apply_rotary_pos_emb(q.to(dev), k.to(dev), cos.to(dev), sin.to(dev), unsqueeze_dim=unsqueeze_dim)
    rq, rk = ref.apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=unsqueeze_dim)
    assert qo.shape == q.shape and ko.shape == k.shape
    if dtype == BF16:
        assert _eq(qo, rq) and _eq(ko, rk)
    else:
        assert_fp32_close(qo, rq, "apply_rotary_pos_emb q fp32")
        assert_fp32_close(ko, rk, "apply_rotary_pos_emb k fp32")


@pytest.mark.parametrize("dims", [(1536, 4096, 1536), (4096, 10922, 4096), (1536, 6144, 1536)])
def test_swiglu_ffn_module(dev, model, dims):
    """SwiGLUFFN (action_model/ops.py:137-161) at the MSAT's widths (SA, VL with
    its padded hidden 10922, SS) against an eager bf16 composition on the same
    weights: linear (fp32 sum + bias, one rounding), silu, product, linear.
    w3 is drawn with std 0.01 sqrt(4096 / hidden) so that |y| stays below 4
    (above it one bf16 ulp, 0.031, exceeds the 2e-2 bound, and the GEMM's and
    the CPU's fp32 sums, in different orders, flip a rounding now and then)."""
    from rldx.model.modules.action_model.ops import SwiGLUFFN

    i, h, o = dims
    g = torch.Generator().manual_seed(h)
    m = SwiGLUFFN(i, h, o)
    with torch.no_grad():
        for name, p in m.named_parameters():
            std = 0.01 * (4096 / h) ** 0.5 if name == "w3.weight" else 0.02
            p.copy_(std * torch.randn(p.shape, generator=g))
    m = m.to(dev, BF16)
    x = torch.randn(1, 82, i, generator=g).to(BF16)
    y = m(x.to(dev))
    sd = {k: v.detach().cpu() for k, v in m.state_dict().items()}
    x12 = (x[0].float() @ sd["w12.weight"].float().t() + sd["w12.bias"].float()).to(BF16)
    hid = ref.swiglu(x12)
    r = (hid.float() @ sd["w3.weight"].float().t() + sd["w3.bias"].float()).to(BF16)
    assert y.shape == (1, 82, o)
    assert_bf16_close(y[0], r, f"SwiGLUFFN {dims}")
    with torch.no_grad():  # an in-place weight update repacks
        m.w3.weight.mul_(0.5)
    y2 = m(x.to(dev))
    r2 = (hid.float() @ (sd["w3.weight"].float() * 0.5).to(BF16).float().t() + sd["w3.bias"].float()).to(BF16)
    assert_bf16_close(y2[0], r2, f"SwiGLUFFN {dims} after an in-place update")
