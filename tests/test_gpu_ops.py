"""GPU parity of the torch.library operators under the reference's names that the
other GPU tests do not call: ds::fused_attention_2way (the op the reference's
double-stream chain calls, custom_double_stream_chain.py:57-96),
ss::fused_attention_3way (custom_expanded_single_stream_chain.py:78) and
rldx_amd::swiglu, each against the CPU oracle, with the reference's argument
shapes (3-D `linear1` outputs, column views of the full-width `linear1` buffers,
row counts below the buffer's).  Then every registered op through
torch.library.opcheck: the schema (no input mutated) and the `register_fake`
output (shape, dtype, strides) against the real op.

Tolerances: bf16 max-abs <= 2e-2 and relative L2 <= 1e-2; SwiGLU bit-exact."""

import pytest
import torch

import rldx_amd.ops  # noqa: F401  (registers the ops)
from oracle import cpu_reference as ref
from rldx_amd import workloads as W
from tolerances import assert_bf16_close

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _norm_w(g, D):
    return (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)


def _tables(n, D, axis0):
    ids = torch.zeros(n, 2, dtype=torch.long)
    ids[:, 0] = axis0
    ids[:, 1] = torch.arange(n)
    return W.msat_rope_tables(ids, D)


def _joint_ref(streams, H, D, kv_mask=None):
    q, k, v = ref.msat_qkv_norm_rope(streams, H, D)
    bias = ref.mask_to_bias(kv_mask) if kv_mask is not None else None
    M = q.shape[1]
    return ref.sdpa(q[None], k[None], v[None], key_bias=bias)[0].permute(1, 0, 2).reshape(1, M, H * D)


def _ds_2way_args(seed, n_sa=18, n_vl=64, H=24, D=64, extra_rows=0):
    """Reference DoubleStreamBlock shapes: sa_qkv / vl_qkv are the (1, n, 3*inner)
    outputs of the SA / VL QKV linears (custom_double_stream_chain.py:57-62)."""
    g = torch.Generator().manual_seed(seed)
    inner = H * D
    sa = torch.randn(1, n_sa + extra_rows, 3 * inner, generator=g).to(BF16)
    vl = torch.randn(1, n_vl + extra_rows, 3 * inner, generator=g).to(BF16)
    qs, ks, qv, kv = (_norm_w(g, D) for _ in range(4))
    cos, sin = _tables(n_sa, D, 0)
    return sa, vl, qs, ks, qv, kv, cos, sin


@pytest.mark.parametrize("extra_rows", [0, 5])
def test_ds_fused_attention_2way_op(dev, extra_rows):
    """[VL | SA] joint attention; `n_sa` / `n_vl` below the buffers' row counts
    take the leading rows (the op's `[:n]` slicing)."""
    H, D, n_sa, n_vl = 24, 64, 18, 64
    sa, vl, qs, ks, qv, kv, cos, sin = _ds_2way_args(5, n_sa, n_vl, H, D, extra_rows)
    o = torch.ops.ds.fused_attention_2way(*(t.to(dev) for t in (sa, vl, qs, ks, qv, kv, cos, sin)), n_sa, n_vl)
    assert o.shape == (1, n_vl + n_sa, H * D) and o.dtype == BF16
    r = _joint_ref([(vl[0, :n_vl], qv, kv, None, None), (sa[0, :n_sa], qs, ks, cos, sin)], H, D)
    assert_bf16_close(o, r, "ds::fused_attention_2way")


def test_ds_fused_attention_2way_op_head_kwargs(dev):
    """The additive num_heads / head_dim kwargs at the synthetic step's 12 x 128."""
    H, D, n_sa, n_vl = 12, 128, 64, 512
    sa, vl, qs, ks, qv, kv, cos, sin = _ds_2way_args(6, n_sa, n_vl, H, D)
    o = torch.ops.ds.fused_attention_2way(*(t.to(dev) for t in (sa, vl, qs, ks, qv, kv, cos, sin)), n_sa, n_vl,
                                          num_heads=H, head_dim=D)
    r = _joint_ref([(vl[0], qv, kv, None, None), (sa[0], qs, ks, cos, sin)], H, D)
    assert_bf16_close(o, r, "ds::fused_attention_2way 12x128")


def _ss_3way_args(seed, n_x, n_sa, n_p, H=24, D=64, mlp=12288):
    """Reference ExpandedSingleStreamBlock shapes: x_qkv / p_qkv are column views
    [:, :3*inner] of the full (n, 3*inner + mlp) linear1 outputs
    (custom_expanded_single_stream_chain.py:66-93)."""
    g = torch.Generator().manual_seed(seed)
    inner = H * D
    x_full = torch.randn(n_x, 3 * inner + mlp, generator=g).to(BF16)
    p_full = torch.randn(n_p, 3 * inner + mlp, generator=g).to(BF16)
    xq, xk, pq, pk = (_norm_w(g, D) for _ in range(4))
    sc, ss = _tables(n_sa, D, 0)
    pc, ps = _tables(n_p, D, 1)
    return x_full, p_full, xq, xk, pq, pk, sc, ss, pc, ps


@pytest.mark.parametrize("masked", [False, True])
def test_ss_fused_attention_3way_op(dev, masked):
    """[VL+SA | P]: RoPE on the last n_sa rows of x and on every P row; with a
    kv_mask, masked VL and padded P keys (1 = visible, 0 = padded)."""
    H, D, n_vl, n_sa, n_p = 24, 64, 80, 18, 16
    n_x = n_vl + n_sa
    x_full, p_full, xq, xk, pq, pk, sc, ss, pc, ps = _ss_3way_args(7, n_x, n_sa, n_p, H, D)
    inner = H * D
    xd, pd = x_full.to(dev), p_full.to(dev)
    kv_mask = None
    if masked:
        kv_mask = torch.ones(1, n_x + n_p)
        kv_mask[:, 70:n_vl] = 0
        kv_mask[:, -4:] = 0
    o = torch.ops.ss.fused_attention_3way(xd[:, : 3 * inner], pd[:, : 3 * inner],
                                          *(t.to(dev) for t in (xq, xk, pq, pk, sc, ss, pc, ps)), n_x, n_sa, n_p,
                                          kv_mask=kv_mask.to(dev) if masked else None)
    assert o.shape == (1, n_x + n_p, inner)
    streams = [(x_full[: n_x - n_sa], xq, xk, None, None), (x_full[n_x - n_sa:], xq, xk, sc, ss),
               (p_full, pq, pk, pc, ps)]
    assert_bf16_close(o, _joint_ref(streams, H, D, kv_mask), f"ss::fused_attention_3way masked={masked}")


def test_ss_fused_attention_2way_op_3d(dev):
    """A 3-D (1, M, C) linear1 output: the op flattens the leading dims."""
    H, D, M, n_sa = 24, 64, 82, 18
    g = torch.Generator().manual_seed(11)
    qkv = torch.randn(1, M, 3 * H * D, generator=g).to(BF16)
    qw, kw = _norm_w(g, D), _norm_w(g, D)
    cos, sin = _tables(n_sa, D, 0)
    o = torch.ops.ss.fused_attention_2way(*(t.to(dev) for t in (qkv, qw, kw, cos, sin)), n_sa)
    assert o.shape == (1, M, H * D)
    r = _joint_ref([(qkv[0, : M - n_sa], qw, kw, None, None), (qkv[0, M - n_sa:], qw, kw, cos, sin)], H, D)
    assert_bf16_close(o, r, "ss::fused_attention_2way (3-D qkv)")


@pytest.mark.parametrize("shape", [(64, 2 * 4096), (1, 82, 2 * 6144), (3, 2 * 96)])
def test_rldx_amd_swiglu_op(dev, shape):
    g = torch.Generator().manual_seed(12)
    x = (3 * torch.randn(*shape, generator=g)).to(BF16)
    y = torch.ops.rldx_amd.swiglu(x.to(dev))
    r = ref.swiglu(x)
    assert y.shape == r.shape
    assert torch.equal(y.cpu().view(torch.int16), r.view(torch.int16)), "rldx_amd::swiglu is not bit-exact"


# ---------------------------------------------------------------------------
# register_fake vs the real op (torch.library.opcheck)
# ---------------------------------------------------------------------------
def _opcheck_cases():
    H, D = 24, 64
    sa, vl, qs, ks, qv, kv, cos, sin = _ds_2way_args(21)
    x_full, p_full, xq, xk, pq, pk, sc, ss_, pc, ps = _ss_3way_args(22, 82, 18, 16)
    inner = H * D
    g = torch.Generator().manual_seed(23)
    kv_mask = torch.ones(1, 98)
    kv_mask[:, -3:] = 0
    gc = W.GqaCfg(seq=96, q_heads=8, kv_heads=2)
    gi = W.gqa_inputs(gc)
    rows = lambda m, d: torch.randn(m, d, generator=g).to(BF16)  # noqa: E731
    cases = {
        "ds::fused_attention_2way": (torch.ops.ds.fused_attention_2way, (sa, vl, qs, ks, qv, kv, cos, sin, 18, 64), {}),
        "ds::fused_attention_3way": (torch.ops.ds.fused_attention_3way,
                                     (sa[0, :18], vl[0, :64], p_full[:, : 3 * inner], qs, ks, qv, kv, pq, pk, cos, sin,
                                      pc, ps, 18, 64, 16), {"kv_mask": kv_mask}),
        "ss::fused_attention_2way": (torch.ops.ss.fused_attention_2way,
                                     (x_full[:, : 3 * inner].unsqueeze(0), xq, xk, sc, ss_, 18), {}),
        "ss::fused_attention_3way": (torch.ops.ss.fused_attention_3way,
                                     (x_full[:, : 3 * inner], p_full[:, : 3 * inner], xq, xk, pq, pk, sc, ss_, pc, ps,
                                      82, 18, 16), {"kv_mask": kv_mask}),
        "ds::grouped_swiglu": (torch.ops.ds.grouped_swiglu,
                               (rows(18, 2 * 4096), rows(1, 2 * 4096)[0], rows(64, 2 * 10922), rows(1, 2 * 10922)[0],
                                18, 64, 4096, 10922), {}),
        "ss::fused_mlp_swiglu": (torch.ops.ss.fused_mlp_swiglu,
                                 (rows(82, 1536), 0.02 * rows(2 * 1024, 1536), rows(1, 2048)[0]), {"split_k": 2}),
        "rldx_backbone::fused_attention": (torch.ops.rldx_backbone.fused_attention,
                                           (gi["qkv"], gi["q_norm_w"], W.norm_weight_rot(gi["q_norm_w"]),
                                            gi["k_norm_w"], W.norm_weight_rot(gi["k_norm_w"]), gi["cos"],
                                            W.signed_sin(gi["sin"]), 8, 2, 128), {}),
        "rldx_amd::swiglu": (torch.ops.rldx_amd.swiglu, (rows(5, 2 * 64),), {}),
        "ds::grouped_res_ln": (torch.ops.ds.grouped_res_ln,
                               (rows(18, 1536), rows(1, 1536)[0], rows(18, 1536), rows(64, 4096), rows(1, 4096)[0],
                                rows(64, 4096), 18, 64, 1536, 4096), {}),
        "ds::vl_epilogue_ln": (torch.ops.ds.vl_epilogue_ln,
                               (rows(64, 4096), rows(1, 4096)[0], rows(1, 4096)[0], rows(64, 4096), 64, 4096), {}),
        "ss::fused_epilogue_ln": (torch.ops.ss.fused_epilogue_ln,
                                  (rows(82, 1536).unsqueeze(0), rows(82, 1536).unsqueeze(0)), {}),
        "rldx_backbone::fused_epilogue_add2_rmsnorm": (torch.ops.rldx_backbone.fused_epilogue_add2_rmsnorm,
                                                       (rows(40, 2048), rows(40, 2048), rows(1, 2048)[0]), {}),
        "rldx_backbone::fused_epilogue_add3_rmsnorm": (torch.ops.rldx_backbone.fused_epilogue_add3_rmsnorm,
                                                       (rows(40, 2048), rows(40, 2048), rows(40, 2048),
                                                        rows(1, 2048)[0]), {}),
        "mem::fused_epilogue_add2_rmsnorm": (torch.ops.mem.fused_epilogue_add2_rmsnorm,
                                             (rows(64, 2048), rows(64, 2048), rows(1, 2048)[0]), {}),
    }
    vc = W.VitAttnCfg()
    vi = W.vit_attention_inputs(vc)
    cases["rldx_backbone::vision_attention"] = (torch.ops.rldx_backbone.vision_attention,
                                                (vi["qkv"], vi["rope_cos"], vi["rope_sin"], vi["cu_seqlens"],
                                                 vi["scaling"], vc.heads, vc.head_dim), {})
    mc = W.MemAttnCfg()
    mi = W.memory_attention_inputs(mc)
    cases["mem::fused_attention"] = (torch.ops.mem.fused_attention,
                                     (mi["qkv"], mi["cos"], mi["signed_sin"], mc.heads, mc.head_dim, mc.n_cog), {})
    return cases


OPCHECK_CASES = [
    "ds::fused_attention_2way", "ds::fused_attention_3way", "ss::fused_attention_2way", "ss::fused_attention_3way",
    "ds::grouped_swiglu", "ss::fused_mlp_swiglu", "rldx_backbone::fused_attention", "rldx_amd::swiglu",
    "ds::grouped_res_ln", "ds::vl_epilogue_ln", "ss::fused_epilogue_ln", "rldx_backbone::fused_epilogue_add2_rmsnorm",
    "rldx_backbone::fused_epilogue_add3_rmsnorm", "rldx_backbone::vision_attention", "mem::fused_attention",
    "mem::fused_epilogue_add2_rmsnorm",
]


@pytest.mark.parametrize("name", OPCHECK_CASES)
def test_register_fake_matches_real_op(dev, name):
    op, args, kwargs = _opcheck_cases()[name]
    to = lambda t: t.to(dev) if torch.is_tensor(t) else t  # noqa: E731
    args = tuple(to(a) for a in args)
    kwargs = {k: to(v) for k, v in kwargs.items()}
    torch.library.opcheck(op, args, kwargs, test_utils=("test_schema", "test_faketensor"))
