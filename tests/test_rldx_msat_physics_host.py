"""CPU tests pinning the all-add-ons MSAT oracle (physics stream): the
ExpandedDoubleStreamBlock / ExpandedSingleStreamBlock restatements and
MSAT._forward_physics (blocks.py:705-1089, msat.py:558-775), by properties a
plausible mistake breaks, and the P-stream parameter inventory."""

import torch
import torch.nn.functional as F

from oracle import rldx_msat_ref as R
from rldx_amd import rldx_msat as RM

BF16 = torch.bfloat16


def _tiny(seed, n_vl=5, n_p=4, ds=1, ss=1):
    """A small all-add-ons MSAT; QK-norm weights spread over [0.5, 1.5] so that
    exchanging two streams' norm weights shows."""
    cfg = RM.RldxMsatCfg(heads=2, head_dim=64, ds_blocks=ds, ss_blocks=ss, sa_dim=128, vl_dim=256, output_dim=64,
                         n_vl=n_vl, n_sa_pure=3, use_physics=True, n_physics=n_p)
    sd = RM.make_state_dict(cfg, "cpu", seed=seed)
    g = torch.Generator().manual_seed(seed + 2)
    for k in sd:
        if "norm" in k:
            sd[k] = (0.5 + torch.rand(sd[k].shape, generator=g)).to(BF16)
    return cfg, sd, RM.make_inputs(cfg, "cpu", seed=seed + 1)


def _fwd(cfg, sd, inp, **kw):
    return R.msat_forward_physics(sd, inp["sa"], inp["vl"], inp["p"], inp["temb"], inp["time_token"],
                                  heads=cfg.heads, head_dim=cfg.head_dim, ds_blocks=cfg.ds_blocks,
                                  ss_blocks=cfg.ss_blocks, **kw)


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def test_physics_param_count_matches_the_all_add_ons_release():
    """4 + 8 Expanded blocks at the release widths: the P stream adds 597.9 M
    parameters, 1839.8 M in all read by the chain; the reference reports
    1842.6 M for the all-add-ons MSAT (rldx/inference/action_model/README.md:30),
    which also counts the timestep encoder and time-token projection the chain
    takes as inputs (2.7 M, as in the no-add-ons count of README.md:11)."""
    full = sum(torch.Size(s).numel() for s in RM.RldxMsatCfg(use_physics=True).param_shapes().values())
    assert full == 1_839_808_848
    assert 2.0e6 < 1_842_600_000 - full < 3.5e6


def test_cfg_from_state_dict_sees_the_physics_stream():
    cfg = RM.RldxMsatCfg(ds_blocks=1, ss_blocks=2, use_physics=True)
    got = RM.RldxMsatCfg.from_state_dict({k: torch.empty(s) for k, s in cfg.param_shapes().items()})
    assert got.use_physics and got.param_shapes() == cfg.param_shapes()


def test_expanded_blocks_are_residual_with_zero_weights():
    """Zero linears: every stream of both Expanded blocks passes through bit for bit."""
    cfg, sd, inp = _tiny(3)
    sd = {k: (v if "norm" in k else torch.zeros_like(v)) for k, v in sd.items()}
    sa = torch.cat([inp["time_token"], inp["sa"]], dim=1)
    n = cfg.n_vl + sa.shape[1] + cfg.n_physics
    pe = torch.polar(torch.ones(1, n, 32), torch.rand(1, n, 32))
    sa2, vl2, p2 = R.expanded_ds_block(sd, "double_blocks.0.", sa, inp["vl"], inp["p"], pe, cfg.heads)
    assert torch.equal(sa2, sa) and torch.equal(vl2, inp["vl"]) and torch.equal(p2, inp["p"])
    x = torch.randn(1, 9, cfg.sa_dim).to(BF16)
    x2, p3 = R.expanded_ss_block(sd, "single_blocks.0.", x, inp["p"], pe[:, : 9 + cfg.n_physics], cfg.heads)
    assert torch.equal(x2, x) and torch.equal(p3, inp["p"])


def _swap_names(sd, pairs):
    out = dict(sd)
    for a, b in pairs:
        for k in list(sd):
            if a in k:
                out[k.replace(a, b)] = sd[k]
                out[k] = sd[k.replace(a, b)]
    return out


def test_expanded_ds_block_sa_and_p_streams_are_mirror_images():
    """SA and P enter the 3-way block symmetrically (own pre-LN, QKV, QK norms,
    rows of the joint attention, proj and MLP): running the block with the two
    streams' tokens, weights, RoPE rows and key-mask entries exchanged exchanges
    the outputs.  A P stream that used an SA weight, another stream's RoPE rows
    or no residual breaks this by O(1)."""
    cfg, sd, inp = _tiny(11, n_p=6)
    sa = torch.cat([inp["time_token"], inp["sa"]], dim=1)
    nv, ns, npp = cfg.n_vl, sa.shape[1], cfg.n_physics
    g = torch.Generator().manual_seed(2)
    pe = torch.polar(torch.ones(1, nv + ns + npp, 32), 6.0 * torch.rand(1, nv + ns + npp, 32, generator=g))
    kb = torch.zeros(1, nv + ns + npp, dtype=BF16)
    kb[0, 1] = float("-inf")
    kb[0, nv + ns + 2] = float("-inf")
    sa2, vl2, p2 = R.expanded_ds_block(sd, "double_blocks.0.", sa, inp["vl"], inp["p"], pe, cfg.heads, kb)
    sw = _swap_names(sd, [(".sa_qkv.", ".p_qkv."), (".sa_proj.", ".p_proj."), (".sa_mlp.", ".p_mlp."),
                          ("q_norm_sa", "q_norm_p"), ("k_norm_sa", "k_norm_p")])
    perm = torch.cat([torch.arange(nv), torch.arange(nv + ns, nv + ns + npp), torch.arange(nv, nv + ns)])
    sb, vb, pb = R.expanded_ds_block(sw, "double_blocks.0.", inp["p"], inp["vl"], sa, pe[:, perm], cfg.heads,
                                     kb[:, perm])
    assert _rel(pb, sa2) < 2e-3 and _rel(sb, p2) < 2e-3 and _rel(vb, vl2) < 2e-3
    # and the P stream matters: dropping its keys changes SA's output
    kb2 = kb.clone()
    kb2[0, nv + ns:] = float("-inf")
    sa3, _, _ = R.expanded_ds_block(sd, "double_blocks.0.", sa, inp["vl"], inp["p"], pe, cfg.heads, kb2)
    assert _rel(sa3, sa2) > 1e-2


def test_expanded_ss_block_x_and_p_streams_are_mirror_images():
    """The same exchange for the [VL+SA | P] single-stream block: x's linear1 /
    q_norm / k_norm / mlp_proj / linear2 against P's p_* parameters."""
    cfg, sd, inp = _tiny(21, n_p=7)
    nx, npp = 9, cfg.n_physics
    x = torch.randn(1, nx, cfg.sa_dim, generator=torch.Generator().manual_seed(4)).to(BF16)
    g = torch.Generator().manual_seed(5)
    pe = torch.polar(torch.ones(1, nx + npp, 32), 6.0 * torch.rand(1, nx + npp, 32, generator=g))
    kb = torch.zeros(1, nx + npp, dtype=BF16)
    kb[0, 3] = float("-inf")
    x2, p2 = R.expanded_ss_block(sd, "single_blocks.0.", x, inp["p"], pe, cfg.heads, kb)
    sw = _swap_names(sd, [(".linear1.", ".p_linear1."), (".mlp_proj.", ".p_mlp_proj."), (".linear2.", ".p_linear2."),
                          (".q_norm.", ".p_q_norm."), (".k_norm.", ".p_k_norm.")])
    perm = torch.cat([torch.arange(nx, nx + npp), torch.arange(nx)])
    xb, pb = R.expanded_ss_block(sw, "single_blocks.0.", inp["p"], x, pe[:, perm], cfg.heads, kb[:, perm])
    assert _rel(pb, x2) < 2e-3 and _rel(xb, p2) < 2e-3


def test_physics_masked_out_leaves_the_action_path_of_the_plain_msat():
    """physics_attention_mask = 0 removes every P key (blocks.py:855-858,
    msat.py:731-736), so the action output equals the no-add-ons forward on
    the same SA / VL weights; with the P stream visible it does not."""
    cfg, sd, inp = _tiny(31, ds=2, ss=2)
    kw = dict(heads=cfg.heads, head_dim=cfg.head_dim, ds_blocks=2, ss_blocks=2)
    plain = R.msat_forward(sd, inp["sa"], inp["vl"], inp["temb"], inp["time_token"], **kw)
    act0, _ = _fwd(cfg, sd, inp, physics_attention_mask=torch.zeros(1))
    act1, _ = _fwd(cfg, sd, inp)
    assert _rel(act0, plain) < 2e-3
    assert _rel(act1, plain) > 1e-2
    assert torch.equal(_fwd(cfg, sd, inp, physics_attention_mask=torch.ones(1))[0], act1)


def test_physics_mask_and_vl_mask_compose():
    """Masked VL tokens cannot reach either output with the P stream present."""
    cfg, sd, inp = _tiny(41)
    mask = torch.tensor([[1.0, 0.0, 1.0, 1.0, 0.0]])
    a, p = _fwd(cfg, sd, inp, encoder_attention_mask=mask)
    inp2 = dict(inp, vl=inp["vl"].clone())
    inp2["vl"][:, [1, 4]] = (4.0 * torch.randn(1, 2, cfg.vl_dim)).to(BF16)
    a2, p2 = _fwd(cfg, sd, inp2, encoder_attention_mask=mask)
    assert torch.equal(a, a2) and torch.equal(p, p2)
    a3, p3 = _fwd(cfg, sd, inp2)
    assert not torch.equal(a3, a) and not torch.equal(p3, p)


def test_physics_output_projection_closed_form():
    """Zero blocks: physics = proj_out_physics_2(LN(p) * (1 + scale) + shift),
    shift | scale = proj_out_physics_1(silu(temb)) (msat.py:771-775), in fp64."""
    cfg, sd, inp = _tiny(51, ds=0, ss=0)
    _, ph = _fwd(cfg, sd, inp)
    t = inp["temb"].double()
    ss = F.silu(t) @ sd["proj_out_physics_1.weight"].double().t() + sd["proj_out_physics_1.bias"].double()
    shift, scale = ss[:, : cfg.sa_dim], ss[:, cfg.sa_dim:]
    p = inp["p"].double()[0]
    ln = (p - p.mean(-1, keepdim=True)) / torch.sqrt(p.var(-1, unbiased=False, keepdim=True) + 1e-6)
    y = (ln * (1 + scale) + shift) @ sd["proj_out_physics_2.weight"].double().t() + \
        sd["proj_out_physics_2.bias"].double()
    assert (ph[0].double() - y).abs().max() < 0.05 * y.abs().max()


def test_physics_rows_are_told_apart_from_sa_rows_by_position():
    """P rows sit at RoPE axis-0 position 1 (msat.py:630-632, :706-710): with a
    P stream that duplicates the SA stream (same tokens, same weights, so the
    same axis-1 positions 0 .. n_sa - 1), the P outputs differ from the SA
    outputs (rel-L2 3e-3 here); at axis-0 position 0 they would be the same
    rows, bit for bit."""
    cfg, sd, inp = _tiny(61, n_p=4, ds=1, ss=0)
    for k in list(sd):
        for a, b in ((".sa_qkv.", ".p_qkv."), (".sa_proj.", ".p_proj."), (".sa_mlp.", ".p_mlp."),
                     ("q_norm_sa", "q_norm_p"), ("k_norm_sa", "k_norm_p"), ("proj_out_1.", "proj_out_physics_1."),
                     ("proj_out_2.", "proj_out_physics_2.")):
            if a in k:
                sd[k.replace(a, b)] = sd[k]
    dup = torch.cat([inp["time_token"], inp["sa"]], dim=1)
    kw = dict(heads=cfg.heads, head_dim=cfg.head_dim, ds_blocks=1, ss_blocks=0)
    for quirk in (True, False):
        act, ph = R.msat_forward_physics(sd, inp["sa"], inp["vl"], dup, inp["temb"], inp["time_token"],
                                         bf16_quirk=quirk, **kw)
        assert _rel(ph[:, 1:], act) > 1e-3
