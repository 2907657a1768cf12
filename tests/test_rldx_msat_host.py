"""CPU tests of the RLDX-1 MSAT chain's host side: parameter names and shapes,
local safetensors loading, RoPE tables against the oracle's eager position ids
(with and without the bf16 quirk), and the oracle's block structure."""

import torch

from oracle import rldx_msat_ref as R
from rldx_amd import rldx_msat as RM


def _small():
    return RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1)


def test_param_count_matches_the_release():
    """4 DS + 8 SS blocks at 24 x 64, SA 1536, VL 4096: 1241.9 M parameters read by
    the chain; the reference reports 1244.6 M for the MSAT with its timestep
    encoder and time-token projection (rldx/inference/action_model/README.md:11),
    which the chain takes as inputs (2.7 M)."""
    n = sum(torch.Size(s).numel() for s in RM.RldxMsatCfg().param_shapes().values())
    assert n == 1_241_871_184
    assert 2.0e6 < 1_244_600_000 - n < 3.5e6


def test_cfg_from_state_dict_roundtrip():
    cfg = RM.RldxMsatCfg(ds_blocks=2, ss_blocks=3)
    shapes = {k: torch.empty(s) for k, s in cfg.param_shapes().items()}
    got = RM.RldxMsatCfg.from_state_dict(shapes)
    assert got.param_shapes() == cfg.param_shapes()
    assert (got.heads, got.head_dim, got.ds_blocks, got.ss_blocks, got.vl_ffn) == (24, 64, 2, 3, 10922)


def test_load_msat_state_dict_from_local_safetensors(tmp_path):
    from safetensors.torch import save_file

    cfg = _small()
    sd = RM.make_state_dict(cfg, "cpu", seed=3)
    full = {f"action_model.model.{k}": v for k, v in sd.items()}
    full["backbone.some.weight"] = torch.zeros(4, dtype=torch.bfloat16)
    keys = sorted(full)
    save_file({k: full[k] for k in keys[: len(keys) // 2]}, str(tmp_path / "model-00001.safetensors"))
    save_file({k: full[k] for k in keys[len(keys) // 2:]}, str(tmp_path / "model-00002.safetensors"))
    got = RM.load_msat_state_dict(str(tmp_path))
    assert set(got) == set(sd)
    assert all(torch.equal(got[k], sd[k]) for k in sd)


def _eager_pe(cfg, quirk, single):
    tabs = R.rope_freq_tables(cfg.head_dim, cfg.rope_theta, cfg.max_seq_len, quirk)
    N, nv, nt = cfg.tokens, cfg.n_vl, cfg.num_temb_tokens
    ids = torch.zeros(1, N, 2, dtype=torch.long)
    ids[:, nv:nv + nt, 1] = torch.arange(nt)
    start = nt + 1 if single else nt
    ids[:, nv + nt:, 1] = torch.arange(start, start + cfg.n_sa_pure)
    return R.rope_pe(tabs, ids)[0]


def test_rope_tables_equal_the_eager_embedder_rows():
    """The chain's DS / SS tables (SA rows) are the eager RoPEEmbedder1D values at
    the eager position ids (msat.py:376-487); VL rows are the identity there."""
    cfg = RM.RldxMsatCfg()
    for quirk in (True, False):
        for single, pos in ((False, torch.arange(cfg.n_sa)),
                            (True, torch.cat([torch.arange(1), torch.arange(2, 2 + cfg.n_sa_pure)]))):
            pe = _eager_pe(cfg, quirk, single)
            c, s = RM.rope_tables(cfg, pos, quirk)
            sa = pe[cfg.n_vl:]
            if quirk:
                assert sa.dtype == torch.bfloat16
                assert torch.equal(sa.float(), c) and not s.any()
                assert torch.equal(pe[: cfg.n_vl].float(), torch.ones_like(pe[: cfg.n_vl].float()))
            else:
                assert torch.equal(sa.real, c) and torch.equal(sa.imag, s)
                assert torch.equal(pe[: cfg.n_vl], torch.ones_like(pe[: cfg.n_vl]))


def test_bf16_quirk_is_the_complex_to_bf16_cast():
    """A bf16 cast of the complex64 buffers keeps the real part (what
    model.to(torch.bfloat16) does to RoPEEmbedder1D's buffers)."""
    exact = R.rope_freq_tables(64, 1e4, 64, False)
    quirk = R.rope_freq_tables(64, 1e4, 64, True)
    for e, q in zip(exact, quirk):
        assert torch.equal(e.real.to(torch.bfloat16), q)
        assert torch.equal(e.to(torch.bfloat16), q)  # torch's complex -> real cast discards imag


def test_oracle_blocks_are_residual_with_zero_weights():
    """With every linear weight and bias zero, a DS block and an SS block return
    their inputs bit for bit (residual structure; identity modulation)."""
    cfg = _small()
    sd = {k: (v if "norm" in k else torch.zeros_like(v)) for k, v in RM.make_state_dict(cfg, "cpu").items()}
    inp = RM.make_inputs(cfg, "cpu")
    sa = torch.cat([inp["time_token"], inp["sa"]], dim=1)
    pe = _eager_pe(cfg, True, False)[None]
    sa2, vl2 = R.ds_block(sd, "double_blocks.0.", sa, inp["vl"], pe, cfg.heads)
    assert torch.equal(sa2, sa) and torch.equal(vl2, inp["vl"])
    x = torch.randn(1, cfg.tokens, cfg.sa_dim).to(torch.bfloat16)
    assert torch.equal(R.ss_block(sd, "single_blocks.0.", x, pe, cfg.heads), x)


def test_oracle_output_projection_closed_form():
    """Zero blocks: out = proj_out_2(LN(sa) * (1 + scale) + shift), shift | scale =
    proj_out_1(silu(temb)) — checked in fp64 against the oracle's bf16 chain."""
    cfg = RM.RldxMsatCfg(ds_blocks=0, ss_blocks=0)
    sd = RM.make_state_dict(cfg, "cpu", seed=5, std=0.05)
    inp = RM.make_inputs(cfg, "cpu")
    o = R.msat_forward(sd, inp["sa"], inp["vl"], inp["temb"], inp["time_token"], heads=24, head_dim=64,
                       ds_blocks=0, ss_blocks=0)
    t = inp["temb"].double()
    ss = torch.nn.functional.silu(t) @ sd["proj_out_1.weight"].double().t() + sd["proj_out_1.bias"].double()
    shift, scale = ss[:, :1536], ss[:, 1536:]
    sa = inp["sa"].double()[0]
    ln = (sa - sa.mean(-1, keepdim=True)) / torch.sqrt(sa.var(-1, unbiased=False, keepdim=True) + 1e-6)
    y = (ln * (1 + scale) + shift) @ sd["proj_out_2.weight"].double().t() + sd["proj_out_2.bias"].double()
    assert (o[0].double() - y).abs().max() < 0.05 * y.abs().max()


def test_oracle_sa_output_invariant_to_vl_token_order():
    """VL rows carry identity RoPE and no mask, so the action outputs cannot
    depend on the order of the cognition tokens (a swapped [VL | SA] order or
    RoPE on the wrong rows breaks this)."""
    cfg = RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1)
    sd = RM.make_state_dict(cfg, "cpu", seed=7)
    inp = RM.make_inputs(cfg, "cpu", seed=8)
    kw = dict(heads=24, head_dim=64, ds_blocks=1, ss_blocks=1, bf16_quirk=False)
    o = R.msat_forward(sd, inp["sa"], inp["vl"], inp["temb"], inp["time_token"], **kw).double()
    perm = torch.randperm(cfg.n_vl, generator=torch.Generator().manual_seed(0))
    op = R.msat_forward(sd, inp["sa"], inp["vl"][:, perm], inp["temb"], inp["time_token"], **kw).double()
    assert (o - op).norm() / o.norm() < 1e-2


def _tiny_oracle_inputs(seed, n_vl=5):
    cfg = RM.RldxMsatCfg(heads=2, head_dim=64, ds_blocks=1, ss_blocks=1, sa_dim=128, vl_dim=128, output_dim=64,
                         n_vl=n_vl, n_sa_pure=3)
    sd = RM.make_state_dict(cfg, "cpu", seed=seed)
    inp = RM.make_inputs(cfg, "cpu", seed=seed + 1)
    return cfg, sd, inp


def _run(cfg, sd, inp, mask=None, vl=None):
    return R.msat_forward(sd, inp["sa"], inp["vl"] if vl is None else vl, inp["temb"], inp["time_token"],
                          heads=cfg.heads, head_dim=cfg.head_dim, ds_blocks=cfg.ds_blocks, ss_blocks=cfg.ss_blocks,
                          encoder_attention_mask=mask)


def test_oracle_vl_mask_semantics():
    """encoder_attention_mask in the oracle (blocks.py:558-575, msat.py:517-531):
    an all-ones mask equals no mask bit for bit; masked VL tokens cannot reach
    the output (changing their values leaves it bit-identical), while the same
    change without the mask does change it."""
    cfg, sd, inp = _tiny_oracle_inputs(81)
    base = _run(cfg, sd, inp)
    assert torch.equal(_run(cfg, sd, inp, torch.ones(1, 5)), base)
    mask = torch.tensor([[1.0, 0.0, 1.0, 0.0, 1.0]])
    vl2 = inp["vl"].clone()
    vl2[:, [1, 3]] = 5.0 * torch.randn(1, 2, cfg.vl_dim).to(vl2.dtype)
    assert torch.equal(_run(cfg, sd, inp, mask), _run(cfg, sd, inp, mask, vl=vl2))
    assert not torch.equal(_run(cfg, sd, inp), _run(cfg, sd, inp, vl=vl2))


def test_dispatcher_falls_back_for_good_when_the_build_fails():
    """MsatDispatcher on a CPU module: the first call is served by the module's own
    forward; building the chain needs the GPU kernels and fails here, so every
    later call stays on the module's own forward (serve_optimization.py:464-472)."""
    cfg = RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1)
    shapes = cfg.param_shapes()
    root = torch.nn.Module()
    for k, s in shapes.items():
        *path, leaf = k.split(".")
        m = root
        for part in path:
            if not hasattr(m, part):
                m.add_module(part, torch.nn.Module())
            m = getattr(m, part)
        m.register_buffer(leaf, torch.zeros(s, dtype=torch.bfloat16))
    calls = []
    root.forward = lambda *a, **k: calls.append((a, k)) or "own"
    d = RM.install(root)
    sa, vl = torch.zeros(1, cfg.n_sa_pure, cfg.sa_dim), torch.zeros(1, cfg.n_vl, cfg.vl_dim)
    assert root(sa, vl, torch.zeros(1)) == "own" and d.failed and d.chain is None
    assert root(sa, vl, torch.zeros(1), encoder_attention_mask=torch.ones(1, cfg.n_vl)) == "own"
    assert len(calls) == 2 and d.served == 0 and d.fallbacks == 2
    # the reference keyword arguments reach the module's own forward unchanged
    assert calls[1][0][4] is not None


def test_dispatcher_unserved_calls():
    d = RM.MsatDispatcher(torch.nn.Module(), max_batch=4)
    x3 = torch.zeros(1, 17, 8)
    mixed = "inputs are not [B, tokens, width] with one batch size"
    assert d._unserved(x3, x3, True, None, None) == "return_all_hidden_states"
    # batches up to max_batch run on a chain of their own size
    assert d._unserved(torch.zeros(2, 17, 8), torch.zeros(2, 17, 8), False, None, None) is None
    assert d._unserved(torch.zeros(4, 17, 8), torch.zeros(4, 17, 8), False, None, None) is None
    assert d._unserved(torch.zeros(5, 17, 8), torch.zeros(5, 17, 8), False, None, None) == "batch above max_batch (4)"
    assert d._unserved(torch.zeros(2, 17, 8), torch.zeros(1, 17, 8), False, None, None) == mixed
    assert d._unserved(torch.zeros(17, 8), torch.zeros(17, 8), False, None, None) == mixed
    assert d._unserved(x3, x3, False, torch.zeros(1, 4, 8), None) is None  # module without use_physics ignores them
    d.msat.use_physics = True
    assert d._unserved(x3, x3, False, torch.zeros(1, 4, 8), None) is None  # served by the all-add-ons chain
    assert d._n_physics(torch.zeros(1, 4, 8)) == 4 and d._n_physics(None) == 0
    assert d._unserved(x3, x3, False, torch.zeros(2, 4, 8), None) == mixed

    class _Built:  # a chain built for 17 SA, 17 VL and 4 physics tokens
        np_ = 4
        cfg = RM.RldxMsatCfg(n_vl=17, n_sa_pure=17)

    d.chain = _Built()
    assert d._unserved(x3, x3, False, torch.zeros(1, 4, 8), None) is None
    assert d._unserved(x3, x3, False, torch.zeros(1, 5, 8), None) == "token counts differ from the chain's"
    assert d._unserved(x3, x3, False, None, None) == "token counts differ from the chain's"


# ---------------------------------------------------------------------------
# The action head oracle (R.action_head): Euler update in closed form, the RTC
# prefix path against the unsliced re-lock composition, vlln written out.
# ---------------------------------------------------------------------------
def _tiny_head(seed, horizon=6, steps=2, **kw):
    mc = RM.RldxMsatCfg(heads=2, head_dim=64, ds_blocks=1, ss_blocks=1, sa_dim=128, vl_dim=128, output_dim=64,
                        n_vl=5, n_sa_pure=1 + horizon)
    hc = RM.RldxHeadCfg(state_dim=8, action_dim=8, action_horizon=horizon, hidden_size=64, num_embodiments=2,
                        steps=steps, **kw)
    sd = {k: v.float() for k, v in RM.make_state_dict(mc, "cpu", seed=seed).items()}
    hsd = {k: v.float() for k, v in RM.make_head_state_dict(mc, hc, "cpu", seed=seed + 1).items()}
    g = torch.Generator().manual_seed(seed + 2)
    io = dict(vl=torch.randn(1, mc.n_vl, mc.vl_dim, generator=g), state=torch.randn(1, 1, hc.state_dim, generator=g),
              x0=torch.randn(1, horizon, hc.action_dim, generator=g),
              prefix=torch.randn(1, max(hc.prefix_len, 1), hc.action_dim, generator=g)[:, :hc.prefix_len])
    return mc, hc, sd, hsd, io


def _head(mc, hc, sd, hsd, io, e=1, **kw):
    return R.action_head(hsd, sd, io["vl"], io["state"], io["x0"], steps=hc.steps, heads=mc.heads,
                         head_dim=mc.head_dim, ds_blocks=mc.ds_blocks, ss_blocks=mc.ss_blocks, e=e,
                         prefix=io["prefix"] if hc.prefix_len > 0 else None, use_vlln=hc.use_vlln, **kw)


def test_oracle_action_head_euler_closed_form():
    """A decoder whose last layer has zero weights predicts its bias c[e] for
    every row at every step, so `steps` Euler steps of dt = 1/steps move each
    free row by exactly c[e]; the prefix rows equal the prefix exactly.  A wrong
    dt, decode slice, embodiment index or prefix re-lock fails this."""
    for d in (0, 2):
        mc, hc, sd, hsd, io = _tiny_head(5, steps=4, prefix_len=d)
        hsd["action_decoder.layer2.W"].zero_()
        c = torch.tensor([[0.5] * 8, [-0.25 * (i + 1) for i in range(8)]])
        hsd["action_decoder.layer2.b"].copy_(c)
        act = _head(mc, hc, sd, hsd, io, e=1)
        assert torch.equal(act[:d], io["prefix"][0])
        assert torch.allclose(act[d:], io["x0"][0, d:] + c[1], atol=1e-6, rtol=0)


def _relock_composition(mc, hc, sd, hsd, io, e=1):
    """RTC trained mode without the chain's slicing (rldx/model/core/rldx.py:609-610
    re-lock semantics): every step encodes all `horizon` rows with per-row time
    (1 for the prefix rows, the step's time for the rest), runs the MSAT, decodes
    every row, advances all rows, then writes the prefix back."""
    H, d, w = hc.action_horizon, hc.prefix_len, mc.sa_dim

    def lin(x, name):
        return torch.addmm(hsd[f"{name}.b"][e], x, hsd[f"{name}.W"][e])

    state_feat = lin(torch.relu(lin(io["state"][0], "state_encoder.layer1")), "state_encoder.layer2")
    act = io["x0"][0].clone()
    act[:d] = io["prefix"][0]
    for i in range(hc.steps):
        t = torch.full((H,), i / hc.steps)
        t[:d] = 1.0
        half = w // 2
        fr = t[:, None] * torch.exp(-torch.arange(half, dtype=torch.float) * (torch.log(torch.tensor(10000.0)) / half))
        tau = torch.cat([torch.sin(fr), torch.cos(fr)], dim=-1)
        h = lin(torch.cat([lin(act, "action_encoder.W1"), tau], dim=-1), "action_encoder.W2")
        feat = lin(h * torch.sigmoid(h), "action_encoder.W3") + hsd["position_embedding.weight"]
        out = R.msat_forward(sd, torch.cat([state_feat, feat])[None], io["vl"], hsd["static_tembs"][i],
                             hsd["static_time_tokens"][i], heads=mc.heads, head_dim=mc.head_dim,
                             ds_blocks=mc.ds_blocks, ss_blocks=mc.ss_blocks)[0]
        act = act + lin(torch.relu(lin(out, "action_decoder.layer1")), "action_decoder.layer2")[-H:] / hc.steps
        act[:d] = io["prefix"][0]
    return act


def test_oracle_action_head_prefix_equals_the_relock_composition():
    """The prefix path (prefix features encoded once at time 1, postfix-only
    encode / decode) equals the unsliced composition to fp32 rounding, and
    the prefix changes the free rows (its tokens are attended)."""
    mc, hc, sd, hsd, io = _tiny_head(17, prefix_len=3)
    got = _head(mc, hc, sd, hsd, io)
    ref = _relock_composition(mc, hc, sd, hsd, io)
    assert torch.allclose(got, ref, atol=1e-5, rtol=1e-5), (got - ref).abs().max()
    io2 = dict(io, prefix=io["prefix"] + 0.5)
    assert (_head(mc, hc, sd, hsd, io2)[3:] - got[3:]).abs().max() > 1e-5
    # x0's prefix rows never matter
    io3 = dict(io, x0=io["x0"].clone())
    io3["x0"][:, :3] = 7.0
    assert torch.equal(_head(mc, hc, sd, hsd, io3), got)


def test_oracle_action_head_vlln_is_layer_norm_of_the_vl_tokens():
    """use_vlln equals the head without it on VL tokens normalised by hand:
    (x - mean) / sqrt(var + 1e-5) * w + b per token, biased variance."""
    mc, hc, sd, hsd, io = _tiny_head(29, use_vlln=True)
    x = io["vl"].double()
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    vl_n = ((x - mu) / torch.sqrt(var + 1e-5) * hsd["vlln.weight"].double() + hsd["vlln.bias"].double()).float()
    got = _head(mc, hc, sd, hsd, io)
    hc_off = RM.RldxHeadCfg(**{**hc.__dict__, "use_vlln": False})
    ref = _head(mc, hc_off, sd, hsd, dict(io, vl=vl_n))
    assert torch.allclose(got, ref, atol=1e-5, rtol=1e-5), (got - ref).abs().max()
    assert (_head(mc, hc_off, sd, hsd, io) - got).abs().max() > 1e-5


def test_action_head_dispatcher_unserved_calls():
    """The per-call refusals of the action-head dispatcher (no build needed)."""
    m = torch.nn.Module()
    m.gs_msat = torch.nn.Module()
    m.gs_msat.n_vl = 64
    m.prefix_len = 0
    d = RM.ActionHeadDispatcher(m, max_batch=4)
    vl, st = torch.zeros(1, 64, 8), torch.zeros(1, 4)
    mixed = "inputs of different batch sizes"
    assert d._unserved(vl, st, None, None) is None
    assert d._unserved(torch.zeros(2, 64, 8), torch.zeros(2, 4), None, None) is None  # a head for 2 robots
    assert d._unserved(torch.zeros(5, 64, 8), torch.zeros(5, 4), None, None) == "batch above max_batch (4)"
    assert d._unserved(torch.zeros(2, 64, 8), torch.zeros(1, 4), None, None) == mixed
    assert d._unserved(torch.zeros(2, 64, 8), torch.zeros(2, 4), torch.zeros(1, 3, 8), None) == mixed
    assert d._unserved(torch.zeros(64, 8), st, None, None) == mixed
    assert d._unserved(torch.zeros(1, 63, 8), st, None, None) == "VL token count differs from the module's"
    m.prefix_len = 3
    assert d._unserved(vl, st, None, None) == "prefix_len > 0 without prefix_actions"
    assert d._unserved(vl, st, torch.zeros(1, 3, 8), None) is None
    m.use_physics = True
    assert d._unserved(vl, st, torch.zeros(1, 3, 8), None) == "physics model without physics_hist"
    assert d._unserved(vl, st, torch.zeros(1, 3, 8), torch.zeros(1, 1, 5)) is None


def test_action_head_dispatcher_detects_weight_changes():
    """weights_changed(): in-place updates, replaced parameters and new buffers
    after the stamp (no build needed); refresh() clears the stamp."""
    m = torch.nn.Module()
    m.lin = torch.nn.Linear(4, 4)
    m.register_buffer("steps", torch.arange(4.0))
    d = RM.ActionHeadDispatcher(m, check_weights=True)
    assert d.weights_changed()  # never built
    d._stamp = d._weights_stamp()
    assert not d.weights_changed()
    with torch.no_grad():
        m.lin.weight.add_(1.0)  # in place
    assert d.weights_changed()
    d._stamp = d._weights_stamp()
    m.lin.bias = torch.nn.Parameter(torch.zeros(4))  # replaced
    assert d.weights_changed()
    d._stamp = d._weights_stamp()
    m.register_buffer("extra", torch.zeros(1))  # added
    assert d.weights_changed()
    d.refresh()
    assert d._stamp is None and d.rebuilds == 0  # nothing built yet, nothing counted
