"""GPU parity of the RLDX-1 MSAT chain (rldx_amd.rldx_msat.RldxMsat: the
reference's own 24 x 64, 4 DS + 8 SS architecture on the rldx_amd kernels)
against the CPU oracle (oracle/rldx_msat_ref.py) on the same weights."""

import pytest
import torch

from oracle import rldx_msat_ref as R
from rldx_amd import rldx_msat as RM
from tolerances import BF16_REL_L2, assert_bf16_close, stats

pytestmark = pytest.mark.gpu


def _oracle(sd, inp, cfg, quirk, mask=None):
    cpu = {k: v.cpu() for k, v in sd.items()}
    return R.msat_forward(cpu, inp["sa"].cpu(), inp["vl"].cpu(), inp["temb"].cpu(), inp["time_token"].cpu(),
                          heads=cfg.heads, head_dim=cfg.head_dim, ds_blocks=cfg.ds_blocks, ss_blocks=cfg.ss_blocks,
                          theta=cfg.rope_theta, max_seq_len=cfg.max_seq_len, bf16_quirk=quirk,
                          encoder_attention_mask=None if mask is None else mask.cpu())


def _rel(a, b):
    return ((a - b).norm() / b.norm()).item()


def assert_as_accurate_as_eager_bf16(o, sd, inp, cfg, quirk, what, mask=None):
    """Over several blocks the bf16 roundings of any evaluation order compound
    (the bf16 oracle itself is 6e-3 / 8e-3 / 1.5e-2 rel-L2 from an fp32
    evaluation at 1+1 / 2+2 / 4+8 blocks).  Bound: the GPU chain is no further
    from the fp32 evaluation of the same weights and inputs than 1.5x the eager
    bf16 evaluation is, and its cosine to the bf16 oracle is >= 0.999."""
    o = o.detach().cpu().double()
    r16 = _oracle(sd, inp, cfg, quirk, mask).double()
    sd32 = {k: v.float() for k, v in sd.items()}
    inp32 = {k: v.float() for k, v in inp.items()}
    r32 = _oracle(sd32, inp32, cfg, quirk, mask).double()
    floor, got = _rel(r16, r32), _rel(o, r32)
    cos = torch.nn.functional.cosine_similarity(o.flatten(), r16.flatten(), dim=0).item()
    print(f"{what}: rel-L2 to fp32 {got:.2e} (eager bf16: {floor:.2e}), to the bf16 oracle {_rel(o, r16):.2e}, "
          f"cos {cos:.6f}")
    assert torch.isfinite(o).all() and got <= 1.5 * floor and cos >= 0.999, what


@pytest.mark.parametrize("quirk", [True, False])
def test_rldx_msat_one_block_each(dev, quirk):
    """1 DS + 1 SS block on unscaled random weights (outputs reach |y| ~ 3,
    where one bf16 ulp is 0.0156, so independently rounded sums differ by more
    than the unit-scale max-abs bound of 2e-2).  Bounds: rel-L2 <= 1e-2 to the
    bf16 oracle, and the fp32 referee (no further from an fp32 evaluation than
    1.5x the eager bf16 oracle, cosine >= 0.999); max-abs is printed."""
    cfg = RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1)
    sd = RM.make_state_dict(cfg, dev, seed=21)
    inp = RM.make_inputs(cfg, dev, seed=22)
    chain = RM.RldxMsat(sd, cfg, dev, bf16_quirk=quirk)
    o = chain.forward(inp["sa"], inp["vl"], inp["temb"], inp["time_token"]).clone()
    s = stats(o, _oracle(sd, inp, cfg, quirk))
    print(f"RLDX MSAT 1 DS + 1 SS, quirk={quirk}: to the bf16 oracle {s}")
    assert s["nonfinite_mismatch"] == 0 and s["rel_l2"] <= BF16_REL_L2, s
    assert_as_accurate_as_eager_bf16(o, sd, inp, cfg, quirk, f"RLDX MSAT 1 DS + 1 SS, quirk={quirk}")


def test_rldx_msat_full_model(dev):
    """4 DS + 8 SS blocks at the release dimensions."""
    cfg = RM.RldxMsatCfg()
    sd = RM.make_state_dict(cfg, dev, seed=31)
    inp = RM.make_inputs(cfg, dev, seed=32)
    chain = RM.RldxMsat(sd, cfg, dev)
    o = chain.forward(inp["sa"], inp["vl"], inp["temb"], inp["time_token"]).clone()
    assert_as_accurate_as_eager_bf16(o, sd, inp, cfg, True, "full MSAT")


def test_rldx_msat_graph_replay(dev):
    cfg = RM.RldxMsatCfg(ds_blocks=2, ss_blocks=2)
    sd = RM.make_state_dict(cfg, dev, seed=41)
    chain = RM.RldxMsat(sd, cfg, dev)
    chain.capture()
    for rep in range(3):
        inp = RM.make_inputs(cfg, dev, seed=50 + rep)
        for k in ("sa", "vl", "temb", "time_token"):
            chain.inputs[k].copy_(inp[k])
        got = chain.replay().clone()
        torch.cuda.synchronize()
        eager = chain.forward(inp["sa"], inp["vl"], inp["temb"], inp["time_token"]).clone()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16)), f"replay {rep}"
    assert_as_accurate_as_eager_bf16(got, sd, inp, cfg, True, "graph replay, 2 DS + 2 SS")


def _stack(inps):
    return {k: torch.cat([i[k] for i in inps]) for k in inps[0]}


def test_rldx_msat_batch_of_robots(dev):
    """A chain for three robots (RldxMsat.for_batch: the batch-1 chain's packed
    weights, shared) with different inputs and VL masks per robot.  Each
    robot's output agrees with the batch-1 chain run on that robot alone
    (rel-L2 <= 1e-2: the GEMMs of the larger batch may take other tiles or
    splits, which order the sums differently), and the batch is as accurate
    as the eager bf16 evaluation of the same batch (the referee above)."""
    cfg = RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1)
    sd = RM.make_state_dict(cfg, dev, seed=61)
    one = RM.RldxMsat(sd, cfg, dev, vl_mask=True)
    three = one.for_batch(3)
    assert three.batch == 3 and three.ds is one.ds and three.w is one.w
    inps = [RM.make_inputs(cfg, dev, seed=70 + b) for b in range(3)]
    mask = torch.ones(3, cfg.n_vl, device=dev)
    mask[1, 5:9] = 0
    mask[2, -3:] = 0
    alone = [one.forward(i["sa"], i["vl"], i["temb"], i["time_token"], mask[b:b + 1]).clone()
             for b, i in enumerate(inps)]
    batch = _stack(inps)
    o = three.forward(batch["sa"], batch["vl"], batch["temb"], batch["time_token"], mask).clone()
    assert o.shape == (3, cfg.n_sa_pure, cfg.output_dim)
    for b in range(3):
        s = stats(o[b], alone[b][0])
        same = (o[b].view(torch.int16) == alone[b][0].view(torch.int16)).float().mean().item()
        print(f"robot {b}: batch of 3 vs alone {s}, bit-identical elements {same:.4f}")
        assert s["nonfinite_mismatch"] == 0 and s["rel_l2"] <= BF16_REL_L2, (b, s)
    assert_as_accurate_as_eager_bf16(o, sd, batch, cfg, True, "3 robots, 1 DS + 1 SS", mask=mask)


def _module_tree(sd):
    """nn.Module tree whose state_dict() has exactly the keys of `sd` (what a
    loaded reference MSAT exposes)."""
    root = torch.nn.Module()
    for k, v in sd.items():
        *path, leaf = k.split(".")
        m = root
        for part in path:
            if not hasattr(m, part):
                m.add_module(part, torch.nn.Module())
            m = getattr(m, part)
        m.register_parameter(leaf, torch.nn.Parameter(v, requires_grad=False))
    return root


def _tree_with_time_modules(cfg, sd, dev, seed):
    """A module tree with the reference MSAT's state-dict keys, a timestep encoder,
    a time-token projection, and (as its own forward) the oracle evaluated on the
    CPU: the dispatcher's fallback path then returns the reference's result."""
    msat = _module_tree(sd)
    g = torch.Generator(device=dev).manual_seed(seed)
    wt = (0.02 * torch.randn(cfg.inner, 1, generator=g, device=dev)).to(torch.bfloat16)
    wtt = (0.02 * torch.randn(cfg.sa_dim, cfg.inner, generator=g, device=dev)).to(torch.bfloat16)
    msat.timestep_encoder = lambda t: (t[:, None].to(torch.bfloat16) @ wt.t())
    msat.time_token_proj = lambda temb: temb @ wtt.t()
    msat.calls = []

    def own_forward(hidden_states, encoder_hidden_states, timestep=None, return_all_hidden_states=False,
                    encoder_attention_mask=None, physics_embs=None, physics_attention_mask=None):
        msat.calls.append(dict(return_all_hidden_states=return_all_hidden_states,
                               masked=encoder_attention_mask is not None))
        temb = msat.timestep_encoder(timestep)
        tt = msat.time_token_proj(temb).unsqueeze(1)
        c = RM.RldxMsatCfg.from_state_dict(sd, n_vl=encoder_hidden_states.shape[1],
                                           n_sa_pure=hidden_states.shape[1])
        inp = dict(sa=hidden_states, vl=encoder_hidden_states, temb=temb, time_token=tt)
        out = _oracle(sd, inp, c, True, mask=encoder_attention_mask).to(dev)
        return (out, []) if return_all_hidden_states else out

    msat.forward = own_forward
    return msat


def _time_inputs(msat, t):
    temb = msat.timestep_encoder(t)
    return temb, msat.time_token_proj(temb).unsqueeze(1)


def test_install_on_a_module_tree(dev):
    """install() with token counts builds the chain now; msat(...) keeps the
    reference forward signature and uses the module's own time embedding and
    time-token projection."""
    cfg = RM.RldxMsatCfg(ds_blocks=1, ss_blocks=2)
    sd = RM.make_state_dict(cfg, dev, seed=61)
    msat = _tree_with_time_modules(cfg, sd, dev, 62)
    d = RM.install(msat, n_vl=cfg.n_vl, n_sa_pure=cfg.n_sa_pure, bf16_quirk=True)
    assert d.chain.cfg.param_shapes() == cfg.param_shapes()
    inp = RM.make_inputs(cfg, dev, seed=63)
    t = torch.tensor([0.25], device=dev)
    o = msat(inp["sa"], inp["vl"], t).clone()
    assert d.served == 1 and msat.calls == []
    temb, tt = _time_inputs(msat, t)
    ref_inp = dict(sa=inp["sa"], vl=inp["vl"], temb=temb, time_token=tt)
    assert_as_accurate_as_eager_bf16(o, sd, ref_inp, cfg, True, "installed MSAT forward, 1 DS + 2 SS")


@pytest.mark.parametrize("n_vl", [64, 80])
def test_dispatcher_serves_masks_and_falls_back(dev, n_vl):
    """The lazy dispatcher (graph replay): the first call is the module's own
    forward; then encoder_attention_mask is served by the chain (masked VL keys
    carry -inf); return_all_hidden_states and token counts other than the
    chain's go to the module's own forward.  n_vl = 80 is not a multiple of 32:
    the chain pads the VL rows with masked keys."""
    cfg = RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1, n_vl=n_vl)
    sd = RM.make_state_dict(cfg, dev, seed=64)
    msat = _tree_with_time_modules(cfg, sd, dev, 65)
    d = RM.install(msat, bf16_quirk=True, graph=True)  # the tree has no RoPE buffers to detect the quirk from
    inp = RM.make_inputs(cfg, dev, seed=66)
    t = torch.tensor([0.5], device=dev)
    first = msat(inp["sa"], inp["vl"], t).clone()
    assert d.chain is not None and d.served == 0 and len(msat.calls) == 1
    temb, tt = _time_inputs(msat, t)
    ref_inp = dict(sa=inp["sa"], vl=inp["vl"], temb=temb, time_token=tt)
    o = msat(inp["sa"], inp["vl"], t).clone()
    assert d.served == 1 and len(msat.calls) == 1
    assert_as_accurate_as_eager_bf16(o, sd, ref_inp, cfg, True, f"dispatcher, n_vl={n_vl}")
    mask = torch.ones(1, n_vl, device=dev)
    mask[:, 5:n_vl:3] = 0
    om = msat(inp["sa"], inp["vl"], t, encoder_attention_mask=mask).clone()
    assert d.served == 2 and len(msat.calls) == 1
    assert_as_accurate_as_eager_bf16(om, sd, ref_inp, cfg, True, f"dispatcher with a VL mask, n_vl={n_vl}",
                                     mask=mask)
    assert (om.float() - o.float()).abs().max() > 1e-2, "the mask changed nothing"
    # unchanged inputs without the mask replay the unmasked result bit for bit
    o2 = msat(inp["sa"], inp["vl"], t).clone()
    assert torch.equal(o2.view(torch.int16), o.view(torch.int16))
    msat(inp["sa"], inp["vl"], t, return_all_hidden_states=True)
    assert len(msat.calls) == 2 and msat.calls[-1]["return_all_hidden_states"]
    # two robots (different times and masks) run on a chain of their own, on the same packed weights
    inp2 = RM.make_inputs(cfg, dev, seed=68)
    t2 = torch.tensor([0.5, 0.25], device=dev)
    mask2 = torch.cat([mask, torch.ones(1, n_vl, device=dev)])
    mask2[1, :7] = 0
    sa2, vl2 = torch.cat([inp["sa"], inp2["sa"]]), torch.cat([inp["vl"], inp2["vl"]])
    ob = msat(sa2, vl2, t2, encoder_attention_mask=mask2).clone()
    assert d.served == 4 and len(msat.calls) == 2 and d.chains[2].batch == 2 and d.chains[2].ds is d.chain.ds
    s = stats(ob[0], om[0])
    print(f"robot 0 of a batch of 2 vs alone: {s}")
    assert s["nonfinite_mismatch"] == 0 and s["rel_l2"] <= BF16_REL_L2, s
    temb2, tt2 = _time_inputs(msat, t2)
    assert_as_accurate_as_eager_bf16(ob, sd, dict(sa=sa2, vl=vl2, temb=temb2, time_token=tt2), cfg, True,
                                     f"dispatcher, batch of 2, n_vl={n_vl}", mask=mask2)
    short = RM.make_inputs(RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1, n_vl=32), dev, seed=67)
    msat(inp["sa"], short["vl"], t)
    assert len(msat.calls) == 3 and d.served == 4 and not d.failed


def _head_reference(head_sd, msat_sd, hc, mc, head, e=0, dtype=torch.float32):
    """The oracle's CustomActionHeadChain.forward composition (R.action_head) on the
    head's static inputs, evaluated in `dtype` (fp32, or bf16 eager with a
    rounding after every op)."""
    return R.action_head(head_sd, msat_sd, head.vl, head.state, head.x0, steps=hc.steps, heads=mc.heads,
                         head_dim=mc.head_dim, ds_blocks=mc.ds_blocks, ss_blocks=mc.ss_blocks, e=e,
                         prefix=head.prefix if hc.prefix_len > 0 else None, use_vlln=hc.use_vlln,
                         vlln_eps=hc.vlln_eps, dtype=dtype)


def _head_on_gpu(mc, hc, dev, seed, embodiment):
    sd = RM.make_state_dict(mc, dev, seed=seed)
    hsd = RM.make_head_state_dict(mc, hc, dev, seed=seed + 1)
    head = RM.RldxActionHead(RM.RldxMsat(sd, mc, dev), hsd, hc, embodiment=embodiment)
    g = torch.Generator(device=dev).manual_seed(seed + 2)
    head.vl.copy_(torch.randn(head.vl.shape, generator=g, device=dev))
    head.state.copy_(torch.randn(head.state.shape, generator=g, device=dev))
    head.x0.copy_(torch.randn(head.x0.shape, generator=g, device=dev))
    if hc.prefix_len > 0:
        head.prefix.copy_(torch.randn(head.prefix.shape, generator=g, device=dev))
    head.capture()
    a1 = head.replay().clone()
    a2 = head.replay().clone()
    torch.cuda.synchronize()
    assert torch.equal(a1.view(torch.int16), a2.view(torch.int16)), "graph replays differ"
    return head, sd, hsd, a1


def test_rldx_action_head_graph_matches_fp32_composition(dev):
    """State encoder + 2 denoising steps of action encoder, MSAT (1 DS + 1 SS),
    decoder and Euler update as one hipGraph, against an fp32 CPU composition:
    the actions agree to rel-L2 <= 2e-2 (bf16 path vs fp32) and replays are bitwise stable."""
    mc = RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1)
    hc = RM.RldxHeadCfg(steps=2, num_embodiments=4)
    head, sd, hsd, a1 = _head_on_gpu(mc, hc, dev, 71, 1)
    r = _head_reference(hsd, sd, hc, mc, head, e=1).double()
    rel = _rel(a1[0].cpu().double(), r)
    print(f"action head: rel-L2 to the fp32 composition {rel:.2e}")
    assert torch.isfinite(a1).all() and rel <= 2e-2


@pytest.mark.parametrize("prefix_len,use_vlln", [(4, False), (0, True), (15, True)])
def test_rldx_action_head_prefix_and_vlln_match_fp32_composition(dev, prefix_len, use_vlln):
    """RTC trained mode (the first prefix_len rows frozen to the prefix, encoded
    once at time 1, postfix-only decode) and vlln on the VL tokens, 1 DS + 1 SS,
    2 steps, one hipGraph, against the oracle's fp32 composition: rel-L2 <= 2e-2,
    the prefix rows are the prefix bit for bit, and replays are bitwise stable."""
    mc = RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1)
    hc = RM.RldxHeadCfg(steps=2, num_embodiments=4, prefix_len=prefix_len, use_vlln=use_vlln)
    head, sd, hsd, a1 = _head_on_gpu(mc, hc, dev, 91 + prefix_len, 2)
    r = _head_reference(hsd, sd, hc, mc, head, e=2).double()
    rel = _rel(a1[0].cpu().double(), r)
    print(f"action head (prefix_len={prefix_len}, vlln={use_vlln}): rel-L2 to the fp32 composition {rel:.2e}")
    assert torch.isfinite(a1).all() and rel <= 2e-2
    if prefix_len > 0:
        assert torch.equal(a1[0, :prefix_len], head.prefix[0])


@pytest.mark.parametrize("prefix_len,use_vlln", [(0, False), (4, True)])
def test_rldx_action_head_batch_of_robots(dev, prefix_len, use_vlln):
    """An action head for three robots (for_batch: the same MSAT and head
    weights) with their own VL tokens, states, noise, prefixes and embodiment
    ids (gathered per robot on the device), one hipGraph: each robot's actions
    agree with the batch-1 head run on that robot alone (rel-L2 <= 1e-2; the
    larger batch's GEMMs may order sums differently) and with the oracle's
    fp32 composition for that robot (rel-L2 <= 2e-2, the batch-1 head's
    bound); the prefix rows are each robot's prefix bit for bit."""
    mc = RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1)
    hc = RM.RldxHeadCfg(steps=2, num_embodiments=4, prefix_len=prefix_len, use_vlln=use_vlln)
    head, sd, hsd, _ = _head_on_gpu(mc, hc, dev, 111 + prefix_len, 0)
    three = head.for_batch(3)
    assert three.batch == 3 and three.msat.ds is head.msat.ds and three.sd is head.sd
    g = torch.Generator(device=dev).manual_seed(7)
    names = ["vl", "state", "x0"] + (["prefix"] if prefix_len else [])
    for n in names:
        t = getattr(three, n)
        t.copy_(torch.randn(t.shape, generator=g, device=dev))
    emb = [2, 0, 3]
    three.set_embodiment(emb)
    three.capture()
    a = three.replay().clone()
    for b in range(3):
        for n in names:
            getattr(head, n).copy_(getattr(three, n)[b:b + 1])
        head.set_embodiment(emb[b])
        alone = head.replay().clone()
        rel1 = _rel(a[b].cpu().double(), alone[0].cpu().double())
        rel32 = _rel(a[b].cpu().double(), _head_reference(hsd, sd, hc, mc, head, e=emb[b]).double())
        print(f"action head, robot {b} of 3 (embodiment {emb[b]}): vs alone {rel1:.2e}, to fp32 {rel32:.2e}")
        assert torch.isfinite(a[b]).all() and rel1 <= 1e-2 and rel32 <= 2e-2
        if prefix_len:
            assert torch.equal(a[b, :prefix_len], three.prefix[b])


def test_rldx_action_head_release_shape_as_accurate_as_eager_bf16(dev):
    """The release action head: state encoder + 4 denoising steps of action
    encoder, the 4 DS + 8 SS MSAT (24 x 64, 18 SA + 64 VL tokens) and decoder,
    one hipGraph.  Referee as for the full MSAT: the GPU actions are no further
    from the fp32 composition than 1.5x the eager bf16 composition is (which
    rounds after every op on the CPU), and their cosine to the bf16 composition
    is >= 0.999."""
    mc = RM.RldxMsatCfg()
    hc = RM.RldxHeadCfg(num_embodiments=4)
    head, sd, hsd, a1 = _head_on_gpu(mc, hc, dev, 81, 3)
    o = a1[0].cpu().double()
    r32 = _head_reference(hsd, sd, hc, mc, head, e=3).double()
    r16 = _head_reference(hsd, sd, hc, mc, head, e=3, dtype=torch.bfloat16).double()
    floor, got = _rel(r16, r32), _rel(o, r32)
    cos = torch.nn.functional.cosine_similarity(o.flatten(), r16.flatten(), dim=0).item()
    print(f"release action head: rel-L2 to fp32 {got:.2e} (eager bf16: {floor:.2e}), to the bf16 composition "
          f"{_rel(o, r16):.2e}, max-abs to bf16 {(o - r16).abs().max().item():.3e}, cos {cos:.6f}")
    assert torch.isfinite(a1).all() and got <= 1.5 * floor and cos >= 0.999


def _live_action_model(mc, hc, sd, hsd, dev, seed):
    """A module with GraphSafeActionModel's attributes (graph_safe_action_model.py:
    112-153): gs_msat (_msat with its time modules, n_vl, n_sa_pure, n_physics),
    vlln, the per-embodiment encoders / decoder under CategorySpecificLinear's
    parameter names (W, b), the position embedding, the bf16 schedule; its own
    forward records the call and returns "own"."""
    m = torch.nn.Module()
    gs = torch.nn.Module()
    gs.add_module("_msat", _tree_with_time_modules(mc, sd, dev, seed))
    rope = torch.nn.Module()  # a bf16-cast model's RoPE embedder: real-valued tables (the bf16 quirk)
    rope.theta, rope.max_seq_len = mc.rope_theta, mc.max_seq_len
    rope.register_buffer("freqs_cis_0", torch.zeros(1, dtype=torch.bfloat16, device=dev), persistent=False)
    gs._msat.add_module("rope_embedder", rope)
    gs.n_vl, gs.n_sa_pure, gs.n_physics = mc.n_vl, mc.n_sa_pure, 0
    m.add_module("gs_msat", gs)
    for enc, layers in (("state_encoder", ("layer1", "layer2")), ("action_encoder", ("W1", "W2", "W3")),
                        ("action_decoder", ("layer1", "layer2"))):
        mod = torch.nn.Module()
        for layer in layers:
            sub = torch.nn.Module()
            sub.W = torch.nn.Parameter(hsd[f"{enc}.{layer}.W"], requires_grad=False)
            sub.b = torch.nn.Parameter(hsd[f"{enc}.{layer}.b"], requires_grad=False)
            mod.add_module(layer, sub)
        m.add_module(enc, mod)
    pe = torch.nn.Embedding(hc.action_horizon + 8, mc.sa_dim, device=dev, dtype=torch.bfloat16)
    pe.weight.data[:hc.action_horizon] = hsd["position_embedding.weight"]
    m.add_module("position_embedding", pe)
    m.static_pos_ids = torch.arange(hc.action_horizon, device=dev)
    m.static_timesteps = torch.tensor([t / hc.steps for t in range(hc.steps)], dtype=torch.bfloat16, device=dev)
    if hc.use_vlln:
        ln = torch.nn.LayerNorm(mc.vl_dim, device=dev, dtype=torch.bfloat16)
        ln.weight.data.copy_(hsd["vlln.weight"])
        ln.bias.data.copy_(hsd["vlln.bias"])
        m.add_module("vlln", ln)
    else:
        m.add_module("vlln", torch.nn.Identity())
    m.action_horizon, m.action_dim, m.num_inference_timesteps = hc.action_horizon, hc.action_dim, hc.steps
    m.prefix_len, m.dt = hc.prefix_len, 1.0 / hc.steps
    m.calls = []
    m.forward = lambda *a, **k: m.calls.append((a, k)) or "own"
    return m


def test_install_action_head_on_a_live_model(dev):
    """install_action_head builds the head from a live action model (weights,
    baked position embedding and time embeddings, vlln) and serves batch-1
    calls with the reference signature, RTC prefix and vlln included, against
    the oracle's fp32 composition (rel-L2 <= 2e-2, prefix rows exact), for two
    embodiments through one captured graph; a batch of two robots with their
    own embodiments runs on a head of its own (same weights) to the same bound;
    a missing prefix is refused to the module's own forward, an embodiment id
    out of range raises IndexError without disabling the dispatcher."""
    mc = RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1)
    hc = RM.RldxHeadCfg(steps=2, num_embodiments=3, prefix_len=2, use_vlln=True)
    sd = RM.make_state_dict(mc, dev, seed=101)
    hsd = RM.make_head_state_dict(mc, hc, dev, seed=102)
    m = _live_action_model(mc, hc, sd, hsd, dev, 103)
    d = RM.install_action_head(m)  # the bf16 quirk detected from the RoPE tables
    h = d.head
    for k in hsd:
        if not k.startswith("static_"):
            assert torch.equal(h.sd[k], hsd[k]), k
    msat = m.gs_msat._msat
    for i, t in enumerate(m.static_timesteps):
        temb, tt = _time_inputs(msat, t.reshape(1))
        assert torch.equal(h.sd["static_tembs"][i], temb) and torch.equal(h.sd["static_time_tokens"][i, :, :1], tt)
    g = torch.Generator(device=dev).manual_seed(104)

    def rnd(*s):
        return torch.randn(*s, generator=g, device=dev).to(torch.bfloat16)

    for e in (2, 0):
        vl, state = rnd(1, mc.n_vl, mc.vl_dim), rnd(1, hc.state_dim)
        x0, prefix = rnd(1, hc.action_horizon, hc.action_dim), rnd(1, 2, hc.action_dim)
        out = m(vl, state, torch.tensor([e]), init_noise=x0, prefix_actions=prefix)
        ref = R.action_head(h.sd, sd, vl, state[:, None], x0, steps=hc.steps, heads=mc.heads, head_dim=mc.head_dim,
                            ds_blocks=mc.ds_blocks, ss_blocks=mc.ss_blocks, e=e, prefix=prefix, use_vlln=True).double()
        rel = _rel(out[0].cpu().double(), ref)
        print(f"installed action head, embodiment {e}: rel-L2 to the fp32 composition {rel:.2e}")
        assert torch.isfinite(out).all() and rel <= 2e-2
        assert torch.equal(out[0, :2], prefix[0])
    assert d.served == 2 and m.calls == []
    # two robots with embodiments 0 and 1: a head for the batch, on the same weights, captured on first use
    vl2, state2 = rnd(2, mc.n_vl, mc.vl_dim), rnd(2, hc.state_dim)
    x02, prefix2 = rnd(2, hc.action_horizon, hc.action_dim), rnd(2, 2, hc.action_dim)
    out2 = m(vl2, state2, torch.tensor([0, 1]), init_noise=x02, prefix_actions=prefix2)
    assert d.served == 3 and m.calls == [] and d.heads[2].batch == 2 and d.heads[2].msat.ds is h.msat.ds
    for b in range(2):
        ref = R.action_head(h.sd, sd, vl2[b:b + 1], state2[b:b + 1, None], x02[b:b + 1], steps=hc.steps,
                            heads=mc.heads, head_dim=mc.head_dim, ds_blocks=mc.ds_blocks, ss_blocks=mc.ss_blocks,
                            e=b, prefix=prefix2[b:b + 1], use_vlln=True).double()
        rel = _rel(out2[b].cpu().double(), ref)
        print(f"installed action head, robot {b} of 2 (embodiment {b}): rel-L2 to the fp32 composition {rel:.2e}")
        assert torch.isfinite(out2[b]).all() and rel <= 2e-2
        assert torch.equal(out2[b, :2], prefix2[b])
    assert m(vl, state, torch.tensor([1]), init_noise=x0) == "own"
    assert d.refusals == {"prefix_len > 0 without prefix_actions": 1}
    with pytest.raises(IndexError):
        m(vl, state, torch.tensor([3]), init_noise=x0, prefix_actions=prefix)
    with pytest.raises(ValueError):  # one embodiment id per robot
        m(vl2, state2, torch.tensor([0]), init_noise=x02, prefix_actions=prefix2)
    out = m(vl, state, torch.tensor([1]), prefix_actions=prefix)  # noise drawn here
    assert not d.failed and d.served == 4 and torch.isfinite(out).all() and torch.equal(out[0, :2], prefix[0])
    # the mirrored CustomActionHeadChain (the reference's build function) on an identical model: the same bits
    from rldx_amd.compat.inference.action_model.engine.custom_action_model_chain import \
        build_custom_action_model_chain
    chain = build_custom_action_model_chain(_live_action_model(mc, hc, sd, hsd, dev, 103), dev)
    a = chain(vl, state, torch.tensor([0]), init_noise=x0, prefix_actions=prefix)
    b = m(vl, state, torch.tensor([0]), init_noise=x0, prefix_actions=prefix)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    # check_weights: an in-place update of a live weight drops the head; the call
    # that notices it rebuilds the head and is served by the module's own
    # forward, the next one by the rebuilt head, which matches a head built
    # from the updated weights
    d.check_weights = True
    with torch.no_grad():
        m.action_decoder.layer2.b.mul_(0.5)
    assert m(vl, state, torch.tensor([0]), init_noise=x0, prefix_actions=prefix) == "own"
    assert d.rebuilds == 1 and d.head is not None and d.refusals["building the head"] == 1
    c = m(vl, state, torch.tensor([0]), init_noise=x0, prefix_actions=prefix)
    assert d.head is not None and not d.failed
    # a head built from a snapshot of the updated weights (the fake model's
    # parameters share storage with hsd, so the snapshot is taken from it now)
    hsd2 = {k: v.clone() for k, v in hsd.items()}
    fresh = RM.install_action_head(_live_action_model(mc, hc, sd, hsd2, dev, 103), graph=False)
    e2 = fresh.model(vl, state, torch.tensor([0]), init_noise=x0, prefix_actions=prefix)
    assert torch.equal(c.view(torch.int16), e2.view(torch.int16))
    assert not torch.equal(c.view(torch.int16), b.view(torch.int16))
