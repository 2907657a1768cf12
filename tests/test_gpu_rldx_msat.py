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
    short = RM.make_inputs(RM.RldxMsatCfg(ds_blocks=1, ss_blocks=1, n_vl=32), dev, seed=67)
    msat(inp["sa"], short["vl"], t)
    assert len(msat.calls) == 3 and d.served == 3 and not d.failed


def _head_reference(head_sd, msat_sd, hc, mc, vl, state, x0, e=0, dtype=torch.float32):
    """CPU composition of CustomActionHeadChain.forward (custom_action_model_chain.py:81-171)
    from the oracle MSAT and the per-embodiment MLPs of embodiment_conditioned_mlp.py,
    evaluated in `dtype` (fp32, or bf16 eager with a rounding after every op)."""
    f = {k: v.cpu().to(dtype) for k, v in head_sd.items()}
    sd = {k: v.cpu().to(dtype) for k, v in msat_sd.items()}

    def lin(x, name):  # CategorySpecificLinear, batch 1
        return torch.addmm(f[f"{name}.b"][e], x, f[f"{name}.W"][e])

    def tau(t, width):  # SinusoidalPositionalEncoding (fp32), cast to the model dtype
        half = width // 2
        ex = torch.exp(-torch.arange(half, dtype=torch.float) * (torch.log(torch.tensor(10000.0)) / half))
        fr = torch.full((hc.action_horizon, 1), t) * ex
        return torch.cat([torch.sin(fr), torch.cos(fr)], dim=-1).to(dtype)

    state_feat = lin(torch.relu(lin(state.cpu().to(dtype)[0], "state_encoder.layer1")), "state_encoder.layer2")
    act = x0.cpu().to(dtype)[0].clone()
    for i in range(hc.steps):
        a = lin(act, "action_encoder.W1")
        x = lin(torch.cat([a, tau(i / hc.steps, mc.sa_dim)], dim=-1), "action_encoder.W2")
        a = lin(x * torch.sigmoid(x), "action_encoder.W3") + f["position_embedding.weight"]
        sa = torch.cat([state_feat, a])[None]
        out = R.msat_forward(sd, sa, vl.cpu().to(dtype), f["static_tembs"][i], f["static_time_tokens"][i],
                             heads=mc.heads, head_dim=mc.head_dim, ds_blocks=mc.ds_blocks, ss_blocks=mc.ss_blocks)
        v = lin(torch.relu(lin(out[0], "action_decoder.layer1")), "action_decoder.layer2")[-hc.action_horizon:]
        act.add_(v, alpha=1.0 / hc.steps)
    return act


def _head_on_gpu(mc, hc, dev, seed, embodiment):
    sd = RM.make_state_dict(mc, dev, seed=seed)
    hsd = RM.make_head_state_dict(mc, hc, dev, seed=seed + 1)
    head = RM.RldxActionHead(RM.RldxMsat(sd, mc, dev), hsd, hc, embodiment=embodiment)
    g = torch.Generator(device=dev).manual_seed(seed + 2)
    head.vl.copy_(torch.randn(head.vl.shape, generator=g, device=dev))
    head.state.copy_(torch.randn(head.state.shape, generator=g, device=dev))
    head.x0.copy_(torch.randn(head.x0.shape, generator=g, device=dev))
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
    r = _head_reference(hsd, sd, hc, mc, head.vl, head.state, head.x0, e=1).double()
    rel = _rel(a1[0].cpu().double(), r)
    print(f"action head: rel-L2 to the fp32 composition {rel:.2e}")
    assert torch.isfinite(a1).all() and rel <= 2e-2


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
    r32 = _head_reference(hsd, sd, hc, mc, head.vl, head.state, head.x0, e=3).double()
    r16 = _head_reference(hsd, sd, hc, mc, head.vl, head.state, head.x0, e=3, dtype=torch.bfloat16).double()
    floor, got = _rel(r16, r32), _rel(o, r32)
    cos = torch.nn.functional.cosine_similarity(o.flatten(), r16.flatten(), dim=0).item()
    print(f"release action head: rel-L2 to fp32 {got:.2e} (eager bf16: {floor:.2e}), to the bf16 composition "
          f"{_rel(o, r16):.2e}, max-abs to bf16 {(o - r16).abs().max().item():.3e}, cos {cos:.6f}")
    assert torch.isfinite(a1).all() and got <= 1.5 * floor and cos >= 0.999
