"""GPU parity of the all-add-ons RLDX-1 MSAT chain (RldxMsat with a physics
stream: ExpandedDoubleStreamBlocks over [VL | SA | P], ExpandedSingleStreamBlocks
over [VL+SA | P]) against the CPU oracle's MSAT._forward_physics restatement
(oracle/rldx_msat_ref.py) on the same weights, at the reference's all-add-ons
token counts (N_vl = 80, rldx/inference/action_model/README.md:28-37; 17
physics tokens: 1 history + 16 future, physics_head.py:107-109)."""

import pytest
import torch

from oracle import rldx_msat_ref as R
from rldx_amd import rldx_msat as RM
from tolerances import assert_bf16_close

pytestmark = pytest.mark.gpu


def _cfg(**kw):
    base = dict(n_vl=80, use_physics=True, n_physics=17)
    base.update(kw)
    return RM.RldxMsatCfg(**base)


def _oracle(sd, inp, cfg, quirk=True, mask=None, pmask=None):
    cpu = {k: v.cpu() for k, v in sd.items()}
    return R.msat_forward_physics(cpu, inp["sa"].cpu(), inp["vl"].cpu(), inp["p"].cpu(), inp["temb"].cpu(),
                                  inp["time_token"].cpu(), heads=cfg.heads, head_dim=cfg.head_dim,
                                  ds_blocks=cfg.ds_blocks, ss_blocks=cfg.ss_blocks, theta=cfg.rope_theta,
                                  max_seq_len=cfg.max_seq_len, bf16_quirk=quirk,
                                  encoder_attention_mask=None if mask is None else mask.cpu(),
                                  physics_attention_mask=None if pmask is None else pmask.cpu())


def _run(chain, inp, mask=None, pmask=None):
    o = chain.forward(inp["sa"], inp["vl"], inp["temb"], inp["time_token"], mask, inp["p"], pmask)
    return o["action"].clone(), o["physics"].clone()


def _rel(a, b):
    return ((a - b).norm() / b.norm()).item()


def _as_accurate_as_eager_bf16(outs, sd, inp, cfg, what, quirk=True, mask=None, pmask=None):
    """Bound as for the no-add-ons chain: each output is no further from the
    fp32 evaluation of the same weights and inputs than 1.5x the eager bf16
    evaluation is, and its cosine to the bf16 oracle is >= 0.999."""
    r16 = _oracle(sd, inp, cfg, quirk, mask, pmask)
    sd32 = {k: v.float() for k, v in sd.items()}
    inp32 = {k: v.float() for k, v in inp.items()}
    r32 = _oracle(sd32, inp32, cfg, quirk, mask, pmask)
    for name, o, a16, a32 in zip(("action", "physics"), outs, r16, r32):
        o, a16, a32 = o.detach().cpu().double(), a16.double(), a32.double()
        floor, got = _rel(a16, a32), _rel(o, a32)
        cos = torch.nn.functional.cosine_similarity(o.flatten(), a16.flatten(), dim=0).item()
        print(f"{what} / {name}: rel-L2 to fp32 {got:.2e} (eager bf16: {floor:.2e}), to the bf16 oracle "
              f"{_rel(o, a16):.2e}, max-abs {(o - a16).abs().max().item():.3e}, cos {cos:.6f}")
        assert torch.isfinite(o).all() and got <= 1.5 * floor and cos >= 0.999, f"{what} / {name}"


@pytest.mark.parametrize("quirk", [True, False])
def test_physics_msat_one_block_each(dev, quirk):
    """1 Expanded DS + 1 Expanded SS block; the bf16 contract on both outputs
    (output projections drawn with std 0.01, as for the no-add-ons test)."""
    cfg = _cfg(ds_blocks=1, ss_blocks=1)
    sd = RM.make_state_dict(cfg, dev, seed=121)
    for k in ("proj_out_2.weight", "proj_out_physics_2.weight"):
        sd[k] = (sd[k].float() * 0.5).to(torch.bfloat16)
    inp = RM.make_inputs(cfg, dev, seed=122)
    chain = RM.RldxMsat(sd, cfg, dev, bf16_quirk=quirk)
    a, p = _run(chain, inp)
    ra, rp = _oracle(sd, inp, cfg, quirk)
    assert_bf16_close(a, ra, f"all-add-ons MSAT 1 + 1 action, quirk={quirk}")
    assert_bf16_close(p, rp, f"all-add-ons MSAT 1 + 1 physics, quirk={quirk}")


def test_physics_msat_full_model(dev):
    """4 Expanded DS + 8 Expanded SS blocks at the release widths (1839.8 M
    parameters), N_vl = 80, 17 physics tokens."""
    cfg = _cfg()
    sd = RM.make_state_dict(cfg, dev, seed=131)
    inp = RM.make_inputs(cfg, dev, seed=132)
    chain = RM.RldxMsat(sd, cfg, dev)
    _as_accurate_as_eager_bf16(_run(chain, inp), sd, inp, cfg, "all-add-ons MSAT")


def test_physics_msat_masks_in_graph_replay(dev):
    """encoder_attention_mask and physics_attention_mask through the captured
    graph: replays equal eager runs bit for bit, each matches the oracle with
    the same masks, and a masked physics stream changes the action output."""
    cfg = _cfg(ds_blocks=2, ss_blocks=2)
    sd = RM.make_state_dict(cfg, dev, seed=141)
    inp = RM.make_inputs(cfg, dev, seed=142)
    chain = RM.RldxMsat(sd, cfg, dev, vl_mask=True)
    chain.capture()
    vmask = torch.ones(1, cfg.n_vl, device=dev)
    vmask[:, 3:cfg.n_vl:4] = 0
    cases = [(None, None), (vmask, None), (None, torch.zeros(1, device=dev)), (vmask, torch.ones(1, device=dev))]
    outs = []
    for mask, pmask in cases:
        for k in ("sa", "vl", "temb", "time_token", "p"):
            chain.inputs[k].copy_(inp[k])
        chain.inputs["vl_mask"].copy_(torch.ones_like(vmask) if mask is None else mask)
        chain.inputs["physics_mask"].fill_(1.0 if pmask is None else float(pmask.item()))
        g = chain.replay()
        got = (g["action"].clone(), g["physics"].clone())
        torch.cuda.synchronize()
        eager = _run(chain, inp, mask, pmask)
        torch.cuda.synchronize()
        for x, y in zip(got, eager):
            assert torch.equal(x.view(torch.int16), y.view(torch.int16)), f"replay, masks {mask is not None}, {pmask}"
        _as_accurate_as_eager_bf16(got, sd, inp, cfg, f"graph, vl mask {mask is not None}, physics mask {pmask}",
                                   mask=mask, pmask=pmask)
        outs.append(got)
    assert (outs[2][0].float() - outs[0][0].float()).abs().max() > 1e-2, "the physics mask changed nothing"
    assert (outs[1][0].float() - outs[0][0].float()).abs().max() > 1e-2, "the VL mask changed nothing"


def test_dispatcher_serves_physics_calls(dev):
    """A physics-enabled module tree (use_physics = True): the dispatcher builds
    the all-add-ons chain from the first physics call and serves the later
    ones (graph replay) with both masks; a call with another physics token
    count, or none, goes to the module's own forward."""
    cfg = _cfg(ds_blocks=1, ss_blocks=1, n_physics=9)
    sd = RM.make_state_dict(cfg, dev, seed=151)
    root = torch.nn.Module()
    for k, v in sd.items():
        *path, leaf = k.split(".")
        m = root
        for part in path:
            if not hasattr(m, part):
                m.add_module(part, torch.nn.Module())
            m = getattr(m, part)
        m.register_parameter(leaf, torch.nn.Parameter(v, requires_grad=False))
    root.use_physics = True
    g = torch.Generator(device=dev).manual_seed(152)
    wt = (0.02 * torch.randn(cfg.inner, 1, generator=g, device=dev)).to(torch.bfloat16)
    wtt = (0.02 * torch.randn(cfg.sa_dim, cfg.inner, generator=g, device=dev)).to(torch.bfloat16)
    root.timestep_encoder = lambda t: (t[:, None].to(torch.bfloat16) @ wt.t())
    root.time_token_proj = lambda temb: temb @ wtt.t()
    calls = []

    def own_forward(hidden_states, encoder_hidden_states, timestep=None, return_all_hidden_states=False,
                    encoder_attention_mask=None, physics_embs=None, physics_attention_mask=None):
        calls.append(physics_embs is None)
        return None

    root.forward = own_forward
    d = RM.install(root, bf16_quirk=True, graph=True)
    inp = RM.make_inputs(cfg, dev, seed=153)
    t = torch.tensor([0.25], device=dev)
    root(inp["sa"], inp["vl"], t, physics_embs=inp["p"])
    assert d.chain is not None and d.chain.phys and d.chain.np_ == 9 and calls == [False]
    temb = root.timestep_encoder(t)
    ref = dict(inp, temb=temb, time_token=root.time_token_proj(temb).unsqueeze(1))
    pmask = torch.zeros(1, device=dev)
    vmask = torch.ones(1, cfg.n_vl, device=dev)
    vmask[:, :7] = 0
    o = root(inp["sa"], inp["vl"], t, encoder_attention_mask=vmask, physics_embs=inp["p"],
             physics_attention_mask=pmask)
    assert d.served == 1 and len(calls) == 1
    _as_accurate_as_eager_bf16((o["action"].clone(), o["physics"].clone()), sd, ref, cfg, "dispatcher physics",
                               mask=vmask, pmask=pmask)
    root(inp["sa"], inp["vl"], t, physics_embs=inp["p"][:, :5])
    root(inp["sa"], inp["vl"], t)
    assert calls == [False, False, True] and d.served == 1 and not d.failed


def _head_reference_physics(head_sd, msat_sd, hc, mc, vl, state, x0, hist, px0, e=0, dtype=torch.float32):
    """CPU composition of CustomExpandedActionHeadChain.forward without the RTC
    prefix (custom_expanded_action_model_chain.py:92-219): per-embodiment
    encoders / decoder (embodiment_conditioned_mlp.py), the physics encoders
    and decoder (physics.py:9-72) and the oracle's _forward_physics, evaluated
    in `dtype` (fp32, or bf16 eager with a rounding after every op)."""
    f = {k: v.cpu().to(dtype) for k, v in head_sd.items()}
    sd = {k: v.cpu().to(dtype) for k, v in msat_sd.items()}
    F = torch.nn.functional

    def lin(x, name):  # CategorySpecificLinear, batch 1
        return torch.addmm(f[f"{name}.b"][e], x, f[f"{name}.W"][e])

    def nn_lin(x, name):
        return F.linear(x, f[f"{name}.weight"], f[f"{name}.bias"])

    def sin_enc(t, width):  # SinusoidalPositionalEncoding over positions t [T] (fp32), cast to the model dtype
        half = width // 2
        ex = torch.exp(-torch.arange(half, dtype=torch.float) * (torch.log(torch.tensor(10000.0)) / half))
        fr = t.float()[:, None] * ex
        return torch.cat([torch.sin(fr), torch.cos(fr)], dim=-1).to(dtype)

    def penc(x, pos, enc):
        h = nn_lin(x, f"physics.{enc}.W1")
        return nn_lin(F.silu(nn_lin(torch.cat([h, pos], dim=-1), f"physics.{enc}.W2")), f"physics.{enc}.W3")

    state_feat = lin(torch.relu(lin(state.cpu().to(dtype)[0], "state_encoder.layer1")), "state_encoder.layer2")
    act = x0.cpu().to(dtype)[0].clone()
    hist_tok = penc(hist.cpu().to(dtype)[0], sin_enc(torch.arange(hc.physics_hist_len), mc.sa_dim),
                    "physics_cond_encoder")
    fut = px0.cpu().to(dtype)[0].clone()
    for i in range(hc.steps):
        t = i / hc.steps
        tau = sin_enc(torch.full((hc.action_horizon,), t), mc.sa_dim)
        a = lin(act, "action_encoder.W1")
        x = lin(torch.cat([a, tau], dim=-1), "action_encoder.W2")
        a = lin(x * torch.sigmoid(x), "action_encoder.W3") + f["position_embedding.weight"]
        sa = torch.cat([state_feat, a])[None]
        p_embs = torch.cat([hist_tok, penc(fut, tau[: hc.physics_fut_len], "physics_fut_encoder")])[None]
        out, ph = R.msat_forward_physics(sd, sa, vl.cpu().to(dtype), p_embs, f["static_tembs"][i],
                                         f["static_time_tokens"][i], heads=mc.heads, head_dim=mc.head_dim,
                                         ds_blocks=mc.ds_blocks, ss_blocks=mc.ss_blocks)
        v = lin(torch.relu(lin(out[0], "action_decoder.layer1")), "action_decoder.layer2")[-hc.action_horizon:]
        act.add_(v, alpha=1.0 / hc.steps)
        pv = nn_lin(F.silu(nn_lin(ph[0, -hc.physics_fut_len:], "physics.physics_decoder.net.0")),
                    "physics.physics_decoder.net.2")
        fut.add_(pv, alpha=1.0 / hc.steps)
    return act, fut


def _physics_head_on_gpu(mc, hc, dev, seed, embodiment):
    sd = RM.make_state_dict(mc, dev, seed=seed)
    hsd = RM.make_head_state_dict(mc, hc, dev, seed=seed + 1)
    head = RM.RldxActionHead(RM.RldxMsat(sd, mc, dev), hsd, hc, embodiment=embodiment)
    g = torch.Generator(device=dev).manual_seed(seed + 2)
    for t in (head.vl, head.state, head.x0, head.physics_hist, head.physics_x0):
        t.copy_(torch.randn(t.shape, generator=g, device=dev))
    head.capture()
    a1 = head.replay().clone()
    f1 = head.physics_fut.clone()
    a2 = head.replay().clone()
    torch.cuda.synchronize()
    assert torch.equal(a1.view(torch.int16), a2.view(torch.int16)), "graph replays differ"
    return head, sd, hsd, a1, f1


def test_all_add_ons_action_head_graph_matches_fp32_composition(dev):
    """State encoder, physics history encoder, then 2 denoising steps of action
    and physics-future encoders, all-add-ons MSAT (1 + 1 Expanded blocks, N_vl
    80, 1 + 16 physics tokens), action and physics decoders and both Euler
    updates as one hipGraph, against an fp32 CPU composition: actions and the
    physics future agree to rel-L2 <= 2e-2 and replays are bitwise stable."""
    hc = RM.RldxHeadCfg(steps=2, num_embodiments=4, physics_dim=37, physics_hist_len=1)
    mc = _cfg(ds_blocks=1, ss_blocks=1, n_physics=hc.physics_hist_len + hc.physics_fut_len)
    head, sd, hsd, a1, f1 = _physics_head_on_gpu(mc, hc, dev, 171, 2)
    ra, rf = _head_reference_physics(hsd, sd, hc, mc, head.vl, head.state, head.x0, head.physics_hist,
                                     head.physics_x0, e=2)
    rel_a, rel_f = _rel(a1[0].cpu().double(), ra.double()), _rel(f1[0].cpu().double(), rf.double())
    print(f"all-add-ons action head: actions rel-L2 {rel_a:.2e}, physics future rel-L2 {rel_f:.2e}")
    assert torch.isfinite(a1).all() and torch.isfinite(f1).all() and rel_a <= 2e-2 and rel_f <= 2e-2


def test_all_add_ons_action_head_full_depth_as_accurate_as_eager_bf16(dev):
    """The all-add-ons action head at full depth: 4 denoising steps through the
    4 + 8 Expanded-block MSAT (N_vl 80, 1 + 16 physics tokens) with both
    decoders and Euler updates, one hipGraph.  Referee as for the full MSAT:
    actions and physics future are each no further from the fp32 composition
    than 1.5x the eager bf16 composition is, with cosine >= 0.999 to the latter."""
    hc = RM.RldxHeadCfg(num_embodiments=4, physics_dim=37, physics_hist_len=1)
    mc = _cfg(n_physics=hc.physics_hist_len + hc.physics_fut_len)
    head, sd, hsd, a1, f1 = _physics_head_on_gpu(mc, hc, dev, 181, 1)
    args = (hsd, sd, hc, mc, head.vl, head.state, head.x0, head.physics_hist, head.physics_x0)
    r32 = _head_reference_physics(*args, e=1)
    r16 = _head_reference_physics(*args, e=1, dtype=torch.bfloat16)
    for name, o, a16, a32 in zip(("actions", "physics future"), (a1[0], f1[0]), r16, r32):
        o, a16, a32 = o.cpu().double(), a16.double(), a32.double()
        floor, got = _rel(a16, a32), _rel(o, a32)
        cos = torch.nn.functional.cosine_similarity(o.flatten(), a16.flatten(), dim=0).item()
        print(f"all-add-ons action head / {name}: rel-L2 to fp32 {got:.2e} (eager bf16: {floor:.2e}), to the bf16 "
              f"composition {_rel(o, a16):.2e}, max-abs to bf16 {(o - a16).abs().max().item():.3e}, cos {cos:.6f}")
        assert torch.isfinite(o).all() and got <= 1.5 * floor and cos >= 0.999, name


def test_physics_chain_batch_of_robots(dev):
    """The all-add-ons chain for three robots (for_batch) with different
    inputs, VL masks and physics masks per robot: each robot's action and
    physics outputs agree with the batch-1 chain run on that robot alone
    (rel-L2 <= 1e-2; the larger batch's GEMMs may order sums differently) and
    the batch is as accurate as the eager bf16 batch.  Robot b's SA padding
    rows (its 18 SA rows are padded to 32 in the joint sequence) read the next
    robot's QKV rows: their keys are masked and their outputs not stored, so
    they reach no output."""
    cfg = _cfg(ds_blocks=1, ss_blocks=1)
    sd = RM.make_state_dict(cfg, dev, seed=63)
    one = RM.RldxMsat(sd, cfg, dev, vl_mask=True)
    three = one.for_batch(3)
    inps = [RM.make_inputs(cfg, dev, seed=80 + b) for b in range(3)]
    mask = torch.ones(3, cfg.n_vl, device=dev)
    mask[0, 7:11] = 0
    mask[2, -5:] = 0
    pmask = torch.tensor([1.0, 0.0, 1.0], device=dev)
    alone = [_run(one, i, mask[b:b + 1], pmask[b:b + 1]) for b, i in enumerate(inps)]
    batch = {k: torch.cat([i[k] for i in inps]) for k in inps[0]}
    outs = _run(three, batch, mask, pmask)
    for b in range(3):
        for name, o, a in zip(("action", "physics"), outs, alone[b]):
            rel = _rel(o[b].double().cpu(), a[0].double().cpu())
            print(f"robot {b} / {name}: batch of 3 vs alone rel-L2 {rel:.2e}")
            assert torch.isfinite(o[b]).all() and rel <= 1e-2, (b, name, rel)
    _as_accurate_as_eager_bf16(outs, sd, batch, cfg, "3 robots, physics chain", mask=mask, pmask=pmask)
