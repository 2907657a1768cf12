"""CPU oracle of the synthetic MSAT action step — TEST INFRASTRUCTURE ONLY.

Eager composition of the reference block (ExpandedDoubleStreamBlock.forward with
identity modulation, rldx/model/modules/action_model/blocks.py:705-891) and the
denoising loop (GraphSafeActionModel.forward,
rldx/inference/action_model/model/graph_safe_action_model.py:430-485), in CPU
bf16 torch.  Weights and inputs are the same tensors the GPU step uses
(rldx_amd.msat_step.make_weights / make_inputs, copied to the host).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .cpu_reference import layer_norm, merge_heads, msat_qkv_norm_rope, sdpa

STREAMS = ("vl", "sa", "p")


def block(cfg, w, L, xs, inp):
    """One triple-stream block on per-stream residuals xs = {vl, sa, p}."""
    qkv = {s: F.linear(layer_norm(xs[s], cfg.eps), w[f"{s}.qkv.w"][L], w[f"{s}.qkv.b"][L]) for s in STREAMS}
    streams = [
        (qkv["vl"], w["vl.q_norm"][L], w["vl.k_norm"][L], None, None),
        (qkv["sa"], w["sa.q_norm"][L], w["sa.k_norm"][L], inp["sa_cos"], inp["sa_sin"]),
        (qkv["p"], w["p.q_norm"][L], w["p.k_norm"][L], inp["p_cos"], inp["p_sin"]),
    ]
    q, k, v = msat_qkv_norm_rope(streams, cfg.heads, cfg.head_dim, cfg.eps)
    o = merge_heads(sdpa(q[None], k[None], v[None], key_bias=inp["key_bias"]))[0]
    n_vl, n_sa = cfg.n_vl, cfg.n_sa
    parts = {"vl": o[:n_vl], "sa": o[n_vl:n_vl + n_sa], "p": o[n_vl + n_sa:]}
    out = {}
    for s in STREAMS:
        x = xs[s] + F.linear(parts[s], w[f"{s}.proj.w"][L], w[f"{s}.proj.b"][L])
        u = F.linear(layer_norm(x, cfg.eps), w[f"{s}.w12.w"][L], w[f"{s}.w12.b"][L])
        x1, x2 = u.chunk(2, dim=-1)
        out[s] = x + F.linear(F.silu(x1) * x2, w[f"{s}.w3.w"][L], w[f"{s}.w3.b"][L])
    return out


def action_step(cfg, w, inp, steps=None, blocks=None):
    """Full action step: `steps` Euler iterations over `blocks` blocks."""
    steps = cfg.steps if steps is None else steps
    blocks = cfg.blocks if blocks is None else blocks
    act = inp["x0"].clone()
    dt = 1.0 / cfg.steps
    for t in range(steps):
        sa = F.linear(act, w["act_in.w"], w["act_in.b"]) + inp["temb"][t]
        sa = sa + inp["pos"]
        xs = {"vl": inp["vl"], "sa": sa, "p": inp["p"]}
        for L in range(blocks):
            xs = block(cfg, w, L, xs, inp)
        vel = F.linear(layer_norm(xs["sa"], cfg.eps), w["act_out.w"], w["act_out.b"])
        act = act + dt * vel
    return act
