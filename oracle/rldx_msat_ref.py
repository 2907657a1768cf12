"""CPU oracle of the RLDX-1 MSAT forward — TEST INFRASTRUCTURE ONLY.

Eager restatement, in CPU bf16 torch, of MSAT._forward_inner with the
`input_token` time conditioning and `rope_sa_only` positions
(rldx/model/modules/action_model/msat.py:291-556, :777-781), its
DoubleStreamBlock.forward and SingleStreamBlock.forward with identity
modulation (rldx/model/modules/action_model/blocks.py:166-254, :383-609), the
RoPE embedder and rotary product (rldx/model/modules/action_model/ops.py:11-119),
RMSNorm (rldx/model/modules/norms.py:7-22) and SwiGLUFFN (ops.py:137-161).

The all-add-ons forward (`msat_forward_physics`) restates MSAT._forward_physics
(msat.py:558-775) with ExpandedDoubleStreamBlock.forward over [VL | SA | P]
(blocks.py:705-891) and ExpandedSingleStreamBlock.forward over [VL+SA | P]
(blocks.py:970-1089), identity modulation on every stream.

Weights are a state dict under the reference module's own names
(`double_blocks.{i}.sa_qkv.weight`, `single_blocks.{i}.linear1.bias`, ...).
The time embedding `temb` and the time token are inputs, as in the reference's
inference chain (custom_msat_chain.py:109-126), which bakes them per step.
With identity modulation, (1 + 0) * y + 0 and 1 * y reproduce y exactly in
bf16, so the modulation products are not spelled out.

`action_head` composes the MSAT with the action head around it
(CustomActionHeadChain.forward, custom_action_model_chain.py:81-171): vlln,
the state / action encoders, the RTC trained-mode prefix, the decoder and the
Euler update.  Its pins (tests/test_rldx_msat_host.py): the Euler update in
closed form (a decoder with zero weights moves every free row by exactly its
bias, the prefix rows not at all), the prefix path against the unsliced
re-lock composition (encode every row with per-row time, decode every row,
re-lock the prefix after each step), and vlln against LayerNorm written out.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .cpu_reference import apply_rotary_emb, layer_norm, merge_heads, msat_rmsnorm, sdpa, split_heads, swiglu


def rope_freq_tables(head_dim: int, theta: float, max_seq_len: int, bf16_quirk: bool):
    """RoPEEmbedder1D buffers for axes [D/4, 3D/4] (msat.py:883-893; ops.py:11-25,
    :82-103): precompute_freqs_cis per axis, complex64 [max_seq_len, axis_dim/2].
    bf16_quirk: the buffers of a model loaded with torch_dtype=bfloat16 — the cast
    keeps the real part (cos) in bf16 and drops the imaginary part
    (custom_msat_chain.py:15-54)."""
    tables = []
    for dim in (head_dim // 4, head_dim - head_dim // 4):
        freqs = 1.0 / (theta ** (torch.arange(0, dim, 2)[: (dim // 2)].float() / dim))
        t = torch.arange(max_seq_len)
        freqs = torch.outer(t, freqs).float()
        fc = torch.polar(torch.ones_like(freqs), freqs)
        tables.append(fc.real.to(torch.bfloat16) if bf16_quirk else fc)
    return tables


def rope_pe(tables, ids: torch.Tensor) -> torch.Tensor:
    """RoPEEmbedder1D.forward (ops.py:105-118): ids [B, N, 2] -> [B, N, D/2]."""
    return torch.cat([tables[i][ids[..., i]] for i in range(len(tables))], dim=-1)


def _linear(x, sd, name):
    return F.linear(x, sd[f"{name}.weight"], sd.get(f"{name}.bias"))


def _swiglu_ffn(x, sd, name):
    """SwiGLUFFN.forward (ops.py:155-161): w3(silu(x1) * x2), x1 | x2 = w12(x)."""
    return _linear(swiglu(_linear(x, sd, f"{name}.w12")), sd, f"{name}.w3")


def _qk_norm(x, w):
    """per-head RMSNorm over [B, H, N, Dh] (blocks.py:525-537)."""
    return msat_rmsnorm(x, w)


def key_bias_of(mask: torch.Tensor, n_rest: int, dtype) -> torch.Tensor:
    """Joint-attention key mask of an encoder (VL) mask: cat([mask, ones]) then
    -inf where 0 and 0 elsewhere, in the activation dtype (blocks.py:558-575,
    msat.py:517-531).  mask [B, N_vl] -> [B, N_vl + n_rest]."""
    kv = torch.cat([mask, torch.ones(mask.shape[0], n_rest, dtype=mask.dtype)], dim=1)
    return torch.where(kv == 0, torch.tensor(float("-inf"), dtype=dtype), torch.tensor(0.0, dtype=dtype))


def ds_block(sd: dict, p: str, sa: torch.Tensor, vl: torch.Tensor, pe: torch.Tensor, heads: int, key_bias=None):
    """DoubleStreamBlock.forward, identity modulation (blocks.py:383-609).
    sa [B, N_sa, sa_dim] (time token first), vl [B, N_vl, vl_dim]; pe [B, N_vl + N_sa, Dh/2];
    key_bias [B, N_vl + N_sa] additive or None."""
    sa_qkv = _linear(layer_norm(sa), sd, f"{p}sa_qkv")
    vl_qkv = _linear(layer_norm(vl), sd, f"{p}vl_qkv")
    sa_q, sa_k, sa_v = (split_heads(t, heads) for t in sa_qkv.chunk(3, dim=-1))
    vl_q, vl_k, vl_v = (split_heads(t, heads) for t in vl_qkv.chunk(3, dim=-1))
    sa_q, sa_k = _qk_norm(sa_q, sd[f"{p}q_norm_sa.weight"]), _qk_norm(sa_k, sd[f"{p}k_norm_sa.weight"])
    vl_q, vl_k = _qk_norm(vl_q, sd[f"{p}q_norm_vl.weight"]), _qk_norm(vl_k, sd[f"{p}k_norm_vl.weight"])
    q = torch.cat([vl_q, sa_q], dim=2)
    k = torch.cat([vl_k, sa_k], dim=2)
    v = torch.cat([vl_v, sa_v], dim=2)
    q, k = apply_rotary_emb(q, k, pe)
    o = sdpa(q, k, v, key_bias=key_bias)
    n_vl = vl.shape[1]
    sa = sa + _linear(merge_heads(o[:, :, n_vl:]), sd, f"{p}sa_proj")
    vl = vl + _linear(merge_heads(o[:, :, :n_vl]), sd, f"{p}vl_proj")
    sa = sa + _swiglu_ffn(layer_norm(sa), sd, f"{p}sa_mlp")
    vl = vl + _swiglu_ffn(layer_norm(vl), sd, f"{p}vl_mlp")
    return sa, vl


def ss_block(sd: dict, p: str, x: torch.Tensor, pe: torch.Tensor, heads: int, key_bias=None):
    """SingleStreamBlock.forward with SwiGLU, identity modulation (blocks.py:166-254)."""
    inner = sd[f"{p}linear2.weight"].shape[1] - sd[f"{p}mlp_proj.weight"].shape[0]
    h = _linear(layer_norm(x), sd, f"{p}linear1")
    qkv, mlp = h[..., : 3 * inner], h[..., 3 * inner:]
    q, k, v = (split_heads(t, heads) for t in qkv.chunk(3, dim=-1))
    q, k = _qk_norm(q, sd[f"{p}q_norm.weight"]), _qk_norm(k, sd[f"{p}k_norm.weight"])
    q, k = apply_rotary_emb(q, k, pe)
    attn = merge_heads(sdpa(q, k, v, key_bias=key_bias))
    mlp_out = _linear(swiglu(mlp), sd, f"{p}mlp_proj")
    return x + _linear(torch.cat([attn, mlp_out], dim=-1), sd, f"{p}linear2")


def msat_forward(sd: dict, sa_embs: torch.Tensor, vl_embs: torch.Tensor, temb: torch.Tensor,
                 time_token: torch.Tensor, *, heads: int, head_dim: int, ds_blocks: int, ss_blocks: int,
                 theta: float = 10000.0, max_seq_len: int = 1024, bf16_quirk: bool = True,
                 encoder_attention_mask=None) -> torch.Tensor:
    """MSAT._forward_inner, non-physics path, temb_type input_token, rope_sa_only
    (msat.py:291-556) and _output_projection (:777-781).
    sa_embs [B, N_sa_pure, sa_dim], vl_embs [B, N_vl, vl_dim], temb [B, inner],
    time_token [B, num_temb_tokens, sa_dim]; encoder_attention_mask [B, N_vl]
    (1 = visible) or None; returns [B, N_sa_pure, output_dim]."""
    tables = rope_freq_tables(head_dim, theta, max_seq_len, bf16_quirk)
    num_temb = time_token.shape[1]
    B, n_vl = vl_embs.shape[:2]
    sa = torch.cat([time_token, sa_embs], dim=1)
    n_sa = sa.shape[1]
    # position ids (msat.py:376-422): VL rows (0, 0); time tokens axis 1 = 0..; SA rows after them
    ids = torch.zeros(B, n_vl + n_sa, 2, dtype=torch.long)
    ids[:, n_vl:n_vl + num_temb, 1] = torch.arange(num_temb)
    ids[:, n_vl + num_temb:, 1] = torch.arange(num_temb, n_sa)
    pe = rope_pe(tables, ids)
    kb = None if encoder_attention_mask is None else key_bias_of(encoder_attention_mask, n_sa, vl_embs.dtype)
    vl = vl_embs
    for i in range(ds_blocks):
        sa, vl = ds_block(sd, f"double_blocks.{i}.", sa, vl, pe, heads, kb)
    time_tok = sa[:, :num_temb]
    sa = sa[:, num_temb:]
    x = torch.cat([_linear(vl, sd, "vl_proj_to_sa"), time_tok, sa], dim=1)
    # single-stream position ids (msat.py:465-487): time tokens 0..; action rows from num_temb + 1
    n_pure = sa.shape[1]
    ids_s = torch.zeros(B, x.shape[1], 2, dtype=torch.long)
    ids_s[:, n_vl:n_vl + num_temb, 1] = torch.arange(num_temb)
    ids_s[:, x.shape[1] - n_pure:, 1] = torch.arange(num_temb + 1, num_temb + 1 + n_pure)
    pe_s = rope_pe(tables, ids_s)
    for i in range(ss_blocks):
        x = ss_block(sd, f"single_blocks.{i}.", x, pe_s, heads, kb)
    sa = x[:, -n_pure:]
    shift, scale = _linear(F.silu(temb), sd, "proj_out_1").chunk(2, dim=1)
    sa = layer_norm(sa) * (1 + scale[:, None]) + shift[:, None]
    return _linear(sa, sd, "proj_out_2")


# ---------------------------------------------------------------------------
# All add-ons: physics (P) stream
# ---------------------------------------------------------------------------
def key_bias_3(vl_mask, n_vl: int, n_sa: int, physics_mask, n_p: int, dtype):
    """Key mask of the [VL | SA | P] (or [VL+SA | P]) joint sequence
    (blocks.py:843-864, msat.py:716-743): VL rows from encoder_attention_mask
    [B, n_vl] (1 visible) or ones, the n_sa rows after them ones, the n_p physics
    rows the per-sample physics_attention_mask [B] broadcast over them, or ones;
    -inf where 0, 0 elsewhere, in the activation dtype.  None when both masks
    are None (the eager blocks then pass attn_mask=None)."""
    if vl_mask is None and physics_mask is None:
        return None
    B = (vl_mask if vl_mask is not None else physics_mask).shape[0]
    vm = vl_mask if vl_mask is not None else torch.ones(B, n_vl, dtype=dtype)
    pm = physics_mask[:, None].expand(-1, n_p).to(vm.dtype) if physics_mask is not None else \
        torch.ones(B, n_p, dtype=vm.dtype)
    kv = torch.cat([vm, torch.ones(B, n_sa, dtype=vm.dtype), pm], dim=1)
    return torch.where(kv == 0, torch.tensor(float("-inf"), dtype=dtype), torch.tensor(0.0, dtype=dtype))


def expanded_ds_block(sd: dict, p: str, sa, vl, ph, pe, heads: int, key_bias=None):
    """ExpandedDoubleStreamBlock.forward with p_tokens, identity modulation
    (blocks.py:729-891): per-stream pre-LN and QKV, per-stream QK-RMSNorm
    (q_norm_p / k_norm_p on P), joint attention over [VL | SA | P] with RoPE from
    pe [B, N_vl + N_sa + N_p, Dh/2], then per-stream proj + residual and SwiGLU
    MLP + residual.  Returns (sa, vl, ph)."""
    n_vl, n_sa = vl.shape[1], sa.shape[1]
    qkvs = [_linear(layer_norm(x), sd, f"{p}{n}_qkv") for x, n in ((vl, "vl"), (sa, "sa"), (ph, "p"))]
    q, k, v = [], [], []
    for t, n in zip(qkvs, ("vl", "sa", "p")):
        tq, tk, tv = (split_heads(u, heads) for u in t.chunk(3, dim=-1))
        q.append(_qk_norm(tq, sd[f"{p}q_norm_{n}.weight"]))
        k.append(_qk_norm(tk, sd[f"{p}k_norm_{n}.weight"]))
        v.append(tv)
    q, k = apply_rotary_emb(torch.cat(q, dim=2), torch.cat(k, dim=2), pe)
    o = sdpa(q, k, torch.cat(v, dim=2), key_bias=key_bias)
    vl = vl + _linear(merge_heads(o[:, :, :n_vl]), sd, f"{p}vl_proj")
    sa = sa + _linear(merge_heads(o[:, :, n_vl:n_vl + n_sa]), sd, f"{p}sa_proj")
    ph = ph + _linear(merge_heads(o[:, :, n_vl + n_sa:]), sd, f"{p}p_proj")
    sa = sa + _swiglu_ffn(layer_norm(sa), sd, f"{p}sa_mlp")
    vl = vl + _swiglu_ffn(layer_norm(vl), sd, f"{p}vl_mlp")
    ph = ph + _swiglu_ffn(layer_norm(ph), sd, f"{p}p_mlp")
    return sa, vl, ph


def expanded_ss_block(sd: dict, p: str, x, ph, pe, heads: int, key_bias=None):
    """ExpandedSingleStreamBlock.forward with p_tokens, SwiGLU, identity
    modulation (blocks.py:970-1089): linear1 / p_linear1 split into QKV | MLP,
    QK-RMSNorm (q_norm, k_norm / p_q_norm, p_k_norm), joint attention over
    [x | P] with RoPE from pe [B, N_x + N_p, Dh/2], then linear2 / p_linear2 of
    [attention | mlp_proj(SwiGLU)] + residual.  Returns (x, ph)."""
    inner = sd[f"{p}linear2.weight"].shape[1] - sd[f"{p}mlp_proj.weight"].shape[0]
    n_x = x.shape[1]
    h = _linear(layer_norm(x), sd, f"{p}linear1")
    hp = _linear(layer_norm(ph), sd, f"{p}p_linear1")
    q, k, v = [], [], []
    for t, qn, kn in ((h, "q_norm", "k_norm"), (hp, "p_q_norm", "p_k_norm")):
        tq, tk, tv = (split_heads(u, heads) for u in t[..., : 3 * inner].chunk(3, dim=-1))
        q.append(_qk_norm(tq, sd[f"{p}{qn}.weight"]))
        k.append(_qk_norm(tk, sd[f"{p}{kn}.weight"]))
        v.append(tv)
    q, k = apply_rotary_emb(torch.cat(q, dim=2), torch.cat(k, dim=2), pe)
    o = sdpa(q, k, torch.cat(v, dim=2), key_bias=key_bias)
    x_mlp = _linear(swiglu(h[..., 3 * inner:]), sd, f"{p}mlp_proj")
    p_mlp = _linear(swiglu(hp[..., 3 * inner:]), sd, f"{p}p_mlp_proj")
    x = x + _linear(torch.cat([merge_heads(o[:, :, :n_x]), x_mlp], dim=-1), sd, f"{p}linear2")
    ph = ph + _linear(torch.cat([merge_heads(o[:, :, n_x:]), p_mlp], dim=-1), sd, f"{p}p_linear2")
    return x, ph


def _adaln_out(x, temb, sd, proj1: str, proj2: str):
    """AdaLN-zero output projection (msat.py:771-781): LN(x) * (1 + scale) + shift,
    shift | scale = proj1(silu(temb)), then proj2."""
    shift, scale = _linear(F.silu(temb), sd, proj1).chunk(2, dim=1)
    return _linear(layer_norm(x) * (1 + scale[:, None]) + shift[:, None], sd, proj2)


def msat_forward_physics(sd: dict, sa_embs, vl_embs, p_embs, temb, time_token, *, heads: int, head_dim: int,
                         ds_blocks: int, ss_blocks: int, theta: float = 10000.0, max_seq_len: int = 1024,
                         bf16_quirk: bool = True, encoder_attention_mask=None, physics_attention_mask=None):
    """MSAT._forward_physics, temb_type input_token, rope_sa_only (msat.py:558-775).
    sa_embs [B, N_sa_pure, sa_dim], vl_embs [B, N_vl, vl_dim], p_embs [B, N_p,
    sa_dim], temb [B, inner], time_token [B, num_temb, sa_dim];
    encoder_attention_mask [B, N_vl] and physics_attention_mask [B] (1 visible)
    or None.  Returns (action [B, N_sa_pure, output_dim], physics [B, N_p,
    output_dim])."""
    tables = rope_freq_tables(head_dim, theta, max_seq_len, bf16_quirk)
    num_temb = time_token.shape[1]
    B, n_vl = vl_embs.shape[:2]
    n_p = p_embs.shape[1]
    sa = torch.cat([time_token, sa_embs], dim=1)
    n_sa = sa.shape[1]
    # lower ids (msat.py:595-639): SA axis 1 = 0 .. n_sa - 1; P axis 0 = 1, axis 1 = 0 .. n_p - 1
    ids = torch.zeros(B, n_vl + n_sa + n_p, 2, dtype=torch.long)
    ids[:, n_vl:n_vl + n_sa, 1] = torch.arange(n_sa)
    ids[:, n_vl + n_sa:, 0] = 1
    ids[:, n_vl + n_sa:, 1] = torch.arange(n_p)
    pe = rope_pe(tables, ids)
    kb = key_bias_3(encoder_attention_mask, n_vl, n_sa, physics_attention_mask, n_p, vl_embs.dtype)
    vl, ph = vl_embs, p_embs
    for i in range(ds_blocks):
        sa, vl, ph = expanded_ds_block(sd, f"double_blocks.{i}.", sa, vl, ph, pe, heads, kb)
    time_tok, sa = sa[:, :num_temb], sa[:, num_temb:]
    x = torch.cat([_linear(vl, sd, "vl_proj_to_sa"), time_tok, sa], dim=1)
    n_pure, n_x = sa.shape[1], x.shape[1]
    # upper ids (msat.py:679-712): time tokens 0 ..; action rows from num_temb + 1; P as below
    ids_s = torch.zeros(B, n_x + n_p, 2, dtype=torch.long)
    ids_s[:, n_vl:n_vl + num_temb, 1] = torch.arange(num_temb)
    ids_s[:, n_x - n_pure:n_x, 1] = torch.arange(num_temb + 1, num_temb + 1 + n_pure)
    ids_s[:, n_x:, 0] = 1
    ids_s[:, n_x:, 1] = torch.arange(n_p)
    pe_s = rope_pe(tables, ids_s)
    kb_s = key_bias_3(encoder_attention_mask, n_vl, n_x - n_vl, physics_attention_mask, n_p, vl_embs.dtype)
    for i in range(ss_blocks):
        x, ph = expanded_ss_block(sd, f"single_blocks.{i}.", x, ph, pe_s, heads, kb_s)
    action = _adaln_out(x[:, -n_pure:], temb, sd, "proj_out_1", "proj_out_2")
    physics = _adaln_out(ph, temb, sd, "proj_out_physics_1", "proj_out_physics_2")
    return action, physics


# ---------------------------------------------------------------------------
# The action head around the MSAT, CustomActionHeadChain.forward
# (rldx/inference/action_model/engine/custom_action_model_chain.py:81-171), batch
# 1, no physics: vlln, state encoder, the RTC trained-mode prefix, and per
# denoising step action encoder + position embedding, MSAT, action decoder and
# the Euler update.  Per-embodiment MLPs as CategorySpecificLinear
# (rldx/model/modules/action_model/embodiment_conditioned_mlp.py): x W[e] + b[e].
# ---------------------------------------------------------------------------
def sinusoidal_time(t: float, rows: int, width: int, dtype) -> torch.Tensor:
    """SinusoidalPositionalEncoding of a per-token time (embodiment_conditioned_mlp.py:14-33),
    fp32, for `rows` tokens at time t, cast to the model dtype."""
    half = width // 2
    ex = torch.exp(-torch.arange(half, dtype=torch.float) * (torch.log(torch.tensor(10000.0)) / half))
    fr = torch.full((rows, 1), float(t)) * ex
    return torch.cat([torch.sin(fr), torch.cos(fr)], dim=-1).to(dtype)


def action_head(head_sd: dict, msat_sd: dict, vl, state, x0, *, steps: int, heads: int, head_dim: int,
                ds_blocks: int, ss_blocks: int, e: int = 0, prefix=None, use_vlln: bool = False,
                vlln_eps: float = 1e-5, dtype=torch.float32):
    """Actions [horizon, action_dim] of one inference, evaluated in `dtype` (fp32, or bf16
    eager with a rounding after every op).  vl [1, n_vl, vl_dim], state [1, 1, state_dim],
    x0 [1, horizon, action_dim]; prefix [1, d, action_dim] or None (RTC trained mode:
    rows < d are the prefix for the whole call, encoded once at time 1 (:98-121); each
    step encodes rows >= d at the step's time, decodes only the last horizon - d
    outputs and advances only those rows (:131-170)); use_vlln: affine LayerNorm of
    the VL embeddings (head_sd vlln.weight / vlln.bias) first (:84)."""
    f = {k: v.cpu().to(dtype) for k, v in head_sd.items()}
    sd = {k: v.cpu().to(dtype) for k, v in msat_sd.items()}

    def lin(x, name):
        return torch.addmm(f[f"{name}.b"][e], x, f[f"{name}.W"][e])

    def encode(x, tau):  # MultiEmbodimentActionEncoder: W3(swish(W2([W1 x | tau])))
        h = lin(torch.cat([lin(x, "action_encoder.W1"), tau], dim=-1), "action_encoder.W2")
        return lin(h * torch.sigmoid(h), "action_encoder.W3")

    vl = vl.cpu().to(dtype)
    if use_vlln:
        vl = F.layer_norm(vl, (vl.shape[-1],), f["vlln.weight"], f["vlln.bias"], vlln_eps)
    horizon, width = x0.shape[1], f["position_embedding.weight"].shape[1]
    pos = f["position_embedding.weight"]
    d = 0 if prefix is None else prefix.shape[1]
    state_feat = lin(torch.relu(lin(state.cpu().to(dtype)[0], "state_encoder.layer1")), "state_encoder.layer2")
    act = x0.cpu().to(dtype)[0].clone()
    if d > 0:
        act[:d] = prefix.cpu().to(dtype)[0]
        prefix_feat = encode(act[:d], sinusoidal_time(1.0, d, width, dtype)) + pos[:d]
    for i in range(steps):
        # the schedule i / steps is a bf16 buffer (graph_safe_action_model.py:147-153)
        t = float(torch.tensor(i / float(steps), dtype=torch.bfloat16))
        tau = sinusoidal_time(t, horizon, width, dtype)
        post = encode(act[d:], tau[d:]) + pos[d:]
        feat = torch.cat([prefix_feat, post]) if d > 0 else post
        sa = torch.cat([state_feat, feat])[None]
        out = msat_forward(sd, sa, vl, f["static_tembs"][i], f["static_time_tokens"][i], heads=heads,
                           head_dim=head_dim, ds_blocks=ds_blocks, ss_blocks=ss_blocks)[0]
        if d > 0:
            v = lin(torch.relu(lin(out[-(horizon - d):], "action_decoder.layer1")), "action_decoder.layer2")
        else:
            v = lin(torch.relu(lin(out, "action_decoder.layer1")), "action_decoder.layer2")[-horizon:]
        act[d:] = act[d:] + v * (1.0 / steps)
    return act
