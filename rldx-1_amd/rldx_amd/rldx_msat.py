"""The RLDX-1 MSAT (no add-ons) on the rldx_amd kernels, built from the
reference's own weights.

`RldxMsat` is the counterpart of the reference's CustomOpMSAT
(rldx/inference/action_model/engine/custom_msat_chain.py:56-126): the same
forward(hidden_states, encoder_hidden_states, temb, time_token) with the time
embedding and time token baked by the caller, 4 DoubleStreamBlocks over
[VL | time | SA] and 8 SingleStreamBlocks over [VL->SA | time | SA]
(rldx/model/modules/action_model/blocks.py:166-254, :383-609; msat.py:291-556),
then the AdaLN output projection (msat.py:777-781).  It is built from a state
dict under the reference module's names (`double_blocks.0.sa_qkv.weight`, ...),
read from local safetensors files by `load_msat_state_dict` (no hub access), or
taken from a live module by `install`.

RoPE: the rope_sa_only tables of RoPEEmbedder1D.  A model loaded in bfloat16
has its complex frequency buffers cast to bf16, which keeps cos and drops sin;
`bf16_quirk=True` (the default, as the reference chain assumes) reproduces that
(cos rounded to bf16, sin = 0), False uses the exact fp32 tables.

Per DoubleStreamBlock (8 launches; the SA and VL streams have different
widths, so each linear is one launch of groups with their own n and k):
    LayerNorm -> packed h_s, both      rldx_layernorm_pack_many_bf16
    QKV linears (+ bias)               rldx_grouped_gemm_mixed_bf16
    QK-RMSNorm + RoPE (SA rows) + K/V  rldx_msat_qkv_norm_rope_bf16
    joint attention -> packed o        rldx_attention_packed_fwd_bf16
    proj + residual (in place)         rldx_grouped_gemm_mixed_bf16 (residual)
    LayerNorm -> packed h_s, both      rldx_layernorm_pack_many_bf16
    w12 + SwiGLU -> packed             rldx_grouped_gemm_mixed_bf16 (swiglu)
    w3 + residual (in place)           rldx_grouped_gemm_mixed_bf16 (residual)
Per SingleStreamBlock (7 launches):
    LayerNorm -> packed h; linear1's QKV columns (+ bias); linear1's MLP columns
    + SwiGLU -> packed; QK-RMSNorm + RoPE; attention -> columns [0, inner) of
    the packed linear2 operand; mlp_proj (+ bias) -> its columns [inner, ...);
    linear2 + residual (in place).
VL rows are padded to a multiple of 32 (whole 32-row blocks of the packed
activations, so the SA rows of a packed matrix start at a block boundary); the
padding rows start at zero every forward and their keys carry a -inf key bias,
so they never reach a real row.  The same key-bias vector carries the
`encoder_attention_mask` of the eager MSAT (1 = visible VL token, 0 = masked;
msat.py:517-531, blocks.py:558-575) when the chain is built with vl_mask=True.
The GEMMs have 18, 64 or 82 rows, so their launches have only 24-144 output
tiles: each is split over K (split_for) towards 256 workgroups, partials summed
in a fixed order in one shared workspace.
The SwiGLU widths of the double-stream FFNs (SA 4096, VL 10922) are padded
with zero weight rows / columns to a multiple of 128 (silu(0) * 0 = 0, so the
padding contributes nothing).  The output projection's tiny modulation
(F.silu(temb) -> proj_out_1, LayerNorm * (1 + scale) + shift) runs as torch ops.
"""

from __future__ import annotations

import math
import os
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F

from . import functional as Fn
from .workloads import msat_freqs_cis

BF16 = torch.bfloat16


@dataclass
class RldxMsatCfg:
    """MSAT dimensions (rldx/configs/model/rldx.py:94-112; Appendix values of the
    RLDX-1 release: 24 x 64 heads, 4 + 8 blocks, SA 1536, VL 4096)."""

    heads: int = 24
    head_dim: int = 64
    ds_blocks: int = 4
    ss_blocks: int = 8
    sa_dim: int = 1536
    vl_dim: int = 4096
    mlp_ratio: float = 4.0
    vl_mlp_ratio: Optional[float] = None
    output_dim: int = 1024
    n_vl: int = 64          # cognition tokens
    n_sa_pure: int = 17     # state token + action horizon 16
    num_temb_tokens: int = 1
    rope_theta: float = 10000.0
    max_seq_len: int = 1024
    eps: float = 1e-6
    use_physics: bool = False  # Expanded blocks with a P stream (msat.py:928-989)
    n_physics: int = 0         # P tokens per call (physics history + future); 0 = no P stream

    @property
    def inner(self) -> int:
        return self.heads * self.head_dim

    @property
    def sa_ffn(self) -> int:  # blocks.py:317-319
        return int(2 / 3 * int(self.sa_dim * self.mlp_ratio))

    @property
    def vl_ffn(self) -> int:  # blocks.py:349-351
        r = self.vl_mlp_ratio if self.vl_mlp_ratio is not None else self.mlp_ratio
        return int(2 / 3 * int(self.vl_dim * r))

    @property
    def ss_expanded(self) -> int:  # blocks.py:100-114
        return int(self.sa_dim * self.mlp_ratio)

    @property
    def ss_hidden(self) -> int:
        return int(2 / 3 * self.ss_expanded)

    @property
    def n_sa(self) -> int:
        return self.n_sa_pure + self.num_temb_tokens

    @property
    def tokens(self) -> int:
        return self.n_vl + self.n_sa

    def param_shapes(self) -> dict:
        """Parameter names and shapes of the reference MSAT (no add-ons,
        temb_type input_token, qk_norm rms_norm, SwiGLU) that the chain reads."""
        d, v, i = self.sa_dim, self.vl_dim, self.inner
        s = {}
        for b in range(self.ds_blocks):
            p = f"double_blocks.{b}."
            s.update({p + "sa_qkv.weight": (3 * i, d), p + "sa_qkv.bias": (3 * i,),
                      p + "vl_qkv.weight": (3 * i, v), p + "vl_qkv.bias": (3 * i,),
                      p + "sa_proj.weight": (d, i), p + "sa_proj.bias": (d,),
                      p + "vl_proj.weight": (v, i), p + "vl_proj.bias": (v,),
                      p + "sa_mlp.w12.weight": (2 * self.sa_ffn, d), p + "sa_mlp.w12.bias": (2 * self.sa_ffn,),
                      p + "sa_mlp.w3.weight": (d, self.sa_ffn), p + "sa_mlp.w3.bias": (d,),
                      p + "vl_mlp.w12.weight": (2 * self.vl_ffn, v), p + "vl_mlp.w12.bias": (2 * self.vl_ffn,),
                      p + "vl_mlp.w3.weight": (v, self.vl_ffn), p + "vl_mlp.w3.bias": (v,)})
            for n in ("q_norm_sa", "k_norm_sa", "q_norm_vl", "k_norm_vl"):
                s[p + n + ".weight"] = (self.head_dim,)
        e, hs = self.ss_expanded, self.ss_hidden
        for b in range(self.ss_blocks):
            p = f"single_blocks.{b}."
            s.update({p + "linear1.weight": (3 * i + 2 * e, d), p + "linear1.bias": (3 * i + 2 * e,),
                      p + "mlp_proj.weight": (hs, e), p + "mlp_proj.bias": (hs,),
                      p + "linear2.weight": (d, i + hs), p + "linear2.bias": (d,),
                      p + "q_norm.weight": (self.head_dim,), p + "k_norm.weight": (self.head_dim,)})
        s.update({"vl_proj_to_sa.weight": (d, v), "vl_proj_to_sa.bias": (d,),
                  "proj_out_1.weight": (2 * d, i), "proj_out_1.bias": (2 * d,),
                  "proj_out_2.weight": (self.output_dim, d), "proj_out_2.bias": (self.output_dim,)})
        if self.use_physics:
            s.update(self.physics_param_shapes())
        return s

    def physics_param_shapes(self) -> dict:
        """The P-stream parameters of the all-add-ons MSAT (p_dim = sa_dim,
        msat.py:938-989): ExpandedDoubleStreamBlock p_* (blocks.py:665-697, the P
        SwiGLU width that of SA), ExpandedSingleStreamBlock p_* (blocks.py:942-964)
        and the physics output projection."""
        d, i, hd = self.sa_dim, self.inner, self.head_dim
        s = {}
        for b in range(self.ds_blocks):
            p = f"double_blocks.{b}."
            s.update({p + "p_qkv.weight": (3 * i, d), p + "p_qkv.bias": (3 * i,),
                      p + "p_proj.weight": (d, i), p + "p_proj.bias": (d,),
                      p + "p_mlp.w12.weight": (2 * self.sa_ffn, d), p + "p_mlp.w12.bias": (2 * self.sa_ffn,),
                      p + "p_mlp.w3.weight": (d, self.sa_ffn), p + "p_mlp.w3.bias": (d,),
                      p + "q_norm_p.weight": (hd,), p + "k_norm_p.weight": (hd,)})
        e, hs = self.ss_expanded, self.ss_hidden
        for b in range(self.ss_blocks):
            p = f"single_blocks.{b}."
            s.update({p + "p_linear1.weight": (3 * i + 2 * e, d), p + "p_linear1.bias": (3 * i + 2 * e,),
                      p + "p_mlp_proj.weight": (hs, e), p + "p_mlp_proj.bias": (hs,),
                      p + "p_linear2.weight": (d, i + hs), p + "p_linear2.bias": (d,),
                      p + "p_q_norm.weight": (hd,), p + "p_k_norm.weight": (hd,)})
        s.update({"proj_out_physics_1.weight": (2 * d, i), "proj_out_physics_1.bias": (2 * d,),
                  "proj_out_physics_2.weight": (self.output_dim, d), "proj_out_physics_2.bias": (self.output_dim,)})
        return s

    @staticmethod
    def from_state_dict(sd: dict, **overrides) -> "RldxMsatCfg":
        """Dimensions read off the parameter shapes (token counts from overrides)."""
        ds = sum(1 for k in sd if k.startswith("double_blocks.") and k.endswith(".sa_qkv.weight"))
        ss = sum(1 for k in sd if k.startswith("single_blocks.") and k.endswith(".linear1.weight"))
        hd = sd["double_blocks.0.q_norm_sa.weight"].shape[0]
        inner = sd["double_blocks.0.sa_qkv.weight"].shape[0] // 3
        sa_dim, vl_dim = sd["double_blocks.0.sa_qkv.weight"].shape[1], sd["double_blocks.0.vl_qkv.weight"].shape[1]
        kw = dict(heads=inner // hd, head_dim=hd, ds_blocks=ds, ss_blocks=ss, sa_dim=sa_dim, vl_dim=vl_dim,
                  output_dim=sd["proj_out_2.weight"].shape[0], use_physics="proj_out_physics_2.weight" in sd,
                  mlp_ratio=sd["double_blocks.0.sa_mlp.w12.weight"].shape[0] * 3 / 4 / sa_dim)
        kw.update(overrides)
        cfg = RldxMsatCfg(**kw)
        if int(cfg.sa_dim * cfg.mlp_ratio) != sd["double_blocks.0.sa_mlp.w12.weight"].shape[0] * 3 // 4:
            cfg.mlp_ratio = 4.0  # the ratio is only recoverable up to the int() of blocks.py; the release uses 4
        vl_w12 = sd["double_blocks.0.vl_mlp.w12.weight"].shape[0] // 2
        if cfg.vl_ffn != vl_w12:
            cfg.vl_mlp_ratio = math.ceil(vl_w12 * 3 / 2) / vl_dim
        return cfg


def make_state_dict(cfg: RldxMsatCfg, device, seed: int = 11, std: float = 0.02) -> dict:
    """Random-init parameters under the reference names: weights and biases
    ~ N(0, std), norm weights 1 + N(0, 0.02); bf16 on `device`."""
    g = torch.Generator(device=device).manual_seed(seed)
    sd = {}
    for k, shape in cfg.param_shapes().items():
        r = torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
        sd[k] = (1.0 + 0.02 * r if "norm" in k else std * r).to(BF16)
    return sd


def make_inputs(cfg: RldxMsatCfg, device, seed: int = 12) -> dict:
    """SA embeddings (state + action tokens), VL (cognition) tokens, a time
    embedding and its time token, and with n_physics > 0 the physics tokens
    `p` [1, n_physics, sa_dim]; bf16, batch 1."""
    g = torch.Generator(device=device).manual_seed(seed)

    def rnd(*shape, std=1.0):
        return (std * torch.randn(*shape, generator=g, device=device, dtype=torch.float32)).to(BF16)

    inp = dict(sa=rnd(1, cfg.n_sa_pure, cfg.sa_dim), vl=rnd(1, cfg.n_vl, cfg.vl_dim),
               temb=rnd(1, cfg.inner, std=0.5), time_token=rnd(1, cfg.num_temb_tokens, cfg.sa_dim, std=0.5))
    if cfg.n_physics > 0:
        inp["p"] = rnd(1, cfg.n_physics, cfg.sa_dim)
    return inp


def load_msat_state_dict(path: str, prefix: str = "action_model.model.", device="cpu") -> dict:
    """MSAT parameters from local safetensors file(s) (a file, or every
    *.safetensors file of a directory) of an RLDX checkpoint: keys under
    `prefix` (the MSAT of RLDX.action_model, rldx/model/core/rldx.py:75, :892),
    prefix stripped, cast to bf16.  Reads tensors only (no code is executed)."""
    from safetensors.torch import load_file

    files = [path] if os.path.isfile(path) else sorted(
        os.path.join(path, f) for f in os.listdir(path) if f.endswith(".safetensors"))
    Fn._require(len(files) > 0, f"no .safetensors file at {path}")
    sd = {}
    for f in files:
        for k, v in load_file(f, device=str(device)).items():
            if k.startswith(prefix):
                sd[k[len(prefix):]] = v.to(BF16)
    Fn._require(len(sd) > 0, f"no parameter under prefix '{prefix}' in {path}")
    return sd


def rope_tables(cfg: RldxMsatCfg, positions: torch.Tensor, bf16_quirk: bool, axis0: int = 0):
    """fp32 cos / sin [N, D/2] of the rope_sa_only embedder (axes [D/4, 3D/4])
    at axis-0 position `axis0` (0 for SA rows, 1 for physics rows) and the
    given axis-1 positions (RoPEEmbedder1D, ops.py:70-119); with bf16_quirk,
    cos rounded to bf16 and sin = 0 (custom_msat_chain.py:15-54)."""
    parts = []
    for i, ad in enumerate((cfg.head_dim // 4, cfg.head_dim - cfg.head_dim // 4)):
        fc = msat_freqs_cis(ad, cfg.max_seq_len, cfg.rope_theta)
        idx = torch.full_like(positions, axis0) if i == 0 else positions
        parts.append(fc[idx])
    pe = torch.cat(parts, dim=-1)
    if bf16_quirk:
        return pe.real.to(BF16).float().contiguous(), torch.zeros(pe.shape, dtype=torch.float32)
    return pe.real.float().contiguous(), pe.imag.float().contiguous()


def _pad_rows(w: torch.Tensor, rows: int) -> torch.Tensor:
    return w if w.shape[0] == rows else torch.cat([w, w.new_zeros(rows - w.shape[0], *w.shape[1:])])


def _pad_cols(w: torch.Tensor, cols: int) -> torch.Tensor:
    return w if w.shape[1] == cols else torch.cat([w, w.new_zeros(w.shape[0], cols - w.shape[1])], dim=1)


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


class RldxMsat:
    """Static-buffer executor of the RLDX-1 MSAT forward; `forward` launches it
    eagerly (capturable in a hipGraph), `capture` / `replay` record and replay it.

    With cfg.use_physics and cfg.n_physics > 0 it is the all-add-ons MSAT
    (CustomOpExpandedMSAT, rldx/inference/action_model/engine/
    custom_expanded_msat_chain.py:19-115; eager MSAT._forward_physics,
    msat.py:558-775): 4 ExpandedDoubleStreamBlocks over [VL | SA | P] and 8
    ExpandedSingleStreamBlocks over [VL+SA | P].  The P stream has the SA
    stream's widths, so every SA GEMM and its P counterpart run as one grouped
    launch (two groups sharing n and k), as do the x and P GEMMs of the single
    blocks and the two output projections; the joint attention is one launch
    over [VL | SA | P].  The SA rows of the joint sequence are padded to a
    multiple of 32 so that the P rows of the packed attention output start on
    a 32-row block (the A operand of the P GEMMs): padding rows of Q/K/V are
    zero and their keys carry -inf."""

    # packed weights and RoPE tables: shared by the chains of one model for every batch size
    _WEIGHTS = ("w", "sa_ffn_p", "vl_ffn_p", "ds", "ss", "vl_proj_to_sa", "proj_out_2", "proj_out_physics_2",
                "ds_cos", "ds_sin", "ss_cos", "ss_sin", "p_cos", "p_sin")

    def __init__(self, sd: Optional[dict], cfg: RldxMsatCfg, device, bf16_quirk: bool = True, vl_mask: bool = False,
                 batch: int = 1, weights_of: Optional["RldxMsat"] = None):
        self.cfg, self.dev = cfg, torch.device(device)
        H, D, inner = cfg.heads, cfg.head_dim, cfg.inner
        Fn._require(D in (64, 128), "head_dim must be 64 or 128")
        Fn._require(cfg.n_vl >= 1 and cfg.n_sa_pure >= 1, "the chain needs VL and SA tokens")
        self.phys = cfg.use_physics and cfg.n_physics > 0
        Fn._require(cfg.n_physics == 0 or cfg.use_physics, "physics tokens need the P-stream parameters")
        # joint sequence: [VL padded to 32 | SA (padded to 32 with a P stream) | P]
        self.nv = _round_up(cfg.n_vl, 32)
        self.ns = _round_up(cfg.n_sa, 32) if self.phys else cfg.n_sa
        self.np_ = cfg.n_physics if self.phys else 0
        self.p0 = self.nv + self.ns                  # first P row
        self.N = self.p0 + self.np_
        self.nx = self.nv + cfg.n_sa                 # rows of the single-stream x = [VL->SA | time | SA]
        self.vl_mask = vl_mask
        self.masked = vl_mask or self.nv != cfg.n_vl or self.phys
        self.bf16_quirk = bf16_quirk
        Fn._require(int(batch) >= 1, "batch must be >= 1")
        self.batch = int(batch)
        if weights_of is None:
            Fn._require(sd is not None, "a state dict, or weights_of (a chain whose packed weights to share)")
            self._pack_weights(sd)
        else:
            Fn._require(weights_of.cfg == cfg and weights_of.dev == self.dev and weights_of.bf16_quirk == bf16_quirk,
                        "weights_of must be a chain of the same configuration, device and RoPE tables")
            for name in self._WEIGHTS:
                setattr(self, name, getattr(weights_of, name, None))
        self._alloc()

    def for_batch(self, batch: int) -> "RldxMsat":
        """A chain of this model for `batch` robots on the same packed weights
        (nothing of them is copied): its own activation buffers, masks and plans."""
        return RldxMsat(None, self.cfg, self.dev, self.bf16_quirk, self.vl_mask, batch=batch, weights_of=self)

    def _pack_weights(self, sd: dict) -> None:
        cfg, bf16_quirk = self.cfg, self.bf16_quirk
        H, D, inner = cfg.heads, cfg.head_dim, cfg.inner
        for k, shape in cfg.param_shapes().items():
            Fn._require(k in sd, f"missing parameter {k}")
            Fn._require(tuple(sd[k].shape) == tuple(shape), f"{k}: shape {tuple(sd[k].shape)}, expected {shape}")
        names = cfg.param_shapes() if self.phys else {k: v for k, v in cfg.param_shapes().items()
                                                      if k not in cfg.physics_param_shapes()}
        w = {k: sd[k].to(device=self.dev, dtype=BF16).contiguous() for k in names}
        self.w = w
        self.sa_ffn_p, self.vl_ffn_p = _round_up(cfg.sa_ffn, 128), _round_up(cfg.vl_ffn, 128)
        for dim in (cfg.sa_dim, cfg.vl_dim, inner, cfg.ss_expanded, cfg.ss_hidden + inner, cfg.output_dim):
            Fn._require(dim % 64 == 0, f"width {dim} is not a multiple of 64")
        for dim in (cfg.sa_dim, cfg.vl_dim, inner, cfg.ss_expanded, inner + cfg.ss_hidden):
            Fn._require(dim % 128 == 0, f"GEMM depth {dim} is not a multiple of 128")

        def swiglu_w(w12, b12, ffn, ffn_p):
            g, u = w12[:ffn], w12[ffn:]
            gb, ub = b12[:ffn], b12[ffn:]
            wp = torch.cat([_pad_rows(g, ffn_p), _pad_rows(u, ffn_p)])
            bp = torch.cat([_pad_rows(gb[:, None], ffn_p)[:, 0], _pad_rows(ub[:, None], ffn_p)[:, 0]])
            return Fn.pack_weight(wp, swiglu_pairs=True), bp.contiguous()

        streams = ("sa", "vl", "p") if self.phys else ("sa", "vl")
        self.ds = []
        for b in range(cfg.ds_blocks):
            p = f"double_blocks.{b}."
            blk = {}
            for st in streams:
                ffn, ffn_p = (cfg.vl_ffn, self.vl_ffn_p) if st == "vl" else (cfg.sa_ffn, self.sa_ffn_p)
                for n in ("q_norm", "k_norm"):
                    blk[f"{n}_{st}.weight"] = w[f"{p}{n}_{st}.weight"]
                for n in ("qkv", "proj"):
                    blk[f"{st}_{n}"] = Fn.pack_weight(w[f"{p}{st}_{n}.weight"])
                    blk[f"{st}_{n}.bias"] = w[f"{p}{st}_{n}.bias"]
                blk[f"{st}_w12"], blk[f"{st}_w12.bias"] = swiglu_w(w[f"{p}{st}_mlp.w12.weight"],
                                                                  w[f"{p}{st}_mlp.w12.bias"], ffn, ffn_p)
                blk[f"{st}_w3"] = Fn.pack_weight(_pad_cols(w[f"{p}{st}_mlp.w3.weight"], ffn_p))
                blk[f"{st}_mlp.w3.bias"] = w[f"{p}{st}_mlp.w3.bias"]
            self.ds.append(blk)
        self.ss = []
        for b in range(cfg.ss_blocks):
            p = f"single_blocks.{b}."
            blk = {}
            for pre in (("", "p_") if self.phys else ("",)):
                w1, b1 = w[f"{p}{pre}linear1.weight"], w[f"{p}{pre}linear1.bias"]
                blk.update({f"{pre}q_norm": w[f"{p}{pre}q_norm.weight"], f"{pre}k_norm": w[f"{p}{pre}k_norm.weight"],
                            f"{pre}qkv": Fn.pack_weight(w1[: 3 * inner].contiguous()),
                            f"{pre}qkv.bias": b1[: 3 * inner].contiguous(),
                            f"{pre}mlp": Fn.pack_weight(w1[3 * inner:].contiguous(), swiglu_pairs=True),
                            f"{pre}mlp.bias": b1[3 * inner:].contiguous(),
                            f"{pre}mlp_proj": Fn.pack_weight(w[f"{p}{pre}mlp_proj.weight"]),
                            f"{pre}mlp_proj.bias": w[f"{p}{pre}mlp_proj.bias"],
                            f"{pre}linear2": Fn.pack_weight(w[f"{p}{pre}linear2.weight"]),
                            f"{pre}linear2.bias": w[f"{p}{pre}linear2.bias"]})
            self.ss.append(blk)
        self.vl_proj_to_sa = Fn.pack_weight(w["vl_proj_to_sa.weight"])
        self.proj_out_2 = Fn.pack_weight(w["proj_out_2.weight"])
        # RoPE: DS rows [time | SA] at axis-1 positions 0 .. n_sa - 1; SS rows [time | SA]
        # at 0 and num_temb + 1 ... (custom_msat_chain.py:81-105, the eager ids of msat.py:376-487);
        # P rows at axis 0 = 1, axis 1 = 0 .. n_p - 1 in both (custom_expanded_msat_chain.py:44-85,
        # msat.py:630-632, :706-710).  Tables of padding rows: cos 1, sin 0 (their Q/K are zero).
        nt = cfg.num_temb_tokens
        ds_pos = torch.arange(cfg.n_sa)
        ss_pos = torch.cat([torch.arange(nt), torch.arange(nt + 1, nt + 1 + cfg.n_sa_pure)])

        def tables(pos, axis0=0, rows=None):
            c, sn = rope_tables(cfg, pos, bf16_quirk, axis0)
            if rows is not None and rows > c.shape[0]:
                c = torch.cat([c, torch.ones(rows - c.shape[0], c.shape[1])])
                sn = torch.cat([sn, torch.zeros(rows - sn.shape[0], sn.shape[1])])
            return c.contiguous().to(self.dev), sn.contiguous().to(self.dev)

        self.ds_cos, self.ds_sin = tables(ds_pos, rows=self.ns)
        self.ss_cos, self.ss_sin = tables(ss_pos, rows=self.ns)
        if self.phys:
            self.p_cos, self.p_sin = tables(torch.arange(self.np_), axis0=1)
        self.proj_out_physics_2 = Fn.pack_weight(w["proj_out_physics_2.weight"]) if self.phys else None

    def _alloc(self) -> None:
        """Activation buffers, masks and GEMM plans for self.batch robots.  Rows
        of a batch: each stream's rows of every robot, robot after robot
        (robot b's row r of a stream at b * rows + r), so that one GEMM covers a
        stream for the whole batch; the joint attention writes its output back
        into that order by row segments."""
        cfg = self.cfg
        H, D, inner = cfg.heads, cfg.head_dim, cfg.inner
        B, nt = self.batch, cfg.num_temb_tokens
        N, nv, ns, nx, npp = self.N, self.nv, cfg.n_sa, self.nx, self.np_
        ebuf = lambda *s: torch.empty(*s, dtype=BF16, device=self.dev)  # noqa: E731
        # x = [VL->SA | time | SA] of the single-stream blocks (B nv rows, then B n_sa); its SA rows are the SA
        # residual stream of the double-stream blocks (no copy between the two)
        self.x = ebuf(B * nx, cfg.sa_dim)
        self.x_sa, self.x_vl = self.x[B * nv:], ebuf(B * nv, cfg.vl_dim)
        self.h_sa = Fn.PackedAct.empty(B * ns, cfg.sa_dim, self.dev)
        self.h_vl = Fn.PackedAct.empty(B * nv, cfg.vl_dim, self.dev)
        # QKV rows of SA: the GEMM writes B n_sa rows; robot b's joint sequence reads self.ns rows from b n_sa,
        # so with a P stream its padding rows are the next robot's first rows (their keys are masked and their
        # outputs not stored) or, for the last robot, the zero rows at the end
        self.qkv_sa_buf = torch.zeros(B * ns + self.ns - ns, 3 * inner, dtype=BF16, device=self.dev)
        self.qkv_sa, self.qkv_vl = self.qkv_sa_buf[:B * ns], ebuf(B * nv, 3 * inner)
        self.q = ebuf(B, H, N, D)
        self.kvp = ebuf(B, H, Fn.kv_packed_elems(N, D))
        # attention output (and the single blocks' [attention | MLP] operand): B nv VL rows, B n_sa SA rows,
        # then from the next 32-row block (pa) B np P rows
        self.pa = _round_up(B * (nv + ns), 32)
        self.segments = [(0, nv, 0), (nv, ns, B * nv)] + ([(self.p0, npp, self.pa)] if self.phys else [])
        self.att = Fn.PackedAct.empty(self.pa + B * npp, inner, self.dev)
        self.gl_sa = Fn.PackedAct.empty(B * ns, self.sa_ffn_p, self.dev)
        self.gl_vl = Fn.PackedAct.empty(B * nv, self.vl_ffn_p, self.dev)
        self.vl_packed = Fn.PackedAct.empty(B * nv, cfg.vl_dim, self.dev)
        self.h = Fn.PackedAct.empty(B * nx, cfg.sa_dim, self.dev)
        self.qkv_buf = torch.zeros(B * nx + self.ns - ns, 3 * inner, dtype=BF16, device=self.dev)
        self.qkv = self.qkv_buf[:B * nx]
        self.gl = Fn.PackedAct.empty(B * nx, cfg.ss_expanded, self.dev)
        self.cat = Fn.PackedAct.empty(self.pa + B * npp, inner + cfg.ss_hidden, self.dev)
        self.mod = ebuf(B * cfg.n_sa_pure, cfg.sa_dim)
        self.mod_packed = Fn.PackedAct.empty(B * cfg.n_sa_pure, cfg.sa_dim, self.dev)
        self.out = ebuf(B, cfg.n_sa_pure, cfg.output_dim)
        self.inputs = dict(sa=ebuf(B, cfg.n_sa_pure, cfg.sa_dim), vl=ebuf(B, cfg.n_vl, cfg.vl_dim),
                           temb=ebuf(B, inner), time_token=ebuf(B, nt, cfg.sa_dim))
        if self.phys:
            self.x_p = ebuf(B * npp, cfg.sa_dim)
            self.h_p = Fn.PackedAct.empty(B * npp, cfg.sa_dim, self.dev)
            self.qkv_p = ebuf(B * npp, 3 * inner)
            self.gl_p = Fn.PackedAct.empty(B * npp, self.sa_ffn_p, self.dev)
            self.gl_p_ss = Fn.PackedAct.empty(B * npp, cfg.ss_expanded, self.dev)
            self.mod_p = ebuf(B * npp, cfg.sa_dim)
            self.mod_p_packed = Fn.PackedAct.empty(B * npp, cfg.sa_dim, self.dev)
            self.out_p = ebuf(B, npp, cfg.output_dim)
            self.inputs["p"] = ebuf(B, npp, cfg.sa_dim)
        if self.vl_mask:
            self.inputs["vl_mask"] = torch.ones(B, cfg.n_vl, dtype=torch.float32, device=self.dev)
            if self.phys:
                self.inputs["physics_mask"] = torch.ones(B, dtype=torch.float32, device=self.dev)
        # additive key bias of each robot's N attention rows: 0, or -inf on padding, masked VL and masked P keys
        self.key_bias = torch.zeros(B, N, dtype=torch.float32, device=self.dev)
        self.key_bias[:, cfg.n_vl:nv] = float("-inf")
        self.key_bias[:, nv + ns:self.p0] = float("-inf")
        self._ninf = torch.full((), float("-inf"), dtype=torch.float32, device=self.dev)
        self._zero = torch.zeros((), dtype=torch.float32, device=self.dev)
        self.graph = None
        # the pre-norms of a block's streams, one launch each time
        self.ds_norms = [(self.x_sa, self.h_sa), (self.x_vl, self.h_vl)] + ([(self.x_p, self.h_p)] if self.phys else [])
        self.ss_norms = [(self.x, self.h)] + ([(self.x_p, self.h_p)] if self.phys else [])
        # every GEMM of the forward on its static buffers, with its split-K factor
        self.ds_gemms = [self._ds_gemm_items(blk) for blk in self.ds]
        self.ss_gemms = [self._ss_gemm_items(blk) for blk in self.ss]
        self.vl_proj_gemm = self._planned(
            [(self.vl_packed, self.vl_proj_to_sa, self.w["vl_proj_to_sa.bias"], self.x[:B * nv], None)], "bias")
        out_items = [(self.mod_packed, self.proj_out_2, self.w["proj_out_2.bias"],
                      self.out.view(B * cfg.n_sa_pure, cfg.output_dim), None)]
        if self.phys:
            out_items.append((self.mod_p_packed, self.proj_out_physics_2, self.w["proj_out_physics_2.bias"],
                              self.out_p.view(B * npp, cfg.output_dim), None))
        self.out_gemm = self._planned(out_items, "bias")
        plans = [g for d in self.ds_gemms + self.ss_gemms for g in d.values()] + [self.vl_proj_gemm, self.out_gemm]
        self.ws = Fn.GemmWorkspace(max(Fn.grouped_gemm_workspace_bytes(it, epi, sk, wide) for it, epi, sk, wide in plans),
                                   self.dev)

    @staticmethod
    def split_for(m, n: int, k: int) -> int:
        """Split-K factor for a launch (m: the rows of each group, or one int):
        the 82-, 64- and 18-row GEMMs of this model have 24-344 output tiles;
        where K is long (>= 4096) a tile streams a long slice of K on one CU,
        and splitting K by the largest power of two <= min(8, K / 1024) that
        keeps tiles x split <= 256 (one workgroup per CU) pays; with shorter K
        the partial-sum traffic costs more than the added workgroups gain.
        Measured per GEMM at the release shape (us per launch, weights
        streaming from HBM, split 1 / chosen): vl_qkv 15.3 / 12.7, sa_w3 11.7 /
        9.1, vl_w3 52.1 / 23.9, mlp_proj 26.3 / 19.3, linear2 17.1 / 11.1; the
        short-K GEMMs were fastest unsplit.  Tiles as the planner cuts them:
        32 x 64 for up to 32 rows, else 64 x 64, summed over the groups."""
        if k < 4096:
            return 1
        ms = [m] if isinstance(m, int) else list(m)
        tiles = sum(((r + 31) // 32 if r <= 32 else (r + 63) // 64) for r in ms) * (n // 64)
        split = 1
        while split < 8 and split * 2 <= k // 1024 and tiles * split * 2 <= 256:
            split *= 2
        return split

    @staticmethod
    def wide_for(n: int, epi: str, split: int) -> bool:
        """64 x 128 / 32 x 128 tiles (RLDX_GEMM_WIDE_TILES, the same results bit
        for bit) for the wide unsplit SwiGLU GEMMs: measured per GEMM at the
        release shape, DS vl_w12 (64 x 22016 x 4096) 47.9 -> 42.2 us and SS mlp
        (82 x 12288 x 1536) 17.6 -> 16.2 us; every other GEMM of the model was
        slower with them (vl_w3 23.9 -> 31.1, sa_w12 9.7 -> 11.6)."""
        return epi.startswith("swiglu") and n >= 12288 and split == 1

    def _planned(self, items, epi):
        w = items[0][1]
        split = self.split_for([it[0].m for it in items], w.n, w.k)
        return (items, epi, split, self.wide_for(w.n, epi, split))

    @staticmethod
    def _joined(sa_plan, vl_plan):
        """The SA (+ P) and VL GEMMs of a double-stream block as one launch
        (rldx_grouped_gemm_mixed_bf16: each group its own n, k and split; wide
        tiles if either plan takes them).  Graph replays run launches one after
        the other, so the short SA GEMMs on their own leave most CUs idle; beside
        the VL GEMM they fill them.  Measured per GEMM pair at the release shape
        (us, weights streaming from HBM, two launches / one): qkv 20.4 / 14.9,
        proj 16.1 / 8.9, w12 54.6 / 45.3, w3 37.1 / 30.4; with the P stream
        29.8 / 23.3, 16.4 / 8.9, 73.3 / 62.5, 43.3 / 37.5.  Each group keeps the
        split of its own plan: no other split or tile choice was faster by more
        than 2 %."""
        (sa_items, epi, sa_split, sa_wide), (vl_items, _, vl_split, vl_wide) = sa_plan, vl_plan
        return (sa_items + vl_items, epi, [sa_split] * len(sa_items) + [vl_split] * len(vl_items),
                sa_wide or vl_wide)

    def _ds_gemm_items(self, blk: dict) -> dict:
        g = self._ds_gemm_pairs(blk)
        return {name: self._joined(g["sa_" + name], g["vl_" + name]) for name in ("qkv", "proj", "w12", "w3")}

    def _ds_gemm_pairs(self, blk: dict) -> dict:
        B, nv, ns, pa, npp = self.batch, self.nv, self.cfg.n_sa, self.pa, self.np_
        att_vl, att_sa, att_p = self.att.rows(0, B * nv), self.att.rows(B * nv, B * (nv + ns)), self.att.rows(
            pa, pa + B * npp)

        def grp(sa_item, p_item):
            return [sa_item, p_item] if self.phys else [sa_item]

        P = self.phys
        return {
            "sa_qkv": self._planned(grp((self.h_sa, blk["sa_qkv"], blk["sa_qkv.bias"], self.qkv_sa, None),
                                        P and (self.h_p, blk["p_qkv"], blk["p_qkv.bias"], self.qkv_p, None)), "bias"),
            "vl_qkv": self._planned([(self.h_vl, blk["vl_qkv"], blk["vl_qkv.bias"], self.qkv_vl, None)], "bias"),
            "sa_proj": self._planned(grp((att_sa, blk["sa_proj"], blk["sa_proj.bias"], self.x_sa, self.x_sa),
                                         P and (att_p, blk["p_proj"], blk["p_proj.bias"], self.x_p, self.x_p)),
                                     "residual"),
            "vl_proj": self._planned([(att_vl, blk["vl_proj"], blk["vl_proj.bias"], self.x_vl, self.x_vl)],
                                     "residual"),
            "sa_w12": self._planned(grp((self.h_sa, blk["sa_w12"], blk["sa_w12.bias"], self.gl_sa, None),
                                        P and (self.h_p, blk["p_w12"], blk["p_w12.bias"], self.gl_p, None)),
                                    "swiglu_packed"),
            "vl_w12": self._planned([(self.h_vl, blk["vl_w12"], blk["vl_w12.bias"], self.gl_vl, None)],
                                    "swiglu_packed"),
            "sa_w3": self._planned(grp((self.gl_sa, blk["sa_w3"], blk["sa_mlp.w3.bias"], self.x_sa, self.x_sa),
                                       P and (self.gl_p, blk["p_w3"], blk["p_mlp.w3.bias"], self.x_p, self.x_p)),
                                   "residual"),
            "vl_w3": self._planned([(self.gl_vl, blk["vl_w3"], blk["vl_mlp.w3.bias"], self.x_vl, self.x_vl)],
                                   "residual"),
        }

    def _ss_gemm_items(self, blk: dict) -> dict:
        inner, hs = self.cfg.inner, self.cfg.ss_hidden
        B, nx, pa = self.batch, self.nx, self.pa
        cx, cp = self.cat.rows(0, B * nx), (self.cat.rows(pa, pa + B * self.np_) if self.phys else None)

        def grp(x_item, p_item):
            return [x_item, p_item] if self.phys else [x_item]

        P = self.phys
        return {
            "qkv": self._planned(grp((self.h, blk["qkv"], blk["qkv.bias"], self.qkv, None),
                                     P and (self.h_p, blk["p_qkv"], blk["p_qkv.bias"], self.qkv_p, None)), "bias"),
            "mlp": self._planned(grp((self.h, blk["mlp"], blk["mlp.bias"], self.gl, None),
                                     P and (self.h_p, blk["p_mlp"], blk["p_mlp.bias"], self.gl_p_ss, None)),
                                 "swiglu_packed"),
            "mlp_proj": self._planned(grp((self.gl, blk["mlp_proj"], blk["mlp_proj.bias"], cx.cols(inner, inner + hs),
                                           None),
                                          P and (self.gl_p_ss, blk["p_mlp_proj"], blk["p_mlp_proj.bias"],
                                                 cp.cols(inner, inner + hs), None)), "bias_packed"),
            "linear2": self._planned(grp((cx, blk["linear2"], blk["linear2.bias"], self.x, self.x),
                                         P and (cp, blk["p_linear2"], blk["p_linear2.bias"], self.x_p, self.x_p)),
                                     "residual"),
        }

    def _gemm(self, plan) -> None:
        items, epi, split, wide = plan
        most = max(split) if isinstance(split, list) else split
        Fn.grouped_gemm(items, epi, split_k=split, workspace=self.ws if most > 1 else None, wide_tiles=wide)

    # -- blocks ---------------------------------------------------------------
    def _kb(self):
        return self.key_bias if self.masked else None

    def _qkv_norm_rope(self, streams) -> None:
        """Q and the packed K/V tiles of every robot's joint sequence from the QKV
        rows of its streams, one launch: streams = [(qkv rows of the whole batch,
        rows per robot, rows in the joint sequence, q_norm, k_norm, cos, sin)] in
        joint order."""
        cfg, B = self.cfg, self.batch
        specs = [Fn.StreamSpec(qkv[:rows], qn, kn, cos, sin) for qkv, per, rows, qn, kn, cos, sin in streams]
        if B == 1:
            Fn.msat_qkv_norm_rope(specs, cfg.heads, cfg.head_dim, cfg.eps, out=(self.q[0], self.kvp[0]), kv_packed=True)
        else:
            Fn.msat_qkv_norm_rope(specs, cfg.heads, cfg.head_dim, cfg.eps, out=(self.q, self.kvp), kv_packed=True,
                                  batch=B, batch_rows=[st[1] for st in streams])

    def _ds_block(self, blk: dict, gm: dict) -> None:
        cfg = self.cfg
        nv, ns = self.nv, cfg.n_sa
        Fn.layernorm_pack_many(self.ds_norms, cfg.eps)
        self._gemm(gm["qkv"])
        streams = [(self.qkv_vl, nv, nv, blk["q_norm_vl.weight"], blk["k_norm_vl.weight"], None, None),
                   (self.qkv_sa_buf, ns, self.ns, blk["q_norm_sa.weight"], blk["k_norm_sa.weight"], self.ds_cos,
                    self.ds_sin)]
        if self.phys:
            streams.append((self.qkv_p, self.np_, self.np_, blk["q_norm_p.weight"], blk["k_norm_p.weight"], self.p_cos,
                            self.p_sin))
        self._qkv_norm_rope(streams)
        Fn.attention_packed(self.q, self.kvp, self.N, key_bias=self._kb(), out=self.att, segments=self.segments)
        self._gemm(gm["proj"])
        Fn.layernorm_pack_many(self.ds_norms, cfg.eps)
        self._gemm(gm["w12"])
        self._gemm(gm["w3"])

    def _ss_block(self, blk: dict, gm: dict) -> None:
        cfg = self.cfg
        B, nv, ns, inner = self.batch, self.nv, cfg.n_sa, cfg.inner
        Fn.layernorm_pack_many(self.ss_norms, cfg.eps)
        self._gemm(gm["qkv"])
        self._gemm(gm["mlp"])
        streams = [(self.qkv_buf, nv, nv, blk["q_norm"], blk["k_norm"], None, None),
                   (self.qkv_buf[B * nv:], ns, self.ns, blk["q_norm"], blk["k_norm"], self.ss_cos, self.ss_sin)]
        if self.phys:
            streams.append((self.qkv_p, self.np_, self.np_, blk["p_q_norm"], blk["p_k_norm"], self.p_cos, self.p_sin))
        self._qkv_norm_rope(streams)
        Fn.attention_packed(self.q, self.kvp, self.N, key_bias=self._kb(), out=self.cat.cols(0, inner),
                            segments=self.segments)
        self._gemm(gm["mlp_proj"])
        self._gemm(gm["linear2"])

    # -- forward --------------------------------------------------------------
    def forward(self, hidden_states: torch.Tensor, encoder_hidden_states: torch.Tensor, temb: torch.Tensor,
                time_token: torch.Tensor, encoder_attention_mask: Optional[torch.Tensor] = None,
                physics_embs: Optional[torch.Tensor] = None, physics_attention_mask: Optional[torch.Tensor] = None,
                adaln: Optional[tuple] = None):
        """CustomOpMSAT.forward (custom_msat_chain.py:109-126) for the chain's
        batch of B robots: hidden_states [B, n_sa_pure, sa_dim],
        encoder_hidden_states [B, n_vl, vl_dim], temb [B, inner], time_token
        [B, num_temb_tokens, sa_dim] -> [B, n_sa_pure, output_dim] (a static
        buffer, overwritten by the next call).  Robots do not interact: each
        one's joint attention runs over its own tokens.
        encoder_attention_mask [B, n_vl] (1 = visible, 0 = masked; a chain built
        with vl_mask=True): masks VL keys in every block as the eager MSAT does
        (msat.py:517-531, blocks.py:558-575); None = every VL token visible.
        With a P stream (CustomOpExpandedMSAT.forward,
        custom_expanded_msat_chain.py:87-115): physics_embs [B, n_physics,
        sa_dim] is required and the result is {"action": [B, n_sa_pure,
        output_dim], "physics": [B, n_physics, output_dim]};
        physics_attention_mask [B] (1 = visible; a chain built with
        vl_mask=True) masks every P key of a robot (msat.py:716-743).  adaln: the
        output AdaLN's (shift, scale[, physics shift, physics scale]) for this
        temb, precomputed with adaln_of(temb) (None: computed here)."""
        cfg = self.cfg
        B, nt, nv, d = self.batch, cfg.num_temb_tokens, cfg.n_vl, cfg.sa_dim
        Fn._require(tuple(hidden_states.shape) == (B, cfg.n_sa_pure, d) and
                    tuple(encoder_hidden_states.shape) == (B, nv, cfg.vl_dim) and
                    tuple(temb.shape) == (B, cfg.inner) and tuple(time_token.shape) == (B, nt, d),
                    f"input shapes do not match the chain's configuration (batch {B})")
        if self.phys:
            Fn._require(physics_embs is not None and tuple(physics_embs.shape) == (B, self.np_, d),
                        "physics_embs must be [B, n_physics, sa_dim] for a chain with a P stream")
        else:
            Fn._require(physics_embs is None and physics_attention_mask is None,
                        "physics inputs need a chain built with use_physics and n_physics > 0")
        if self.vl_mask:
            if encoder_attention_mask is None:
                self.key_bias[:, :nv].zero_()
            else:
                Fn._require(tuple(encoder_attention_mask.shape) == (B, nv), "encoder_attention_mask must be [B, n_vl]")
                torch.where(encoder_attention_mask == 0, self._ninf, self._zero, out=self.key_bias[:, :nv])
            if self.phys:
                if physics_attention_mask is None:
                    self.key_bias[:, self.p0:].zero_()
                else:
                    Fn._require(physics_attention_mask.numel() == B, "physics_attention_mask must be [B]")
                    torch.where(physics_attention_mask.reshape(B, 1).expand(B, self.np_) == 0, self._ninf, self._zero,
                                out=self.key_bias[:, self.p0:])
        else:
            Fn._require(encoder_attention_mask is None and physics_attention_mask is None,
                        "attention masks need a chain built with vl_mask=True")
        x_sa = self.x_sa.view(B, cfg.n_sa, d)
        x_sa[:, :nt].copy_(time_token)
        x_sa[:, nt:].copy_(hidden_states)
        x_vl = self.x_vl.view(B, self.nv, cfg.vl_dim)
        x_vl[:, :nv].copy_(encoder_hidden_states)
        if self.nv > nv:
            x_vl[:, nv:].zero_()
        if self.phys:
            self.x_p.view(B, self.np_, d).copy_(physics_embs)
        for blk, gm in zip(self.ds, self.ds_gemms):
            self._ds_block(blk, gm)
        # x = [vl_proj_to_sa(vl) | time token | SA]
        Fn.pack_act(self.x_vl, out=self.vl_packed)
        self._gemm(self.vl_proj_gemm)  # rows [0, B nv) of x; rows [B nv, B nx) already hold the SA stream
        for blk, gm in zip(self.ss, self.ss_gemms):
            self._ss_block(blk, gm)
        # AdaLN output projections (msat.py:771-781)
        shift, scale, *pmod = self.adaln_of(temb) if adaln is None else adaln
        sa = F.layer_norm(x_sa[:, nt:], (d,), eps=1e-6)
        torch.add(sa * (1 + scale[:, None]), shift[:, None], out=self.mod.view(B, cfg.n_sa_pure, d))
        Fn.pack_act(self.mod, out=self.mod_packed)
        if self.phys:
            pshift, pscale = pmod
            ph = F.layer_norm(self.x_p.view(B, self.np_, d), (d,), eps=1e-6)
            torch.add(ph * (1 + pscale[:, None]), pshift[:, None], out=self.mod_p.view(B, self.np_, d))
            Fn.pack_act(self.mod_p, out=self.mod_p_packed)
        self._gemm(self.out_gemm)
        if self.phys:
            return {"action": self.out, "physics": self.out_p}
        return self.out

    __call__ = forward

    def adaln_of(self, temb: torch.Tensor) -> tuple:
        """(shift, scale) of the output AdaLN for `temb` [B, inner] (and the physics
        output's pair with a P stream): F.silu(temb) -> proj_out_1 (msat.py:771-781).
        A caller whose temb is fixed per step (the action head's static time
        embeddings) computes them once and passes them to forward(adaln=...)."""
        silu_t = F.silu(temb)
        shift, scale = F.linear(silu_t, self.w["proj_out_1.weight"], self.w["proj_out_1.bias"]).chunk(2, dim=1)
        if not self.phys:
            return shift, scale
        pshift, pscale = F.linear(silu_t, self.w["proj_out_physics_1.weight"],
                                  self.w["proj_out_physics_1.bias"]).chunk(2, dim=1)
        return shift, scale, pshift, pscale

    def _forward_static(self):
        i = self.inputs
        return self.forward(i["sa"], i["vl"], i["temb"], i["time_token"], i.get("vl_mask"), i.get("p"),
                            i.get("physics_mask"))

    def capture(self, warmup: int = 2) -> None:
        """Record forward() on the static `inputs` buffers (with the `vl_mask`
        and `physics_mask` buffers when built with vl_mask=True) into one hipGraph."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(warmup):
                self._forward_static()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._forward_static()
        torch.cuda.synchronize()

    def replay(self):
        self.graph.replay()
        return {"action": self.out, "physics": self.out_p} if self.phys else self.out


def chain_for_module(msat: torch.nn.Module, n_vl: int, n_sa_pure: int, n_physics: int = 0,
                     bf16_quirk: Optional[bool] = None, vl_mask: bool = False) -> RldxMsat:
    """An RldxMsat chain from a live MSAT module's state_dict() for these token
    counts: dimensions read off the parameter shapes, RoPE theta / table length
    off its rope_embedder; bf16_quirk=None detects the quirk from the RoPE
    buffers (real-valued: the model was cast to bf16)."""
    sd = {k: v for k, v in msat.state_dict().items()}
    rope = getattr(msat, "rope_embedder", None)
    if bf16_quirk is None:
        bf16_quirk = rope is not None and not getattr(rope, "freqs_cis_0").is_complex()
    overrides = dict(n_vl=n_vl, n_sa_pure=n_sa_pure, n_physics=n_physics)
    if rope is not None:
        overrides.update(rope_theta=float(rope.theta), max_seq_len=int(rope.max_seq_len))
    cfg = RldxMsatCfg.from_state_dict(sd, **overrides)
    dev = next(iter(sd.values())).device
    return RldxMsat(sd, cfg, dev, bf16_quirk=bf16_quirk, vl_mask=vl_mask)


class MsatDispatcher:
    """Replacement of a live MSAT module's forward by the rldx_amd chain, with
    the behaviour of the reference's path-D dispatcher (_CompiledDispatcher,
    rldx/inference/serve_optimization.py:251-516) at the MSAT boundary:

    * the first call is served by the module's own forward while the chain is
      built from msat.state_dict() for that call's token counts (and, with
      graph=True, captured as one hipGraph);
    * later calls compute temb / the time token with the module's own
      timestep_encoder / time_token_proj, copy every input into the chain's
      static buffers and run (or replay) the chain;
    * a batch of B robots runs on a chain for B (RldxMsat.for_batch: the
      same packed weights, its own buffers and, with graph=True, its own
      graph), built on the first call of that batch size; up to max_batch;
    * calls the chain does not serve go to the module's own forward:
      return_all_hidden_states=True, a batch above max_batch, or token counts
      (VL, SA or physics) other than the chain's (shape drift would corrupt
      the static buffers);
    * a failure while building or running switches the dispatcher to the
      module's own forward for good, as the reference does.
    Weights: the chain holds packed copies of msat.state_dict() taken when it
    is built.  msat.load_state_dict() (wrapped by install) and refresh() drop
    the chain, which is rebuilt from the new weights on the next call (that
    call is served by the module's own forward); with check_weights=True every
    call also compares each parameter's storage and version counter with the
    ones the chain was built from (~0.1 ms of host time per call), which
    catches in-place updates such as param.data.copy_().
    encoder_attention_mask and physics_attention_mask are served: the chain is
    built with vl_mask=True.  Physics tokens on a physics-enabled module are
    served by the all-add-ons chain (the first call's physics token count),
    which returns {"action", "physics"} as the eager _forward_physics does.
    The returned tensors are the chain's static output buffers, overwritten by
    the next call."""

    def __init__(self, msat: torch.nn.Module, bf16_quirk: Optional[bool] = None, graph: bool = False,
                 verbose: bool = False, check_weights: bool = False, max_batch: int = 16):
        self.msat, self.orig = msat, msat.forward
        self.bf16_quirk, self.graph, self.verbose = bf16_quirk, graph, verbose
        self.check_weights, self.max_batch = check_weights, int(max_batch)
        self.chain: Optional[RldxMsat] = None   # the first chain built (batch 1), owner of the packed weights
        self.chains: dict = {}                  # batch size -> chain on those weights
        self.failed = False
        self.served = 0      # calls run on the chain
        self.fallbacks = 0   # calls sent to the module's own forward
        self.rebuilds = 0    # chains dropped because the weights changed
        self._dims = None    # (n_vl, n_sa_pure, n_physics) of the chain
        self._stamp = None   # [(tensor, data_ptr, _version)] the chain was built from

    def _weights_stamp(self) -> list:
        return [(t, t.data_ptr(), t._version) for t in self.msat.state_dict(keep_vars=True).values()]

    def weights_changed(self) -> bool:
        """True when a parameter or buffer was replaced or modified in place since the build."""
        cur = self.msat.state_dict(keep_vars=True).values()
        if self._stamp is None or len(self._stamp) != len(cur):
            return True
        return any(t is not u or t.data_ptr() != p or t._version != v for (t, p, v), u in zip(self._stamp, cur))

    def refresh(self) -> None:
        """Drop the chains; the next call rebuilds them from the module's current weights."""
        if self.chain is not None:
            self.rebuilds += 1
        self.chain = None
        self.chains = {}
        self._stamp = None

    def _log(self, msg: str) -> None:
        if self.verbose:
            print(f"[rldx_amd.MsatDispatcher] {msg}", flush=True)

    def build(self, n_vl: int, n_sa_pure: int, n_physics: int = 0) -> RldxMsat:
        chain = chain_for_module(self.msat, n_vl, n_sa_pure, n_physics, self.bf16_quirk, vl_mask=True)
        if self.graph:
            chain.capture()
        self.chain = chain
        self.chains = {1: chain}
        self._dims = (n_vl, n_sa_pure, n_physics)
        self._stamp = self._weights_stamp()
        return chain

    def chain_for(self, batch: int) -> RldxMsat:
        """The chain for `batch` robots, built on the weights of self.chain when first needed."""
        c = self.chains.get(batch)
        if c is None:
            c = self.chain.for_batch(batch)
            if self.graph:
                c.capture()
            self.chains[batch] = c
        return c

    def _unserved(self, hidden_states, encoder_hidden_states, return_all_hidden_states, physics_embs,
                  physics_attention_mask) -> Optional[str]:
        if return_all_hidden_states:
            return "return_all_hidden_states"
        B = hidden_states.shape[0] if hidden_states.dim() == 3 else -1
        if B < 1 or encoder_hidden_states.dim() != 3 or encoder_hidden_states.shape[0] != B:
            return "inputs are not [B, tokens, width] with one batch size"
        if B > self.max_batch:
            return f"batch above max_batch ({self.max_batch})"
        if physics_embs is not None and (physics_embs.dim() != 3 or physics_embs.shape[0] != B):
            return "inputs are not [B, tokens, width] with one batch size"
        c = self.chain
        if c is not None and (encoder_hidden_states.shape[1] != c.cfg.n_vl or hidden_states.shape[1] != c.cfg.n_sa_pure
                              or self._n_physics(physics_embs) != c.np_):
            return "token counts differ from the chain's"
        return None

    def _n_physics(self, physics_embs) -> int:
        """P tokens the eager forward would use: the physics path runs only on a
        physics-enabled module given physics_embs (msat.py:351-363)."""
        if physics_embs is None or not getattr(self.msat, "use_physics", False):
            return 0
        return int(physics_embs.shape[1])

    def __call__(self, hidden_states, encoder_hidden_states, timestep=None, return_all_hidden_states=False,
                 encoder_attention_mask=None, physics_embs=None, physics_attention_mask=None):
        args = (hidden_states, encoder_hidden_states, timestep, return_all_hidden_states, encoder_attention_mask,
                physics_embs, physics_attention_mask)
        if self.failed:
            self.fallbacks += 1
            return self.orig(*args)
        if self.chain is not None and self.check_weights and self.weights_changed():
            self._log("weights changed since the build: rebuilding the chain")
            self.refresh()
        why = self._unserved(hidden_states, encoder_hidden_states, return_all_hidden_states, physics_embs,
                             physics_attention_mask)
        if why is not None:
            self._log(f"served by the module's own forward: {why}")
            self.fallbacks += 1
            return self.orig(*args)
        if self.chain is None:
            out = self.orig(*args)
            self.fallbacks += 1
            try:
                self.build(encoder_hidden_states.shape[1], hidden_states.shape[1], self._n_physics(physics_embs))
            except Exception as e:  # noqa: BLE001 — any build failure means the module's own forward from now on
                self.failed = True
                self._log(f"build failed ({e}); the module's own forward serves every call")
            return out
        try:
            c = self.chain_for(hidden_states.shape[0])
            B = c.batch
            msat = self.msat
            temb = msat.timestep_encoder(timestep)
            tt = msat.time_token_proj(temb).unsqueeze(1).repeat(1, c.cfg.num_temb_tokens, 1)
            mask = encoder_attention_mask
            p_embs, p_mask = (physics_embs, physics_attention_mask) if c.phys else (None, None)
            if self.graph:
                i = c.inputs
                i["sa"].copy_(hidden_states)
                i["vl"].copy_(encoder_hidden_states)
                i["temb"].copy_(temb)
                i["time_token"].copy_(tt)
                if mask is None:
                    i["vl_mask"].fill_(1.0)
                else:
                    i["vl_mask"].copy_(mask.reshape(B, -1))
                if c.phys:
                    i["p"].copy_(p_embs)
                    if p_mask is None:
                        i["physics_mask"].fill_(1.0)
                    else:
                        i["physics_mask"].copy_(p_mask.reshape(B))
                out = c.replay()
            else:
                out = c.forward(hidden_states, encoder_hidden_states, temb, tt, mask, p_embs, p_mask)
            self.served += 1
            return out
        except Exception as e:  # noqa: BLE001 — as the reference: fall back for good on a hot-path failure
            self.failed = True
            self._log(f"hot-path failure ({e}); the module's own forward serves every call")
            self.fallbacks += 1
            return self.orig(*args)


def install(msat: torch.nn.Module, n_vl: Optional[int] = None, n_sa_pure: Optional[int] = None,
            bf16_quirk: Optional[bool] = None, graph: bool = False, verbose: bool = False,
            n_physics: int = 0, check_weights: bool = False, max_batch: int = 16) -> MsatDispatcher:
    """Route a live MSAT module's forward through an MsatDispatcher (what the
    reference's path-D dispatcher does with CustomOpMSAT,
    rldx/inference/serve_optimization.py:251-601).  With n_vl and n_sa_pure the
    chain is built now; without them, on the first call (served by the
    module's own forward); n_physics > 0 builds the all-add-ons chain for
    that many physics tokens.  msat.forward keeps the reference signature
    forward(hidden_states, encoder_hidden_states, timestep,
    return_all_hidden_states, encoder_attention_mask, physics_embs,
    physics_attention_mask) (msat.py:1058-1082).  bf16_quirk=None detects it
    from the RoPE buffers (real-valued: the model was cast to bf16).
    msat.load_state_dict is wrapped so that new weights drop the chain (rebuilt
    on the next call); check_weights=True also catches in-place updates."""
    d = MsatDispatcher(msat, bf16_quirk=bf16_quirk, graph=graph, verbose=verbose, check_weights=check_weights,
                       max_batch=max_batch)
    if n_vl is not None and n_sa_pure is not None:
        d.build(n_vl, n_sa_pure, n_physics)
    msat.forward = d
    msat.rldx_amd_dispatcher = d
    load = msat.load_state_dict

    def load_state_dict(*args, **kwargs):  # new weights: the chain is rebuilt on the next call
        res = load(*args, **kwargs)
        d.refresh()
        return res

    msat.load_state_dict = load_state_dict
    return d


# ---------------------------------------------------------------------------
# The action head around the MSAT: CustomActionHeadChain.forward
# (rldx/inference/action_model/engine/custom_action_model_chain.py:81-171):
# vlln on the VL embeddings, state encoder once, the RTC trained-mode prefix
# encoded once, then per denoising step action encoder + baked position
# embedding, MSAT, action decoder and the Euler update.
# ---------------------------------------------------------------------------
@dataclass
class RldxHeadCfg:
    """rldx/configs/model/rldx.py:80-112, :111-118."""

    state_dim: int = 64       # max_state_dim
    action_dim: int = 64      # max_action_dim
    action_horizon: int = 16
    hidden_size: int = 1024   # decoder width (= MSAT output_dim)
    num_embodiments: int = 32
    steps: int = 4
    # all add-ons: physics signal width (sum of physics_dims, e.g. 30 tactile + 7 torque;
    # rldx/configs/model/rldx.py:264-285) and its history / future token counts
    # (physics_head.py:106-109; future length = action horizon); 0 = no physics head
    physics_dim: int = 0
    physics_hist_len: int = 1
    # RTC trained mode: the first prefix_len action rows are frozen to the
    # previous chunk's actions (custom_action_model_chain.py:38, :98-121, :131-165)
    prefix_len: int = 0
    # vlln: LayerNorm of the VL embeddings at the head's entry (rldx/model/core/rldx.py:100-102;
    # nn.LayerNorm(backbone_embedding_dim), affine, eps 1e-5); the release config leaves it off
    use_vlln: bool = False
    vlln_eps: float = 1e-5

    @property
    def physics_fut_len(self) -> int:
        return self.action_horizon if self.physics_dim > 0 else 0


def make_head_state_dict(msat_cfg: RldxMsatCfg, cfg: RldxHeadCfg, device, seed: int = 13) -> dict:
    """Per-embodiment encoder / decoder parameters under the reference names
    (embodiment_conditioned_mlp.py CategorySpecificLinear W [E, in, out], b
    [E, out]; rldx/model/core/rldx.py:82-106), the position embedding, and
    per-step baked time embeddings / time tokens; bf16."""
    g = torch.Generator(device=device).manual_seed(seed)
    E, d, hs = cfg.num_embodiments, msat_cfg.sa_dim, cfg.hidden_size

    def rnd(*shape, std=0.02):
        return (std * torch.randn(*shape, generator=g, device=device, dtype=torch.float32)).to(BF16)

    sd = {"state_encoder.layer1.W": rnd(E, cfg.state_dim, hs), "state_encoder.layer1.b": rnd(E, hs),
          "state_encoder.layer2.W": rnd(E, hs, d), "state_encoder.layer2.b": rnd(E, d),
          "action_encoder.W1.W": rnd(E, cfg.action_dim, d), "action_encoder.W1.b": rnd(E, d),
          "action_encoder.W2.W": rnd(E, 2 * d, d), "action_encoder.W2.b": rnd(E, d),
          "action_encoder.W3.W": rnd(E, d, d), "action_encoder.W3.b": rnd(E, d),
          "action_decoder.layer1.W": rnd(E, msat_cfg.output_dim, hs), "action_decoder.layer1.b": rnd(E, hs),
          "action_decoder.layer2.W": rnd(E, hs, cfg.action_dim), "action_decoder.layer2.b": rnd(E, cfg.action_dim),
          "position_embedding.weight": rnd(cfg.action_horizon, d),
          "static_tembs": rnd(cfg.steps, 1, msat_cfg.inner, std=0.5),
          "static_time_tokens": rnd(cfg.steps, 1, msat_cfg.num_temb_tokens, d, std=0.5)}
    if cfg.use_vlln:
        sd["vlln.weight"] = (1.0 + rnd(msat_cfg.vl_dim).float()).to(BF16)
        sd["vlln.bias"] = rnd(msat_cfg.vl_dim)
    if cfg.physics_dim > 0:
        # PhysicsHead (physics_head.py:111-113; physics.py:9-72): encoders physics_dim -> d -> d,
        # decoder output_dim -> d -> physics_dim; nn.Linear weights [out, in]
        pd, od = cfg.physics_dim, msat_cfg.output_dim
        for enc in ("physics_cond_encoder", "physics_fut_encoder"):
            sd.update({f"physics.{enc}.W1.weight": rnd(d, pd), f"physics.{enc}.W1.bias": rnd(d),
                       f"physics.{enc}.W2.weight": rnd(d, 2 * d), f"physics.{enc}.W2.bias": rnd(d),
                       f"physics.{enc}.W3.weight": rnd(d, d), f"physics.{enc}.W3.bias": rnd(d)})
        sd.update({"physics.physics_decoder.net.0.weight": rnd(d, od), "physics.physics_decoder.net.0.bias": rnd(d),
                   "physics.physics_decoder.net.2.weight": rnd(pd, d), "physics.physics_decoder.net.2.bias": rnd(pd)})
    return sd


# CategorySpecificLinear layers of the head (embodiment_conditioned_mlp.py:60-82), W [E, in, out], b [E, out]
_CAT_LINEARS = ("state_encoder.layer1", "state_encoder.layer2", "action_encoder.W1", "action_encoder.W2",
                "action_encoder.W3", "action_decoder.layer1", "action_decoder.layer2")


def bf16_timesteps(steps: int) -> list:
    """The denoising schedule t = i / steps as the reference bakes it: a bf16
    tensor (graph_safe_action_model.py:147-153), read back as floats."""
    return torch.tensor([i / float(steps) for i in range(steps)], dtype=BF16).float().tolist()


def sinusoidal_time(t: torch.Tensor, width: int) -> torch.Tensor:
    """SinusoidalPositionalEncoding.forward (embodiment_conditioned_mlp.py:14-33): [T] -> [T, width] fp32."""
    half = width // 2
    exponent = -torch.arange(half, dtype=torch.float, device=t.device) * (torch.log(torch.tensor(10000.0)) / half)
    freqs = t.float().unsqueeze(-1) * exponent.exp()
    return torch.cat([torch.sin(freqs), torch.cos(freqs)], dim=-1)


class RldxActionHead:
    """Flow-matching action head of RLDX-1 with the MSAT on the rldx_amd chain;
    `run` launches one action inference (state encoder + `steps` denoising
    iterations) on static buffers, `capture` / `replay` as one hipGraph.
    Batch: the MSAT chain's (msat.batch = B robots, RldxMsat.for_batch); the
    static buffers hold the B robots' inputs (vl [B, n_vl, vl_dim], state
    [B, 1, state_dim], x0 [B, horizon, action_dim], prefix [B, prefix_len,
    action_dim], e_idx [B] the robots' embodiment ids).  The embodiments are
    read on the device: run() gathers each robot's encoder / decoder weights
    (W[e], b[e] of every CategorySpecificLinear) into static buffers first, so
    one captured graph serves every choice of embodiments.
    timesteps: the denoising times (default: bf16_timesteps(cfg.steps), the
    reference's bf16 schedule).

    cfg.use_vlln: the VL embeddings go through the affine LayerNorm vlln
    (head_sd "vlln.weight" / "vlln.bias") first (custom_action_model_chain.py:84).
    cfg.prefix_len = d > 0 (RTC trained mode, :98-121, :131-165): the first d
    action rows are `prefix` for the whole call; their encoder features (time
    t = 1) are computed once, each step encodes and decodes only the last
    horizon - d rows, and the Euler update advances only those.

    With a physics head (cfg.physics_dim > 0, an MSAT chain with a P stream of
    physics_hist_len + physics_fut_len tokens) it is CustomExpandedActionHeadChain
    .forward (rldx/inference/action_model/engine/
    custom_expanded_action_model_chain.py:84-219): the history tokens are
    encoded once, and per step the future physics state is encoded at the
    step's time, the MSAT returns action and physics hidden states, and the
    physics decoder's velocity advances the future state by the Euler step."""

    def __init__(self, msat: RldxMsat, head_sd: dict, cfg: RldxHeadCfg, embodiment: int = 0,
                 timesteps: Optional[list] = None):
        self.msat, self.cfg, self.sd = msat, cfg, head_sd
        dev, mc = msat.dev, msat.cfg
        Fn._require(mc.n_sa_pure == 1 + cfg.action_horizon, "MSAT SA tokens = state token + action horizon")
        Fn._require(head_sd["action_decoder.layer1.W"].shape[1] == mc.output_dim, "MSAT output_dim feeds the action decoder")
        self.phys = cfg.physics_dim > 0
        Fn._require(self.phys == msat.phys, "a physics head needs an MSAT chain with a P stream, and only then")
        if self.phys:
            Fn._require(msat.np_ == cfg.physics_hist_len + cfg.physics_fut_len,
                        "MSAT physics tokens = physics history + future")
        self.dt = 1.0 / cfg.steps
        self.timesteps = bf16_timesteps(cfg.steps) if timesteps is None else [float(t) for t in timesteps]
        Fn._require(len(self.timesteps) == cfg.steps, "one timestep per denoising step")
        E = cfg.num_embodiments
        for name in _CAT_LINEARS:
            Fn._require(tuple(head_sd[f"{name}.W"].shape[:1]) == (E,) and tuple(head_sd[f"{name}.b"].shape[:1]) == (E,),
                        f"{name}: one weight per embodiment ({E})")
        Fn._require(0 <= embodiment < E, "embodiment id out of range")
        B = self.batch = msat.batch
        self.e_idx = torch.full((B,), embodiment, dtype=torch.long, device=dev)
        # each robot's embodiment weights, gathered at the top of run()
        self.w_e = {n: torch.empty((B, *head_sd[f"{n}.W"].shape[1:]), dtype=head_sd[f"{n}.W"].dtype, device=dev)
                    for n in _CAT_LINEARS}
        self.b_e = {n: torch.empty((B, 1, *head_sd[f"{n}.b"].shape[1:]), dtype=head_sd[f"{n}.b"].dtype, device=dev)
                    for n in _CAT_LINEARS}
        Fn._require(0 <= cfg.prefix_len < cfg.action_horizon, "0 <= prefix_len < action_horizon")
        Fn._require(not cfg.use_vlln or ("vlln.weight" in head_sd and "vlln.bias" in head_sd),
                    "use_vlln needs vlln.weight and vlln.bias")
        e = lambda *s: torch.empty(*s, dtype=BF16, device=dev)  # noqa: E731
        self.vl, self.state = e(B, mc.n_vl, mc.vl_dim), e(B, 1, cfg.state_dim)
        self.vl_n = e(B, mc.n_vl, mc.vl_dim) if cfg.use_vlln else self.vl  # the MSAT's VL input
        self.d = cfg.prefix_len
        if self.d > 0:
            self.prefix = e(B, self.d, cfg.action_dim)
            # the prefix rows' time is 1 (custom_action_model_chain.py:117-121), baked
            self.tau_one = sinusoidal_time(torch.ones(self.d, device=dev), mc.sa_dim).to(BF16).expand(B, -1, -1)
        self.x0 = e(B, cfg.action_horizon, cfg.action_dim)
        self.act = e(B, cfg.action_horizon, cfg.action_dim)
        self.sa = e(B, mc.n_sa_pure, mc.sa_dim)
        # tau encodings of each step's time, baked (same every call)
        self.tau = [sinusoidal_time(torch.full((cfg.action_horizon,), t, device=dev), mc.sa_dim).to(BF16)
                    .expand(B, -1, -1) for t in self.timesteps]
        if self.phys:
            self.physics_hist = e(B, cfg.physics_hist_len, cfg.physics_dim)
            self.physics_x0 = e(B, cfg.physics_fut_len, cfg.physics_dim)
            self.physics_fut = e(B, cfg.physics_fut_len, cfg.physics_dim)
            self.p_embs = e(B, msat.np_, mc.sa_dim)
            # history positions 0 .. T_hist - 1 (physics.py:19-25), baked
            self.hist_pos = sinusoidal_time(torch.arange(cfg.physics_hist_len, device=dev), mc.sa_dim).to(BF16)\
                .expand(B, -1, -1)
        # every robot's static time embedding / time token of each step (custom_action_model_chain.py:125-127,
        # expanded over the batch) and the output AdaLN of each, computed once
        self.tembs = [head_sd["static_tembs"][i].expand(B, -1) for i in range(cfg.steps)]
        self.time_tokens = [head_sd["static_time_tokens"][i].expand(B, -1, -1) for i in range(cfg.steps)]
        self.adaln = [msat.adaln_of(t) for t in self.tembs]
        self.graph = None

    def for_batch(self, batch: int) -> "RldxActionHead":
        """This head for `batch` robots: an MSAT chain for the batch on the same
        packed weights, the same head weights, buffers of its own."""
        return RldxActionHead(self.msat.for_batch(batch), self.sd, self.cfg, timesteps=self.timesteps)

    def _lin(self, x, name):
        return F.linear(x, self.sd[f"{name}.weight"], self.sd[f"{name}.bias"])

    def _physics_encoder(self, x, pos, enc):
        """PhysicalSignalEncoder / PhysicsNoiseEncoder.forward (physics.py:19-25,
        :54-72): W3(silu(W2([W1 x | pos])))."""
        h = self._lin(x, f"physics.{enc}.W1")
        return self._lin(F.silu(self._lin(torch.cat([h, pos], dim=-1), f"physics.{enc}.W2")), f"physics.{enc}.W3")

    def set_embodiment(self, e) -> None:
        """Select the embodiment of every robot (an int) or of each robot (a
        sequence of B ints) for the next run / replay; range-checked on the host:
        the gather must never index past W's first dimension."""
        ids = [int(e)] * self.batch if isinstance(e, int) else [int(v) for v in e]
        if len(ids) != self.batch:
            raise ValueError(f"{len(ids)} embodiment ids for a batch of {self.batch}")
        for v in ids:
            if not 0 <= v < self.cfg.num_embodiments:
                raise IndexError(f"embodiment id {v} out of range [0, {self.cfg.num_embodiments})")
        self.e_idx.copy_(torch.tensor(ids, dtype=torch.long))

    def _cat(self, x, name):
        """CategorySpecificLinear.forward (embodiment_conditioned_mlp.py:72-82):
        x [B, T, in] -> x W[e_b] + b[e_b] per robot b, with the gathered weights."""
        return torch.baddbmm(self.b_e[name], x, self.w_e[name])

    def _encode(self, x, tau):
        """MultiEmbodimentActionEncoder.forward (embodiment_conditioned_mlp.py:191-227):
        W3(swish(W2([W1 x | tau])))."""
        a = self._cat(x, "action_encoder.W1")
        h = self._cat(torch.cat([a, tau], dim=-1), "action_encoder.W2")
        return self._cat(h * torch.sigmoid(h), "action_encoder.W3")

    def run(self) -> torch.Tensor:
        sd, mc, cfg = self.sd, self.msat.cfg, self.cfg
        d, H = self.d, cfg.action_horizon
        for n in _CAT_LINEARS:
            torch.index_select(sd[f"{n}.W"], 0, self.e_idx, out=self.w_e[n])
            torch.index_select(sd[f"{n}.b"], 0, self.e_idx, out=self.b_e[n][:, 0])
        if cfg.use_vlln:
            self.vl_n.copy_(F.layer_norm(self.vl, (mc.vl_dim,), sd["vlln.weight"], sd["vlln.bias"], cfg.vlln_eps))
        h = F.relu(self._cat(self.state, "state_encoder.layer1"))
        self.sa[:, :1].copy_(self._cat(h, "state_encoder.layer2"))
        self.act.copy_(self.x0)
        if d > 0:  # the frozen prefix: its actions and (once) its encoder features
            self.act[:, :d].copy_(self.prefix)
            torch.add(self._encode(self.prefix, self.tau_one), sd["position_embedding.weight"][:d],
                      out=self.sa[:, 1:1 + d])
        if self.phys:
            nh = cfg.physics_hist_len
            self.p_embs[:, :nh].copy_(self._physics_encoder(self.physics_hist, self.hist_pos, "physics_cond_encoder"))
            self.physics_fut.copy_(self.physics_x0)
        for i in range(cfg.steps):
            torch.add(self._encode(self.act[:, d:], self.tau[i][:, d:]), sd["position_embedding.weight"][d:],
                      out=self.sa[:, 1 + d:])
            if self.phys:
                # the step's time for every future row: the same encoding as the actions' tau
                self.p_embs[:, nh:].copy_(self._physics_encoder(self.physics_fut, self.tau[i][:, :cfg.physics_fut_len],
                                                                "physics_fut_encoder"))
                o = self.msat.forward(self.sa, self.vl_n, self.tembs[i], self.time_tokens[i],
                                      physics_embs=self.p_embs, adaln=self.adaln[i])
                out = o["action"]
                ph = o["physics"][:, -cfg.physics_fut_len:]
                pv = self._lin(F.silu(self._lin(ph, "physics.physics_decoder.net.0")), "physics.physics_decoder.net.2")
                self.physics_fut.add_(pv, alpha=self.dt)
            else:
                out = self.msat.forward(self.sa, self.vl_n, self.tembs[i], self.time_tokens[i], adaln=self.adaln[i])
            if d > 0:  # only the postfix rows are decoded and advanced (:156-170)
                hd = F.relu(self._cat(out[:, -(H - d):], "action_decoder.layer1"))
                v = self._cat(hd, "action_decoder.layer2")
            else:
                hd = F.relu(self._cat(out, "action_decoder.layer1"))
                v = self._cat(hd, "action_decoder.layer2")[:, -H:]
            self.act[:, d:].add_(v, alpha=self.dt)
        return self.act

    def capture(self, warmup: int = 2) -> None:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(warmup):
                self.run()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.run()
        torch.cuda.synchronize()

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        return self.act


class ActionHeadDispatcher:
    """Replacement of a live action model's forward -- GraphSafeActionModel.forward
    (rldx/inference/action_model/model/graph_safe_action_model.py:171-315), the
    module the reference's chains bake (custom_action_model_chain.py:23-171,
    custom_expanded_action_model_chain.py:84-219) -- by an RldxActionHead on the
    rldx_amd MSAT chain, built from the module's weights at install.

    Served (a batch of B <= max_batch robots; each batch size on a head of its
    own, RldxActionHead.for_batch: the same packed weights, its own buffers and
    graph, built on the first call of that size): vl_embs [B, n_vl, vl_dim]
    with the module's n_vl; state [B, state_dim] or [B, 1, state_dim];
    embodiment_id [B] (read on the host and range-checked -- one stream sync
    when it lives on the GPU -- an id out of range raises IndexError);
    init_noise [B, horizon, action_dim] or None (then drawn here, as the module
    does); with prefix_len d > 0, prefix_actions [B, d, action_dim]; on a
    physics model, physics_hist [B, hist_len, physics_dim] and
    physics_init_noise or None.  The result is a new tensor [B, horizon,
    action_dim].
    Refused per call, to the module's own forward (counted in `fallbacks`,
    logged with verbose=True): inputs of different batch sizes, a batch above
    max_batch, a VL token count other
    than the module's, prefix_len > 0 without prefix_actions, a physics model
    called without physics_hist (its forward then runs with no history
    tokens).  A build failure (a module the head does not mirror: a vlln other
    than LayerNorm / Identity, physics encoder widths other than the MSAT's
    SA width, a physics future length other than the action horizon) sends
    every call to the module's own forward for good, and so does a failure
    while running, as the reference's dispatcher does
    (rldx/inference/serve_optimization.py:251-516).
    Weights are copied at the build; refresh() drops the head, which is
    rebuilt from the module's current weights on the next call (served by the
    module's own forward); with check_weights=True every call first checks
    the module's parameters and buffers for replacement or in-place change
    (tensor identity, data_ptr, _version) and refreshes on a change."""

    def __init__(self, model: torch.nn.Module, bf16_quirk: Optional[bool] = None, graph: bool = True,
                 verbose: bool = False, check_weights: bool = False, max_batch: int = 16):
        self.model, self.orig = model, model.forward
        self.bf16_quirk, self.graph, self.verbose = bf16_quirk, graph, verbose
        self.check_weights, self.max_batch = check_weights, int(max_batch)
        self.head: Optional[RldxActionHead] = None  # the first head built (batch 1), owner of the packed weights
        self.heads: dict = {}                        # batch size -> head on those weights
        self.failed = False
        self.served = 0
        self.fallbacks = 0
        self.rebuilds = 0    # heads dropped because the weights changed
        self.refusals: dict = {}  # reason -> calls
        self._stamp = None   # [(tensor, data_ptr, _version)] the head was built from

    def _weights_stamp(self) -> list:
        return [(t, t.data_ptr(), t._version) for t in self.model.state_dict(keep_vars=True).values()]

    def weights_changed(self) -> bool:
        """True when a parameter or buffer was replaced or modified in place since the build."""
        cur = self.model.state_dict(keep_vars=True).values()
        if self._stamp is None or len(self._stamp) != len(cur):
            return True
        return any(t is not u or t.data_ptr() != p or t._version != v for (t, p, v), u in zip(self._stamp, cur))

    def _log(self, msg: str) -> None:
        if self.verbose:
            print(f"[rldx_amd.ActionHeadDispatcher] {msg}", flush=True)

    def head_inputs(self) -> tuple:
        """(head_sd, RldxHeadCfg, RldxMsat chain) of the module as it is now."""
        m = self.model
        gs = m.gs_msat
        msat = gs._msat
        phys = bool(getattr(m, "use_physics", False))
        n_phys = int(getattr(gs, "n_physics", 0)) if phys else 0
        chain = chain_for_module(msat, int(gs.n_vl), int(gs.n_sa_pure), n_phys, self.bf16_quirk)
        mc = chain.cfg
        dev = chain.dev
        hsd = {}
        with torch.no_grad():
            for name in ("state_encoder", "action_encoder", "action_decoder"):
                for k, v in getattr(m, name).state_dict().items():
                    hsd[f"{name}.{k}"] = v.to(device=dev, dtype=BF16)
            # the baked values of CustomActionHeadChain.__init__ (custom_action_model_chain.py:46-66)
            hsd["position_embedding.weight"] = m.position_embedding(m.static_pos_ids).to(device=dev, dtype=BF16)
            tembs, tts = [], []
            for t in m.static_timesteps:
                temb = msat.timestep_encoder(t.unsqueeze(0))
                tts.append(msat.time_token_proj(temb).unsqueeze(1).repeat(1, mc.num_temb_tokens, 1))
                tembs.append(temb)
            hsd["static_tembs"] = torch.stack(tembs).to(device=dev, dtype=BF16)
            hsd["static_time_tokens"] = torch.stack(tts).to(device=dev, dtype=BF16)
            vlln = m.vlln
            if isinstance(vlln, torch.nn.LayerNorm):
                Fn._require(tuple(vlln.normalized_shape) == (mc.vl_dim,), "vlln must normalise the VL width")
                ones = torch.ones(mc.vl_dim, device=dev)
                hsd["vlln.weight"] = (vlln.weight if vlln.weight is not None else ones).to(device=dev, dtype=BF16)
                hsd["vlln.bias"] = (vlln.bias if vlln.bias is not None else 0 * ones).to(device=dev, dtype=BF16)
                use_vlln, eps = True, float(vlln.eps)
            else:
                Fn._require(isinstance(vlln, torch.nn.Identity), "vlln must be nn.LayerNorm or nn.Identity")
                use_vlln, eps = False, 1e-5
            kw = {}
            if phys:
                for enc in ("physics_cond_encoder", "physics_fut_encoder", "physics_decoder"):
                    for k, v in getattr(m, enc).state_dict().items():
                        hsd[f"physics.{enc}.{k}"] = v.to(device=dev, dtype=BF16)
                for enc in ("physics_cond_encoder", "physics_fut_encoder"):
                    Fn._require(hsd[f"physics.{enc}.W1.weight"].shape[0] == mc.sa_dim,
                                "physics encoder width must be the MSAT SA width")
                Fn._require(int(m.physics_fut_len) == int(m.action_horizon) and int(m.physics_hist_len) >= 1,
                            "physics future length = action horizon, and a physics history")
                kw = dict(physics_dim=int(m.physics_dim), physics_hist_len=int(m.physics_hist_len))
        W1 = hsd["state_encoder.layer1.W"]
        hc = RldxHeadCfg(state_dim=W1.shape[1], action_dim=int(m.action_dim), action_horizon=int(m.action_horizon),
                         hidden_size=W1.shape[2], num_embodiments=W1.shape[0], steps=int(m.num_inference_timesteps),
                         prefix_len=int(getattr(m, "prefix_len", 0)), use_vlln=use_vlln, vlln_eps=eps, **kw)
        return hsd, hc, chain

    def _capture(self, head: RldxActionHead) -> None:
        if self.graph:
            for buf in [head.vl, head.state, head.x0] + ([head.prefix] if head.d > 0 else []):
                buf.zero_()
            if head.phys:
                for buf in (head.physics_hist, head.physics_x0):
                    buf.zero_()
            head.capture()

    def build(self) -> RldxActionHead:
        hsd, hc, chain = self.head_inputs()
        head = RldxActionHead(chain, hsd, hc, timesteps=self.model.static_timesteps.float().tolist())
        self._capture(head)
        self.head = head
        self.heads = {1: head}
        self._stamp = self._weights_stamp()
        return head

    def head_for(self, batch: int) -> RldxActionHead:
        """The head for `batch` robots, built on the weights of self.head when first needed."""
        h = self.heads.get(batch)
        if h is None:
            h = self.head.for_batch(batch)
            self._capture(h)
            self.heads[batch] = h
        return h

    def refresh(self) -> None:
        """Drop the heads; the next call rebuilds them from the module's current weights."""
        if self.head is not None:
            self.rebuilds += 1
        self.head = None
        self.heads = {}
        self._stamp = None

    def _unserved(self, vl_embs, state, prefix_actions, physics_hist) -> Optional[str]:
        m = self.model
        B = vl_embs.shape[0] if vl_embs.dim() == 3 else -1
        if B < 1 or state.shape[0] != B or any(t is not None and t.shape[0] != B for t in (prefix_actions, physics_hist)):
            return "inputs of different batch sizes"
        if B > self.max_batch:
            return f"batch above max_batch ({self.max_batch})"
        if vl_embs.shape[1] != int(m.gs_msat.n_vl):
            return "VL token count differs from the module's"
        if int(getattr(m, "prefix_len", 0)) > 0 and prefix_actions is None:
            return "prefix_len > 0 without prefix_actions"
        if getattr(m, "use_physics", False) and physics_hist is None:
            return "physics model without physics_hist"
        return None

    def _refuse(self, why: str, args, kwargs):
        self.refusals[why] = self.refusals.get(why, 0) + 1
        self.fallbacks += 1
        self._log(f"served by the module's own forward: {why}")
        return self.orig(*args, **kwargs)

    def __call__(self, vl_embs, state, embodiment_id, init_noise=None, physics_hist=None, physics_init_noise=None,
                 prefix_actions=None):
        args = (vl_embs, state, embodiment_id)
        kwargs = dict(init_noise=init_noise, physics_hist=physics_hist, physics_init_noise=physics_init_noise,
                      prefix_actions=prefix_actions)
        if self.failed:
            self.fallbacks += 1
            return self.orig(*args, **kwargs)
        if self.head is not None and self.check_weights and self.weights_changed():
            self._log("weights changed since the build: rebuilding the head")
            self.refresh()
        why = self._unserved(vl_embs, state, prefix_actions, physics_hist)
        if why is not None:
            return self._refuse(why, args, kwargs)
        if self.head is None:
            try:
                self.build()
            except Exception as e:  # noqa: BLE001 -- any build failure means the module's own forward from now on
                self.failed = True
                self._log(f"build failed ({e}); the module's own forward serves every call")
            return self._refuse("building the head", args, kwargs)
        B = vl_embs.shape[0]
        try:
            h = self.head_for(B)
        except Exception as e:  # noqa: BLE001 -- a head for this batch that cannot be built: this call only
            self._log(f"no head for a batch of {B} ({e})")
            return self._refuse(f"building the head for a batch of {B}", args, kwargs)
        h.set_embodiment(torch.as_tensor(embodiment_id).reshape(-1).tolist())  # IndexError out of range
        try:
            h.vl.copy_(vl_embs)
            h.state.copy_(state.reshape(h.state.shape))
            if init_noise is None:
                h.x0.normal_()
            else:
                h.x0.copy_(init_noise)
            if h.d > 0:
                h.prefix.copy_(prefix_actions)
            if h.phys:
                h.physics_hist.copy_(physics_hist)
                if physics_init_noise is None:
                    h.physics_x0.normal_()
                else:
                    h.physics_x0.copy_(physics_init_noise)
            out = (h.replay() if h.graph is not None else h.run()).clone()
            self.served += 1
            return out
        except Exception as e:  # noqa: BLE001 -- as the reference: fall back for good on a hot-path failure
            self.failed = True
            self._log(f"hot-path failure ({e}); the module's own forward serves every call")
            self.fallbacks += 1
            return self.orig(*args, **kwargs)


def install_action_head(model: torch.nn.Module, bf16_quirk: Optional[bool] = None, graph: bool = True,
                        verbose: bool = False, build: bool = True,
                        check_weights: bool = False, max_batch: int = 16) -> ActionHeadDispatcher:
    """Route a live action model's forward (a GraphSafeActionModel: gs_msat
    with _msat / n_vl / n_sa_pure / n_physics, vlln, state_encoder,
    action_encoder, action_decoder, position_embedding, static_pos_ids,
    static_timesteps, action_horizon, action_dim, num_inference_timesteps,
    prefix_len and, with use_physics, the physics encoders / decoder and their
    lengths) through an ActionHeadDispatcher.  build=True builds (and with
    graph=True captures) the head now; otherwise the first call is served by
    the module's own forward while it is built.  model.forward keeps the
    reference signature forward(vl_embs, state, embodiment_id, init_noise,
    physics_hist, physics_init_noise, prefix_actions)
    (graph_safe_action_model.py:171-180); model.load_state_dict is wrapped so
    that new weights drop the head (rebuilt on the next call);
    check_weights=True also catches in-place updates."""
    d = ActionHeadDispatcher(model, bf16_quirk=bf16_quirk, graph=graph, verbose=verbose,
                             check_weights=check_weights, max_batch=max_batch)
    if build:
        d.build()
    model.forward = d
    model.rldx_amd_dispatcher = d
    load = model.load_state_dict

    def load_state_dict(*args, **kwargs):  # new weights: the head is rebuilt on the next call
        res = load(*args, **kwargs)
        d.refresh()
        return res

    model.load_state_dict = load_state_dict
    return d
