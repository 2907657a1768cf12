"""Synthetic MSAT action step on one GPU, capturable as one hipGraph.

Workload: 16 triple-stream blocks, hidden 1536 for every stream, 12 heads x 128,
SwiGLU FFN with intermediate 4096 (biases everywhere), streams of 512 cognition
(VL), 64 action (SA) and 32 physics (P, last 8 padded) tokens, 4 flow-matching
Euler iterations x <- x + dt * v(x, t), t in {0, 1/4, 2/4, 3/4}, batch 1, bf16,
random-init weights.

Block = ExpandedDoubleStreamBlock.forward with identity modulation (the
`input_token` time conditioning, rldx/model/modules/action_model/blocks.py:705-891):
    h_s   = LayerNorm(x_s)                              (no affine, eps 1e-6)
    qkv_s = Linear_s(h_s)
    q, k  = per-stream RMSNorm, interleaved 2-axis RoPE on SA and P rows
    o     = SDPA([VL | SA | P], key padding mask on the padded P keys)
    x_s  += Proj_s(o_s)
    x_s  += W3_s(SwiGLU(W12_s(LayerNorm(x_s))))
Around the blocks (GraphSafeActionModel.forward denoising loop,
rldx/inference/action_model/model/graph_safe_action_model.py:430-485):
    SA tokens = ActionIn(x_t) + temb[t] + pos     (temb precomputed per step)
    v         = ActionOut(LayerNorm(SA out));   x_{t+1} = x_t + dt * v

Every block runs on the rldx_amd HIP kernels (LayerNorm, grouped GEMMs with
fused bias / residual / SwiGLU epilogues, QK-RMSNorm + RoPE, joint attention);
the tiny action in/out projections around the blocks are one HIP launch each
per iteration (fused_io; torch.addmm and torch elementwise ops otherwise).
Activations of the three streams share one [608, 1536] buffer (rows VL | SA |
P) so every launch covers all streams.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import functional as Fn
from .workloads import msat_rope_tables

BF16 = torch.bfloat16
STREAMS = ("vl", "sa", "p")


@dataclass
class MsatStepCfg:
    blocks: int = 16
    hidden: int = 1536
    heads: int = 12
    head_dim: int = 128
    ffn: int = 4096
    n_vl: int = 512
    n_sa: int = 64
    n_p: int = 32
    n_p_pad: int = 8
    action_dim: int = 32
    steps: int = 4
    eps: float = 1e-6
    rope_theta: float = 10000.0
    seed: int = 5
    weight_std: float = 0.02

    @property
    def tokens(self) -> int:
        return self.n_vl + self.n_sa + self.n_p

    @property
    def inner(self) -> int:
        return self.heads * self.head_dim

    def rows(self, s: str) -> slice:
        if s == "vl":
            return slice(0, self.n_vl)
        if s == "sa":
            return slice(self.n_vl, self.n_vl + self.n_sa)
        return slice(self.n_vl + self.n_sa, self.tokens)

    def flops_per_step(self) -> int:
        """Matmul + attention flops of one action step (all denoising iterations)."""
        d, i, n = self.hidden, self.ffn, self.tokens
        per_tok = 2 * (d * 3 * self.inner + self.inner * d + d * 2 * i + i * d)
        attn = 4 * self.heads * n * n * self.head_dim
        io = 2 * self.n_sa * (self.action_dim * d + d * self.action_dim)
        return self.steps * (self.blocks * (n * per_tok + attn) + io)

    def weight_bytes(self) -> int:
        d, i = self.hidden, self.ffn
        per_stream = (3 * self.inner * d + 3 * self.inner) + (self.inner * d + d) + (2 * i * d + 2 * i) + (i * d + d) \
            + 2 * self.head_dim
        return 2 * (self.blocks * 3 * per_stream + 2 * self.action_dim * d)


def make_weights(cfg: MsatStepCfg, device, dtype=BF16) -> dict:
    """Random-init weights ~ N(0, weight_std) (biases too), norm weights 1 + N(0, 0.02).
    Generated on `device` with a seeded generator; stacked over blocks per stream."""
    g = torch.Generator(device=device).manual_seed(cfg.seed)
    d, i, L = cfg.hidden, cfg.ffn, cfg.blocks

    def rnd(*shape, std=cfg.weight_std):
        return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std).to(dtype)

    w = {}
    for s in STREAMS:
        w[f"{s}.qkv.w"] = rnd(L, 3 * cfg.inner, d)
        w[f"{s}.qkv.b"] = rnd(L, 3 * cfg.inner)
        w[f"{s}.q_norm"] = (1.0 + rnd(L, cfg.head_dim, std=0.02).float()).to(dtype)
        w[f"{s}.k_norm"] = (1.0 + rnd(L, cfg.head_dim, std=0.02).float()).to(dtype)
        w[f"{s}.proj.w"] = rnd(L, d, cfg.inner)
        w[f"{s}.proj.b"] = rnd(L, d)
        w[f"{s}.w12.w"] = rnd(L, 2 * i, d)
        w[f"{s}.w12.b"] = rnd(L, 2 * i)
        w[f"{s}.w3.w"] = rnd(L, d, i)
        w[f"{s}.w3.b"] = rnd(L, d)
    w["act_in.w"] = rnd(d, cfg.action_dim)
    w["act_in.b"] = rnd(d)
    w["act_out.w"] = rnd(cfg.action_dim, d)
    w["act_out.b"] = rnd(cfg.action_dim)
    return w


def make_inputs(cfg: MsatStepCfg, device) -> dict:
    """Cognition / physics tokens, action noise, per-step time embeddings,
    action position embeddings, RoPE tables and the key-padding bias."""
    g = torch.Generator(device=device).manual_seed(cfg.seed + 1)
    d = cfg.hidden

    def rnd(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std).to(BF16)

    inp = {
        "vl": rnd(cfg.n_vl, d),
        "p": rnd(cfg.n_p, d),
        "x0": rnd(cfg.n_sa, cfg.action_dim),
        "temb": rnd(cfg.steps, d, std=0.5),
        "pos": rnd(cfg.n_sa, d, std=0.5),
    }
    sa_ids = torch.zeros(cfg.n_sa, 2, dtype=torch.long)
    sa_ids[:, 1] = torch.arange(cfg.n_sa)
    p_ids = torch.zeros(cfg.n_p, 2, dtype=torch.long)
    p_ids[:, 0] = 1
    p_ids[:, 1] = torch.arange(cfg.n_p)
    sc, ss = msat_rope_tables(sa_ids, cfg.head_dim, cfg.rope_theta)
    pc, ps = msat_rope_tables(p_ids, cfg.head_dim, cfg.rope_theta)
    inp.update({"sa_cos": sc.to(device), "sa_sin": ss.to(device), "p_cos": pc.to(device), "p_sin": ps.to(device)})
    bias = torch.zeros(cfg.tokens, dtype=torch.float32)
    bias[cfg.tokens - cfg.n_p_pad:] = float("-inf")
    inp["key_bias"] = bias.to(device)
    return inp


class MsatActionStep:
    """Static-buffer executor of one action step; `run()` launches it eagerly,
    `capture()` records the same launches into one hipGraph.

    Per block (ln_fold=True, the default), 5 launches, each covering all three
    streams; the residual stream x stays in the packed activation order:
        QKV linears of LN(x) (+ bias)  rldx_grouped_gemm_qkv_norm_rope_ln_bf16:
          with QK-RMSNorm + RoPE,        the pre-LayerNorm folded into the GEMM
          K/V tiles                      (row statistics from the A chunks it streams)
        joint attention -> packed o    rldx_attention_packed_fwd_bf16
        Proj linears, x += (in place)  rldx_grouped_gemm_bf16 (packed residual epilogue)
        W12 linears of LN(x) + SwiGLU  rldx_grouped_gemm_ln_bf16 (SwiGLU epilogue)
        W3 linears, x += (in place)    rldx_grouped_gemm_bf16 (packed residual epilogue)
    ln_fold=False runs the eager rounding of the pre-norm instead: x row-major,
    LayerNorm -> packed h (rldx_layernorm_pack_bf16) before the QKV and W12
    GEMMs (7 launches per block).  fused_qkv=False splits the QKV launch into
    rldx_grouped_gemm_bf16 (or _ln_bf16) and rldx_msat_qkv_norm_rope_bf16.
    fused_io (with ln_fold): each iteration's action encoder, position
    embedding and operand packing of the three streams are one launch
    (rldx_action_encode_pack_bf16) and its decoder + Euler update another
    (rldx_action_decode_euler_bf16), instead of eleven torch / pack launches.
    warm_w3: the attention launch also reads the block's W3 weight panels into
    the memory-side cache (rldx_attention_packed_fwd_warm_bf16), so the W3 GEMM
    after Proj and W12 finds them there instead of in HBM.
    The weights are packed once, at construction, into the GEMM's operand order."""

    def __init__(self, cfg: MsatStepCfg, weights: dict, inputs: dict, fused_qkv: bool = True, ln_fold: bool = True,
                 warm_w3: tuple = STREAMS, fused_io: bool = True):
        self.cfg, self.w, self.inp = cfg, weights, inputs
        self.fused_qkv, self.ln_fold, self.warm_w3 = fused_qkv, ln_fold, tuple(warm_w3)
        self.fused_io = fused_io and ln_fold
        dev = inputs["vl"].device
        n, d, H, D = cfg.tokens, cfg.hidden, cfg.heads, cfg.head_dim
        e = lambda *s: torch.empty(*s, dtype=BF16, device=dev)  # noqa: E731
        self.x = e(n, d)            # residual stream, rows VL | SA | P (with ln_fold: the row-major staging of
        self.xp = Fn.PackedAct.empty(n, d, dev)  # each iteration's inputs; the stream itself is xp, packed)
        # LayerNorm statistics of each stream's rows of xp (written by their producers)
        self.xst = {s: Fn.ln_stats_empty(cfg.rows(s).stop - cfg.rows(s).start, d, dev) for s in STREAMS}
        self.qkv = e(n, 3 * cfg.inner)
        self.q = e(H, n, D)
        self.kvp = e(H, Fn.kv_packed_elems(n, D))  # K/V in the attention kernel's packed tiles
        self.h = Fn.PackedAct.empty(n, d, dev)           # LayerNorm output, GEMM operand order
        self.att = Fn.PackedAct.empty(n, cfg.inner, dev)  # attention output, GEMM operand order
        self.gl = Fn.PackedAct.empty(n, cfg.ffn, dev)     # SwiGLU output, GEMM operand order
        self.act = e(cfg.n_sa, cfg.action_dim)   # x_t, updated in place
        self.vel = e(cfg.n_sa, cfg.action_dim)
        self.sa_in = e(cfg.n_sa, d)
        self.pw = {}
        for s in STREAMS:
            for name in ("qkv", "proj", "w12", "w3"):
                self.pw[f"{s}.{name}"] = [Fn.pack_weight(weights[f"{s}.{name}.w"][L], swiglu_pairs=(name == "w12"))
                                          for L in range(cfg.blocks)]
        self.graph = None

    def _stats(self) -> list:
        return [self.xst[s] for s in STREAMS]

    def _gemms(self, L: int) -> dict:
        """The four grouped GEMMs of block L: (items, epilogue)."""
        cfg, w, pw = self.cfg, self.w, self.pw
        rows = [(s, cfg.rows(s)) for s in STREAMS]
        if self.ln_fold:
            xp = self.xp
            return {
                "qkv": ([(xp.rows(r.start, r.stop), pw[f"{s}.qkv"][L], w[f"{s}.qkv.b"][L], self.qkv[r], None)
                         for s, r in rows], "bias"),
                "proj": ([(self.att.rows(r.start, r.stop), pw[f"{s}.proj"][L], w[f"{s}.proj.b"][L],
                           xp.rows(r.start, r.stop), xp.rows(r.start, r.stop)) for s, r in rows], "residual_packed"),
                "w12": ([(xp.rows(r.start, r.stop), pw[f"{s}.w12"][L], w[f"{s}.w12.b"][L],
                          self.gl.rows(r.start, r.stop), None) for s, r in rows], "swiglu_packed"),
                "w3": ([(self.gl.rows(r.start, r.stop), pw[f"{s}.w3"][L], w[f"{s}.w3.b"][L],
                         xp.rows(r.start, r.stop), xp.rows(r.start, r.stop)) for s, r in rows], "residual_packed"),
            }
        return {
            "qkv": ([(self.h.rows(r.start, r.stop), pw[f"{s}.qkv"][L], w[f"{s}.qkv.b"][L], self.qkv[r], None)
                     for s, r in rows], "bias"),
            "proj": ([(self.att.rows(r.start, r.stop), pw[f"{s}.proj"][L], w[f"{s}.proj.b"][L], self.x[r], self.x[r])
                      for s, r in rows], "residual"),
            "w12": ([(self.h.rows(r.start, r.stop), pw[f"{s}.w12"][L], w[f"{s}.w12.b"][L],
                      self.gl.rows(r.start, r.stop), None) for s, r in rows], "swiglu_packed"),
            "w3": ([(self.gl.rows(r.start, r.stop), pw[f"{s}.w3"][L], w[f"{s}.w3.b"][L], self.x[r], self.x[r])
                    for s, r in rows], "residual"),
        }

    # -- one block -----------------------------------------------------------
    def _block(self, L: int) -> None:
        cfg, w = self.cfg, self.w
        gemm = self._gemms(L)
        ln = cfg.eps if self.ln_fold else None
        if not self.ln_fold:
            Fn.layernorm_pack(self.x, cfg.eps, out=self.h)
        specs = [
            Fn.StreamSpec(self.qkv[cfg.rows("vl")], w["vl.q_norm"][L], w["vl.k_norm"][L]),
            Fn.StreamSpec(self.qkv[cfg.rows("sa")], w["sa.q_norm"][L], w["sa.k_norm"][L],
                          self.inp["sa_cos"], self.inp["sa_sin"]),
            Fn.StreamSpec(self.qkv[cfg.rows("p")], w["p.q_norm"][L], w["p.k_norm"][L],
                          self.inp["p_cos"], self.inp["p_sin"]),
        ]
        st = self._stats() if self.ln_fold else None
        if self.fused_qkv:
            items = [(a, wt, b) for a, wt, b, _, _ in gemm["qkv"][0]]
            Fn.grouped_gemm_qkv_norm_rope(items, specs, cfg.heads, cfg.head_dim, cfg.eps, out=(self.q, self.kvp),
                                          ln_eps=ln, ln_stats=st)
        else:
            Fn.grouped_gemm(*gemm["qkv"], ln_eps=ln, ln_stats=st)
            Fn.msat_qkv_norm_rope(specs, cfg.heads, cfg.head_dim, cfg.eps, out=(self.q, self.kvp), kv_packed=True)
        warm = [self.pw[f"{s}.w3"][L].data for s in self.warm_w3]
        Fn.attention_packed(self.q.unsqueeze(0), self.kvp.unsqueeze(0), cfg.tokens, key_bias=self.inp["key_bias"],
                            out=self.att, warm=warm)
        Fn.grouped_gemm(*gemm["proj"], stats_out=st)
        if not self.ln_fold:
            Fn.layernorm_pack(self.x, cfg.eps, out=self.h)
        Fn.grouped_gemm(*gemm["w12"], ln_eps=ln, ln_stats=st)
        Fn.grouped_gemm(*gemm["w3"], stats_out=st)

    # -- one action step ------------------------------------------------------
    def run(self, steps: int | None = None, blocks: int | None = None) -> torch.Tensor:
        """Launch one action step (optionally truncated to `steps` iterations of
        `blocks` blocks, for parity tests) on the current stream."""
        cfg, w, inp = self.cfg, self.w, self.inp
        steps = cfg.steps if steps is None else steps
        blocks = cfg.blocks if blocks is None else blocks
        sa = cfg.rows("sa")
        self.act.copy_(inp["x0"])
        dt = 1.0 / cfg.steps
        if self.ln_fold:  # the VL and P rows of the staging buffer stay as they are
            self.x[cfg.rows("vl")].copy_(inp["vl"])
            self.x[cfg.rows("p")].copy_(inp["p"])
        for t in range(steps):
            if not self.ln_fold:
                self.x[cfg.rows("vl")].copy_(inp["vl"])
                self.x[cfg.rows("p")].copy_(inp["p"])
            if self.fused_io:
                others = [(self.x[cfg.rows(s)], self.xp.rows(cfg.rows(s).start, cfg.rows(s).stop), self.xst[s])
                          for s in ("vl", "p")]
                Fn.action_encode_pack(self.act, w["act_in.w"], w["act_in.b"], inp["temb"][t], inp["pos"],
                                      self.xp.rows(sa.start, sa.stop), self.xst["sa"], others)
            else:
                torch.addmm(w["act_in.b"], self.act, w["act_in.w"].t(), out=self.sa_in)
                self.sa_in.add_(inp["temb"][t])
                torch.add(self.sa_in, inp["pos"], out=self.x[sa])
                if self.ln_fold:
                    for s in STREAMS:
                        r = cfg.rows(s)
                        Fn.pack_act(self.x[r], out=self.xp.rows(r.start, r.stop), stats=self.xst[s])
            for L in range(blocks):
                self._block(L)
            if self.fused_io:
                Fn.action_decode_euler(self.xp.rows(sa.start, sa.stop), w["act_out.w"], w["act_out.b"], self.act, dt,
                                       cfg.eps)
                continue
            x_sa = self.xp.rows(sa.start, sa.stop).unpack() if self.ln_fold else self.x[sa]
            hs = F.layer_norm(x_sa, (cfg.hidden,), eps=cfg.eps)
            torch.addmm(w["act_out.b"], hs, w["act_out.w"].t(), out=self.vel)
            self.vel.mul_(dt)
            self.act.add_(self.vel)
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
