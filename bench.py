"""Benchmark: ms per MSAT action step (batch 1, one MI355X) + kernel roofline fractions.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Workload (value): the synthetic MSAT action step — 16 triple-stream blocks,
hidden 1536, 12 heads x 128, SwiGLU 4096, 512 cognition / 64 action / 32 physics
tokens, 4 Euler denoising iterations, bf16, random-init weights — captured as
one hipGraph; K replays are timed after W warm-up replays.

Kernel lines (roofline): each hand-written kernel at its workload shape is
captured N times back to back into a hipGraph and timed with HIP events on the
launch stream; achieved = algorithmic bytes or flops per launch / mean launch
time.  The step's four grouped GEMMs are timed on the step's own packed
weights, one launch per block (16 weight sets, 1.2-2.9 GB, so every launch
streams its weights from HBM as in the step).  `roofline` is the dominant kernel
of the step: the W12 + SwiGLU grouped GEMM (3 streams x [8192 x 1536] weights),
whose arithmetic intensity (~186 flop/B) puts it under the HBM roof.
`roofline.traffic` is the measured L2-miss bytes per launch of that kernel
(rocprofv3 FETCH_SIZE + WRITE_SIZE, scaled by the same counters' reading for a
copy of known size: bytes the L2s exchange with the memory side, served by the
256 MB MALL or by HBM), read from profiles/gemm_w12_swiglu_traffic.json when
that file is present.  cpu_baseline: the CPU oracle of the same step (torch bf16 on
the host cores).

Profiling helpers (no JSON line):
    python bench.py --profile-kernel w12    # the dominant kernel alone, 4 x 16 launches
    python bench.py --copy-calibration      # one 256 MiB device copy, 4 times
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "rldx-1_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--kernel-reps", type=int, default=50)
    ap.add_argument("--profile-kernel", choices=["qkv", "proj", "w12", "w3"] + list(PROFILE_KERNELS), default=None,
                    help="run one kernel alone, 64 launches (for counter passes), and exit")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a 256 MiB device-to-device copy 4 times (traffic counter calibration) and exit")
    return ap.parse_args()


PROFILE_KERNELS = ("joint_attn", "gqa_attn", "gqa_op", "gqa_op_169", "step_attn", "vit_attn", "mem_attn", "swiglu",
                   "rmsnorm_rope", "rmsnorm_rope_64k", "res_ln", "vl_ln", "add2_rmsnorm")


def profile_launch(name: str, torch):
    """A zero-argument launcher of one kernel at its workload shape, for counter
    passes (inputs built once; every call is one launch of the kernel under test,
    plus the K-side launch of the backbone operator for gqa_op)."""
    from rldx_amd import functional as Fn
    from rldx_amd import workloads as W
    from rldx_amd.msat_step import MsatStepCfg

    dev = torch.device("cuda:0")
    if name == "swiglu":  # 2048 x 11008
        x = W.swiglu_inputs(W.SwigluCfg())["x"].to(dev)
        y = torch.empty(x.shape[0], x.shape[1] // 2, dtype=torch.bfloat16, device=dev)
        return lambda: Fn.swiglu(x, out=y)
    if name in ("rmsnorm_rope", "rmsnorm_rope_64k"):  # fp32 16384 (or 65536) x 16 x 64, the HBM-bound sweep points
        rs = W.RmsRopeCfg(seq=65536 if name == "rmsnorm_rope_64k" else 16384)
        shape = (rs.batch, rs.seq, rs.heads, rs.head_dim)
        q, k = torch.randn(shape, device=dev), torch.randn(shape, device=dev)
        cs, sn = (t.to(dev) for t in W.qwen_rope_cos_sin(rs.seq, rs.head_dim, rs.theta))
        w = torch.ones(rs.head_dim, device=dev)
        qo, ko = torch.empty_like(q), torch.empty_like(k)
        return lambda: Fn.qk_rmsnorm_rope_half(q, k, w, w, cs, sn, rs.eps, q_out=qo, k_out=ko)
    if name == "joint_attn":  # 16 x 608 x 128, 8 masked keys
        jc = W.JointAttnCfg()
        ji = W.joint_attn_inputs(jc)
        q, k, v = (ji[n].to(dev) for n in ("q", "k", "v"))
        bias = torch.where(ji["kv_mask"] == 0, float("-inf"), 0.0).float().to(dev)
        o = torch.empty_like(q)
        kvp = Fn.kv_pack(k, v)
        return lambda: Fn.attention_packed(q, kvp, jc.tokens, key_bias=bias, out=o)
    if name == "step_attn":  # 12 x 608 x 128, 8 masked keys
        sc = MsatStepCfg()
        n = sc.tokens
        q, k, v = (torch.randn(1, sc.heads, n, sc.head_dim, device=dev).to(torch.bfloat16) for _ in range(3))
        bias = torch.zeros(n, device=dev)
        bias[n - sc.n_p_pad:] = float("-inf")
        o = torch.empty_like(q)
        kvp = Fn.kv_pack(k, v)
        return lambda: Fn.attention_packed(q, kvp, n, key_bias=bias, out=o)
    if name == "vit_attn":  # 2 x 196 patches, 16 x 72: pack launch + varlen attention
        vc = W.VitAttnCfg()
        vi = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in W.vit_attention_inputs(vc).items()}
        vws = torch.empty(Fn.vision_attention_workspace_bytes(vc.tokens, vc.images, vc.heads, vc.head_dim),
                          dtype=torch.uint8, device=dev)
        vo = torch.empty(vc.tokens, vc.heads * vc.head_dim, dtype=torch.bfloat16, device=dev)
        return lambda: Fn.vision_attention(vi["qkv"], vi["rope_cos"], vi["rope_sin"], vi["cu_seqlens"],
                                           vi["scaling"], vc.heads, vc.head_dim, out=vo, workspace=vws)
    if name == "mem_attn":  # 64 tokens, 16 x 256, block-causal (block 16)
        mc = W.MemAttnCfg()
        mi = W.memory_attention_inputs(mc)
        mq, mcos, msin = mi["qkv"].to(dev), mi["cos"].to(dev), mi["signed_sin"].to(dev)
        mo = torch.empty(mc.tokens, mc.heads * mc.head_dim, dtype=torch.bfloat16, device=dev)
        return lambda: Fn.memory_attention(mq, mcos, msin, mc.heads, mc.head_dim, mc.n_cog, out=mo)
    if name in ("res_ln", "vl_ln", "add2_rmsnorm"):  # the residual-add + norm epilogues of the kernel lines
        def rows(m, d):
            return torch.randn(m, d, device=dev).to(torch.bfloat16)

        if name == "res_ln":
            sr, sp, sb = rows(18, 1536), rows(18, 1536), rows(1, 1536)[0]
            vr, vp, vb = rows(128, 4096), rows(128, 4096), rows(1, 4096)[0]
            return lambda: Fn.fused_grouped_res_ln(sr, sb, sp, vr, vb, vp)
        if name == "vl_ln":
            vr, vp, vb = rows(128, 4096), rows(128, 4096), rows(1, 4096)[0]
            nv, lv = torch.empty_like(vr), torch.empty_like(vr)
            return lambda: Fn.fused_vl_epilogue_ln(vr, vb, vb, vp, new_vl_out=nv, ln_vl_out=lv)
        lh, lr, lw = rows(1280, 2048), rows(1280, 2048), rows(1, 2048)[0]
        return lambda: Fn.fused_add2_rmsnorm(lh, lr, lw)
    gc = W.GqaCfg(q_heads=32, kv_heads=8, seq=169) if name == "gqa_op_169" else W.GqaCfg()
    if name == "gqa_attn":  # causal 28/4 x 1280 x 128 on pre-normalised Q/K
        M, Hq, Hkv, D = gc.seq, gc.q_heads, gc.kv_heads, gc.head_dim
        q = torch.randn(1, M, Hq, D, device=dev).to(torch.bfloat16)
        k = torch.randn(1, M, Hkv, D, device=dev).to(torch.bfloat16)
        v = torch.randn(1, M, Hkv, D, device=dev).to(torch.bfloat16)
        o = torch.empty_like(q)
        kvp = Fn.kv_pack(k, v, layout="bshd")
        return lambda: Fn.attention_packed(q, kvp, M, causal=True, layout="bshd", out=o)
    # gqa_op / gqa_op_169: rldx_backbone::fused_attention (K norm + K/V tiles, then attention with
    # the Q norm) at 28/4 x 1280 x 128 / at the reference backbone's 32/8 x 169 x 128
    import rldx_amd.ops as ops

    gi = W.gqa_inputs(gc)
    args = (gi["qkv"].to(dev), gi["q_norm_w"].to(dev), None, gi["k_norm_w"].to(dev), None, gi["cos"].to(dev),
            W.signed_sin(gi["sin"]).to(dev))
    ob = torch.empty(gc.seq, gc.q_heads * gc.head_dim, dtype=torch.bfloat16, device=dev)
    return lambda: ops.llm_fused_attention(*args, num_heads=gc.q_heads, num_kv_heads=gc.kv_heads,
                                           head_dim=gc.head_dim, out=ob)


def graph_time_ms(fn, reps: int, torch) -> float:
    """Mean duration of one `fn()` launch sequence: `reps` copies captured into a
    hipGraph, replayed, timed with events on the capture/launch stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    best = math.inf
    for _ in range(3):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1) / reps)
    return best


def vendor_sdpa(torch, q, k, v, *, causal=False, mask=None, reps=20):
    """torch.nn.functional.scaled_dot_product_attention on the same bf16 shape
    (B, H, S, D): the library attention a PyTorch-ROCm user gets, timed like the
    kernel lines.  Only the fused backends are tried (flash = AOTriton, then
    memory-efficient), with the same key-padding mask where the line has one;
    `flash_unmasked_us` is the flash backend without the mask (it takes none),
    a lower bound for the library on that shape."""
    import warnings

    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    res = {}
    for name, be in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel([be]), warnings.catch_warnings():
                warnings.simplefilter("ignore")  # the backend's reasons for declining a case
                ms = graph_time_ms(lambda: F.scaled_dot_product_attention(q, k, v, attn_mask=mask,
                                                                          is_causal=causal), reps, torch)
            res.update(us=ms * 1e3, backend=name)
            break
        except RuntimeError:
            continue
    if mask is not None and res.get("backend") != "flash":
        try:
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION]), warnings.catch_warnings():
                warnings.simplefilter("ignore")
                ms = graph_time_ms(lambda: F.scaled_dot_product_attention(q, k, v, is_causal=causal), reps, torch)
            res["flash_unmasked_us"] = ms * 1e3
        except RuntimeError:
            pass
    return res or None


def kernel_lines(torch, reps: int):
    from rldx_amd import functional as Fn
    from rldx_amd import workloads as W
    from rldx_amd.msat_step import MsatStepCfg

    dev = torch.device("cuda:0")
    out = {}

    # SwiGLU 2048 x 11008 (rotate 3 input copies so the 256 MB MALL cannot hold them)
    cfg = W.SwigluCfg()
    x = W.swiglu_inputs(cfg)["x"].to(dev)
    xs = [x] + [x.clone() for _ in range(2)]
    ys = [torch.empty(cfg.tokens, cfg.n_half, dtype=torch.bfloat16, device=dev) for _ in range(3)]
    it = {"i": 0}

    def sw():
        i = it["i"] % 3
        it["i"] += 1
        Fn.swiglu(xs[i], out=ys[i])

    ms = graph_time_ms(sw, 30, torch)
    gbs = W.swiglu_bytes(cfg) / (ms * 1e-3) / 1e9
    out["swiglu_2048x11008"] = dict(us=ms * 1e3, achieved=gbs, unit="GB/s", bound="hbm", peak=HBM_PEAK_GBS,
                                    frac=gbs / HBM_PEAK_GBS, bytes=W.swiglu_bytes(cfg))
    del xs, ys, x
    cfg64 = W.SwigluCfg(tokens=64)
    x64 = W.swiglu_inputs(cfg64)["x"].to(dev)
    y64 = torch.empty(64, cfg64.n_half, dtype=torch.bfloat16, device=dev)
    ms = graph_time_ms(lambda: Fn.swiglu(x64, out=y64), reps, torch)
    gbs = W.swiglu_bytes(cfg64) / (ms * 1e-3) / 1e9
    out["swiglu_64x11008"] = dict(us=ms * 1e3, achieved=gbs, unit="GB/s", bound="hbm", peak=HBM_PEAK_GBS,
                                  frac=gbs / HBM_PEAK_GBS, bytes=W.swiglu_bytes(cfg64))

    # RMSNorm + rotate-half RoPE, fp32, q/k [1, 256, 16, 64]
    rc = W.RmsRopeCfg()
    ri = {k: v.to(dev) for k, v in W.rmsnorm_rope_inputs(rc).items()}
    qo = torch.empty_like(ri["q"])
    ko = torch.empty_like(ri["k"])
    ms = graph_time_ms(lambda: Fn.qk_rmsnorm_rope_half(ri["q"], ri["k"], ri["w"], ri["w"], ri["cos"], ri["sin"],
                                                       rc.eps, q_out=qo, k_out=ko), reps, torch)
    gbs = W.rmsnorm_rope_bytes(rc) / (ms * 1e-3) / 1e9
    out["rmsnorm_rope_f32_256x16x64"] = dict(us=ms * 1e3, achieved=gbs, unit="GB/s", bound="hbm", peak=HBM_PEAK_GBS,
                                             frac=gbs / HBM_PEAK_GBS, bytes=W.rmsnorm_rope_bytes(rc))
    # the same kernel on long sequences (the 256-token case above is launch-bound)
    for seq in (16384, 65536):
        rs = W.RmsRopeCfg(seq=seq)
        shape = (rs.batch, rs.seq, rs.heads, rs.head_dim)
        qs_, ks_ = torch.randn(shape, device=dev), torch.randn(shape, device=dev)
        cs_, sn_ = (t.to(dev) for t in W.qwen_rope_cos_sin(rs.seq, rs.head_dim, rs.theta))
        ws_ = ri["w"]
        qo_, ko_ = torch.empty_like(qs_), torch.empty_like(ks_)
        ms = graph_time_ms(lambda: Fn.qk_rmsnorm_rope_half(qs_, ks_, ws_, ws_, cs_, sn_, rs.eps, q_out=qo_, k_out=ko_),
                           reps, torch)
        gbs = W.rmsnorm_rope_bytes(rs) / (ms * 1e-3) / 1e9
        out[f"rmsnorm_rope_f32_{seq}x16x64"] = dict(us=ms * 1e3, achieved=gbs, unit="GB/s", bound="hbm",
                                                    peak=HBM_PEAK_GBS, frac=gbs / HBM_PEAK_GBS,
                                                    bytes=W.rmsnorm_rope_bytes(rs))
        del qs_, ks_, qo_, ko_

    # MSAT joint attention 16 x 608 x 128, masked
    jc = W.JointAttnCfg()
    ji = W.joint_attn_inputs(jc)
    q, k, v = (ji[n].to(dev) for n in ("q", "k", "v"))
    bias = torch.where(ji["kv_mask"] == 0, float("-inf"), 0.0).float().to(dev)
    o = torch.empty_like(q)
    kvp = Fn.kv_pack(k, v)  # packed K/V tiles, as the MSAT QKV kernel produces them
    ms = graph_time_ms(lambda: Fn.attention_packed(q, kvp, jc.tokens, key_bias=bias, out=o), reps, torch)
    tf = W.joint_attn_flops(jc) / (ms * 1e-3) / 1e12
    out["joint_attention_16x608x128"] = dict(us=ms * 1e3, achieved=tf, unit="TFLOP/s", bound="mfma",
                                              peak=BF16_MFMA_PEAK_TFLOPS, frac=tf / BF16_MFMA_PEAK_TFLOPS,
                                              flops=W.joint_attn_flops(jc))
    sdpa_mask = bias.to(torch.bfloat16).view(1, 1, 1, -1).expand(1, 1, jc.tokens, jc.tokens).contiguous()
    out["joint_attention_16x608x128"]["vendor_sdpa"] = vendor_sdpa(torch, q, k, v, mask=sdpa_mask)
    ms = graph_time_ms(lambda: Fn.attention(q, k, v, key_bias=bias, out=o), reps, torch)
    tf = W.joint_attn_flops(jc) / (ms * 1e-3) / 1e12
    out["joint_attention_16x608x128_with_kv_pack"] = dict(us=ms * 1e3, achieved=tf, unit="TFLOP/s",
                                                               bound="mfma", peak=BF16_MFMA_PEAK_TFLOPS,
                                                               frac=tf / BF16_MFMA_PEAK_TFLOPS,
                                                               flops=W.joint_attn_flops(jc))

    # GQA causal prefill 28/4 x 1280 x 128 (rldx_backbone::fused_attention: prologue + attention)
    import rldx_amd.ops as ops

    gc = W.GqaCfg()
    gi = W.gqa_inputs(gc)
    qkv = gi["qkv"].to(dev)
    args = (qkv, gi["q_norm_w"].to(dev), None, gi["k_norm_w"].to(dev), None, gi["cos"].to(dev),
            W.signed_sin(gi["sin"]).to(dev))
    ob = torch.empty(gc.seq, gc.q_heads * gc.head_dim, dtype=torch.bfloat16, device=dev)
    ms = graph_time_ms(lambda: ops.llm_fused_attention(*args, num_heads=gc.q_heads, num_kv_heads=gc.kv_heads,
                                                       head_dim=gc.head_dim, out=ob), reps, torch)
    tf = W.gqa_flops(gc) / (ms * 1e-3) / 1e12
    out["gqa_prefill_op_28x4x1280x128"] = dict(us=ms * 1e3, achieved=tf, unit="TFLOP/s", bound="mfma",
                                               peak=BF16_MFMA_PEAK_TFLOPS, frac=tf / BF16_MFMA_PEAK_TFLOPS,
                                               flops=W.gqa_flops(gc))
    # the same operator at the reference backbone's own attention shape: 32 / 8 heads x 128, 169 tokens
    # (rldx/inference/backbone/llm/engine/kernels/fused_llm_attention.py:14, rldx/inference/backbone/README.md:5)
    gs = W.GqaCfg(q_heads=32, kv_heads=8, seq=169)
    gsi = W.gqa_inputs(gs)
    sargs = (gsi["qkv"].to(dev), gsi["q_norm_w"].to(dev), None, gsi["k_norm_w"].to(dev), None, gsi["cos"].to(dev),
             W.signed_sin(gsi["sin"]).to(dev))
    osb = torch.empty(gs.seq, gs.q_heads * gs.head_dim, dtype=torch.bfloat16, device=dev)
    ms = graph_time_ms(lambda: ops.llm_fused_attention(*sargs, num_heads=gs.q_heads, num_kv_heads=gs.kv_heads,
                                                       head_dim=gs.head_dim, out=osb), reps, torch)
    tf = W.gqa_flops(gs) / (ms * 1e-3) / 1e12
    out["gqa_prefill_op_32x8x169x128"] = dict(us=ms * 1e3, achieved=tf, unit="TFLOP/s", bound="mfma",
                                              peak=BF16_MFMA_PEAK_TFLOPS, frac=tf / BF16_MFMA_PEAK_TFLOPS,
                                              flops=W.gqa_flops(gs))
    # attention kernel alone on pre-normalised Q/K
    M, Hq, Hkv, D = gc.seq, gc.q_heads, gc.kv_heads, gc.head_dim
    qn = torch.randn(1, M, Hq, D, device=dev).to(torch.bfloat16)
    kn = torch.randn(1, M, Hkv, D, device=dev).to(torch.bfloat16)
    vn = torch.randn(1, M, Hkv, D, device=dev).to(torch.bfloat16)
    on = torch.empty_like(qn)
    kvpn = Fn.kv_pack(kn, vn, layout="bshd")
    ms = graph_time_ms(lambda: Fn.attention_packed(qn, kvpn, M, causal=True, layout="bshd", out=on), reps, torch)
    tf = W.gqa_flops(gc) / (ms * 1e-3) / 1e12
    out["gqa_attention_28x4x1280x128"] = dict(us=ms * 1e3, achieved=tf, unit="TFLOP/s", bound="mfma",
                                              peak=BF16_MFMA_PEAK_TFLOPS, frac=tf / BF16_MFMA_PEAK_TFLOPS,
                                              flops=W.gqa_flops(gc))
    g = Hq // Hkv  # the library kernels take K / V expanded to the query heads
    out["gqa_attention_28x4x1280x128"]["vendor_sdpa"] = vendor_sdpa(
        torch, qn.transpose(1, 2), kn.repeat_interleave(g, dim=2).transpose(1, 2).contiguous(),
        vn.repeat_interleave(g, dim=2).transpose(1, 2).contiguous(), causal=True)

    # the step's own attention shape: 12 x 608 x 128, masked
    sc = MsatStepCfg()
    n = sc.tokens
    qs = torch.randn(1, sc.heads, n, sc.head_dim, device=dev).to(torch.bfloat16)
    ks = torch.randn(1, sc.heads, n, sc.head_dim, device=dev).to(torch.bfloat16)
    vs = torch.randn(1, sc.heads, n, sc.head_dim, device=dev).to(torch.bfloat16)
    bs = torch.zeros(n, device=dev)
    bs[n - sc.n_p_pad:] = float("-inf")
    os_ = torch.empty_like(qs)
    kvps = Fn.kv_pack(ks, vs)
    ms = graph_time_ms(lambda: Fn.attention_packed(qs, kvps, n, key_bias=bs, out=os_), reps, torch)
    fl = 4 * sc.heads * n * n * sc.head_dim
    tf = fl / (ms * 1e-3) / 1e12
    out["step_joint_attention_12x608x128"] = dict(us=ms * 1e3, achieved=tf, unit="TFLOP/s", bound="mfma",
                                                  peak=BF16_MFMA_PEAK_TFLOPS, frac=tf / BF16_MFMA_PEAK_TFLOPS,
                                                  flops=fl)
    out["step_joint_attention_12x608x128"]["vendor_sdpa"] = vendor_sdpa(
        torch, qs, ks, vs, mask=bs.to(torch.bfloat16).view(1, 1, 1, -1).expand(1, 1, n, n).contiguous())

    # ViT attention, 2 images x 196 patches, 16 heads x 72 (RoPE + K/V packing + varlen attention)
    vc = W.VitAttnCfg()
    vi = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in W.vit_attention_inputs(vc).items()}
    vws = torch.empty(Fn.vision_attention_workspace_bytes(vc.tokens, vc.images, vc.heads, vc.head_dim),
                      dtype=torch.uint8, device=dev)
    vo = torch.empty(vc.tokens, vc.heads * vc.head_dim, dtype=torch.bfloat16, device=dev)
    ms = graph_time_ms(lambda: Fn.vision_attention(vi["qkv"], vi["rope_cos"], vi["rope_sin"], vi["cu_seqlens"],
                                                   vi["scaling"], vc.heads, vc.head_dim, out=vo, workspace=vws),
                       reps, torch)
    tf = W.vit_attention_flops(vc) / (ms * 1e-3) / 1e12
    out["vit_attention_op_2x196_16x72"] = dict(us=ms * 1e3, achieved=tf, unit="TFLOP/s", bound="mfma",
                                               peak=BF16_MFMA_PEAK_TFLOPS, frac=tf / BF16_MFMA_PEAK_TFLOPS,
                                               flops=W.vit_attention_flops(vc))
    # TransformerMemory attention, 4 x 16 tokens, 16 heads x 256, block-causal (block 16)
    mc = W.MemAttnCfg()
    mi = W.memory_attention_inputs(mc)
    mq, mcos, msin = mi["qkv"].to(dev), mi["cos"].to(dev), mi["signed_sin"].to(dev)
    mo = torch.empty(mc.tokens, mc.heads * mc.head_dim, dtype=torch.bfloat16, device=dev)
    ms = graph_time_ms(lambda: Fn.memory_attention(mq, mcos, msin, mc.heads, mc.head_dim, mc.n_cog, out=mo),
                       reps, torch)
    tf = W.memory_attention_flops(mc) / (ms * 1e-3) / 1e12
    out["memory_attention_op_64_16x256_block16"] = dict(us=ms * 1e3, achieved=tf, unit="TFLOP/s", bound="mfma",
                                                        peak=BF16_MFMA_PEAK_TFLOPS, frac=tf / BF16_MFMA_PEAK_TFLOPS,
                                                        flops=W.memory_attention_flops(mc))

    # RLDX-1 action head at the release MSAT shape (24 x 64 heads, 4 DS + 8 SS blocks, SA 1536,
    # VL 4096, 64 + 18 tokens): state encoder + 4 x (action encoder, MSAT, decoder, Euler), one hipGraph
    from rldx_amd import rldx_msat as RM

    rmc, rhc = RM.RldxMsatCfg(), RM.RldxHeadCfg()
    rhead = RM.RldxActionHead(RM.RldxMsat(RM.make_state_dict(rmc, dev), rmc, dev),
                              RM.make_head_state_dict(rmc, rhc, dev), rhc)
    gr = torch.Generator(device=dev).manual_seed(14)
    for t in (rhead.vl, rhead.state, rhead.x0):
        t.copy_(torch.randn(t.shape, generator=gr, device=dev))
    ms = graph_time_ms(rhead.run, 1, torch)
    msat_ms = graph_time_ms(lambda: rhead.msat.forward(rhead.sa, rhead.vl, rhead.sd["static_tembs"][0],
                                                       rhead.sd["static_time_tokens"][0]), 4, torch)
    out["rldx_action_head_release_shape"] = dict(
        ms=ms, msat_forward_ms=msat_ms, unit="ms per action (4 denoising steps)",
        reference_published_ms=9.66, reference_hardware="RTX 5090, path D (rldx/inference/action_model/README.md:11-18)",
        msat_params=sum(torch.Size(s_).numel() for s_ in rmc.param_shapes().values()))
    # four robots at once (for_batch: the same packed weights, one graph; the GEMMs cover the batch)
    rhead4 = rhead.for_batch(4)
    for t in (rhead4.vl, rhead4.state, rhead4.x0):
        t.copy_(torch.randn(t.shape, generator=gr, device=dev))
    rhead4.set_embodiment([e % rhc.num_embodiments for e in range(4)])
    ms4 = graph_time_ms(rhead4.run, 1, torch)
    out["rldx_action_head_release_shape_4_robots"] = dict(
        ms=ms4, ms_per_robot=ms4 / 4, batch1_ms=ms, unit="ms per call of 4 robots (4 denoising steps each)")
    del rhead, rhead4

    # the same head with all add-ons: Expanded blocks with the physics stream, N_vl = 80 (cognition +
    # memory tokens), 1 + 16 physics tokens of 37 signals (30 tactile + 7 torque), physics encoders and decoder
    rhc = RM.RldxHeadCfg(physics_dim=37, physics_hist_len=1)
    rmc = RM.RldxMsatCfg(n_vl=80, use_physics=True, n_physics=rhc.physics_hist_len + rhc.physics_fut_len)
    rhead = RM.RldxActionHead(RM.RldxMsat(RM.make_state_dict(rmc, dev), rmc, dev),
                              RM.make_head_state_dict(rmc, rhc, dev), rhc)
    for t in (rhead.vl, rhead.state, rhead.x0, rhead.physics_hist, rhead.physics_x0):
        t.copy_(torch.randn(t.shape, generator=gr, device=dev))
    ms = graph_time_ms(rhead.run, 1, torch)
    msat_ms = graph_time_ms(lambda: rhead.msat.forward(rhead.sa, rhead.vl, rhead.sd["static_tembs"][0],
                                                       rhead.sd["static_time_tokens"][0],
                                                       physics_embs=rhead.p_embs), 4, torch)
    out["rldx_action_head_all_add_ons"] = dict(
        ms=ms, msat_forward_ms=msat_ms, unit="ms per action (4 denoising steps)",
        reference_published_ms=10.25, reference_hardware="RTX 5090, path D (rldx/inference/action_model/README.md:28-37)",
        msat_params=sum(torch.Size(s_).numel() for s_ in rmc.param_shapes().values()), n_vl=80,
        physics_tokens=rmc.n_physics)
    del rhead

    # residual-add + norm epilogues: the reference's block-boundary shapes (launch-bound)
    # and the Qwen3-VL prefill shape 1280 x 2048 (HBM-bound)
    def rows(m, d, std=1.0):
        return (std * torch.randn(m, d, device=dev)).to(torch.bfloat16)

    def hbm_line(name, fn, nbytes):
        t = graph_time_ms(fn, reps, torch)
        g = nbytes / (t * 1e-3) / 1e9
        out[name] = dict(us=t * 1e3, achieved=g, unit="GB/s", bound="hbm", peak=HBM_PEAK_GBS, frac=g / HBM_PEAK_GBS,
                         bytes=nbytes)

    sr, sp, sb = rows(18, 1536), rows(18, 1536), rows(1, 1536)[0]
    vr, vp, vb = rows(128, 4096), rows(128, 4096), rows(1, 4096)[0]
    hbm_line("grouped_res_ln_18x1536+128x4096",
             lambda: Fn.fused_grouped_res_ln(sr, sb, sp, vr, vb, vp),
             3 * 2 * (18 * 1536 + 128 * 4096) + 2 * (1536 + 4096))
    nv, lv = torch.empty_like(vr), torch.empty_like(vr)
    hbm_line("vl_epilogue_ln_128x4096",
             lambda: Fn.fused_vl_epilogue_ln(vr, vb, vb, vp, new_vl_out=nv, ln_vl_out=lv),
             4 * 2 * 128 * 4096 + 2 * 2 * 4096)
    lh, lr, lw = rows(1280, 2048), rows(1280, 2048), rows(1, 2048)[0]
    hbm_line("add2_rmsnorm_1280x2048", lambda: Fn.fused_add2_rmsnorm(lh, lr, lw), 4 * 2 * 1280 * 2048 + 2 * 2048)
    return out


def step_gemms(step, pw=None):
    """The four grouped-GEMM launches of a block of `step`, as {name: (launch(L), flops, bytes)}:
    algorithmic flops and HBM bytes (weights + biases of the 3 streams, activations
    in, outputs out, residual in) of one launch.  pw: packed weights to use instead
    of the step's (a dict with the same keys, e.g. copies of them)."""
    from rldx_amd import functional as Fn

    cfg, w = step.cfg, step.w
    pw = step.pw if pw is None else pw
    n, d, inner, ffn = cfg.tokens, cfg.hidden, cfg.inner, cfg.ffn
    rows = [(s, cfg.rows(s)) for s in ("vl", "sa", "p")]

    fold = step.ln_fold  # the pre-LayerNorm folded into QKV / W12, the residual stream packed (as in the step)
    a_in = step.xp if fold else step.h
    st = step._stats() if fold else None
    ln = cfg.eps if fold else None

    def qkv(L):  # with the QK-norm / RoPE / K/V-tile epilogue, as in the step
        specs = [Fn.StreamSpec(None, w[f"{s}.q_norm"][L], w[f"{s}.k_norm"][L],
                               *((step.inp[f"{s}_cos"], step.inp[f"{s}_sin"]) if s != "vl" else ())) for s, _ in rows]
        Fn.grouped_gemm_qkv_norm_rope([(a_in.rows(r.start, r.stop), pw[f"{s}.qkv"][L], w[f"{s}.qkv.b"][L])
                                       for s, r in rows], specs, cfg.heads, cfg.head_dim, cfg.eps,
                                      out=(step.q, step.kvp), ln_eps=ln, ln_stats=st)

    def res_items(a, name, L):
        if fold:
            return [(a.rows(r.start, r.stop), pw[f"{s}.{name}"][L], w[f"{s}.{name}.b"][L],
                     step.xp.rows(r.start, r.stop), step.xp.rows(r.start, r.stop)) for s, r in rows]
        return [(a.rows(r.start, r.stop), pw[f"{s}.{name}"][L], w[f"{s}.{name}.b"][L], step.x[r], step.x[r])
                for s, r in rows]

    def proj(L):
        Fn.grouped_gemm(res_items(step.att, "proj", L), "residual_packed" if fold else "residual", stats_out=st)

    def w12(L):
        Fn.grouped_gemm([(a_in.rows(r.start, r.stop), pw[f"{s}.w12"][L], w[f"{s}.w12.b"][L],
                          step.gl.rows(r.start, r.stop), None) for s, r in rows], "swiglu_packed",
                        ln_eps=ln, ln_stats=st)

    def w3(L):
        Fn.grouped_gemm(res_items(step.gl, "w3", L), "residual_packed" if fold else "residual", stats_out=st)

    def cost(nn, k, n_out, residual):
        flops = 2 * n * nn * k
        byts = 2 * (3 * (nn * k + nn) + n * k + n * n_out + (n * n_out if residual else 0))
        return flops, byts

    return {
        "qkv": (qkv, *cost(3 * inner, d, 3 * inner, False)),
        "proj": (proj, *cost(d, inner, d, True)),
        "w12": (w12, *cost(2 * ffn, d, ffn, False)),
        "w3": (w3, *cost(d, ffn, d, True)),
    }


# The memory-side cache (MALL) holds 256 MB: a GEMM line cycles through at least this many bytes of weights,
# so that every launch streams its weights from HBM as it does in the action step.
WEIGHT_CYCLE_BYTES = 768 << 20


def gemm_lines(torch, step) -> dict:
    """Mean launch time of each grouped GEMM over the 16 blocks' weights, repeated with
    copies of them until a graph of launches cycles through WEIGHT_CYCLE_BYTES (the
    Proj weights of the 16 blocks, 227 MB, would otherwise stay in the MALL)."""
    from rldx_amd import functional as Fn

    out = {}
    blocks = step.cfg.blocks
    for name, (fn, flops, byts) in step_gemms(step).items():
        keys = [f"{s}.{name}" for s in ("vl", "sa", "p")]
        wbytes = sum(step.pw[k][0].data.numel() * 2 for k in keys)
        sets = -(-WEIGHT_CYCLE_BYTES // (wbytes * blocks))
        fns = [fn]
        for _ in range(1, sets):
            alt = dict(step.pw)
            for k in keys:
                alt[k] = [Fn.PackedWeight(p.data.clone(), p.n, p.k, p.swiglu_pairs, p.row_sums) for p in step.pw[k]]
            fns.append(step_gemms(step, alt)[name][0])
        it = {"L": 0}

        def run():
            fns[(it["L"] // blocks) % sets](it["L"] % blocks)
            it["L"] += 1

        ms = graph_time_ms(run, blocks * sets, torch)
        t = ms * 1e-3
        roof_t = max(flops / (BF16_MFMA_PEAK_TFLOPS * 1e12), byts / (HBM_PEAK_GBS * 1e9))
        bound = "hbm" if byts / (HBM_PEAK_GBS * 1e9) >= flops / (BF16_MFMA_PEAK_TFLOPS * 1e12) else "mfma"
        out[f"gemm_{name}"] = dict(us=ms * 1e3, flops=flops, bytes=byts, tflops=flops / t / 1e12,
                                   gbs=byts / t / 1e9, bound=bound, roofline_us=roof_t * 1e6, frac=roof_t / t,
                                   weight_sets=sets, weight_cycle_mb=wbytes * blocks * sets / 1e6)
        del fns
    return out


def host_info(torch) -> dict:
    """The host the CPU legs ran on: CPU model, logical cores, torch threads used."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(cpu_model=model, logical_cores=os.cpu_count(), torch_threads=torch.get_num_threads())


def _median_ms(fn, reps: int) -> float:
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    ts.sort()
    return ts[len(ts) // 2]


def cpu_kernel_baselines(torch) -> dict:
    """The CPU oracle of configs 1-4 (the eager formulas in torch on the host
    cores, the same seeded inputs as the GPU lines): 3 warm-ups, median of 10
    runs (5 for the GQA prefill).  Reported beside the GPU lines, never a gate."""
    from oracle import cpu_reference as ref
    from rldx_amd import workloads as W

    cores = min(os.cpu_count() or 1, 64)
    torch.set_num_threads(cores)
    out = {}

    def leg(name, fn, inputs, reps=10):
        for _ in range(3):
            fn()
        out[name] = dict(ms=_median_ms(fn, reps), cores=torch.get_num_threads(), kind="port",
                         inputs_sha256=W.sha256_of(*inputs))

    rc = W.RmsRopeCfg()
    ri = W.rmsnorm_rope_inputs(rc)
    # the hashed tensor sets are those of tests/golden/workloads.json, so the two can be cross-checked
    leg("rmsnorm_rope_f32_256x16x64",
        lambda: ref.qk_rmsnorm_rope_half(ri["q"], ri["k"], ri["w"], ri["w"], ri["cos"], ri["sin"], rc.eps),
        [ri["q"], ri["k"], ri["w"], ri["cos"], ri["sin"]])
    sx = W.swiglu_inputs(W.SwigluCfg())["x"]
    leg("swiglu_2048x11008", lambda: ref.swiglu(sx), [sx])
    jc = W.JointAttnCfg()
    ji = W.joint_attn_inputs(jc)
    jb = ref.mask_to_bias(ji["kv_mask"])
    leg("joint_attention_16x608x128", lambda: ref.sdpa(ji["q"], ji["k"], ji["v"], key_bias=jb),
        [ji["q"], ji["k"], ji["v"], ji["kv_mask"]])
    gc = W.GqaCfg()
    gi = W.gqa_inputs(gc)
    leg("gqa_prefill_op_28x4x1280x128",
        lambda: ref.llm_fused_attention(gi["qkv"], gi["q_norm_w"], gi["k_norm_w"], gi["cos"], gi["sin"], gc.q_heads,
                                        gc.kv_heads, gc.head_dim),
        [gi["qkv"], gi["q_norm_w"], gi["k_norm_w"], gi["cos"], gi["sin"]], reps=5)
    gs = W.GqaCfg(q_heads=32, kv_heads=8, seq=169)
    gsi = W.gqa_inputs(gs)
    leg("gqa_prefill_op_32x8x169x128",
        lambda: ref.llm_fused_attention(gsi["qkv"], gsi["q_norm_w"], gsi["k_norm_w"], gsi["cos"], gsi["sin"],
                                        gs.q_heads, gs.kv_heads, gs.head_dim),
        [gsi["qkv"], gsi["q_norm_w"], gsi["k_norm_w"], gsi["cos"], gsi["sin"]])
    return out


def read_probe_gbs(torch, nbytes: int = 512 << 20, copies: int = 3, reps: int = 8) -> float:
    """HBM read rate of the library's streaming read kernel (rldx_read_probe:
    16-byte loads, 8 in flight per thread, one workgroup per CU, nothing written),
    over `copies` rotated buffers of `nbytes` so the 256 MB MALL cannot hold
    them; graph-timed like the kernel lines."""
    from rldx_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    bufs = [torch.ones(nbytes // 2, dtype=torch.bfloat16, device=dev) for _ in range(copies)]
    words = lib.rldx_read_probe_sink_words()
    sink = torch.zeros(words, dtype=torch.int32, device=dev)
    it = {"i": 0}

    def run():
        b = bufs[it["i"] % copies]
        it["i"] += 1
        _lib.check(lib.rldx_read_probe(b.data_ptr(), nbytes, sink.data_ptr(), words,
                                       torch.cuda.current_stream().cuda_stream), "rldx_read_probe")

    ms = graph_time_ms(run, reps * copies, torch)
    del bufs
    return nbytes / (ms * 1e-3) / 1e9


def measured_peaks(torch) -> dict:
    """Peaks measured on this GPU, beside the published ones: device-to-device
    copy bandwidth (1 GiB, read + write bytes), the HBM read rate of a plain
    streaming read kernel (3 rotated 512 MiB buffers, `read_probe_gbs`), and the
    bf16 MFMA throughput of a library GEMM (torch.matmul 8192 x 8192 x 8192,
    hipBLASLt)."""
    dev = torch.device("cuda:0")
    a = torch.empty(512 << 20, dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(a)
    ms = graph_time_ms(lambda: b.copy_(a), 8, torch)
    copy_gbs = 2 * a.numel() * 2 / (ms * 1e-3) / 1e9
    del a, b
    read_gbs = read_probe_gbs(torch)
    n = 8192
    x = torch.randn(n, n, device=dev).to(torch.bfloat16)
    y = torch.randn(n, n, device=dev).to(torch.bfloat16)
    z = torch.empty(n, n, dtype=torch.bfloat16, device=dev)
    ms = graph_time_ms(lambda: torch.matmul(x, y, out=z), 8, torch)
    tflops = 2 * n ** 3 / (ms * 1e-3) / 1e12
    return dict(copy_gbs=copy_gbs, read_gbs=read_gbs, stream_gbs=stream_same_bytes(torch, 1 << 30)["gbs"],
                matmul_bf16_tflops=tflops,
                published=dict(hbm_gbs=HBM_PEAK_GBS, bf16_mfma_tflops=BF16_MFMA_PEAK_TFLOPS))


def stream_same_bytes(torch, nbytes: int, reps: int = 8) -> dict:
    """A plain elementwise kernel moving `nbytes` (torch.neg over bf16: half read,
    half written), timed like the kernel lines: the HBM rate that size reaches
    with library code, launch and ramp included.  From 64 MB up, three buffer
    pairs are rotated so the 256 MB MALL cannot hold the working set."""
    dev = torch.device("cuda:0")
    n = max(nbytes // 4, 1)
    copies = 3 if nbytes >= (64 << 20) else 1
    src = [torch.ones(n, dtype=torch.bfloat16, device=dev) for _ in range(copies)]
    dst = [torch.empty_like(src[0]) for _ in range(copies)]
    it = {"i": 0}

    def run():
        i = it["i"] % copies
        it["i"] += 1
        torch.neg(src[i], out=dst[i])

    ms = graph_time_ms(run, reps * copies, torch)
    del src, dst
    return dict(us=ms * 1e3, gbs=4 * n / (ms * 1e-3) / 1e9)


def step_parity(torch, cfg, w, inp, gpu_act, r16=None) -> dict:
    """The action step's parity record, written into the bench line.  The bf16
    bound of the operator configs (max-abs <= 2e-2, rel-L2 <= 1e-2) holds per
    kernel and over 2 blocks; over the full 16 blocks x 4 iterations bf16
    roundings compound in any evaluation order (the eager bf16 oracle itself
    lands ~2.7e-2 max-abs from an fp32 evaluation), so the full step is judged
    against an fp32 evaluation of the same weights and inputs: rel-L2 to it at
    most 1.5x the bf16 oracle's, and cosine to the bf16 oracle >= 0.999."""
    from oracle import msat_step_ref as R

    def cmp(a, b):
        d = a - b
        return dict(max_abs=d.abs().max().item(), rel_l2=(d.norm() / b.norm()).item(),
                    cos=torch.nn.functional.cosine_similarity(a.flatten(), b.flatten(), dim=0).item())

    if r16 is None:
        r16 = R.action_step(cfg, w, inp)
    r32 = R.action_step(cfg, {k: v.float() for k, v in w.items()}, {k: v.float() for k, v in inp.items()})
    out, r16, r32 = gpu_act.detach().cpu().double(), r16.double(), r32.double()
    vs16, vs32, floor = cmp(out, r16), cmp(out, r32), cmp(r16, r32)
    ok = vs32["rel_l2"] <= 1.5 * floor["rel_l2"] and vs16["cos"] >= 0.999
    return dict(vs_bf16_oracle=vs16, vs_fp32=vs32, bf16_oracle_vs_fp32=floor, passed=bool(ok),
                contract="full step: rel-L2 to the fp32 evaluation <= 1.5 x the bf16 oracle's, cos to the bf16 "
                         "oracle >= 0.999 (max-abs 2e-2 is the per-kernel and 2-block bound)")


def cpu_baseline(torch, cfg, weights, inputs, gpu_act=None, budget_s: float = 20.0):
    """Time the CPU oracle step on the host cores; bounded sample, scaled to ms per action step.
    With `gpu_act` (the GPU step's actions on the same inputs) also the step's parity record."""
    from oracle import msat_step_ref as R

    cores = os.cpu_count() or 1
    cores = min(cores, 64)
    torch.set_num_threads(cores)
    w = {k: v.cpu() for k, v in weights.items()}
    inp = {k: v.cpu() for k, v in inputs.items()}
    # one iteration of one block first, to size the sample
    R.action_step(cfg, w, inp, steps=1, blocks=1)
    t0 = time.perf_counter()
    R.action_step(cfg, w, inp, steps=1, blocks=1)
    one = time.perf_counter() - t0
    per_step_est = one * cfg.blocks * cfg.steps
    r16 = None
    if per_step_est <= budget_s / 2:
        reps = max(1, int(budget_s / 2 / max(per_step_est, 1e-3)))
        reps = min(reps, 5)
        t0 = time.perf_counter()
        for _ in range(reps):
            r16 = R.action_step(cfg, w, inp)
        ms = (time.perf_counter() - t0) / reps * 1e3
        sample = f"{reps} full action step(s) ({cfg.blocks} blocks x {cfg.steps} iterations)"
    else:
        blocks = max(1, min(cfg.blocks, int(budget_s / max(one, 1e-3))))
        t0 = time.perf_counter()
        R.action_step(cfg, w, inp, steps=1, blocks=blocks)
        ms = (time.perf_counter() - t0) * cfg.blocks * cfg.steps / blocks * 1e3
        sample = f"1 iteration x {blocks} blocks, scaled x{cfg.blocks * cfg.steps / blocks:.1f} to a full step"
    from rldx_amd import workloads as W

    res = dict(value=ms, unit="ms per MSAT action step", cores=torch.get_num_threads(), kind="port",
               sample=sample + " of the CPU oracle (torch bf16 eager restatement)",
               inputs_sha256=W.sha256_of(*(inp[k] for k in sorted(inp))))
    if gpu_act is not None:
        res["step_parity"] = step_parity(torch, cfg, w, inp, gpu_act, r16)
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the action step is batch-1 single-GPU; multi-GPU would be data parallel over sessions).",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import rldx_amd
    from rldx_amd.msat_step import MsatActionStep, MsatStepCfg, make_inputs, make_weights

    rldx_amd.load()
    dev = torch.device("cuda:0")
    if args.profile_kernel in PROFILE_KERNELS:
        fn = profile_launch(args.profile_kernel, torch)
        for _ in range(64):
            fn()
        torch.cuda.synchronize()
        print(f"[bench] {args.profile_kernel}: 64 launches", file=sys.stderr, flush=True)
        return
    if args.copy_calibration:
        a = torch.empty(128 << 20, dtype=torch.bfloat16, device=dev)
        b = torch.empty_like(a)
        for _ in range(4):
            b.copy_(a)
        torch.cuda.synchronize()
        print("[bench] copied 4 x 256 MiB", file=sys.stderr, flush=True)
        return
    cfg = MsatStepCfg()
    print(f"[bench] building step weights ({cfg.weight_bytes() / 1e9:.2f} GB bf16)", file=sys.stderr, flush=True)
    weights = make_weights(cfg, dev)
    inputs = make_inputs(cfg, dev)
    step = MsatActionStep(cfg, weights, inputs)
    if args.profile_kernel:
        step.run(steps=1, blocks=1)  # fills the activation buffers
        fn = step_gemms(step)[args.profile_kernel][0]
        for _ in range(4):
            for L in range(cfg.blocks):
                fn(L)
        torch.cuda.synchronize()
        print(f"[bench] {args.profile_kernel}: {4 * cfg.blocks} launches", file=sys.stderr, flush=True)
        return
    step.capture()
    print("[bench] graph captured", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        step.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        step.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    act = step.act.clone()  # the replays' actions, for the parity record of the CPU leg
    assert torch.isfinite(act.float()).all(), "non-finite actions"
    print(f"[bench] action step {ms:.3f} ms", file=sys.stderr, flush=True)

    gl = gemm_lines(torch, step)
    kl = kernel_lines(torch, args.kernel_reps)
    kl.update(gl)
    print("[bench] kernel lines done", file=sys.stderr, flush=True)
    dom = gl["gemm_w12"]
    traffic = None
    tf = ROOT / "profiles" / "gemm_w12_swiglu_traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("l2_miss_bytes_per_launch")
    # traffic: L2-miss bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated on a copy):
    # what the L2s fetch from / write to the memory side, served by the MALL or by HBM
    roofline = dict(kernel="gemm_kernel<SWIGLU_PACKED, LN fold>: W12 + SwiGLU grouped GEMM with the pre-LayerNorm "
                           "folded in, 3 streams (512/64/32 rows: 128x128 / 64x64 / 32x64 tiles) x [8192 x 1536] "
                           "weights" if step.ln_fold else
                    "gemm_kernel<SWIGLU_PACKED>: W12 + SwiGLU grouped GEMM, 3 streams "
                    "(512/64/32 rows: 128x128 / 64x64 / 32x64 tiles) x [8192 x 1536] weights",
                    bound="hbm", achieved=dom["gbs"], peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=dom["gbs"] / HBM_PEAK_GBS, traffic=traffic,
                    traffic_kind="L2-miss bytes per launch (MALL + HBM): rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                 "scaled by a device copy of known size",
                    algorithmic_bytes=dom["bytes"],
                    flops=dom["flops"], us=dom["us"])

    peaks = measured_peaks(torch)
    for v in kl.values():  # fractions against the measured peaks as well
        if isinstance(v, dict) and v.get("unit") == "GB/s":
            v["frac_of_measured_copy"] = v["achieved"] / peaks["copy_gbs"]
            v["frac_of_measured_read"] = v["achieved"] / peaks["read_gbs"]
            if "bytes" in v:  # and against a plain elementwise kernel moving the same bytes
                ref = stream_same_bytes(torch, v["bytes"])
                v["stream_same_bytes_us"] = ref["us"]
                v["frac_of_stream_same_bytes"] = ref["us"] / v["us"]
        elif isinstance(v, dict) and v.get("unit") == "TFLOP/s":
            v["frac_of_measured_matmul"] = v["achieved"] / peaks["matmul_bf16_tflops"]
        elif isinstance(v, dict) and "gbs" in v:  # the step GEMMs: weight streaming against the read rate
            v["frac_of_measured_read"] = v["gbs"] / peaks["read_gbs"]
    roofline["frac_of_measured_read"] = dom["gbs"] / peaks["read_gbs"]
    print(f"[bench] measured peaks: copy {peaks['copy_gbs']:.0f} GB/s, read {peaks['read_gbs']:.0f} GB/s, "
          f"stream {peaks['stream_gbs']:.0f} GB/s, "
          f"bf16 matmul {peaks['matmul_bf16_tflops']:.0f} TFLOP/s", file=sys.stderr, flush=True)

    cpu = None
    host = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, cfg, weights, inputs, gpu_act=act)
        print(f"[bench] cpu baseline {cpu['value']:.1f} ms; step parity {cpu['step_parity']}", file=sys.stderr,
              flush=True)
        for name, leg in cpu_kernel_baselines(torch).items():
            kl[name]["cpu"] = leg
            if "us" in kl[name]:
                kl[name]["gpu_speedup_vs_cpu"] = leg["ms"] * 1e3 / kl[name]["us"]
        host = host_info(torch)
        cpu["cpu_model"] = host["cpu_model"]
        print("[bench] cpu kernel baselines done", file=sys.stderr, flush=True)

    line = {
        "metric": "ms per MSAT action step (bs=1, 1 GPU); kernel % HBM/MFMA roofline",
        "value": ms,
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded randn inputs, random-init weights N(0, 0.02))",
        "config": {
            "workload": "msat_action_step",
            "blocks": cfg.blocks, "hidden": cfg.hidden, "heads": cfg.heads, "head_dim": cfg.head_dim,
            "ffn": cfg.ffn, "tokens": {"cognition": cfg.n_vl, "action": cfg.n_sa, "physics": cfg.n_p,
                                       "physics_padded": cfg.n_p_pad},
            "denoise_iterations": cfg.steps, "batch": 1, "graph": "one hipGraph per action step",
            "step_tflop": cfg.flops_per_step() / 1e12, "weight_gb": cfg.weight_bytes() / 1e9,
        },
        "roofline": roofline,
        "measured_peaks": peaks,
        "kernels": kl,
        "cpu_baseline": cpu,
        "host": host,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
