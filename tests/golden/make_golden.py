"""Writes tests/golden/workloads.json: SHA-256 of every seeded workload input and
small slices of the CPU oracle's outputs (the reference ships no golden data for
this path, so these fixtures pin the build's own inputs and oracle across
machines).  Run from the repository root:  python tests/golden/make_golden.py
"""

import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "rldx-1_amd")]

import torch  # noqa: E402

from oracle import cpu_reference as ref  # noqa: E402
from rldx_amd import workloads as W  # noqa: E402


def sl(t, n=16):
    return [float(v) for v in t.detach().float().flatten()[:n]]


def build():
    out = {"torch": torch.__version__}
    r = W.rmsnorm_rope_inputs()
    q, k = ref.qk_rmsnorm_rope_half(r["q"], r["k"], r["w"], r["w"], r["cos"], r["sin"])
    out["rmsnorm_rope_f32"] = {"inputs_sha256": W.sha256_of(r["q"], r["k"], r["w"], r["cos"], r["sin"]),
                               "q_out_head": sl(q), "k_out_tail": sl(k.flatten()[-16:])}
    s = W.swiglu_inputs(W.SwigluCfg(tokens=64))
    y = ref.swiglu(s["x"])
    out["swiglu_64"] = {"inputs_sha256": W.sha256_of(s["x"]), "out_sha256": W.sha256_of(y), "out_head": sl(y)}
    s2 = W.swiglu_inputs()
    out["swiglu_2048"] = {"inputs_sha256": W.sha256_of(s2["x"])}
    j = W.joint_attn_inputs()
    o = ref.sdpa(j["q"], j["k"], j["v"], key_bias=ref.mask_to_bias(j["kv_mask"]))
    out["joint_attention"] = {"inputs_sha256": W.sha256_of(j["q"], j["k"], j["v"], j["kv_mask"]),
                              "out_head": sl(o), "out_row607_head": sl(o[0, 0, 607])}
    g = W.gqa_inputs()
    og = ref.llm_fused_attention(g["qkv"], g["q_norm_w"], g["k_norm_w"], g["cos"], g["sin"], 28, 4, 128)
    out["gqa_prefill"] = {"inputs_sha256": W.sha256_of(g["qkv"], g["q_norm_w"], g["k_norm_w"], g["cos"], g["sin"]),
                          "out_head": sl(og), "out_last_row_head": sl(og[-1])}
    return out


if __name__ == "__main__":
    path = Path(__file__).with_name("workloads.json")
    path.write_text(json.dumps(build(), indent=1) + "\n")
    print("wrote", path)
