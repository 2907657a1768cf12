"""Committed fixtures: seeded workload inputs are bit-stable (SHA-256) and the
CPU oracle reproduces its recorded output slices."""

import json
from pathlib import Path

import pytest
import torch

from oracle import cpu_reference as ref
from rldx_amd import workloads as W

GOLD = json.loads((Path(__file__).parent / "golden" / "workloads.json").read_text())


def close(vals, gold, tol):
    return max(abs(a - b) for a, b in zip(vals, gold)) <= tol


def test_input_hashes():
    r = W.rmsnorm_rope_inputs()
    assert W.sha256_of(r["q"], r["k"], r["w"], r["cos"], r["sin"]) == GOLD["rmsnorm_rope_f32"]["inputs_sha256"]
    assert W.sha256_of(W.swiglu_inputs(W.SwigluCfg(tokens=64))["x"]) == GOLD["swiglu_64"]["inputs_sha256"]
    j = W.joint_attn_inputs()
    assert W.sha256_of(j["q"], j["k"], j["v"], j["kv_mask"]) == GOLD["joint_attention"]["inputs_sha256"]
    g = W.gqa_inputs()
    assert W.sha256_of(g["qkv"], g["q_norm_w"], g["k_norm_w"], g["cos"], g["sin"]) == GOLD["gqa_prefill"]["inputs_sha256"]


def test_oracle_output_slices():
    r = W.rmsnorm_rope_inputs()
    q, k = ref.qk_rmsnorm_rope_half(r["q"], r["k"], r["w"], r["w"], r["cos"], r["sin"])
    assert close([float(v) for v in q.flatten()[:16]], GOLD["rmsnorm_rope_f32"]["q_out_head"], 1e-6)
    y = ref.swiglu(W.swiglu_inputs(W.SwigluCfg(tokens=64))["x"])
    assert W.sha256_of(y) == GOLD["swiglu_64"]["out_sha256"]
    j = W.joint_attn_inputs()
    o = ref.sdpa(j["q"], j["k"], j["v"], key_bias=ref.mask_to_bias(j["kv_mask"]))
    assert close([float(v) for v in o.flatten()[:16]], GOLD["joint_attention"]["out_head"], 2e-3)


@pytest.mark.gpu
def test_gpu_matches_golden_slices(dev):
    from rldx_amd import functional as Fn

    y = Fn.swiglu(W.swiglu_inputs(W.SwigluCfg(tokens=64))["x"].to(dev)).cpu()
    assert W.sha256_of(y) == GOLD["swiglu_64"]["out_sha256"]
    j = W.joint_attn_inputs()
    bias = ref.mask_to_bias(j["kv_mask"]).to(dev)
    o = Fn.attention(j["q"].to(dev), j["k"].to(dev), j["v"].to(dev), key_bias=bias).cpu()
    assert close([float(v) for v in o.flatten()[:16]], GOLD["joint_attention"]["out_head"], 2e-2)
    assert close([float(v) for v in o[0, 0, 607]][:16], GOLD["joint_attention"]["out_row607_head"], 2e-2)
