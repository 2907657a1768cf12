"""The allocation-free entry point rldx_llm_fused_attention_noalloc_bf16, called
through the C ABI, against rldx_llm_fused_attention_bf16 (caller workspace) on
the same inputs: bit-identical outputs on two calls in a row, the second with a
smaller input (the scratch array keeps the first call's contents), and calls
issued back to back on two streams, which the library serialises on the device
(they share the scratch array).  The size limit is checked on the host
(tests/test_capi_host.py)."""

import pytest
import torch

from rldx_amd import _lib
from rldx_amd import functional as Fn
from rldx_amd import workloads as W

pytestmark = pytest.mark.gpu


def _inputs(dev, seq, hq, hkv, seed):
    cfg = W.GqaCfg(seq=seq, q_heads=hq, kv_heads=hkv, seed=seed)
    gi = W.gqa_inputs(cfg)
    return cfg, {k: v.to(dev) for k, v in gi.items()}


def _noalloc(lib, gi, cfg, out, stream=None):
    if "ssin" not in gi:
        gi["ssin"] = W.signed_sin(gi["sin"])
    stream = torch.cuda.current_stream() if stream is None else stream
    return lib.rldx_llm_fused_attention_noalloc_bf16(
        gi["qkv"].data_ptr(), gi["qkv"].stride(0), gi["q_norm_w"].data_ptr(), gi["k_norm_w"].data_ptr(),
        gi["cos"].data_ptr(), gi["ssin"].data_ptr(), gi["cos"].stride(0), 1, out.data_ptr(), out.stride(0), cfg.seq,
        cfg.q_heads, cfg.kv_heads, cfg.head_dim, float(cfg.eps), stream.cuda_stream)


def _with_workspace(gi, cfg):
    return Fn.llm_fused_attention(gi["qkv"], gi["q_norm_w"], gi["k_norm_w"], gi["cos"], W.signed_sin(gi["sin"]),
                                  cfg.q_heads, cfg.kv_heads, cfg.head_dim, eps=cfg.eps)


def test_noalloc_matches_workspace_entry_point_on_two_calls(dev):
    lib = _lib.load()
    for seq, hq, hkv, seed in ((1280, 28, 4, 2), (169, 32, 8, 3)):  # the second call is the smaller one
        cfg, gi = _inputs(dev, seq, hq, hkv, seed)
        out = torch.full((seq, hq * cfg.head_dim), float("nan"), dtype=torch.bfloat16, device=dev)
        assert _noalloc(lib, gi, cfg, out) == 0
        ref = _with_workspace(gi, cfg)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"seq {seq}"


def test_noalloc_calls_on_two_streams_are_serialised(dev):
    """Calls issued on two streams without any host synchronisation between them
    share the scratch array; each must still equal the workspace entry point
    bit for bit (the second call's K/V tiles may not overwrite the first's
    while its attention reads them)."""
    lib = _lib.load()
    cases = [_inputs(dev, 1280, 28, 4, 4), _inputs(dev, 1024, 28, 4, 5)]
    for _, gi in cases:
        gi["ssin"] = W.signed_sin(gi["sin"])
    refs = [_with_workspace(gi, cfg) for cfg, gi in cases]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[torch.full((cfg.seq, cfg.q_heads * cfg.head_dim), float("nan"), dtype=torch.bfloat16, device=dev)
             for _ in range(3)] for cfg, _ in cases]
    for r in range(3):
        for i, (cfg, gi) in enumerate(cases):
            assert _noalloc(lib, gi, cfg, outs[i][r], streams[i]) == 0
    torch.cuda.synchronize()
    for i, ref in enumerate(refs):
        for r in range(3):
            assert torch.equal(outs[i][r].view(torch.int16), ref.view(torch.int16)), f"case {i} round {r}"
