"""GPU parity of mem::fused_attention (rldx_memory_attention_bf16, the
TransformerMemory block-causal attention) against the CPU oracle."""

import pytest
import torch

from oracle import cpu_reference as ref
from rldx_amd import functional as Fn
from rldx_amd import workloads as W
from tolerances import assert_bf16_close

pytestmark = pytest.mark.gpu


def _run(inp, dev, out=None):
    return Fn.memory_attention(inp["qkv"].to(dev), inp["cos"].to(dev), inp["signed_sin"].to(dev), inp["num_heads"],
                               inp["head_dim"], inp["block_attn_size"], out=out)


def test_memory_attention_workload(dev):
    """4 timesteps x 16 cognition tokens, 16 heads x 256, block 16, through the op."""
    import rldx_amd.ops  # noqa: F401

    inp = W.memory_attention_inputs()
    args = (inp["qkv"].to(dev), inp["cos"].to(dev), inp["signed_sin"].to(dev), 16, 256, 16)
    o = torch.ops.mem.fused_attention(*args)
    assert o.shape == (64, 16 * 256)
    assert_bf16_close(o, ref.memory_attention(**inp), "mem::fused_attention")
    o2 = torch.ops.mem.fused_attention(*args)
    assert torch.equal(o.view(torch.int16), o2.view(torch.int16)), "not deterministic"


@pytest.mark.parametrize("T,n_cog,H,D", [(1, 1, 1, 64), (3, 8, 2, 64), (5, 7, 3, 128), (2, 16, 2, 256),
                                         (100, 1, 1, 64), (1, 70, 2, 128), (13, 10, 2, 64), (9, 16, 1, 256)])
def test_memory_attention_shapes(dev, T, n_cog, H, D):
    """Ragged blocks, block 1 (plain causal), one block (full attention), several
    64-key LDS chunks (M up to 144)."""
    cfg = W.MemAttnCfg(memory_length=T, n_cog=n_cog, heads=H, head_dim=D, seed=T * 31 + n_cog)
    inp = W.memory_attention_inputs(cfg)
    o = _run(inp, dev)
    assert_bf16_close(o, ref.memory_attention(**inp), f"memory attention T={T} B={n_cog} H={H} D={D}")


def test_memory_attention_causal_first_row_returns_v(dev):
    """Block size 1: row 0 sees key 0 only, so out[0] == V[0] bit for bit."""
    cfg = W.MemAttnCfg(memory_length=40, n_cog=1, heads=2, head_dim=128, seed=5)
    inp = W.memory_attention_inputs(cfg)
    o = _run(inp, dev).cpu()
    assert torch.equal(o[0].view(torch.int16), inp["qkv"][0, 2 * 2 * 128:].view(torch.int16))


def test_memory_attention_graph_replay(dev):
    cfg = W.MemAttnCfg()
    inp = W.memory_attention_inputs(cfg)
    qkv, cos, ssin = inp["qkv"].to(dev), inp["cos"].to(dev), inp["signed_sin"].to(dev)
    out = torch.empty(64, 16 * 256, dtype=torch.bfloat16, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        Fn.memory_attention(qkv, cos, ssin, 16, 256, 16, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        Fn.memory_attention(qkv, cos, ssin, 16, 256, 16, out=out)
    for rep in range(3):
        new = torch.randn(64, 3 * 16 * 256, generator=torch.Generator().manual_seed(50 + rep)).to(torch.bfloat16)
        qkv.copy_(new.to(dev))
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = Fn.memory_attention(qkv, cos, ssin, 16, 256, 16)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16)), f"replay {rep}"
    assert_bf16_close(got, ref.memory_attention(**{**inp, "qkv": new}), "graph replay vs oracle")
