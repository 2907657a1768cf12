"""GPU parity of rldx_backbone::vision_attention (rldx_vision_attention_bf16)
against the CPU oracle: the RoPE'd Q and packed K/V in the workspace bit-exact,
the attention output within the bf16 tolerance, ragged / empty / single-token
sequences, rows outside every sequence untouched, graph replay."""

import pytest
import torch

from oracle import cpu_reference as ref
from rldx_amd import functional as Fn
from rldx_amd import workloads as W
from test_gpu_kernels import packed_kv_layout
from tolerances import assert_bf16_close

pytestmark = pytest.mark.gpu


def _padded(hd):
    return 64 if hd <= 64 else (96 if hd <= 96 else 128)


def _run(inp, dev, out=None, workspace=None):
    t = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in inp.items()}
    return Fn.vision_attention(t["qkv"], t["rope_cos"], t["rope_sin"], t["cu_seqlens"], t["scaling"],
                               t["num_heads"], t["head_dim"], out=out, workspace=workspace)


def test_vision_attention_workload(dev):
    """2 images x 196 patches, 16 heads x 72 (the RLDX-1 ViT attention), through the op."""
    import rldx_amd.ops  # noqa: F401

    inp = W.vit_attention_inputs()
    t = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in inp.items()}
    o = torch.ops.rldx_backbone.vision_attention(t["qkv"], t["rope_cos"], t["rope_sin"], t["cu_seqlens"],
                                                 t["scaling"], t["num_heads"], t["head_dim"])
    assert o.shape == (392, 16 * 72)
    assert_bf16_close(o, ref.vision_attention(**inp), "rldx_backbone::vision_attention")
    o2 = torch.ops.rldx_backbone.vision_attention(t["qkv"], t["rope_cos"], t["rope_sin"], t["cu_seqlens"],
                                                  t["scaling"], t["num_heads"], t["head_dim"])
    assert torch.equal(o.view(torch.int16), o2.view(torch.int16)), "not deterministic"


@pytest.mark.parametrize("lengths,H,D", [((196, 196), 16, 72), ((33, 1, 64, 95), 2, 72), ((5, 0, 40), 2, 80),
                                         ((129,), 2, 128), ((31, 32, 33), 1, 64)])
def test_vision_workspace_rope_and_packing_bitexact(dev, lengths, H, D):
    """Workspace: RoPE'd Q [H][M][DP] (zero padded) and the packed K/V tiles of
    each (head, sequence) at slot floor((cu[s] + 31 s) / 32), K RoPE'd."""
    cfg = W.VitAttnCfg(lengths=lengths, heads=H, head_dim=D, seed=sum(lengths))
    inp = W.vit_attention_inputs(cfg)
    M, S, DP = cfg.tokens, len(lengths), _padded(D)
    ws = torch.zeros(Fn.vision_attention_workspace_bytes(M, S, H, D), dtype=torch.uint8, device=dev)
    _run(inp, dev, workspace=ws)
    torch.cuda.synchronize()
    ws = ws.cpu()
    q, k, v = inp["qkv"].reshape(M, 3, H, D).unbind(1)
    qr = ref.vision_rope(q, inp["rope_cos"], inp["rope_sin"])
    kr = ref.vision_rope(k, inp["rope_cos"], inp["rope_sin"])
    q_bytes = (H * M * DP * 2 + 255) // 256 * 256
    qpad = ws[: H * M * DP * 2].view(torch.bfloat16).reshape(H, M, DP)
    assert torch.equal(qpad[..., :D].view(torch.int16), qr.transpose(0, 1).view(torch.int16))
    assert not qpad[..., D:].view(torch.int16).any()
    slots = (M + 31 * S) // 32
    tiles = ws[q_bytes: q_bytes + H * slots * 128 * DP].view(torch.bfloat16).reshape(H, slots, 64 * DP)
    cu = inp["cu_seqlens"].tolist()
    for s in range(S):
        a, b = cu[s], cu[s + 1]
        if b == a:
            continue
        base, nt = (a + 31 * s) // 32, (b - a + 31) // 32
        kk = torch.zeros(1, H, b - a, DP, dtype=torch.bfloat16)
        vv = torch.zeros_like(kk)
        kk[0, :, :, :D] = kr[a:b].transpose(0, 1)
        vv[0, :, :, :D] = v[a:b].transpose(0, 1)
        want = packed_kv_layout(kk, vv)[0].reshape(H, nt, 64 * DP)
        assert torch.equal(tiles[:, base: base + nt].view(torch.int16), want.view(torch.int16)), f"sequence {s}"


@pytest.mark.parametrize("lengths,H,D", [((1,), 1, 72), ((33, 1, 64, 95), 2, 72), ((300, 17), 3, 64),
                                         ((5, 0, 40), 2, 80), ((129,), 2, 128), ((31, 32, 33), 1, 8),
                                         ((2, 200, 3), 2, 120), ((64,) * 8, 4, 72),
                                         (tuple((37 * i) % 50 for i in range(70)), 2, 72)])
def test_vision_attention_ragged(dev, lengths, H, D):
    """Ragged, empty and single-token sequences; 70 sequences take the
    binary-search lookup (up to 63 use one load per lane)."""
    cfg = W.VitAttnCfg(lengths=lengths, heads=H, head_dim=D, seed=len(lengths) * 100 + D)
    inp = W.vit_attention_inputs(cfg)
    o = _run(inp, dev)
    assert_bf16_close(o, ref.vision_attention(**inp), f"vision attention {lengths} H={H} D={D}")


def test_vision_attention_single_token_sequences_return_v(dev):
    """A one-token sequence attends only to itself: out == its V, bit for bit."""
    cfg = W.VitAttnCfg(lengths=(1, 1, 7, 1), heads=2, head_dim=72, seed=4)
    inp = W.vit_attention_inputs(cfg)
    o = _run(inp, dev).cpu()
    v = inp["qkv"][:, 2 * 2 * 72:]
    for row in (0, 1, 9):
        assert torch.equal(o[row].view(torch.int16), v[row].view(torch.int16))


def test_vision_attention_rows_outside_sequences_untouched(dev):
    """cu_seqlens [3, 40, 41] over 50 rows: rows 0-2 and 41-49 keep the caller's values."""
    cfg = W.VitAttnCfg(lengths=(50,), heads=2, head_dim=72, seed=8)
    inp = W.vit_attention_inputs(cfg)
    inp["cu_seqlens"] = torch.tensor([3, 40, 41], dtype=torch.int32)
    out = torch.full((50, 144), 3.5, dtype=torch.bfloat16, device=dev)
    _run(inp, dev, out=out)
    o = out.cpu()
    keep = torch.ones(50, dtype=torch.bool)
    keep[3:41] = False
    assert (o[keep] == 3.5).all()
    r = ref.vision_attention(**inp)
    assert_bf16_close(o[3:41], r[3:41], "vision attention, offset sequences")


def test_vision_attention_graph_replay(dev):
    """Captured once, replayed with new inputs copied in: every replay equals the eager call."""
    cfg = W.VitAttnCfg(images=2, heads=4, head_dim=72, seed=21)
    inp = W.vit_attention_inputs(cfg)
    t = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in inp.items()}
    M, S = cfg.tokens, 2
    ws = torch.empty(Fn.vision_attention_workspace_bytes(M, S, 4, 72), dtype=torch.uint8, device=dev)
    out = torch.empty(M, 4 * 72, dtype=torch.bfloat16, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        Fn.vision_attention(t["qkv"], t["rope_cos"], t["rope_sin"], t["cu_seqlens"], t["scaling"], 4, 72, out=out,
                            workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        Fn.vision_attention(t["qkv"], t["rope_cos"], t["rope_sin"], t["cu_seqlens"], t["scaling"], 4, 72, out=out,
                            workspace=ws)
    for rep in range(3):
        gen = torch.Generator().manual_seed(100 + rep)
        new = torch.randn(M, 3 * 4 * 72, generator=gen).to(torch.bfloat16)
        t["qkv"].copy_(new.to(dev))
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = Fn.vision_attention(t["qkv"], t["rope_cos"], t["rope_sin"], t["cu_seqlens"], t["scaling"], 4, 72)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16)), f"replay {rep}"
    assert_bf16_close(got, ref.vision_attention(**{**inp, "qkv": new}), "graph replay vs oracle")


def test_vision_attention_rejects_bad_arguments(dev):
    inp = W.vit_attention_inputs(W.VitAttnCfg(lengths=(10,), heads=1, head_dim=72))
    with pytest.raises(RuntimeError):  # workspace too small
        _run(inp, dev, workspace=torch.empty(64, dtype=torch.uint8, device=dev))
    bad = W.vit_attention_inputs(W.VitAttnCfg(lengths=(10,), heads=1, head_dim=68))
    with pytest.raises(RuntimeError):  # head_dim % 8 != 0
        _run(bad, dev)
