"""GPU parity tests of the grouped GEMM (MSAT block linears) through the C ABI.

Reference: the same GEMM in fp32 on the CPU from the same bf16 operands, then
the eager rounding chain (bf16 output; residual add in bf16; SwiGLU of the bf16
gate / up values with the oracle's SwiGLU).  Tolerance: bf16 max-abs <= 2e-2 and
relative L2 <= 1e-2 (accumulation order differs from the CPU's).
"""

import numpy as np
import pytest
import torch

from oracle import cpu_reference as ref
from rldx_amd import functional as Fn
from tolerances import assert_bf16_close

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def packed_weight_layout(w: torch.Tensor, swiglu_pairs: bool) -> torch.Tensor:
    """CPU construction of the packed weight from its definition: chunk (nb, kb),
    lane l, element i = W[row(nb, l % 32)][16 kb + 8 (l // 32) + i], where row is
    32 nb + l % 32, or with swiglu_pairs (nb % 2) * n/2 + 32 (nb // 2) + l % 32."""
    n, k = w.shape
    nb = torch.arange(n // 32)[:, None, None, None]
    kb = torch.arange(k // 16)[None, :, None, None]
    lane = torch.arange(64)[None, None, :, None]
    i = torch.arange(8)[None, None, None, :]
    if swiglu_pairs:
        row = (nb % 2) * (n // 2) + 32 * (nb // 2) + lane % 32
    else:
        row = 32 * nb + lane % 32
    col = 16 * kb + 8 * (lane // 32) + i
    return w[row.expand(-1, k // 16, 64, 8), col.expand(n // 32, -1, 64, 8)].reshape(-1)


def _rand(shape, g, std=1.0):
    return (std * torch.randn(*shape, generator=g)).to(BF16)


def _linear_ref(a, w, bias):
    y = a.float() @ w.float().t()
    if bias is not None:
        y = y + bias.float()
    return y.to(BF16)


@pytest.mark.parametrize("n,k,pairs", [(4608, 1536, False), (192, 512, False), (8192, 1536, True)])
def test_pack_weight_layout(dev, n, k, pairs):
    g = torch.Generator().manual_seed(n + k)
    w = _rand((n, k), g)
    p = Fn.pack_weight(w.to(dev), swiglu_pairs=pairs)
    assert torch.equal(p.data.cpu(), packed_weight_layout(w, pairs))


@pytest.mark.parametrize("ms,n,k", [((512, 64, 32), 4608, 1536), ((5, 100, 130), 192, 512), ((1,), 64, 512),
                                    ((20,), 128, 384), ((300, 40), 256, 640)])
def test_grouped_gemm_bias(dev, ms, n, k):
    """Includes K ranges of an odd number of 2-k-step stages (20 rows, K 384:
    3 stages of the 32-row tiles' four K-groups), which the one-workgroup-per-CU
    launches run in 2-k-step stages instead of 4."""
    g = torch.Generator().manual_seed(sum(ms) + n)
    items, refs = [], []
    for m in ms:
        a, w, b = _rand((m, k), g), _rand((n, k), g, 0.02), _rand((n,), g, 0.1)
        out = torch.empty(m, n, dtype=BF16, device=dev)
        items.append((a.to(dev), Fn.pack_weight(w.to(dev)), b.to(dev), out, None))
        refs.append(_linear_ref(a, w, b))
    Fn.grouped_gemm(items, "bias")
    for (_, _, _, out, _), r in zip(items, refs):
        assert_bf16_close(out, r, "grouped gemm")


def test_grouped_gemm_residual_in_place(dev):
    """x_s += W3_s(h_s): K = 4096, the output aliases the residual (rows of one buffer)."""
    g = torch.Generator().manual_seed(7)
    n, k = 1536, 4096
    # unit-scale data (|out| < 4): the absolute bf16 bound of 2e-2 is below one
    # bf16 ulp from magnitude 4 on, where any change of accumulation order can
    # flip a rounding
    x = _rand((608, n), g, 0.5)
    h = _rand((608, k), g)
    xd, hd = x.to(dev), h.to(dev)
    items, refs = [], []
    for lo, hi in ((0, 512), (512, 576), (576, 608)):
        w, b = _rand((n, k), g, 0.008), _rand((n,), g, 0.1)
        items.append((hd[lo:hi], Fn.pack_weight(w.to(dev)), b.to(dev), xd[lo:hi], xd[lo:hi]))
        refs.append((x[lo:hi].float() + _linear_ref(h[lo:hi], w, b).float()).to(BF16))
    Fn.grouped_gemm(items, "residual")
    assert_bf16_close(xd, torch.cat(refs), "residual gemm")


def test_grouped_gemm_swiglu(dev):
    g = torch.Generator().manual_seed(9)
    n, k = 8192, 1536
    items, refs = [], []
    for m in (512, 64, 32):
        a, w, b = _rand((m, k), g), _rand((n, k), g, 0.02), _rand((n,), g, 0.1)
        out = torch.empty(m, n // 2, dtype=BF16, device=dev)
        items.append((a.to(dev), Fn.pack_weight(w.to(dev), swiglu_pairs=True), b.to(dev), out, None))
        refs.append(ref.swiglu(_linear_ref(a, w, b)))
    Fn.grouped_gemm(items, "swiglu")
    for (_, _, _, out, _), r in zip(items, refs):
        assert_bf16_close(out, r, "gemm + swiglu")


def test_grouped_gemm_swiglu_epilogue_all_gates_bitexact(dev):
    """The SwiGLU epilogue on every finite normal bf16 gate value.  One-hot A rows
    make each GEMM output exactly one weight element (every other product is 0),
    so with a zero bias the result must equal eager `F.silu(g) * u` of those
    values bit for bit.  Zeros, denormals (the matrix cores may flush them),
    inf and NaN are left out: 0 * inf in the other products would be NaN."""
    bits = np.arange(65536, dtype=np.uint16)
    expo = (bits >> 7) & 0xFF
    keep = (expo != 0) & (expo != 0xFF)
    gates = torch.from_numpy(bits[keep].view(np.int16).copy()).view(BF16)
    n_half, k = 4096, 512
    m = -(-gates.numel() // n_half)
    gate_vals = torch.zeros(m * n_half, dtype=BF16)
    gate_vals[: gates.numel()] = gates
    gate_vals = gate_vals.view(m, n_half)
    up_vals = _rand((m, n_half), torch.Generator().manual_seed(23))
    a = torch.zeros(m, k, dtype=BF16)
    w = torch.zeros(2 * n_half, k, dtype=BF16)
    for r in range(m):
        a[r, 32 * r] = 1.0
        w[:n_half, 32 * r] = gate_vals[r]
        w[n_half:, 32 * r] = up_vals[r]
    out = torch.empty(m, n_half, dtype=BF16, device=dev)
    zero_bias = torch.zeros(2 * n_half, dtype=BF16, device=dev)
    Fn.grouped_gemm([(a.to(dev), Fn.pack_weight(w.to(dev), swiglu_pairs=True), zero_bias, out, None)], "swiglu")
    expect = ref.swiglu(torch.cat([gate_vals, up_vals], dim=1))
    bad = out.cpu().view(torch.int16) != expect.view(torch.int16)
    assert not bool(bad.any()), f"{int(bad.sum())} mismatching words, gates {gate_vals[bad][:4].tolist()}"


def test_grouped_gemm_deterministic(dev):
    g = torch.Generator().manual_seed(3)
    a = _rand((512, 1536), g).to(dev)
    w = Fn.pack_weight(_rand((1536, 1536), g, 0.02).to(dev))
    o1 = torch.empty(512, 1536, dtype=BF16, device=dev)
    o2 = torch.empty_like(o1)
    Fn.grouped_gemm([(a, w, None, o1, None)])
    Fn.grouped_gemm([(a, w, None, o2, None)])
    assert torch.equal(o1, o2)


@pytest.mark.parametrize("epilogue,n,k,split_k", [("residual", 1536, 4096, 8), ("bias", 1536, 1536, 4),
                                                  ("bias", 4608, 1536, 2), ("swiglu", 1536, 1024, 8),
                                                  ("swiglu_packed", 3072, 1536, 4)])
def test_grouped_gemm_split_k(dev, epilogue, n, k, split_k):
    """split_k splits every stream's K range across workgroups (partials summed in
    split order by the last workgroup of a tile): same bf16 tolerance against the
    fp32 reference, bit-identical on repeated launches that share one workspace
    (the tile counters are re-armed), close to the unsplit result."""
    g = torch.Generator().manual_seed(n + k)
    swiglu = epilogue.startswith("swiglu")
    n_out = n // 2 if swiglu else n
    items, refs, outs = [], [], []
    for m in (512, 64, 32):
        a, w, b = _rand((m, k), g), _rand((n, k), g, 0.5 / k ** 0.5), _rand((n,), g, 0.1)
        res = _rand((m, n_out), g, 0.5) if epilogue == "residual" else None
        y = _linear_ref(a, w, b)
        if swiglu:
            r = ref.swiglu(y)
        elif res is not None:
            r = (res.float() + y.float()).to(BF16)
        else:
            r = y
        refs.append(r)
        if epilogue == "swiglu_packed":
            out = Fn.PackedAct.empty(m, n_out, dev)
        else:
            out = res.to(dev) if res is not None else torch.empty(m, n_out, dtype=BF16, device=dev)
        outs.append(out)
        items.append((a.to(dev), Fn.pack_weight(w.to(dev), swiglu_pairs=swiglu), b.to(dev), out,
                      out if res is not None else None))
    need = Fn.grouped_gemm_workspace_bytes(items, epilogue, split_k)
    assert need > 0
    ws = Fn.GemmWorkspace(need, dev)

    def result():
        return [o.unpack().clone() if isinstance(o, Fn.PackedAct) else o.clone() for o in outs]

    base = [o.clone() for o in outs] if epilogue == "residual" else None

    def reset():
        if base is not None:
            for o, b0 in zip(outs, base):
                o.copy_(b0)

    Fn.grouped_gemm(items, epilogue, split_k=split_k, workspace=ws)
    first = result()
    for got, r in zip(first, refs):
        assert_bf16_close(got, r, f"split-K gemm {epilogue}")
    for _ in range(3):  # counters re-armed, partials overwritten: identical results
        reset()
        Fn.grouped_gemm(items, epilogue, split_k=split_k, workspace=ws)
        for x, y in zip(result(), first):
            assert torch.equal(x, y)
    for _ in range(3):  # the splits of every tile on different XCDs: the same bits (device-scope hand-off)
        reset()
        Fn.grouped_gemm(items, epilogue, split_k=split_k, workspace=ws, splits_across_xcds=True)
        for x, y in zip(result(), first):
            assert torch.equal(x, y), "splits across XCDs differ from splits on one XCD"
    reset()
    Fn.grouped_gemm(items, epilogue)  # no split
    for x, y in zip(result(), first):
        assert_bf16_close(x, y, "split vs unsplit")
    assert int(ws.data[:65536].count_nonzero()) == 0  # every tile counter back at zero


def test_grouped_gemm_split_k_workspace_shared_across_shapes(dev):
    """One workspace serves split GEMMs of different shapes in turn (their plans
    place partials at different offsets, counters in the common area): every call
    matches its first result bit for bit and the bf16 reference."""
    g = torch.Generator().manual_seed(77)
    calls = []
    for n, k, epilogue in ((4608, 1536, "bias"), (1536, 1536, "bias"), (1536, 4096, "bias")):
        items, refs = [], []
        for m in (512, 64, 32):
            a, w, b = _rand((m, k), g), _rand((n, k), g, 0.5 / k ** 0.5), _rand((n,), g, 0.1)
            items.append((a.to(dev), Fn.pack_weight(w.to(dev)), b.to(dev), torch.empty(m, n, dtype=BF16, device=dev),
                          None))
            refs.append(_linear_ref(a, w, b))
        calls.append((items, refs, epilogue))
    ws = Fn.GemmWorkspace(max(Fn.grouped_gemm_workspace_bytes(it, ep, 4) for it, _, ep in calls), dev)
    first = None
    for rnd in range(3):
        got = []
        for items, refs, ep in calls:
            Fn.grouped_gemm(items, ep, split_k=4, workspace=ws)
            got.append([it[3].clone() for it in items])
            if rnd == 0:
                for o, r in zip(got[-1], refs):
                    assert_bf16_close(o, r, "split-K, shared workspace")
        if first is None:
            first = got
        else:
            for xs, ys in zip(got, first):
                for x, y in zip(xs, ys):
                    assert torch.equal(x, y)


@pytest.mark.parametrize("m,k", [(608, 1536), (5, 4096), (33, 64)])
def test_act_pack_roundtrip(dev, m, k):
    g = torch.Generator().manual_seed(m + k)
    x = _rand((m, k + 8), g)[:, :k]  # strided rows
    p = Fn.pack_act(x.to(dev))
    assert torch.equal(p.unpack().cpu(), x)
    # layout definition, element by element, on a few rows
    d = p.data.cpu()
    for r in (0, m - 1, m // 2):
        for c in (0, k - 1, k // 3):
            off = ((r // 32) * (k // 16) + c // 16) * 512 + ((r % 32) + 32 * ((c // 8) % 2)) * 8 + c % 8
            assert d[off] == x[r, c]
    # with the LayerNorm statistics (rldx_act_pack_stats_bf16): the same packed bits;
    # slot 0 the row's (sum, sum of squares), the other slots zero
    st = torch.full((k // 64, m, 2), 7.0, device=dev)
    p2 = Fn.pack_act(x.to(dev), stats=st)
    assert torch.equal(p2.unpack(), p.unpack())
    xd = x.double()
    ref = torch.stack([xd.sum(-1), (xd * xd).sum(-1)], dim=-1)
    stc = st.cpu().double()
    assert (stc[0] - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()
    assert not stc[1:].any()


@pytest.mark.parametrize("m,k", [(608, 1536), (7, 4096), (64, 512)])
def test_layernorm_pack(dev, m, k):
    g = torch.Generator().manual_seed(k - m)
    x = (3 * torch.randn(m, k, generator=g) + 0.5).to(BF16)
    p = Fn.layernorm_pack(x.to(dev), 1e-6)
    r = torch.nn.functional.layer_norm(x, (k,), eps=1e-6)
    assert_bf16_close(p.unpack(), r, "layernorm")


@pytest.mark.parametrize("shapes", [((18, 1536), (64, 4096)), ((18, 1536), (96, 4096), (17, 1536)),
                                    ((82, 1536), (17, 1536)), ((300, 8192), (5, 16), (33, 512), (1, 1024))])
def test_layernorm_pack_many_matches_one_at_a_time(dev, shapes):
    """rldx_layernorm_pack_many_bf16 (one launch for a block's streams) gives
    each matrix the bits of rldx_layernorm_pack_bf16 on it alone, including
    matrices narrower than the launch's widest one and strided rows."""
    g = torch.Generator().manual_seed(sum(m * k for m, k in shapes) % 1000)
    xs = []
    for m, k in shapes:
        full = (2 * torch.randn(m, k + 64, generator=g) + 0.25).to(BF16).to(dev)
        xs.append(full[:, :k])  # row stride k + 64
    many = [Fn.PackedAct.empty(m, k, dev) for m, k in shapes]
    Fn.layernorm_pack_many(list(zip(xs, many)), 1e-6)
    one = [Fn.layernorm_pack(x, 1e-6) for x in xs]
    torch.cuda.synchronize()
    for (m, k), a, b in zip(shapes, many, one):
        assert torch.equal(a.unpack().view(torch.int16), b.unpack().view(torch.int16)), f"{m} x {k}"


@pytest.mark.parametrize("n,adim,hidden,others", [(64, 32, 1536, ((512, 0), (32, 8))), (18, 16, 512, ()),
                                                   (37, 64, 2048, ((5, 3),)), (64, 8, 256, ((40, 0), (1, 2), (7, 5)))])
def test_action_encode_pack(dev, n, adim, hidden, others):
    """rldx_action_encode_pack_bf16: the action rows are the eager chain
    bf16(bf16(bf16(act W_in^T + b_in) + temb) + pos) (fp32 dot products: within
    one bf16 rounding of the chain computed with torch in fp32 on the CPU), and
    every matrix's packed rows and statistics are the bits rldx_act_pack_stats_bf16
    gives for the same rows (other matrices with a row stride wider than hidden)."""
    g = torch.Generator().manual_seed(n + adim + hidden)
    act = _rand((n, adim), g).to(dev)
    w_in = _rand((hidden, adim), g, std=adim ** -0.5).to(dev)
    b_in, temb = _rand((hidden,), g, 0.5).to(dev), _rand((hidden,), g, 0.5).to(dev)
    pos = _rand((n, hidden), g, 0.5).to(dev)
    xs = [_rand((m, hidden + pad * 8), g).to(dev)[:, :hidden] for m, pad in others]
    out, st = Fn.PackedAct.empty(n, hidden, dev), Fn.ln_stats_empty(n, hidden, dev)
    o_out = [(x, Fn.PackedAct.empty(x.shape[0], hidden, dev), Fn.ln_stats_empty(x.shape[0], hidden, dev)) for x in xs]
    Fn.action_encode_pack(act, w_in, b_in, temb, pos, out, st, o_out)
    torch.cuda.synchronize()
    y = out.unpack()
    a32, w32 = act.float().cpu(), w_in.float().cpu()
    lin = (a32 @ w32.t()) + b_in.float().cpu()
    ref = (((lin.to(BF16).float() + temb.float().cpu()).to(BF16).float()) + pos.float().cpu()).to(BF16)
    diff = (y.cpu().float() - ref.float()).abs()
    # each of the three roundings may land one ulp apart (the dot products sum in another order): bound by the
    # magnitudes that enter them
    tol = (lin.abs() + temb.float().cpu().abs() + pos.float().cpu().abs()) * 2 ** -7 + 1e-6
    assert (diff <= tol).all(), f"max diff {diff.max().item()}"
    for x, o, s in [(y, out, st)] + o_out:
        rp, rs = Fn.PackedAct.empty(x.shape[0], hidden, dev), Fn.ln_stats_empty(x.shape[0], hidden, dev)
        Fn.pack_act(x.contiguous(), out=rp, stats=rs)
        torch.cuda.synchronize()
        assert torch.equal(o.unpack().view(torch.int16), rp.unpack().view(torch.int16))
        assert torch.equal(s, rs)


@pytest.mark.parametrize("n,adim,hidden", [(64, 32, 1536), (18, 16, 512), (5, 64, 2048)])
def test_action_decode_euler(dev, n, adim, hidden):
    """rldx_action_decode_euler_bf16 against the eager chain on the same packed
    rows: act + dt * (LN(x) W_out^T + b_out) with each of its bf16 roundings
    (torch in fp32 on the CPU): within one bf16 rounding of every step."""
    g = torch.Generator().manual_seed(n * adim + hidden)
    x = (2 * torch.randn(n, hidden, generator=g) + 0.3).to(BF16)
    w_out = _rand((adim, hidden), g, std=hidden ** -0.5).to(dev)
    b_out = _rand((adim,), g, 0.5).to(dev)
    act = _rand((n, adim), g).to(dev)
    act0 = act.clone()
    dt = 0.25
    Fn.action_decode_euler(Fn.pack_act(x.to(dev)), w_out, b_out, act, dt, 1e-6)
    torch.cuda.synchronize()
    hs = torch.nn.functional.layer_norm(x.float(), (hidden,), eps=1e-6).to(BF16).float()
    w32 = w_out.float().cpu()
    vel = (hs @ w32.t() + b_out.float().cpu()).to(BF16).float()
    ref = (act0.float().cpu() + (vel * dt).to(BF16).float()).to(BF16)
    diff = (act.cpu().float() - ref.float()).abs()
    # hs may differ by one ulp per element (another mean / rsqrt evaluation) and the sums run in another order:
    # bound the velocity error by the magnitudes summed, then the two roundings after it
    vel_err = (hs.abs() @ w32.abs().t() + b_out.float().cpu().abs()) * 2 ** -7
    tol = (act0.float().cpu().abs() + dt * vel.abs()) * 2 ** -7 + dt * vel_err + 1e-6
    assert (diff <= tol).all(), f"max diff {diff.max().item()}"


def test_swiglu_packed_epilogue_matches_row_major(dev):
    g = torch.Generator().manual_seed(13)
    n, k = 8192, 1536
    a = _rand((608, k), g).to(dev)
    w = Fn.pack_weight(_rand((n, k), g, 0.02).to(dev), swiglu_pairs=True)
    b = _rand((n,), g, 0.1).to(dev)
    ap = Fn.pack_act(a)
    rm = torch.empty(608, n // 2, dtype=BF16, device=dev)
    pk = Fn.PackedAct.empty(608, n // 2, dev)
    rows = ((0, 512), (512, 576), (576, 608))
    Fn.grouped_gemm([(ap.rows(lo, hi), w, b, rm[lo:hi], None) for lo, hi in rows], "swiglu")
    Fn.grouped_gemm([(ap.rows(lo, hi), w, b, pk.rows(lo, hi), None) for lo, hi in rows], "swiglu_packed")
    assert torch.equal(pk.unpack(), rm)


def test_attention_packed_output(dev):
    g = torch.Generator().manual_seed(17)
    H, S, D = 12, 608, 128
    q = torch.randn(1, H, S, D, generator=g).to(BF16).to(dev)
    k = torch.randn(1, H, S, D, generator=g).to(BF16).to(dev)
    v = torch.randn(1, H, S, D, generator=g).to(BF16).to(dev)
    bias = torch.zeros(S, device=dev)
    bias[-8:] = float("-inf")
    kvp = Fn.kv_pack(k, v)
    o = torch.empty(1, S, H, D, dtype=BF16, device=dev)
    Fn.attention_packed(q, kvp, S, key_bias=bias, out=o.permute(0, 2, 1, 3))
    op = Fn.attention_packed(q, kvp, S, key_bias=bias, out=Fn.PackedAct.empty(S, H * D, dev))
    assert torch.equal(op.unpack(), o.view(S, H * D))


@pytest.mark.parametrize("H,D,S,segs", [(12, 128, 608, [(0, 512), (512, 56), (576, 32)]),
                                        (24, 64, 96, [(0, 64), (64, 17)]),
                                        (24, 64, 82, [(0, 82)])])
def test_attention_packed_segments_batch(dev, H, D, S, segs):
    """rldx_attention_packed_segments_fwd_bf16: three robots' joint sequences
    whose output rows go to one packed matrix stream by stream (a segment's
    rows of robot 0, then robot 1, ..., each segment from a 32-row block;
    rows between the segments, the padding of a stream, not stored) equal
    the strided output of the same attention row for row, bit for bit, and
    packed rows that no segment maps keep their contents."""
    B = 3
    g = torch.Generator().manual_seed(23)
    q = torch.randn(B, H, S, D, generator=g).to(BF16).to(dev)
    k = torch.randn(B, H, S, D, generator=g).to(BF16).to(dev)
    v = torch.randn(B, H, S, D, generator=g).to(BF16).to(dev)
    bias = torch.zeros(B, S)
    for b in range(B):  # a different set of masked keys per robot
        bias[b, S - 4 - 3 * b:S - 3 * b] = float("-inf")
    bias = bias.to(dev)
    kvp = Fn.kv_pack(k, v)
    o = torch.empty(B, S, H, D, dtype=BF16, device=dev)
    Fn.attention_packed(q, kvp, S, key_bias=bias, out=o.permute(0, 2, 1, 3))
    full, base = [], 0
    for off, rows in segs:
        full.append((off, rows, base))
        base = (base + B * rows + 31) // 32 * 32
    m = full[-1][2] + B * full[-1][1]
    pk = Fn.PackedAct.empty(m, H * D, dev)
    pk.data.fill_(7.0)
    Fn.attention_packed(q, kvp, S, key_bias=bias, out=pk, segments=full)
    expect = torch.full((m, H * D), 7.0, dtype=BF16)
    oc = o.cpu()
    for off, rows, first in full:
        for b in range(B):
            expect[first + b * rows:first + (b + 1) * rows] = oc[b, off:off + rows].reshape(rows, H * D)
    assert torch.equal(pk.unpack().cpu().view(torch.int16), expect.view(torch.int16))


@pytest.mark.parametrize("warm_sizes", [(4_718_592, 4_718_592, 4_718_592), (1000,), (0, 129, 12_582_912), (64,)])
def test_attention_packed_warm_up_is_bit_identical(dev, warm_sizes):
    """rldx_attention_packed_fwd_warm_bf16 (extra workgroups reading the lines of
    up to three ranges) returns the bits of the plain launch, with causal and
    key-bias variants; ranges of any length (partial last lines, empty, shorter
    than one line) are read only inside their bytes (the warm tensors are left
    unchanged)."""
    g = torch.Generator().manual_seed(29)
    H, S, D = 12, 608, 128
    q = torch.randn(1, H, S, D, generator=g).to(BF16).to(dev)
    k = torch.randn(1, H, S, D, generator=g).to(BF16).to(dev)
    v = torch.randn(1, H, S, D, generator=g).to(BF16).to(dev)
    bias = torch.zeros(S, device=dev)
    bias[-8:] = float("-inf")
    kvp = Fn.kv_pack(k, v)
    warm = [torch.randint(0, 255, (n,), dtype=torch.uint8, generator=g).to(dev) for n in warm_sizes]
    before = [t.clone() for t in warm]
    for kb, causal in ((bias, False), (None, True)):
        o0 = Fn.attention_packed(q, kvp, S, key_bias=kb, causal=causal, out=Fn.PackedAct.empty(S, H * D, dev))
        o1 = Fn.attention_packed(q, kvp, S, key_bias=kb, causal=causal, out=Fn.PackedAct.empty(S, H * D, dev),
                                 warm=warm)
        torch.cuda.synchronize()
        assert torch.equal(o0.unpack().view(torch.int16), o1.unpack().view(torch.int16)), f"causal {causal}"
    assert all(torch.equal(a, b) for a, b in zip(warm, before))


def test_concatenated_packed_operand_from_attention_and_bias_packed_gemm(dev):
    """The single-stream block's linear2 operand cat([attention, mlp_proj(...)]):
    the attention kernel writes columns [0, 1536) and a bias_packed GEMM columns
    [1536, 5632) of one packed [82, 5632] matrix, each equal bit for bit to its
    row-major output; a swiglu_packed GEMM into a column view likewise."""
    g = torch.Generator().manual_seed(19)
    H, S, D, n2, k2 = 24, 82, 64, 4096, 6144
    q = torch.randn(1, H, S, D, generator=g).to(BF16).to(dev)
    kk = torch.randn(1, H, S, D, generator=g).to(BF16).to(dev)
    v = torch.randn(1, H, S, D, generator=g).to(BF16).to(dev)
    kvp = Fn.kv_pack(kk, v)
    o = torch.empty(1, S, H, D, dtype=BF16, device=dev)
    Fn.attention_packed(q, kvp, S, out=o.permute(0, 2, 1, 3))
    a = _rand((S, k2), g).to(dev)
    w = Fn.pack_weight(_rand((n2, k2), g, 0.02).to(dev))
    b = _rand((n2,), g, 0.1).to(dev)
    rm = torch.empty(S, n2, dtype=BF16, device=dev)
    ap = Fn.pack_act(a)
    Fn.grouped_gemm([(ap, w, b, rm, None)], "bias")
    cat = Fn.PackedAct.empty(S, H * D + n2, dev)
    cat.data.fill_(7.0)
    Fn.attention_packed(q, kvp, S, out=cat.cols(0, H * D))
    Fn.grouped_gemm([(ap, w, b, cat.cols(H * D, H * D + n2), None)], "bias_packed")
    full = cat.unpack()
    assert torch.equal(full[:, : H * D], o.view(S, H * D))
    assert torch.equal(full[:, H * D:], rm)
    # swiglu_packed into the right half of a wider packed matrix
    w12 = Fn.pack_weight(_rand((2 * 1024, k2), g, 0.02).to(dev), swiglu_pairs=True)
    b12 = _rand((2 * 1024,), g, 0.1).to(dev)
    sw = torch.empty(S, 1024, dtype=BF16, device=dev)
    Fn.grouped_gemm([(ap, w12, b12, sw, None)], "swiglu")
    wide = Fn.PackedAct.empty(S, 2048, dev)
    Fn.grouped_gemm([(ap, w12, b12, wide.cols(1024, 2048), None)], "swiglu_packed")
    assert torch.equal(wide.unpack()[:, 1024:], sw)


@pytest.mark.parametrize("ms,H,k,D", [((512, 64, 32), 12, 1536, 128), ((470, 64, 32), 12, 1536, 128),
                                     ((1024, 64, 32), 12, 256, 128),
                                     ((64, 32, 20), 2, 256, 128), ((40,), 3, 384, 128), ((0, 96, 64), 2, 128, 128),
                                     ((64, 18), 24, (4096, 1536), 64), ((96, 32, 17), 24, (4096, 1536, 1536), 64),
                                     ((64, 18), 24, 1536, 64), ((40,), 2, 256, 64), ((32, 20), 4, (384, 256), 64),
                                     ((64, 18), 12, (4096, 1536), 128), ((20, 40, 17), 4, (256, 384, 128), 64),
                                     ((64, 18, 17), 24, 1536, 64)])
def test_grouped_gemm_qkv_norm_rope_matches_two_launches(dev, ms, H, k, D):
    """The QKV epilogue (QK RMSNorm + RoPE + packed K/V tiles in the GEMM) is
    bit-identical to the bias GEMM followed by rldx_msat_qkv_norm_rope_bf16:
    Q (H, M, D) and every element of the packed K/V tiles, including the zero
    padding keys of a last stream whose rows are not a multiple of 32.  Shapes:
    the action step's streams (128 x 128 and 64 x 128 tiles, one workgroup per
    CU; the 128 x 128 tiles finish in registers, also with 470 rows: a partial
    last tile, padding keys 470-479 in its last 32-key tile), 1024 rows (more than 256 workgroups: two per CU), short and single
    streams, an empty stream; head_dim 64 (two heads per tile) with the RLDX-1
    double-stream shapes (VL 4096 | SA 1536 [| P 1536], a K per stream:
    rldx_grouped_gemm_qkv_norm_rope_mixed_bf16) and the single-stream shape.
    Streams before the last with rows % 32 != 0 start the next stream on a
    32-row boundary: the reference gives them zero QKV rows up to it (as the
    RLDX-1 chain pads its SA rows before the P stream); Q is compared on the
    stream rows (the fused launch does not write padding Q rows), and a padding
    key may be -0 in the reference (RoPE of a zero row) where the fused launch
    writes +0."""
    from rldx_amd.msat_step import msat_rope_tables

    ks = list(k) if isinstance(k, tuple) else [k] * len(ms)
    g = torch.Generator().manual_seed(sum(ms) + H + sum(ks) + D)
    n = 3 * H * D
    items, specs, qkv_items, ref_specs, live_rows, M = [], [], [], [], [], 0
    last = max(i for i, m in enumerate(ms) if m)
    for i, m in enumerate(ms):
        k = ks[i]
        mp = (m + 31) // 32 * 32 if i < last else m  # joint rows of the stream
        if m:
            live_rows += list(range((M + 31) // 32 * 32, (M + 31) // 32 * 32 + m))
            M = (M + 31) // 32 * 32 + m
        a = Fn.pack_act(_rand((m, k), g).to(dev)) if m else Fn.PackedAct.empty(0, k, dev)
        w = Fn.pack_weight(_rand((n, k), g, std=k ** -0.5).to(dev))
        b = _rand((n,), g, std=0.5).to(dev)
        qw, kw = (1 + 0.2 * torch.randn(D, generator=g)).to(BF16).to(dev), (1 + 0.2 * torch.randn(D, generator=g)).to(BF16).to(dev)
        cos = sin = None
        if i > 0 and m:  # streams after the first carry RoPE tables
            ids = torch.stack([torch.zeros(mp, dtype=torch.long), torch.arange(mp) + 3 * i], dim=-1)
            cos, sin = (t.to(dev) for t in msat_rope_tables(ids, D, 10000.0))
        qkv = torch.zeros(mp, n, dtype=BF16, device=dev)  # rows past m stay zero (padding keys)
        items.append((a, w, b))
        qkv_items.append((a, w, b, qkv[:m], None))
        specs.append(Fn.StreamSpec(None, qw, kw, cos, sin))
        ref_specs.append(Fn.StreamSpec(qkv, qw, kw, cos, sin))
    q = torch.full((H, M, D), 7.0, dtype=BF16, device=dev)
    kvp = torch.full((H, Fn.kv_packed_elems(M, D)), 5.0, dtype=BF16, device=dev)
    Fn.grouped_gemm_qkv_norm_rope(items, specs, H, D, 1e-6, out=(q, kvp))
    for it in qkv_items:
        if it[0].m:
            Fn.grouped_gemm([it], "bias")
    live = [s for s in ref_specs if s.qkv.shape[0]]
    q2, kvp2 = Fn.msat_qkv_norm_rope(live, H, D, 1e-6, kv_packed=True)
    torch.cuda.synchronize()
    rows = torch.tensor(live_rows, device=dev)
    assert torch.equal(q[:, rows].view(torch.int16), q2[:, rows].view(torch.int16))
    # bits equal everywhere, except that a padding key the reference rotates as a
    # zero row may hold -0 where the fused launch writes +0
    same = (kvp.view(torch.int16) == kvp2.view(torch.int16)) | ((kvp == 0) & (kvp2 == 0))
    assert bool(same.all())


@pytest.mark.parametrize("epilogue,ms,n,k,split", [("swiglu_packed", (64,), 22016, 512, 1),
                                                   ("swiglu_packed", (82, 18), 12288, 256, 1),
                                                   ("residual", (64, 18), 1536, 1024, 4),
                                                   ("bias", (512, 64, 32), 1536, 256, 1),
                                                   ("bias_packed", (40,), 4096, 256, 2)])
def test_grouped_gemm_wide_tiles_bit_identical(dev, epilogue, ms, n, k, split):
    """64 x 128 / 32 x 128 tiles (RLDX_GEMM_WIDE_TILES) keep the K-groups of 64 x 64
    / 32 x 64, so every epilogue gives the same bits as the default plan, with and
    without split-K."""
    swiglu = epilogue.startswith("swiglu")
    n_out = n // 2 if swiglu else n
    packed = epilogue.endswith("packed")
    outs = []
    for wide in (False, True):
        items = []
        gg = torch.Generator().manual_seed(n + k)
        for m in ms:
            a = Fn.pack_act(_rand((m, k), gg).to(dev))
            w = Fn.pack_weight(_rand((n, k), gg, std=k ** -0.5).to(dev), swiglu_pairs=swiglu)
            b = _rand((n,), gg, std=0.5).to(dev)
            res = _rand((m, n_out), gg).to(dev) if epilogue == "residual" else None
            out = Fn.PackedAct.empty(m, n_out, dev) if packed else (res if res is not None else
                                                                   torch.empty(m, n_out, dtype=BF16, device=dev))
            items.append((a, w, b, out, res))
        ws = Fn.GemmWorkspace(Fn.grouped_gemm_workspace_bytes(items, epilogue, split, wide), dev) if split > 1 else None
        Fn.grouped_gemm(items, epilogue, split_k=split, workspace=ws, wide_tiles=wide)
        torch.cuda.synchronize()
        outs.append([(it[3].unpack() if packed else it[3]).clone() for it in items])  # rows < m only
    for x, y in zip(*outs):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))


@pytest.mark.parametrize("epilogue,shapes,splits,wide", [
    ("bias", ((18, 4608, 1536), (64, 4608, 4096)), (1, 2), False),
    ("residual", ((18, 1536, 4096), (18, 1536, 4096), (64, 4096, 2816)), (4, 2, 2), False),
    ("residual_packed", ((18, 1536, 4096), (64, 4096, 2816)), (2, 1), False),
    ("swiglu_packed", ((18, 8192, 1536), (64, 5504, 512)), (1, 1), True),
    ("swiglu_packed", ((40, 512, 256), (300, 256, 384), (5, 1024, 640)), (1, 2, 1), False),
    ("bias_packed", ((100, 1024, 384), (30, 256, 512)), (2, 1), True),
    ("bias", ((0, 1024, 256), (40, 512, 384)), (1, 2), False),
    ("residual", ((33, 256, 1024), (0, 512, 128), (7, 128, 256)), (8, 1, 2), False)])
def test_grouped_gemm_mixed_shapes_bit_identical(dev, epilogue, shapes, splits, wide):
    """One launch of groups with different n, k and split
    (rldx_grouped_gemm_mixed_bf16) gives every group the bits of a launch of that
    group alone with its split; the residual epilogues' row statistics too."""
    swiglu = epilogue.startswith("swiglu")
    packed = epilogue.endswith("packed")
    res_epi = epilogue.startswith("residual")
    gg = torch.Generator().manual_seed(sum(n + k for _, n, k in shapes))
    data = []
    for m, n, k in shapes:
        n_out = n // 2 if swiglu else n
        data.append((m, n_out, _rand((m, k), gg).to(dev), _rand((n, k), gg, std=k ** -0.5).to(dev),
                     _rand((n,), gg, std=0.5).to(dev), _rand((m, n_out), gg).to(dev) if res_epi else None))

    def items():
        out = []
        for m, n_out, a, w, b, r in data:
            if packed:
                o = Fn.pack_act(r) if r is not None else Fn.PackedAct.empty(m, n_out, dev)
                out.append((Fn.pack_act(a), Fn.pack_weight(w, swiglu_pairs=swiglu), b, o, o if res_epi else None))
            else:
                o = r.clone() if r is not None else torch.empty(m, n_out, dtype=BF16, device=dev)
                out.append((Fn.pack_act(a), Fn.pack_weight(w, swiglu_pairs=swiglu), b, o, o if res_epi else None))
        return out

    def stats():
        return [Fn.ln_stats_empty(m, n_out, dev) for m, n_out, *_ in data] if res_epi else None

    mixed, st_mixed = items(), stats()
    ws = Fn.GemmWorkspace(max(1, Fn.grouped_gemm_workspace_bytes(mixed, epilogue, list(splits), wide)), dev)
    Fn.grouped_gemm(mixed, epilogue, split_k=list(splits), workspace=ws, wide_tiles=wide, stats_out=st_mixed)
    alone, st_alone = items(), stats()
    for i, (it, sp) in enumerate(zip(alone, splits)):
        wsi = Fn.GemmWorkspace(Fn.grouped_gemm_workspace_bytes([it], epilogue, sp, wide), dev) if sp > 1 else None
        Fn.grouped_gemm([it], epilogue, split_k=sp, workspace=wsi, wide_tiles=wide,
                        stats_out=[st_alone[i]] if res_epi else None)
        torch.cuda.synchronize()
    torch.cuda.synchronize()
    for i, (x, y) in enumerate(zip(mixed, alone)):
        xo, yo = (x[3].unpack(), y[3].unpack()) if packed else (x[3], y[3])
        assert torch.equal(xo.view(torch.int16), yo.view(torch.int16)), f"group {i} {shapes[i]}"
        if res_epi:
            assert torch.equal(st_mixed[i], st_alone[i]), f"group {i} statistics"
    # and against the CPU product (the layout of each group's output is its own n)
    m, n_out, a, w, b, r = data[0]
    y = _linear_ref(a.cpu(), w.cpu(), b.cpu())
    if not swiglu and not res_epi:
        assert_bf16_close((mixed[0][3].unpack() if packed else mixed[0][3]).cpu(), y)


def test_ss_fused_mlp_swiglu_op(dev):
    import rldx_amd.ops  # noqa: F401  registers ss::fused_mlp_swiglu

    g = torch.Generator().manual_seed(19)
    M, K, NH = 82, 1536, 4096
    x, w, b = _rand((M, K), g), _rand((2 * NH, K), g, 0.02), _rand((2 * NH,), g, 0.1)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    y = torch.ops.ss.fused_mlp_swiglu(xd, wd, bd, 1)
    assert y.shape == (M, NH)
    assert_bf16_close(y, ref.swiglu(_linear_ref(x, w, b)), "ss::fused_mlp_swiglu")
    assert torch.equal(torch.ops.ss.fused_mlp_swiglu(xd, wd, bd, 1), y)  # packed-weight cache hit
    ys = torch.ops.ss.fused_mlp_swiglu(xd, wd, bd, 4)  # split-K: partials summed in a fixed order
    assert_bf16_close(ys, ref.swiglu(_linear_ref(x, w, b)), "ss::fused_mlp_swiglu split_k=4")
    assert torch.equal(torch.ops.ss.fused_mlp_swiglu(xd, wd, bd, 4), ys)
    wd.mul_(0.5)  # in-place update -> repacked
    assert_bf16_close(torch.ops.ss.fused_mlp_swiglu(xd, wd, bd, 1), ref.swiglu(_linear_ref(x, (w.float() * 0.5).to(BF16), b)),
                      "after weight update")


def _ln_ref(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """LayerNorm without affine parameters in fp64, not rounded (the folded GEMM
    skips the bf16 rounding of the normalised rows)."""
    x = x.double()
    mu = x.mean(-1, keepdim=True)
    return (x - mu) / torch.sqrt(x.var(-1, unbiased=False, keepdim=True) + eps)


@pytest.mark.parametrize("epilogue,ms,n,k,wide,shift", [("bias", (512, 64, 32), 4608, 1536, False, 0.0),
                                                        ("swiglu_packed", (512, 64, 32), 8192, 1536, False, 0.0),
                                                        ("swiglu_packed", (82, 18), 12288, 1536, True, 0.0),
                                                        ("bias", (300, 18), 4608, 2048, False, 0.0),
                                                        ("bias", (96, 33), 1024, 512, False, 3.0),
                                                        ("swiglu_packed", (20,), 256, 384, False, -2.0)])
def test_grouped_gemm_layernorm_fold(dev, epilogue, ms, n, k, wide, shift):
    """The pre-LayerNorm folded into the GEMM (rldx_grouped_gemm_ln_bf16): from the
    un-normalised rows x and their statistics (rldx_act_pack_stats_bf16), the
    result matches LN(x) W^T + b (LN in fp64, then the epilogue's eager rounding)
    to the bf16 contract, also for rows whose mean is 3 or 2 standard deviations
    away from 0 (E[x^2] - mean^2 in fp32), and it agrees with the eager path
    (LayerNorm-pack, then the GEMM) to the same bound; tile shapes 128 x 128,
    64 x 64, 32 x 64 and the wide 64 x 128 / 32 x 128, the largest K the fold
    takes (2048, 8 statistics slots per thread at 128-row tiles)."""
    g = torch.Generator().manual_seed(n + k + sum(ms))
    swiglu = epilogue.startswith("swiglu")
    n_out = n // 2 if swiglu else n
    items, eager_items, refs, stats = [], [], [], []
    for m in ms:
        x = (_rand((m, k), g).float() + shift).to(BF16)
        # |outputs| < 4, where one bf16 ulp stays below the 2e-2 bound (the fold and the
        # eager path round the normalised rows differently, so single roundings can flip)
        w = _rand((n, k), g, std=(0.3 if swiglu else 0.5) * k ** -0.5)
        b = _rand((n,), g, 0.1)
        pw = Fn.pack_weight(w.to(dev), swiglu_pairs=swiglu)
        mk = (lambda: Fn.PackedAct.empty(m, n_out, dev)) if swiglu else (
            lambda: torch.empty(m, n_out, dtype=BF16, device=dev))
        st = Fn.ln_stats_empty(m, k, dev)
        items.append((Fn.pack_act(x.to(dev), stats=st), pw, b.to(dev), mk(), None))
        stats.append(st)
        eager_items.append((Fn.layernorm_pack(x.to(dev), 1e-6), pw, b.to(dev), mk(), None))
        y = (_ln_ref(x) @ w.double().t() + b.double()).float().to(BF16)
        refs.append(ref.swiglu(y) if swiglu else y)
    Fn.grouped_gemm(items, epilogue, wide_tiles=wide, ln_eps=1e-6, ln_stats=stats)
    Fn.grouped_gemm(eager_items, epilogue, wide_tiles=wide)
    torch.cuda.synchronize()
    for it, ei, r in zip(items, eager_items, refs):
        got = it[3].unpack() if swiglu else it[3]
        eager = ei[3].unpack() if swiglu else ei[3]
        assert_bf16_close(got, r, f"LayerNorm-folded {epilogue}")
        assert_bf16_close(got, eager, f"LayerNorm-folded {epilogue} vs LayerNorm-pack + GEMM")
    with pytest.raises(RuntimeError):  # the fold does not split K
        Fn.grouped_gemm(items, epilogue, split_k=2, workspace=Fn.GemmWorkspace(1 << 20, dev), ln_eps=1e-6,
                        ln_stats=stats)


@pytest.mark.parametrize("shift", [30.0, 100.0])
def test_grouped_gemm_layernorm_fold_large_row_offsets(dev, shift):
    """Rows whose mean is 30 or 100 standard deviations away from 0: the fold's
    E[x^2] - mean^2 (fp32 over K = 1536) and rstd (x W^T - mean s) cancel
    there.  Bound: the bf16 contract against LN(x) W^T + b with LN in fp64 on
    the same bf16 rows, and against the eager path (LayerNorm-pack, then the
    GEMM).  The bf16 rows themselves are coarse at that offset (one ulp at 100
    is 0.5), which both references see too."""
    g = torch.Generator().manual_seed(int(shift))
    m, n, k = 64, 256, 1536
    x = (_rand((m, k), g).float() + shift).to(BF16)
    w = _rand((n, k), g, std=0.5 * k ** -0.5)
    b = _rand((n,), g, 0.1)
    pw = Fn.pack_weight(w.to(dev))
    st = Fn.ln_stats_empty(m, k, dev)
    fold = torch.empty(m, n, dtype=BF16, device=dev)
    eager = torch.empty(m, n, dtype=BF16, device=dev)
    Fn.grouped_gemm([(Fn.pack_act(x.to(dev), stats=st), pw, b.to(dev), fold, None)], "bias", ln_eps=1e-6,
                    ln_stats=[st])
    Fn.grouped_gemm([(Fn.layernorm_pack(x.to(dev), 1e-6), pw, b.to(dev), eager, None)], "bias")
    torch.cuda.synchronize()
    r = (_ln_ref(x) @ w.double().t() + b.double()).float().to(BF16)
    s = assert_bf16_close(fold, r, f"LayerNorm fold, rows {shift} sigma off zero")
    print(f"LayerNorm fold at {shift} sigma: {s}")
    assert_bf16_close(fold, eager, f"LayerNorm fold vs LayerNorm-pack + GEMM, rows {shift} sigma off zero")


def _slot_sums(x: torch.Tensor) -> torch.Tensor:
    """fp64 (sum, sum of squares) of every 64-column slot of every row, slot-major:
    [k / 64, m, 2]."""
    v = x.double().reshape(x.shape[0], -1, 64)
    return torch.stack([v.sum(-1), (v * v).sum(-1)], dim=-1).transpose(0, 1)


@pytest.mark.parametrize("rows,k", [(((0, 512), (512, 576), (576, 608)), 4096),
                                    (((0, 300), (320, 360), (384, 404)), 1536)])
def test_grouped_gemm_residual_packed_epilogue_bit_identical(dev, rows, k):
    """RLDX_GEMM_EPI_RESIDUAL_PACKED (the residual stream held in the packed
    activation order, updated in place) gives the row-major residual epilogue's
    bits, with and without split-K; with stats_out (rldx_grouped_gemm_stats_bf16)
    the same bits again, and per row and 64-column slot the sum and sum of
    squares of the stored values (fp32 against fp64: relative 1e-5).  Without
    split-K the 64 x 64 tiles of the launch (one workgroup per CU) finish in
    registers; ragged streams (300 / 40 / 20 rows, each starting on a 32-row
    boundary of the packed stream) give them a partial last row tile."""
    g = torch.Generator().manual_seed(23 + k)
    n = 1536
    m_all = rows[-1][1]
    x = _rand((m_all, n), g, 0.5).to(dev)
    h = _rand((m_all, k), g).to(dev)
    ws = [(_rand((n, k), g, 0.008).to(dev), _rand((n,), g, 0.1).to(dev)) for _ in range(3)]
    for split in (1, 4):
        xr, xp = x.clone(), Fn.pack_act(x)
        it_r = [(h[lo:hi], Fn.pack_weight(w), b, xr[lo:hi], xr[lo:hi]) for (lo, hi), (w, b) in zip(rows, ws)]
        it_p = [(h[lo:hi], Fn.pack_weight(w), b, xp.rows(lo, hi), xp.rows(lo, hi)) for (lo, hi), (w, b) in zip(rows, ws)]
        wsr = Fn.GemmWorkspace(Fn.grouped_gemm_workspace_bytes(it_r, "residual", split), dev) if split > 1 else None
        wsp = Fn.GemmWorkspace(Fn.grouped_gemm_workspace_bytes(it_p, "residual_packed", split), dev) if split > 1 \
            else None
        xs = Fn.pack_act(x)
        it_s = [(h[lo:hi], Fn.pack_weight(w), b, xs.rows(lo, hi), xs.rows(lo, hi)) for (lo, hi), (w, b) in zip(rows, ws)]
        sts = [Fn.ln_stats_empty(hi - lo, n, dev) for lo, hi in rows]
        Fn.grouped_gemm(it_r, "residual", split_k=split, workspace=wsr)
        Fn.grouped_gemm(it_p, "residual_packed", split_k=split, workspace=wsp)
        Fn.grouped_gemm(it_s, "residual_packed", split_k=split, workspace=wsp, stats_out=sts)
        torch.cuda.synchronize()
        assert torch.equal(xp.unpack().view(torch.int16), xr.view(torch.int16)), f"split {split}"
        assert torch.equal(xs.unpack().view(torch.int16), xr.view(torch.int16)), f"split {split}, stats"
        for (lo, hi), st in zip(rows, sts):
            ref_st = _slot_sums(xr[lo:hi].cpu())
            err = (st.cpu().double() - ref_st).abs().max().item()
            assert err <= 1e-5 * ref_st.abs().max().item(), f"split {split}, rows {lo}: statistics off by {err}"


@pytest.mark.parametrize("ms,n,ln", [((512, 64, 32), 8192, False), ((512, 64, 32), 8192, True),
                                     ((300, 64, 32), 8256, False), ((300, 64, 32), 8256, True),
                                     ((257,), 16448, True)])
def test_swiglu_packed_register_epilogue_bit_identical(dev, ms, n, ln):
    """The packed SwiGLU epilogue of the 128 x 128 tiles (streams of >= 256 rows)
    finishes in registers in the narrow kernel; the wide kernel runs the same
    tiles and K-groups through the fp32 tile and the store phase.  Both give the
    same bits, with and without the LayerNorm fold, also for a partial last row
    tile (300, 257 rows) and a partial last column tile (n / 2 = 4128, 8224:
    half of the last 64-column tile past the outputs)."""
    g = torch.Generator().manual_seed(sum(ms) + n + ln)
    k = 1536
    data = []
    for m in ms:
        x = _rand((m, k), g).to(dev)
        w = Fn.pack_weight(_rand((n, k), g, std=0.3 * k ** -0.5).to(dev), swiglu_pairs=True)
        b = _rand((n,), g, 0.1).to(dev)
        data.append((x, w, b))
    outs = []
    for wide in (False, True):
        items, stats = [], []
        for x, w, b in data:
            st = Fn.ln_stats_empty(x.shape[0], k, dev) if ln else None
            items.append((Fn.pack_act(x, stats=st) if ln else Fn.pack_act(x), w, b,
                          Fn.PackedAct.empty(x.shape[0], n // 2, dev), None))
            stats.append(st)
        Fn.grouped_gemm(items, "swiglu_packed", wide_tiles=wide, ln_eps=1e-6 if ln else None,
                        ln_stats=stats if ln else None)
        torch.cuda.synchronize()
        outs.append([it[3].unpack().clone() for it in items])
    for x, y in zip(*outs):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))
    if not ln:  # and the row-major SwiGLU epilogue (store phase) gives the same bits as well
        for (x, w, b), got in zip(data, outs[0]):
            rm = torch.empty(x.shape[0], n // 2, dtype=BF16, device=dev)
            Fn.grouped_gemm([(Fn.pack_act(x), w, b, rm, None)], "swiglu")
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16), rm.view(torch.int16))


@pytest.mark.parametrize("ms,H,k", [((512, 64, 32), 12, 1536), ((64, 470), 12, 1536), ((40,), 3, 384)])
def test_grouped_gemm_qkv_norm_rope_layernorm_fold(dev, ms, H, k):
    """The QKV epilogue with the LayerNorm fold is bit-identical to the folded
    bias GEMM followed by rldx_msat_qkv_norm_rope_bf16 (same fold arithmetic in
    both epilogues), and within the bf16 contract of the eager path (LayerNorm-
    pack + QKV epilogue) on Q."""
    from rldx_amd.msat_step import msat_rope_tables

    g = torch.Generator().manual_seed(sum(ms) + H + k + 1)
    D, n = 128, 3 * H * 128
    items, eager, specs, qkv_items, stats = [], [], [], [], []
    for i, m in enumerate(ms):
        x = _rand((m, k), g).to(dev)
        w = Fn.pack_weight(_rand((n, k), g, std=k ** -0.5).to(dev))
        b = _rand((n,), g, std=0.5).to(dev)
        # norm weights ~0.5: |Q|, |K| < 4, where one bf16 ulp stays below the 2e-2 bound
        qw = (0.5 + 0.1 * torch.randn(D, generator=g)).to(BF16).to(dev)
        kw = (0.5 + 0.1 * torch.randn(D, generator=g)).to(BF16).to(dev)
        cos = sin = None
        if i > 0:
            ids = torch.stack([torch.zeros(m, dtype=torch.long), torch.arange(m) + 3 * i], dim=-1)
            cos, sin = (t.to(dev) for t in msat_rope_tables(ids, D, 10000.0))
        qkv = torch.empty(m, n, dtype=BF16, device=dev)
        stats.append(Fn.ln_stats_empty(m, k, dev))
        items.append((Fn.pack_act(x, stats=stats[-1]), w, b))
        eager.append((Fn.layernorm_pack(x, 1e-6), w, b))
        qkv_items.append((Fn.pack_act(x), w, b, qkv, None))
        specs.append(Fn.StreamSpec(qkv, qw, kw, cos, sin))
    q, kvp = Fn.grouped_gemm_qkv_norm_rope(items, specs, H, D, 1e-6, ln_eps=1e-6, ln_stats=stats)
    Fn.grouped_gemm(qkv_items, "bias", ln_eps=1e-6, ln_stats=stats)
    q2, kvp2 = Fn.msat_qkv_norm_rope(specs, H, D, 1e-6, kv_packed=True)
    q3, _ = Fn.grouped_gemm_qkv_norm_rope(eager, specs, H, D, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(q.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(kvp.view(torch.int16), kvp2.view(torch.int16))
    assert_bf16_close(q, q3, "QKV epilogue with the LayerNorm fold vs LayerNorm-pack + QKV epilogue")
