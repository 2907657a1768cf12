"""CPU tests of the C ABI library: it loads, exports every declared symbol, the
device SwiGLU element function is exact on all bf16 inputs (run on the host),
and argument validation rejects bad calls before any GPU work."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import cpu_reference as ref
from rldx_amd import _lib
from rldx_amd import functional as Fn

HEADER = Path(__file__).resolve().parents[1] / "include" / "rldx_amd.h"
HIP_INVALID_VALUE = 1


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:hipError_t|int64_t|int)\s+(rldx_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "rldx_attention_fwd_bf16" in names and len(names) >= 7, names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in rldx_amd.h but not exported"
    assert set(declared_functions()) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"


def test_host_swiglu_exhaustive_bitexact():
    """All 65536 bf16 gate values x several up values: the exact device element
    function, executed on the CPU, reproduces eager `F.silu(x1) * x2` bit for bit."""
    gates = np.arange(65536, dtype=np.uint16)
    g_t = torch.from_numpy(gates.view(np.int16).copy()).view(torch.bfloat16)
    for up in (1.0, -1.0, 2.5, -0.0078125, 7.0, 1e30):
        u_t = torch.full((65536,), up, dtype=torch.bfloat16)
        ups = u_t.view(torch.int16).numpy().view(np.uint16)
        mine = Fn.host_swiglu_bf16_bits(gates, ups)
        r = ref.swiglu(torch.cat([g_t, u_t])[None, :])[0]
        rb = r.view(torch.int16).numpy().view(np.uint16)
        nan = np.isnan(r.float().numpy()) & np.isnan(torch.from_numpy(mine.view(np.int16)).view(torch.bfloat16).float().numpy())
        bad = (mine != rb) & ~nan
        assert not bad.any(), f"up={up}: {int(bad.sum())} mismatches, first gate bits {gates[bad][:5]}"


def test_host_swiglu_random_pairs():
    rng = np.random.default_rng(0)
    g = rng.integers(0, 65536, size=200000, dtype=np.uint16)
    u = rng.integers(0, 65536, size=200000, dtype=np.uint16)
    mine = Fn.host_swiglu_bf16_bits(g, u)
    gt = torch.from_numpy(g.view(np.int16).copy()).view(torch.bfloat16)
    ut = torch.from_numpy(u.view(np.int16).copy()).view(torch.bfloat16)
    r = ref.swiglu(torch.cat([gt, ut])[None, :])[0]
    rb = r.view(torch.int16).numpy().view(np.uint16)
    both_nan = np.isnan(r.float().numpy()) & np.isnan(torch.from_numpy(mine.view(np.int16)).view(torch.bfloat16).float().numpy())
    assert not ((mine != rb) & ~both_nan).any()


def test_epilogue_norm_abi_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    p = 16  # stand-in device address: every call below must fail validation before any launch
    # row wider than 8192
    assert lib.rldx_grouped_res_ln_bf16(p, p, p, p, p, p, p, p, 1, 1, 8200, 16, 1e-6, None) == HIP_INVALID_VALUE
    # negative rows, null operand with work to do, negative eps
    assert lib.rldx_grouped_res_ln_bf16(p, p, p, p, p, p, p, p, -1, 1, 16, 16, 1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_grouped_res_ln_bf16(p, None, p, p, p, p, p, p, 2, 0, 16, 16, 1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_grouped_res_ln_bf16(p, p, p, p, p, p, p, p, 2, 2, 16, 16, -1.0, None) == HIP_INVALID_VALUE
    # zero-width rows with work to do
    assert lib.rldx_ss_epilogue_ln_bf16(p, None, None, p, 3, 0, 1e-6, None) == HIP_INVALID_VALUE
    # missing new-hidden output
    assert lib.rldx_vl_epilogue_ln_bf16(p, p, p, p, None, p, 2, 16, 1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_ss_epilogue_ln_bf16(p, p, None, p, 2, 16, 1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_add_rmsnorm_bf16(p, p, None, p, None, p, 2, 16, 1e-6, None) == HIP_INVALID_VALUE
    # RMSNorm without a weight
    assert lib.rldx_add_rmsnorm_bf16(p, p, None, None, p, p, 2, 16, 1e-6, None) == HIP_INVALID_VALUE
    # nothing to do
    assert lib.rldx_grouped_res_ln_bf16(None, None, None, None, None, None, None, None, 0, 0, 16, 16, 1e-6,
                                        None) == 0
    assert lib.rldx_add_rmsnorm_bf16(None, None, None, None, None, None, 0, 2048, 1e-6, None) == 0


def test_model_ops_abi_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    p = 16  # stand-in device address, 16-byte aligned: every call below must fail validation
    # RMSNorm: width not a multiple of 8 (bf16) / 4 (fp32), wider than 8192, row stride below the width,
    # missing weight, negative eps, misaligned fp32 weight
    assert lib.rldx_rms_norm_bf16(p, 12, p, 1, p, 12, 2, 12, 1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_rms_norm_bf16(p, 8200, p, 1, p, 8200, 2, 8200, 1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_rms_norm_f32(p, 6, p, 1, p, 8, 2, 6, 1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_rms_norm_f32(p, 64, p, 1, p, 32, 2, 64, 1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_rms_norm_bf16(p, 64, None, 1, p, 64, 2, 64, 1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_rms_norm_bf16(p, 64, p, 1, p, 64, 2, 64, -1.0, None) == HIP_INVALID_VALUE
    assert lib.rldx_rms_norm_bf16(p, 64, p + 4, 1, p, 64, 2, 64, 1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_rms_norm_bf16(None, 64, None, 1, None, 64, 0, 64, 1e-6, None) == 0  # nothing to do
    # interleaved RoPE: head_dim not a multiple of 8, odd table stride, table rows narrower than D / 2,
    # misaligned table, missing output
    st = _lib.i64_array([64 * 4 * 8, 64 * 8, 64])
    fs = _lib.i64_array([0, 32])
    args = (p, st, p, st, p, st, p, st, 1, 4, 4, 8)
    assert lib.rldx_rope_interleaved_bf16(*args, 60, p, fs, None) == HIP_INVALID_VALUE
    assert lib.rldx_rope_interleaved_bf16(*args, 64, p, _lib.i64_array([0, 33]), None) == HIP_INVALID_VALUE
    assert lib.rldx_rope_interleaved_bf16(*args, 64, p, _lib.i64_array([0, 16]), None) == HIP_INVALID_VALUE
    assert lib.rldx_rope_interleaved_bf16(*args, 64, p + 8, fs, None) == HIP_INVALID_VALUE
    assert lib.rldx_rope_interleaved_f32(p, st, None, st, p, st, p, st, 1, 4, 4, 8, 64, p, fs,
                                         None) == HIP_INVALID_VALUE
    # rotate-half RoPE alone: weights may be null; unknown flag bits are rejected
    cs = _lib.i64_array([0, 64])
    assert lib.rldx_qk_rmsnorm_rope_half_bf16(p, p, None, None, p, p, p, p, 1, 4, 2, 2, 64, st, st, st, st, cs, 1e-6,
                                              8, None) == HIP_INVALID_VALUE
    assert lib.rldx_qk_rmsnorm_rope_half_bf16(p, p, None, None, p, p, p, p, 1, 4, 2, 2, 64, st, st, st, st, cs, 1e-6,
                                              0, None) == HIP_INVALID_VALUE  # norm without weights


def test_capi_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    # ldx smaller than 2*n_half
    assert lib.rldx_swiglu_bf16(16, 4, None, 16, 8, 2, 8, None) == HIP_INVALID_VALUE
    # negative rows
    assert lib.rldx_swiglu_bf16(16, 16, None, 16, 8, -1, 8, None) == HIP_INVALID_VALUE
    # null pointers with work to do
    assert lib.rldx_swiglu_bf16(None, 16, None, None, 8, 2, 8, None) == HIP_INVALID_VALUE
    st = _lib.i64_array([0, 0, 0])
    # unsupported head_dim
    big = 1 << 30
    assert lib.rldx_attention_fwd_bf16(16, 16, 16, 16, 1, 1, 1, 4, 4, 96, st, st, st, st, None, 0, 1.0, 0, 16, big,
                                       None) == HIP_INVALID_VALUE
    # q heads not a multiple of kv heads
    assert lib.rldx_attention_fwd_bf16(16, 16, 16, 16, 1, 3, 2, 4, 4, 128, st, st, st, st, None, 0, 1.0, 0, 16, big,
                                       None) == HIP_INVALID_VALUE
    # misaligned pointer
    assert lib.rldx_attention_fwd_bf16(18, 16, 16, 16, 1, 2, 2, 4, 4, 128, st, st, st, st, None, 0, 1.0, 0, 16, big,
                                       None) == HIP_INVALID_VALUE
    # workspace too small for the packed K/V copy (1 tile of 32 keys x 2 heads)
    need = lib.rldx_attention_workspace_bytes(1, 2, 4, 128)
    assert need == 2 * 64 * 128 * 2
    assert lib.rldx_attention_kv_packed_elems(33, 64) == 2 * 64 * 64
    assert lib.rldx_attention_fwd_bf16(16, 16, 16, 16, 1, 2, 2, 4, 4, 128, st, st, st, st, None, 0, 1.0, 0, 16,
                                       need - 2, None) == HIP_INVALID_VALUE
    # non-positive softmax scale
    assert lib.rldx_attention_fwd_bf16(16, 16, 16, 16, 1, 2, 2, 4, 4, 128, st, st, st, st, None, 0, 0.0, 0, 16,
                                       need, None) == HIP_INVALID_VALUE
    # packed head stride shorter than the tiles of seq_k = 40 (2 tiles)
    ps = _lib.i64_array([0, 64 * 128])
    assert lib.rldx_attention_packed_fwd_bf16(16, 16, ps, 16, 0, 1, 2, 2, 4, 40, 128, st, st, None, 0, 1.0, 0,
                                              None) == HIP_INVALID_VALUE
    # packed output needs batch 1
    assert lib.rldx_attention_packed_fwd_bf16(16, 16, ps, 16, 1, 2, 2, 2, 4, 32, 128, st, st, None, 0, 1.0, 0,
                                              None) == HIP_INVALID_VALUE
    assert lib.rldx_attention_kv_pack_bf16(16, st, 16, st, 16, ps, 1, 1, 40, 128, None) == HIP_INVALID_VALUE
    # row segments of a packed output: rejected before any launch when absent, out of order, overlapping,
    # past seq_q, without a packed output, or mapping a packed row past 2^31
    ps2 = _lib.i64_array([12 * 64 * 128 * 19, 64 * 128 * 19])

    def seg_call(segs, out_packed=1, batch=3):
        flat = _lib.i64_array([v for sg in segs for v in sg]) if segs else None
        return lib.rldx_attention_packed_segments_fwd_bf16(16, 16, ps2, 16, out_packed, flat, len(segs), batch, 12,
                                                          12, 608, 608, 128, st, None, 0, 1.0, 0, None)
    for segs in ([], [(0, 512, 0), (500, 64, 1536)], [(512, 64, 0), (0, 512, 192)], [(0, 600, 0), (600, 9, 1800)],
                 [(-1, 4, 0)], [(0, 4, -32)], [(0, 4, 0)] * 4, [(0, 608, (1 << 31) - 1000)]):
        assert seg_call(segs) == HIP_INVALID_VALUE, segs
    assert seg_call([(0, 512, 0)], out_packed=0) == HIP_INVALID_VALUE
    assert lib.rldx_msat_qkv_norm_rope_bf16(None, 1, 12, 128, 16, 16, 16, 0, 0, None, 0, 1e-6,
                                            None) == HIP_INVALID_VALUE
    s = _lib.MsatStream(16, 100, 4, 16, 16, None, None, 0)  # row stride < 3*H*D
    assert lib.rldx_msat_qkv_norm_rope_bf16(ctypes.byref(s), 1, 12, 128, 16, 16, 16, 0, 0, None, 0, 1e-6,
                                            None) == HIP_INVALID_VALUE
    # batched form: batch out of range, or a negative row step between batch entries
    s = _lib.MsatStream(16, 4608, 4, 16, 16, None, None, 0)
    for batch, rows in ((65536, 4), (-1, 4), (2, -4)):
        assert lib.rldx_msat_qkv_norm_rope_batch_bf16(ctypes.byref(s), 1, batch, _lib.i64_array([rows]), 12, 128, 16,
                                                      None, None, 0, 0, 0, 16, 64 * 128, 64 * 128, 1e-6,
                                                      None) == HIP_INVALID_VALUE
    assert lib.rldx_msat_qkv_norm_rope_batch_bf16(ctypes.byref(s), 1, 2, None, 12, 128, 16, None, None, 0, 0, 0, 16,
                                                  64 * 128, 64 * 128, 1e-6, None) == HIP_INVALID_VALUE
    s = _lib.MsatStream(16, 4608, 40, 16, 16, None, None, 0)  # packed head stride < 2 tiles
    assert lib.rldx_msat_qkv_norm_rope_bf16(ctypes.byref(s), 1, 12, 128, 16, None, None, 0, 0, 16, 64 * 128,
                                            1e-6, None) == HIP_INVALID_VALUE
    # empty key set with queries present
    ps = _lib.i64_array([0, 0])
    assert lib.rldx_attention_packed_fwd_bf16(16, 16, ps, 16, 0, 1, 2, 2, 4, 0, 128, st, st, None, 0, 1.0, 0,
                                              None) == HIP_INVALID_VALUE
    assert lib.rldx_qk_rmsnorm_rope_half_f32(16, 16, 16, 16, 16, 16, 16, 16, 1, 4, 2, 2, 96, st, st, st, st, st,
                                             1e-6, 0, None) == HIP_INVALID_VALUE
    # fused LLM attention: workspace too small / kv heads not dividing q heads
    assert lib.rldx_llm_fused_attention_bf16(16, 4608, 16, 16, 16, 16, 128, 1, 16, 3584, 1280, 28, 4, 128, 1e-6, 16,
                                             8, None) == HIP_INVALID_VALUE
    assert lib.rldx_llm_fused_attention_bf16(16, 4608, 16, 16, 16, 16, 128, 1, 16, 3584, 1280, 28, 3, 128, 1e-6, 16,
                                             1 << 30, None) == HIP_INVALID_VALUE
    assert lib.rldx_llm_fused_attention_workspace_bytes(1280, 4, 128) == 4 * 40 * 64 * 128 * 2


QKV_INTERNAL = 16  # the fused QKV epilogue's internal code: only rldx_grouped_gemm_qkv_norm_rope_bf16 takes it


def _gemm_groups(ms, a_ptr=256, w_ptr=512, out_ptr=1024, ldo=8192):
    groups = (_lib.GemmGroup * len(ms))()
    for i, m in enumerate(ms):
        groups[i] = _lib.GemmGroup(a_ptr, m, w_ptr, None, out_ptr, ldo, out_ptr, ldo)
    return groups


def test_grouped_gemm_split_plan_and_rejections():
    """The split-K plan is a host-side function of the shapes and split_k: every
    group's K stages are split by the largest power of two <= split_k dividing
    them; a too small, missing or misaligned workspace and unsupported shapes are
    rejected before anything is launched."""
    lib = _lib.load()
    msat = (512, 64, 32)
    # W3 shapes (n 1536, k 4096): 512 rows -> 192 tiles of 64 x 64, 64 rows -> 24,
    # 32 rows -> 24 tiles of 32 x 64; 16 KB of partials per tile and split
    w3 = lib.rldx_grouped_gemm_workspace_bytes(_gemm_groups(msat), 3, 1536, 4096, 1, 8)
    assert w3 == 65536 + (192 + 24 + 24) * 8 * 16384
    assert lib.rldx_grouped_gemm_workspace_bytes(_gemm_groups(msat), 3, 1536, 4096, 1, 1) == 0
    # split_k 6 -> 4; k 1536 gives 12 stages in the 32 x 64 tiles' four K-groups: 8 does not divide them
    assert lib.rldx_grouped_gemm_workspace_bytes(_gemm_groups((32,)), 1, 1536, 4096, 1, 6) == 65536 + 24 * 4 * 16384
    assert lib.rldx_grouped_gemm_workspace_bytes(_gemm_groups((32,)), 1, 1536, 1536, 1, 8) == 65536 + 24 * 4 * 16384
    assert lib.rldx_grouped_gemm_workspace_bytes(_gemm_groups(msat), 3, 8192, 1000, 3, 2) == -1   # k % 128
    assert lib.rldx_grouped_gemm_workspace_bytes(_gemm_groups(msat), 3, 8160, 1536, 0, 2) == -1   # n % 64
    g = _gemm_groups(msat)
    assert lib.rldx_grouped_gemm_ws_bf16(g, 3, 1536, 4096, 1, 8, 4096, w3 - 256, None) == HIP_INVALID_VALUE
    assert lib.rldx_grouped_gemm_ws_bf16(g, 3, 1536, 4096, 1, 8, 4096 + 16, w3, None) == HIP_INVALID_VALUE
    assert lib.rldx_grouped_gemm_ws_bf16(g, 3, 1536, 4096, 1, 8, None, w3, None) == HIP_INVALID_VALUE
    assert lib.rldx_grouped_gemm_ws_bf16(_gemm_groups(msat, a_ptr=264), 3, 1536, 4096, 1, 8, 4096, w3,
                                         None) == HIP_INVALID_VALUE
    assert lib.rldx_grouped_gemm_bf16(_gemm_groups(msat), 3, 1536, 4096, 7, None) == HIP_INVALID_VALUE


def test_grouped_gemm_wide_tiles_plan():
    """RLDX_GEMM_WIDE_TILES: streams below the 128 x 128 threshold take 64 x 128 /
    32 x 128 tiles (W3 shapes, split 8: 96 + 12 tiles of 64 x 128 with 32 KB of
    partials per split, 12 tiles of 32 x 128 with 16 KB); RLDX_GEMM_SPLITS_ACROSS_XCDS
    needs no other workspace; unknown flag bits and the QKV epilogue are rejected."""
    lib = _lib.load()
    msat = (512, 64, 32)
    wide = lib.rldx_grouped_gemm_ex_workspace_bytes(_gemm_groups(msat), 3, 1536, 4096, 1, 8, 1)
    assert wide == 65536 + (96 + 12) * 8 * 32768 + 12 * 8 * 16384
    assert lib.rldx_grouped_gemm_ex_workspace_bytes(_gemm_groups(msat), 3, 1536, 4096, 1, 8, 0) == \
        lib.rldx_grouped_gemm_workspace_bytes(_gemm_groups(msat), 3, 1536, 4096, 1, 8)
    # RLDX_GEMM_SPLITS_ACROSS_XCDS moves workgroups, not partials: the same workspace
    assert lib.rldx_grouped_gemm_ex_workspace_bytes(_gemm_groups(msat), 3, 1536, 4096, 1, 8, 3) == wide
    assert lib.rldx_grouped_gemm_ex_workspace_bytes(_gemm_groups(msat), 3, 1536, 4096, 1, 8, 4) == -1
    assert lib.rldx_grouped_gemm_ex_workspace_bytes(_gemm_groups(msat), 3, 4608, 1536, QKV_INTERNAL, 1, 1) == -1
    assert lib.rldx_grouped_gemm_ex_bf16(_gemm_groups(msat), 3, 1536, 4096, 1, 1, 4, None, 0, None) == HIP_INVALID_VALUE
    assert lib.rldx_grouped_gemm_ex_bf16(_gemm_groups(msat), 3, 1536, 4096, 1, 8, 1, 4096, wide - 256,
                                         None) == HIP_INVALID_VALUE


def test_grouped_gemm_mixed_plan_and_rejections():
    """rldx_grouped_gemm_mixed_bf16: every group its own n, k and split; the
    workspace is the sum of the groups' partials (each as a one-group launch of
    its shape and split), and bad per-group shapes or splits, the QKV epilogue
    and missing shape arrays are rejected before anything is launched."""
    lib = _lib.load()
    i64, i32 = _lib.i64_array, lambda v: (ctypes.c_int32 * len(v))(*v)
    # DS-block W3 shapes: SA 18 x 1536 x 4096 (24 tiles of 32 x 64), VL 64 x 4096 x 11008 (64 tiles of 64 x 64)
    g = _gemm_groups((18, 64))
    ws = lib.rldx_grouped_gemm_mixed_workspace_bytes(g, i64([1536, 4096]), i64([4096, 11008]), i32([4, 2]), 2, 1, 0)
    one = [lib.rldx_grouped_gemm_workspace_bytes(_gemm_groups((m,)), 1, n, k, 1, s)
           for m, n, k, s in ((18, 1536, 4096, 4), (64, 4096, 11008, 2))]
    assert ws == 65536 + sum(o - 65536 for o in one) == 65536 + 24 * 4 * 16384 + 64 * 2 * 16384
    assert lib.rldx_grouped_gemm_mixed_workspace_bytes(g, i64([1536, 4096]), i64([4096, 11008]), i32([1, 1]), 2, 1,
                                                       0) == 0
    bad = [(i64([1536, 4000]), i64([4096, 11008]), i32([1, 1]), 1),      # n % 64
           (i64([1536, 4096]), i64([4096, 11000]), i32([1, 1]), 1),      # k % 128
           (i64([1536, 4096]), i64([4096, 11008]), i32([1, 0]), 1),      # split < 1
           (i64([1536, 4096]), i64([4096, 11008]), i32([1, 65]), 1),     # split > 64
           (None, i64([4096, 11008]), i32([1, 1]), 1),
           (i64([1536, 4096]), None, i32([1, 1]), 1),
           (i64([1536, 4096]), i64([4096, 11008]), i32([1, 1]), QKV_INTERNAL)]
    for ns, ks, sp, epi in bad:
        assert lib.rldx_grouped_gemm_mixed_workspace_bytes(g, ns, ks, sp, 2, epi, 0) == -1
        assert lib.rldx_grouped_gemm_mixed_bf16(g, ns, ks, sp, None, 2, epi, 0, None, 0, None) == HIP_INVALID_VALUE
    assert lib.rldx_grouped_gemm_mixed_bf16(g, i64([1536, 4096]), i64([4096, 11008]), i32([1, 1]), None, 2, 1, 4,
                                            None, 0, None) == HIP_INVALID_VALUE                   # unknown flag
    assert lib.rldx_grouped_gemm_mixed_bf16(g, i64([1536, 4096]), i64([4096, 11008]), i32([4, 2]), None, 2, 1, 0,
                                            4096, ws - 256, None) == HIP_INVALID_VALUE            # workspace short


def test_layernorm_pack_many_rejections():
    """rldx_layernorm_pack_many_bf16 checks every matrix before launching: 1-4
    matrices, k % 16 == 0 and <= 8192, row stride >= k and a multiple of 8,
    16-byte aligned pointers; empty matrices are skipped (nothing to launch)."""
    lib = _lib.load()

    def rows(*specs):
        arr = (_lib.Rows * len(specs))()
        for i, (x, ldx, m, k, p) in enumerate(specs):
            arr[i] = _lib.Rows(x, ldx, m, k, p)
        return arr

    ok = (4096, 1536, 18, 1536, 8192)
    assert lib.rldx_layernorm_pack_many_bf16(rows(ok), 0, 1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_layernorm_pack_many_bf16(rows(ok, ok, ok, ok, ok), 5, 1e-6, None) == HIP_INVALID_VALUE
    for bad in [(4096, 1536, 18, 1544, 8192),       # k % 16
                (4096, 8208, 18, 8208, 8192),       # k > 8192
                (4096, 1532, 18, 1536, 8192),       # ldx < k
                (4096, 1540, 18, 1536, 8192),       # ldx % 8
                (4104, 1536, 18, 1536, 8192),       # x misaligned
                (4096, 1536, 18, 1536, 8200),       # packed misaligned
                (None, 1536, 18, 1536, 8192),
                (4096, 1536, -1, 1536, 8192)]:
        assert lib.rldx_layernorm_pack_many_bf16(rows(ok, bad), 2, 1e-6, None) == HIP_INVALID_VALUE, bad
    # nothing to do: no launch, success
    assert lib.rldx_layernorm_pack_many_bf16(rows((None, 0, 0, 1536, None), (None, 0, 5, 0, None)), 2, 1e-6,
                                             None) == 0


def test_attention_warm_up_rejections():
    """rldx_attention_packed_fwd_warm_bf16 checks its warm-up ranges before
    anything else: 0-3 of them, non-negative lengths, 4-byte aligned non-null
    pointers where a range is not empty."""
    lib = _lib.load()
    st = _lib.i64_array([0, 0, 0])
    ps = _lib.i64_array([0, 64 * 128 * 2 * 19])

    def call(ptrs, nbytes, count):
        p = (ctypes.c_void_p * max(1, len(ptrs)))(*ptrs) if ptrs is not None else None
        b = _lib.i64_array(nbytes) if nbytes is not None else None
        return lib.rldx_attention_packed_fwd_warm_bf16(16, 16, ps, 16, 1, 1, 12, 12, 608, 608, 128, st, st, None, 0,
                                                       0.088, 0, p, b, count, None)

    assert call([256], [4096], 4) == HIP_INVALID_VALUE           # more than three ranges
    assert call([256], [4096], -1) == HIP_INVALID_VALUE
    assert call(None, [4096], 1) == HIP_INVALID_VALUE            # missing pointer array
    assert call([256], None, 1) == HIP_INVALID_VALUE             # missing length array
    assert call([256], [-128], 1) == HIP_INVALID_VALUE           # negative length
    assert call([258], [4096], 1) == HIP_INVALID_VALUE           # misaligned range
    assert call([None], [4096], 1) == HIP_INVALID_VALUE          # null range with bytes
    # a bad attention argument is still caught with valid ranges (scale <= 0)
    assert lib.rldx_attention_packed_fwd_warm_bf16(16, 16, ps, 16, 1, 1, 12, 12, 608, 608, 128, st, st, None, 0,
                                                   0.0, 0, (ctypes.c_void_p * 1)(256), _lib.i64_array([4096]), 1,
                                                   None) == HIP_INVALID_VALUE


def test_action_encode_decode_rejections():
    """rldx_action_encode_pack_bf16 / rldx_action_decode_euler_bf16 check every
    argument before launching: action_dim % 8 and <= 64, hidden % 64 and <= 2048,
    alignment, at most 3 more matrices with hidden columns; empty inputs launch
    nothing."""
    lib = _lib.load()
    A = 4096  # a 16-byte aligned stand-in address (nothing is launched)

    def enc(n=64, adim=32, hidden=1536, act=A, packed=A, stats=A, rows=None, count=0):
        rs = (_lib.Rows * max(1, count))(*(rows or []))
        st = (ctypes.c_void_p * max(1, count))(*([A] * count))
        return lib.rldx_action_encode_pack_bf16(act, n, adim, A, A, A, A, hidden, packed, stats, rs, st, count, None)

    assert enc(adim=30) == HIP_INVALID_VALUE
    assert enc(adim=72) == HIP_INVALID_VALUE
    assert enc(hidden=1500) == HIP_INVALID_VALUE
    assert enc(hidden=4096) == HIP_INVALID_VALUE
    assert enc(act=A + 8) == HIP_INVALID_VALUE
    assert enc(packed=None) == HIP_INVALID_VALUE
    assert enc(stats=A + 4) == HIP_INVALID_VALUE
    assert enc(count=4, rows=[_lib.Rows(A, 1536, 8, 1536, A)] * 4) == HIP_INVALID_VALUE
    assert enc(count=1, rows=[_lib.Rows(A, 1536, 8, 1024, A)]) == HIP_INVALID_VALUE   # k != hidden
    assert enc(count=1, rows=[_lib.Rows(A, 1532, 8, 1536, A)]) == HIP_INVALID_VALUE   # ldx < k
    assert enc(count=1, rows=[_lib.Rows(A + 2, 1536, 8, 1536, A)]) == HIP_INVALID_VALUE
    assert enc(n=0, count=1, rows=[_lib.Rows(None, 1536, 0, 1536, None)]) == 0        # nothing to do

    def dec(n=64, hidden=1536, eps=1e-6, adim=32, packed=A, act=A, b=A, dt=0.25):
        return lib.rldx_action_decode_euler_bf16(packed, n, hidden, eps, A, b, adim, dt, act, None)

    assert dec(adim=12) == HIP_INVALID_VALUE
    assert dec(hidden=2112) == HIP_INVALID_VALUE
    assert dec(eps=-1.0) == HIP_INVALID_VALUE
    assert dec(dt=float("nan")) == HIP_INVALID_VALUE
    assert dec(packed=A + 8) == HIP_INVALID_VALUE
    assert dec(act=None) == HIP_INVALID_VALUE
    assert dec(b=A + 1) == HIP_INVALID_VALUE
    assert dec(n=0) == 0


def _msat_norms(ms, rope_ld=0):
    d = (_lib.MsatStream * len(ms))()
    for i, m in enumerate(ms):
        d[i] = _lib.MsatStream(None, 0, m, 4096, 4352, 8192 if rope_ld else None, 12288 if rope_ld else None, rope_ld)
    return d


def test_grouped_gemm_qkv_norm_rope_rejections():
    """The fused QKV entry checks its arguments before anything is launched; the
    generic grouped GEMM entries do not accept its epilogue."""
    lib = _lib.load()
    msat = (512, 64, 32)

    def call(ms=msat, norm_ms=None, H=12, D=128, k=1536, q=1 << 20, qsh=608 * 128, qsm=128, kvp=1 << 24,
             kvsh=19 * 64 * 128, rope_ld=0):
        return lib.rldx_grouped_gemm_qkv_norm_rope_bf16(_gemm_groups(ms), _msat_norms(norm_ms or ms, rope_ld), len(ms),
                                                        H, D, k, q, qsh, qsm, kvp, kvsh, 1e-6, None)

    assert call(norm_ms=(512, 64, 31)) == HIP_INVALID_VALUE        # rows differ from the GEMM group's
    # streams start 32-key tiles: 20 + 20 + 20 rows take 3 tiles (84 joint rows), not 2
    assert call(ms=(20, 20, 20), kvsh=2 * 64 * 128) == HIP_INVALID_VALUE
    assert call(D=96) == HIP_INVALID_VALUE                          # head_dim 128 or 64
    assert call(D=64, H=3) == HIP_INVALID_VALUE                     # 64 needs an even head count (whole tiles)
    assert call(k=1000) == HIP_INVALID_VALUE                        # k % 128
    assert call(kvsh=19 * 64 * 128 - 8) == HIP_INVALID_VALUE        # packed K/V head stride too small
    assert call(q=(1 << 20) + 8) == HIP_INVALID_VALUE               # Q not 16-byte aligned
    assert call(qsm=132) == HIP_INVALID_VALUE                       # Q row stride % 8
    assert call(rope_ld=60) == HIP_INVALID_VALUE                    # RoPE rows shorter than head_dim / 2
    assert call(H=0) == HIP_INVALID_VALUE
    assert lib.rldx_grouped_gemm_bf16(_gemm_groups(msat), 3, 4608, 1536, QKV_INTERNAL, None) == HIP_INVALID_VALUE
    assert lib.rldx_grouped_gemm_workspace_bytes(_gemm_groups(msat), 3, 4608, 1536, QKV_INTERNAL, 1) == -1
    for internal in (QKV_INTERNAL, QKV_INTERNAL + 1):
        assert lib.rldx_grouped_gemm_bf16(_gemm_groups(msat), 3, 4608, 1536, internal, None) == HIP_INVALID_VALUE

    def mixed(ks, ms=(64, 18), D=64, H=24, kvsh=3 * 64 * 64):
        k = _lib.i64_array(ks) if ks is not None else None
        return lib.rldx_grouped_gemm_qkv_norm_rope_mixed_bf16(_gemm_groups(ms), _msat_norms(ms), len(ms), H, D, k,
                                                              1 << 20, 82 * 64, 64, 1 << 24, kvsh, 1e-6, None)

    # the RLDX-1 double-stream QKV shapes (VL 4096 | SA 1536, 24 x 64 heads), each with one argument wrong
    assert mixed(None) == HIP_INVALID_VALUE                          # no K array
    assert mixed([4096, 1500]) == HIP_INVALID_VALUE                  # k % 128
    assert mixed([4096, 1536], ms=(40, 18), kvsh=2 * 64 * 64) == HIP_INVALID_VALUE  # 40 rows pad to 64: 3 tiles
    assert mixed([4096, 1536], H=23) == HIP_INVALID_VALUE            # odd head count at head_dim 64
    assert mixed([4096, 1536], kvsh=3 * 64 * 64 - 8) == HIP_INVALID_VALUE


def test_vision_attention_workspace_and_rejections():
    lib = _lib.load()
    # 2 x 196 tokens, 16 heads x 72 (padded to 96): Q 16*392*96*2 bytes, 14 slots of 128*96-byte tiles per head
    assert lib.rldx_vision_attention_workspace_bytes(392, 2, 16, 72) == 16 * 392 * 96 * 2 + 16 * 14 * 128 * 96
    assert lib.rldx_vision_attention_workspace_bytes(100, 3, 2, 64) == 25600 + 2 * ((100 + 93) // 32) * 128 * 64
    for hd in (0, 4, 68, 136, -8):
        assert lib.rldx_vision_attention_workspace_bytes(392, 2, 16, hd) == -1
    big = 1 << 30
    ok = dict(qkv=256, cos=512, sin=768, cu=1024, S=2, out=2048, M=392, H=16, D=72, sc=0.1, ws=4096, wsb=big)

    def call(**kw):
        a = {**ok, **kw}
        return lib.rldx_vision_attention_bf16(a["qkv"], a["cos"], a["sin"], a["cu"], a["S"], a["out"], a["M"], a["H"],
                                              a["D"], a["sc"], a["ws"], a["wsb"], None)

    assert call(D=70) == HIP_INVALID_VALUE             # head_dim % 8
    assert call(D=136) == HIP_INVALID_VALUE            # head_dim > 128
    assert call(S=0) == HIP_INVALID_VALUE              # no sequence
    assert call(H=0) == HIP_INVALID_VALUE
    assert call(sc=0.0) == HIP_INVALID_VALUE
    assert call(sc=float("inf")) == HIP_INVALID_VALUE
    assert call(qkv=None) == HIP_INVALID_VALUE
    assert call(cu=None) == HIP_INVALID_VALUE
    assert call(qkv=264) == HIP_INVALID_VALUE          # 16-byte alignment
    assert call(cos=520) == HIP_INVALID_VALUE
    assert call(out=2052) == HIP_INVALID_VALUE         # 8-byte alignment
    assert call(cu=1026) == HIP_INVALID_VALUE
    assert call(wsb=16 * 392 * 96 * 2) == HIP_INVALID_VALUE  # workspace too small
    assert call(M=(1 << 24) + 1) == HIP_INVALID_VALUE
    assert call(M=0, qkv=None, out=None) == 0          # nothing to do


def test_memory_attention_rejections():
    lib = _lib.load()

    def call(qkv=256, cos=512, ssin=768, out=1024, M=64, H=16, D=256, B=16):
        return lib.rldx_memory_attention_bf16(qkv, cos, ssin, out, M, H, D, B, None)

    assert call(D=96) == HIP_INVALID_VALUE      # head_dim not 64 / 128 / 256
    assert call(D=512) == HIP_INVALID_VALUE
    assert call(B=0) == HIP_INVALID_VALUE       # block_attn_size >= 1
    assert call(H=0) == HIP_INVALID_VALUE
    assert call(M=-1) == HIP_INVALID_VALUE
    assert call(qkv=None) == HIP_INVALID_VALUE
    assert call(cos=520) == HIP_INVALID_VALUE   # 16-byte alignment
    assert call(out=1026) == HIP_INVALID_VALUE  # 8-byte alignment
    assert call(M=(1 << 24) + 1) == HIP_INVALID_VALUE
    assert call(M=0, qkv=None, out=None) == 0


def test_packed_output_widths_validated():
    """Packed GEMM outputs take ldo 0 or a packed width (multiple of 16, >= the
    output columns); attention's out_packed 1 or such a width."""
    lib = _lib.load()
    g = _gemm_groups((82,), ldo=0)
    assert lib.rldx_grouped_gemm_workspace_bytes(g, 1, 4096, 6144, 4, 1) == 0      # bias_packed, ldo 0
    g = _gemm_groups((82,), ldo=5632)
    assert lib.rldx_grouped_gemm_workspace_bytes(g, 1, 4096, 6144, 4, 1) == 0      # into a wider matrix
    for bad in (5640, 4080, -16):  # not a multiple of 16, narrower than the output, negative
        g = _gemm_groups((82,), ldo=bad)
        assert lib.rldx_grouped_gemm_workspace_bytes(g, 1, 4096, 6144, 4, 1) == -1
    for bad_epi in (6, 15, 17, -1):  # no such epilogue
        assert lib.rldx_grouped_gemm_workspace_bytes(_gemm_groups((82,)), 1, 4096, 6144, bad_epi, 1) == -1
    st = _lib.i64_array([0, 0, 0])
    ps = _lib.i64_array([0, 24 * 64 * 64 * 3])
    for bad in (-1, 1000, 1536 - 16):
        assert lib.rldx_attention_packed_fwd_bf16(256, 512, ps, 1024, bad, 1, 24, 24, 82, 82, 64, st, st, None, 0,
                                                  0.125, 0, None) == HIP_INVALID_VALUE


def test_zero_sized_calls_are_noops():
    lib = _lib.load()
    st = _lib.i64_array([0, 0, 0])
    assert lib.rldx_swiglu_bf16(None, 0, None, None, 0, 0, 8, None) == 0
    assert lib.rldx_attention_fwd_bf16(None, None, None, None, 0, 2, 2, 4, 4, 128, st, st, st, st, None, 0, 1.0, 0,
                                       None, 0, None) == 0


def test_python_wrappers_refuse_cpu_tensors():
    x = torch.zeros(2, 16, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        Fn.swiglu(x)
    q = torch.zeros(1, 2, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        Fn.attention(q, q, q)


def test_llm_attention_noalloc_rejects_sizes_beyond_its_scratch():
    """rldx_llm_fused_attention_noalloc_bf16 checks the packed K/V size against its
    scratch array (RLDX_LLM_ATTN_NOALLOC_MAX_BYTES = 16 MiB) before anything else:
    one key more than fits is rejected with hipErrorInvalidValue, without touching
    a device (this host has none)."""
    lib = _lib.load()
    max_bytes = 16 << 20
    fits = max_bytes // (8 * 4 * 128)  # 8 KV heads, K + V bf16 = 4 * D bytes per key and head
    assert lib.rldx_llm_fused_attention_workspace_bytes(fits, 8, 128) == max_bytes
    assert lib.rldx_llm_fused_attention_workspace_bytes(fits + 1, 8, 128) > max_bytes
    p = 4096  # never dereferenced: the call must fail on the size first
    assert lib.rldx_llm_fused_attention_noalloc_bf16(p, 48 * 128, p, p, p, p, 128, 1, p, 32 * 128, fits + 1, 32, 8, 128,
                                                    1e-6, None) == HIP_INVALID_VALUE
    assert lib.rldx_llm_fused_attention_noalloc_bf16(p, 48 * 128, p, p, p, p, 128, 1, p, 32 * 128, 1 << 20, 32, 8, 128,
                                                    1e-6, None) == HIP_INVALID_VALUE


def test_residual_packed_epilogue_and_layernorm_fold_rejections():
    """RLDX_GEMM_EPI_RESIDUAL_PACKED takes a packed residual (ldr 0 or a packed
    width, % 16); the LayerNorm-fold entries need every group's row sums and
    statistics, a non-negative eps, the bias / packed-SwiGLU / QKV epilogues,
    k <= 2048 and no other flag than RLDX_GEMM_WIDE_TILES; statistics out need a
    residual epilogue.  Checked before anything is launched."""
    lib = _lib.load()
    for ldr, ok in ((0, True), (1536, True), (3072, True), (1544, False), (1520, False), (-16, False)):
        g = _gemm_groups((608,), ldo=0)
        g[0].ldr = ldr
        assert (lib.rldx_grouped_gemm_workspace_bytes(g, 1, 1536, 4096, _lib.GEMM_EPI_RESIDUAL_PACKED, 1) == 0) == ok
    g = _gemm_groups((608,), ldo=0)
    g[0].residual = None
    assert lib.rldx_grouped_gemm_workspace_bytes(g, 1, 1536, 4096, _lib.GEMM_EPI_RESIDUAL_PACKED, 1) == -1
    ptrs = lambda *p: (ctypes.c_void_p * len(p))(*p)  # noqa: E731
    sums, stats = ptrs(4096, 8192, 12288), ptrs(16384, 20480, 24576)
    missing, odd = ptrs(4096, None, 12288), ptrs(4096, 8194, 12288)
    msat = (512, 64, 32)
    call = lib.rldx_grouped_gemm_ln_bf16
    bias = _lib.GEMM_EPI_BIAS
    inval = HIP_INVALID_VALUE
    assert call(_gemm_groups(msat), None, stats, 3, 4608, 1536, bias, 0, 1e-6, None) == inval
    assert call(_gemm_groups(msat), sums, None, 3, 4608, 1536, bias, 0, 1e-6, None) == inval
    assert call(_gemm_groups(msat), missing, stats, 3, 4608, 1536, bias, 0, 1e-6, None) == inval
    assert call(_gemm_groups(msat), sums, missing, 3, 4608, 1536, bias, 0, 1e-6, None) == inval
    assert call(_gemm_groups(msat), odd, stats, 3, 4608, 1536, bias, 0, 1e-6, None) == inval
    assert call(_gemm_groups(msat), sums, ptrs(16384, 20484, 24576), 3, 4608, 1536, bias, 0, 1e-6, None) == inval
    for epi in (_lib.GEMM_EPI_RESIDUAL, _lib.GEMM_EPI_SWIGLU, _lib.GEMM_EPI_BIAS_PACKED,
                _lib.GEMM_EPI_RESIDUAL_PACKED, QKV_INTERNAL):
        assert call(_gemm_groups(msat), sums, stats, 3, 8192, 1536, epi, 0, 1e-6, None) == inval
    assert call(_gemm_groups(msat), sums, stats, 3, 4608, 1536, bias, 2, 1e-6, None) == inval  # flag 2
    assert call(_gemm_groups(msat), sums, stats, 3, 4608, 1536, bias, 0, -1.0, None) == inval
    assert call(_gemm_groups(msat), sums, stats, 3, 4608, 1000, bias, 0, 1e-6, None) == inval
    assert call(_gemm_groups(msat), sums, stats, 3, 4608, 4096, bias, 0, 1e-6, None) == inval  # k > 2048
    d = _msat_norms(msat)
    qkv = lib.rldx_grouped_gemm_qkv_norm_rope_ln_bf16
    for sm, st in ((None, stats), (sums, None), (missing, stats)):
        assert qkv(_gemm_groups(msat), d, sm, st, 3, 12, 128, 1536, 1 << 20, 608 * 128, 128, 2 << 20,
                   19 * 64 * 128, 1e-6, 1e-6, None) == inval
    st_out = lib.rldx_grouped_gemm_stats_bf16
    assert st_out(_gemm_groups(msat), None, 3, 1536, 4096, _lib.GEMM_EPI_RESIDUAL, 1, 0, None, 0, None) == inval
    for epi in (bias, _lib.GEMM_EPI_SWIGLU_PACKED, _lib.GEMM_EPI_BIAS_PACKED):
        assert st_out(_gemm_groups(msat), stats, 3, 1536, 4096, epi, 1, 0, None, 0, None) == inval
    assert st_out(_gemm_groups(msat), missing, 3, 1536, 4096, _lib.GEMM_EPI_RESIDUAL, 1, 0, None, 0, None) == inval
    pack = lib.rldx_act_pack_stats_bf16
    assert pack(4096, 1536, 10, 1536, 8192, None, None) == inval
    assert pack(4096, 1536, 10, 1552, 8192, 16384, None) == inval  # k % 64
    assert pack(4096, 1536, 10, 1536, 8192, 16388, None) == inval  # stats alignment
