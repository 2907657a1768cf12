"""ctypes binding of librldx_amd.so, the gfx950 C-ABI library (include/rldx_amd.h).

The library is the only compute path: if it is missing or fails to load,
every operator raises.  There is no CPU or PyTorch fallback.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "librldx_amd.so"

c_i64 = ctypes.c_int64
c_i32 = ctypes.c_int32
c_f32 = ctypes.c_float
c_vp = ctypes.c_void_p
c_i64p = ctypes.POINTER(ctypes.c_int64)


class Rows(ctypes.Structure):
    """rldx_rows_t"""

    _fields_ = [("x", ctypes.c_void_p), ("ldx", ctypes.c_int64), ("m", ctypes.c_int64), ("k", ctypes.c_int64),
                ("packed", ctypes.c_void_p)]


class GemmGroup(ctypes.Structure):
    """rldx_gemm_group_t"""

    _fields_ = [
        ("a_packed", ctypes.c_void_p),
        ("m", ctypes.c_int64),
        ("w_packed", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("ldo", ctypes.c_int64),
        ("residual", ctypes.c_void_p),
        ("ldr", ctypes.c_int64),
    ]


class MsatStream(ctypes.Structure):
    """Mirror of `rldx_msat_stream_t`."""

    _fields_ = [
        ("qkv", c_vp),
        ("qkv_row_stride", c_i64),
        ("rows", c_i64),
        ("q_norm_w", c_vp),
        ("k_norm_w", c_vp),
        ("rope_cos", c_vp),
        ("rope_sin", c_vp),
        ("rope_row_stride", c_i64),
    ]


# name -> (restype, argtypes); must stay in sync with include/rldx_amd.h
SIGNATURES = {
    "rldx_read_probe_sink_words": (c_i64, []),
    "rldx_read_probe": (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp]),
    "rldx_swiglu_bf16": (c_i32, [c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp]),
    "rldx_grouped_swiglu_bf16": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp]),
    "rldx_qk_rmsnorm_rope_half_f32": (
        c_i32,
        [c_vp] * 8 + [c_i64] * 5 + [c_i64p] * 5 + [c_f32, c_i32, c_vp],
    ),
    "rldx_qk_rmsnorm_rope_half_bf16": (
        c_i32,
        [c_vp] * 8 + [c_i64] * 5 + [c_i64p] * 5 + [c_f32, c_i32, c_vp],
    ),
    "rldx_msat_qkv_norm_rope_bf16": (
        c_i32,
        [ctypes.POINTER(MsatStream), c_i32, c_i64, c_i64, c_vp, c_vp, c_vp, c_i64, c_i64, c_vp, c_i64, c_f32, c_vp],
    ),
    "rldx_msat_qkv_norm_rope_batch_bf16": (
        c_i32,
        [ctypes.POINTER(MsatStream), c_i32, c_i64, c_i64p, c_i64, c_i64, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp,
         c_i64, c_i64, c_f32, c_vp],
    ),
    "rldx_attention_kv_packed_elems": (c_i64, [c_i64, c_i64]),
    "rldx_attention_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64, c_i64]),
    "rldx_attention_kv_pack_bf16": (c_i32, [c_vp, c_i64p, c_vp, c_i64p, c_vp, c_i64p, c_i64, c_i64, c_i64, c_i64, c_vp]),
    "rldx_attention_fwd_bf16": (
        c_i32,
        [c_vp] * 4 + [c_i64] * 6 + [c_i64p] * 4 + [c_vp, c_i64, c_f32, c_i32, c_vp, c_i64, c_vp],
    ),
    "rldx_attention_packed_fwd_bf16": (
        c_i32,
        [c_vp, c_vp, c_i64p, c_vp, c_i32] + [c_i64] * 6 + [c_i64p] * 2 + [c_vp, c_i64, c_f32, c_i32, c_vp],
    ),
    "rldx_attention_packed_segments_fwd_bf16": (
        c_i32,
        [c_vp, c_vp, c_i64p, c_vp, c_i32, c_i64p, c_i32] + [c_i64] * 6 + [c_i64p] + [c_vp, c_i64, c_f32, c_i32, c_vp],
    ),
    "rldx_attention_packed_fwd_warm_bf16": (
        c_i32,
        [c_vp, c_vp, c_i64p, c_vp, c_i32] + [c_i64] * 6 + [c_i64p] * 2 + [c_vp, c_i64, c_f32, c_i32]
        + [ctypes.POINTER(c_vp), c_i64p, c_i32, c_vp],
    ),
    "rldx_llm_fused_attention_bf16": (
        c_i32,
        [c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_f32, c_vp,
         c_i64, c_vp],
    ),
    "rldx_llm_fused_attention_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64]),
    "rldx_llm_fused_attention_noalloc_bf16": (
        c_i32,
        [c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_f32, c_vp],
    ),
    "rldx_vision_attention_bf16": (
        c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_f32, c_vp, c_i64, c_vp]
    ),
    "rldx_vision_attention_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64, c_i64]),
    "rldx_memory_attention_bf16": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp]),
    "rldx_gemm_pack_weight_bf16": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_i32, c_vp, c_vp]),
    "rldx_act_packed_elems": (c_i64, [c_i64, c_i64]),
    "rldx_act_pack_bf16": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp]),
    "rldx_layernorm_pack_bf16": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_f32, c_vp, c_vp]),
    "rldx_grouped_gemm_bf16": (c_i32, [ctypes.POINTER(GemmGroup), c_i32, c_i64, c_i64, c_i32, c_vp]),
    "rldx_grouped_gemm_workspace_bytes": (c_i64, [ctypes.POINTER(GemmGroup), c_i32, c_i64, c_i64, c_i32, c_i32]),
    "rldx_grouped_gemm_ws_bf16": (c_i32, [ctypes.POINTER(GemmGroup), c_i32, c_i64, c_i64, c_i32, c_i32, c_vp, c_i64,
                                          c_vp]),
    "rldx_grouped_gemm_ex_bf16": (c_i32, [ctypes.POINTER(GemmGroup), c_i32, c_i64, c_i64, c_i32, c_i32, c_i32, c_vp,
                                          c_i64, c_vp]),
    "rldx_grouped_gemm_ex_workspace_bytes": (c_i64, [ctypes.POINTER(GemmGroup), c_i32, c_i64, c_i64, c_i32, c_i32,
                                                     c_i32]),
    "rldx_grouped_gemm_qkv_norm_rope_bf16": (c_i32, [ctypes.POINTER(GemmGroup), ctypes.POINTER(MsatStream), c_i32,
                                                     c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_f32,
                                                     c_vp]),
    "rldx_grouped_gemm_qkv_norm_rope_mixed_bf16": (c_i32, [ctypes.POINTER(GemmGroup), ctypes.POINTER(MsatStream),
                                                           c_i32, c_i64, c_i64, c_i64p, c_vp, c_i64, c_i64, c_vp,
                                                           c_i64, c_f32, c_vp]),
    "rldx_grouped_gemm_ln_bf16": (c_i32, [ctypes.POINTER(GemmGroup), ctypes.POINTER(c_vp), ctypes.POINTER(c_vp), c_i32,
                                          c_i64, c_i64, c_i32, c_i32, c_f32, c_vp]),
    "rldx_grouped_gemm_qkv_norm_rope_ln_bf16": (c_i32, [ctypes.POINTER(GemmGroup), ctypes.POINTER(MsatStream),
                                                        ctypes.POINTER(c_vp), ctypes.POINTER(c_vp), c_i32, c_i64, c_i64,
                                                        c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_f32, c_f32, c_vp]),
    "rldx_grouped_gemm_stats_bf16": (c_i32, [ctypes.POINTER(GemmGroup), ctypes.POINTER(c_vp), c_i32, c_i64, c_i64,
                                             c_i32, c_i32, c_i32, c_vp, c_i64, c_vp]),
    "rldx_act_pack_stats_bf16": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp]),
    "rldx_layernorm_pack_many_bf16": (c_i32, [ctypes.POINTER(Rows), c_i32, c_f32, c_vp]),
    "rldx_action_encode_pack_bf16": (c_i32, [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp,
                                             ctypes.POINTER(Rows), ctypes.POINTER(c_vp), c_i32, c_vp]),
    "rldx_action_decode_euler_bf16": (c_i32, [c_vp, c_i64, c_i64, c_f32, c_vp, c_vp, c_i64, c_f32, c_vp, c_vp]),
    "rldx_grouped_gemm_mixed_bf16": (c_i32, [ctypes.POINTER(GemmGroup), c_i64p, c_i64p, ctypes.POINTER(c_i32),
                                             ctypes.POINTER(c_vp), c_i32, c_i32, c_i32, c_vp, c_i64, c_vp]),
    "rldx_grouped_gemm_mixed_workspace_bytes": (c_i64, [ctypes.POINTER(GemmGroup), c_i64p, c_i64p,
                                                        ctypes.POINTER(c_i32), c_i32, c_i32, c_i32]),
    "rldx_host_swiglu_bf16": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64]),
    "rldx_grouped_res_ln_bf16": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                         c_i64, c_i64, c_i64, c_i64, c_f32, c_vp]),
    "rldx_vl_epilogue_ln_bf16": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_f32, c_vp]),
    "rldx_ss_epilogue_ln_bf16": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_f32, c_vp]),
    "rldx_add_rmsnorm_bf16": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_f32, c_vp]),
    "rldx_rms_norm_bf16": (c_i32, [c_vp, c_i64, c_vp, c_i32, c_vp, c_i64, c_i64, c_i64, c_f32, c_vp]),
    "rldx_rms_norm_f32": (c_i32, [c_vp, c_i64, c_vp, c_i32, c_vp, c_i64, c_i64, c_i64, c_f32, c_vp]),
    "rldx_rope_interleaved_bf16": (c_i32, [c_vp, c_i64p, c_vp, c_i64p, c_vp, c_i64p, c_vp, c_i64p, c_i64, c_i64, c_i64,
                                           c_i64, c_i64, c_vp, c_i64p, c_vp]),
    "rldx_rope_interleaved_f32": (c_i32, [c_vp, c_i64p, c_vp, c_i64p, c_vp, c_i64p, c_vp, c_i64p, c_i64, c_i64, c_i64,
                                          c_i64, c_i64, c_vp, c_i64p, c_vp]),
}

ROPE_SIN_SIGNED = 1  # RLDX_ROPE_SIN_SIGNED
ROPE_NO_NORM = 2  # RLDX_ROPE_NO_NORM
GEMM_EPI_BIAS, GEMM_EPI_RESIDUAL, GEMM_EPI_SWIGLU, GEMM_EPI_SWIGLU_PACKED, GEMM_EPI_BIAS_PACKED = 0, 1, 2, 3, 4
GEMM_EPI_RESIDUAL_PACKED = 5
GEMM_WIDE_TILES = 1  # RLDX_GEMM_WIDE_TILES
GEMM_SPLITS_ACROSS_XCDS = 2  # RLDX_GEMM_SPLITS_ACROSS_XCDS

_lib = None
_hip = None


def lib_path() -> Path:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load librldx_amd.so once; raise a clear error if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"rldx_amd: {LIB_PATH} not found. Build it with `make -C rldx-1_amd` "
            "(or __graft_entry__.build()); there is no fallback path."
        )
    lib = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _hip_runtime() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so", mode=os.RTLD_NOW | os.RTLD_GLOBAL)
        _hip.hipGetErrorString.restype = ctypes.c_char_p
        _hip.hipGetErrorString.argtypes = [ctypes.c_int]
    return _hip


def check(status: int, what: str) -> None:
    if status != 0:
        try:
            msg = _hip_runtime().hipGetErrorString(status).decode()
        except OSError:
            msg = "unknown"
        raise RuntimeError(f"rldx_amd: {what} failed with hipError {status} ({msg})")


def i64_array(values) -> ctypes.Array:
    arr = (ctypes.c_int64 * len(values))(*[int(v) for v in values])
    return arr
