"""Tensor-level launchers for the gfx950 kernels.

Each function validates its tensors on the host (dtype, device, shapes,
strides), then calls the C ABI of librldx_amd.so on the current HIP stream.
PyTorch only provides device memory and the stream.  Outputs are allocated
with `torch.empty` (caching allocator, hipGraph-safe) unless `out=` is given.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence

import torch

from . import _lib

BF16 = torch.bfloat16
F32 = torch.float32


def _stream_ptr(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(f"rldx_amd: {msg}")


def _on_gpu(*ts: Optional[torch.Tensor]) -> None:
    dev = None
    for t in ts:
        if t is None:
            continue
        _require(t.is_cuda, "tensors must live on a ROCm device (the HIP kernels are the only path)")
        if dev is None:
            dev = t.device
        _require(t.device == dev, "all tensors must be on the same device")


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _rows_view(x: torch.Tensor, what: str):
    """Describe x[..., C] as (rows, row_stride) without copying."""
    _require(x.dim() >= 1 and x.stride(-1) == 1, f"{what}: last dimension must be contiguous")
    if x.dim() == 1:
        return 1, x.shape[-1]
    lead = x.shape[:-1]
    rows = int(math.prod(lead))
    ld = x.stride(-2)
    # leading dims must collapse into one strided dimension
    expect = ld
    for size, stride in zip(reversed(lead), reversed(x.stride()[:-1])):
        if size != 1:
            _require(stride == expect, f"{what}: leading dimensions must collapse to one row stride")
        expect = stride * size
    return rows, ld


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
def swiglu(x: torch.Tensor, bias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """`F.silu(x1) * x2` with `x1, x2 = x.chunk(2, -1)`, bf16, eager rounding.

    rldx/model/modules/action_model/ops.py:157-161.  With `bias` ([2*N] bf16)
    each half is first rounded as bf16(x + b)."""
    _on_gpu(x, bias, out)
    _require(x.dtype == BF16, "swiglu expects bfloat16 input")
    _require(x.shape[-1] % 2 == 0, "swiglu: last dimension must be even")
    n_half = x.shape[-1] // 2
    rows, ldx = _rows_view(x, "swiglu input")
    if bias is not None:
        _require(bias.dtype == BF16 and bias.dim() == 1 and bias.shape[0] == 2 * n_half and bias.is_contiguous(),
                 "swiglu bias must be contiguous bf16 [2*N]")
    if out is None:
        out = torch.empty((*x.shape[:-1], n_half), dtype=BF16, device=x.device)
    _require(out.shape == (*x.shape[:-1], n_half) and out.dtype == BF16, "swiglu out has the wrong shape/dtype")
    _, ldy = _rows_view(out, "swiglu out")
    if rows == 0 or n_half == 0:
        return out
    lib = _lib.load()
    _lib.check(lib.rldx_swiglu_bf16(x.data_ptr(), ldx, _ptr(bias), out.data_ptr(), ldy, rows, n_half,
                                    _stream_ptr(x)), "rldx_swiglu_bf16")
    return out


def grouped_swiglu(sa_w12: torch.Tensor, sa_bias: Optional[torch.Tensor], vl_w12: torch.Tensor,
                   vl_bias: Optional[torch.Tensor], m_sa: int, m_vl: int, n_half_sa: int, n_half_vl: int):
    """Two-group SwiGLU in one launch (ds::grouped_swiglu semantics, eager rounding)."""
    _on_gpu(sa_w12, sa_bias, vl_w12, vl_bias)
    for t, m, nh, name in ((sa_w12, m_sa, n_half_sa, "sa_w12"), (vl_w12, m_vl, n_half_vl, "vl_w12")):
        _require(t.dtype == BF16 and t.is_contiguous(), f"{name} must be contiguous bf16")
        _require(t.numel() == m * 2 * nh, f"{name} must hold ({m}, {2 * nh}) elements")
    for b, nh, name in ((sa_bias, n_half_sa, "sa_bias"), (vl_bias, n_half_vl, "vl_bias")):
        if b is not None:
            _require(b.dtype == BF16 and b.is_contiguous() and b.numel() == 2 * nh, f"{name} must be bf16 [{2 * nh}]")
    _require((sa_bias is None) == (vl_bias is None), "biases must be both given or both None")
    sa_out = torch.empty((m_sa, n_half_sa), dtype=BF16, device=sa_w12.device)
    vl_out = torch.empty((m_vl, n_half_vl), dtype=BF16, device=sa_w12.device)
    lib = _lib.load()
    _lib.check(lib.rldx_grouped_swiglu_bf16(sa_w12.data_ptr(), _ptr(sa_bias), vl_w12.data_ptr(), _ptr(vl_bias),
                                            sa_out.data_ptr(), vl_out.data_ptr(), m_sa, m_vl, n_half_sa, n_half_vl,
                                            _stream_ptr(sa_w12)), "rldx_grouped_swiglu_bf16")
    return sa_out, vl_out


# ---------------------------------------------------------------------------
# rotate-half QK-RMSNorm + RoPE
# ---------------------------------------------------------------------------
def qk_rmsnorm_rope_half(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                         cos: torch.Tensor, sin: torch.Tensor, eps: float = 1e-6, *, sin_is_signed: bool = False,
                         q_out: Optional[torch.Tensor] = None, k_out: Optional[torch.Tensor] = None):
    """Qwen3-VL q_norm/k_norm followed by rotate-half RoPE, fused.

    q: [B, S, Hq, D], k: [B, S, Hk, D] (any strides with D contiguous);
    cos/sin: [S, D] or [B, S, D].  fp32 or bf16 (all tensors one dtype).
    `sin_is_signed`: `sin` is the pre-signed table of
    fused_llm_attention.prepare_signed_sin (first half negated).
    rldx/model/modules/backbone/modeling_qwen3_vl.py:356-401."""
    return _rope_half(q, k, q_weight, k_weight, cos, sin, eps, sin_is_signed, q_out, k_out)


def rope_half(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *,
              sin_is_signed: bool = False, q_out: Optional[torch.Tensor] = None,
              k_out: Optional[torch.Tensor] = None):
    """Rotate-half RoPE alone, q' = q cos + rotate_half(q) sin in the input type
    (each product and the sum rounded, as eager bf16), on the same layouts as
    qk_rmsnorm_rope_half (RLDX_ROPE_NO_NORM).
    rldx/model/modules/backbone/modeling_qwen3_vl.py:377-401."""
    return _rope_half(q, k, None, None, cos, sin, 0.0, sin_is_signed, q_out, k_out)


def _rope_half(q, k, q_weight, k_weight, cos, sin, eps, sin_is_signed, q_out, k_out):
    _on_gpu(q, k, q_weight, k_weight, cos, sin, q_out, k_out)
    norm = q_weight is not None
    dt = q.dtype
    _require(dt in (F32, BF16), "rotate-half RoPE supports float32 and bfloat16")
    for t in (k, q_weight, k_weight, cos, sin):
        _require(t is None or t.dtype == dt, "all inputs must share one dtype")
    _require(q.dim() == 4 and k.dim() == 4, "q and k must be [B, S, H, D]")
    B, S, Hq, D = q.shape
    _require(k.shape[0] == B and k.shape[1] == S and k.shape[3] == D, "k must be [B, S, Hk, D] matching q")
    Hk = k.shape[2]
    _require(D in (64, 128), "head_dim must be 64 or 128")
    if norm:
        _require(k_weight is not None and q_weight.shape == (D,) and k_weight.shape == (D,),
                 "norm weights must be [D]")
        _require(q_weight.is_contiguous() and k_weight.is_contiguous(), "norm weights must be contiguous")
    if cos.dim() == 2:
        cos = cos.unsqueeze(0)
        sin = sin.unsqueeze(0)
    _require(cos.dim() == 3 and cos.shape[1:] == (S, D) and cos.shape[0] in (1, B), "cos must be [S, D] or [B, S, D]")
    _require(sin.shape == cos.shape and sin.stride() == cos.stride(), "sin must match cos in shape and strides")
    _require(q.stride(-1) == 1 and k.stride(-1) == 1 and cos.stride(-1) == 1, "last dims must be contiguous")
    if q_out is None:
        q_out = torch.empty((B, S, Hq, D), dtype=dt, device=q.device)
    if k_out is None:
        k_out = torch.empty((B, S, Hk, D), dtype=dt, device=q.device)
    _require(q_out.shape == q.shape and k_out.shape == k.shape, "output shapes must match inputs")
    cb = cos.stride(0) if cos.shape[0] == B and B > 1 else 0
    qs = _lib.i64_array([q.stride(0), q.stride(1), q.stride(2)])
    ks = _lib.i64_array([k.stride(0), k.stride(1), k.stride(2)])
    qos = _lib.i64_array([q_out.stride(0), q_out.stride(1), q_out.stride(2)])
    kos = _lib.i64_array([k_out.stride(0), k_out.stride(1), k_out.stride(2)])
    css = _lib.i64_array([cb, cos.stride(1)])
    if B * S == 0:
        return q_out, k_out
    lib = _lib.load()
    fn = lib.rldx_qk_rmsnorm_rope_half_f32 if dt == F32 else lib.rldx_qk_rmsnorm_rope_half_bf16
    flags = (_lib.ROPE_SIN_SIGNED if sin_is_signed else 0) | (0 if norm else _lib.ROPE_NO_NORM)
    _lib.check(fn(q.data_ptr(), k.data_ptr(), _ptr(q_weight), _ptr(k_weight), cos.data_ptr(), sin.data_ptr(),
                  q_out.data_ptr(), k_out.data_ptr(), B, S, Hq, Hk, D, qs, ks, qos, kos, css, float(eps), flags,
                  _stream_ptr(q)), "rldx_qk_rmsnorm_rope_half")
    return q_out, k_out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RMSNorm with one rounding: (weight * (x * rsqrt(mean(x^2) + eps))).to(x.dtype)
    over the last dimension, fp32 arithmetic; x bf16 or fp32, weight fp32 or bf16
    (rldx/model/modules/norms.py:18-22; rldx_rms_norm_bf16 / _f32)."""
    _on_gpu(x, weight, out)
    dt = x.dtype
    _require(dt in (F32, BF16), "rms_norm supports float32 and bfloat16 inputs")
    _require(weight.dtype in (F32, BF16) and weight.dim() == 1 and weight.is_contiguous(),
             "weight must be a contiguous float32 or bfloat16 vector")
    dim = x.shape[-1]
    _require(weight.numel() == dim, "weight must have the last dimension's size")
    rows, ld = _rows_view(x, "x")
    if out is None:
        out = torch.empty(x.shape, dtype=dt, device=x.device)
    _require(out.shape == x.shape and out.dtype == dt, "out must match x")
    orows, old = _rows_view(out, "out")
    if rows == 0:
        return out
    lib = _lib.load()
    fn = lib.rldx_rms_norm_bf16 if dt == BF16 else lib.rldx_rms_norm_f32
    _lib.check(fn(x.data_ptr(), ld, weight.data_ptr(), 1 if weight.dtype == F32 else 0, out.data_ptr(), old, rows, dim,
                  float(eps), _stream_ptr(x)), "rldx_rms_norm")
    return out


def rope_interleaved(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor):
    """Interleaved (complex) RoPE: pairs (x[2i], x[2i+1]) times freqs_cis[n][i] in
    fp32, rounded once to the input type.  xq [B, Hq, N, D], xk [B, Hk, N, D]
    (bf16 or fp32, D contiguous); freqs_cis complex64 [N, D/2], [1, N, D/2] or
    [B, N, D/2].  Returns new contiguous (xq_out, xk_out)
    (rldx/model/modules/action_model/ops.py:48-67; rldx_rope_interleaved_*)."""
    _on_gpu(xq, xk, freqs_cis)
    dt = xq.dtype
    _require(dt in (F32, BF16) and xk.dtype == dt, "xq and xk must share one dtype, float32 or bfloat16")
    _require(xq.dim() == 4 and xk.dim() == 4, "xq and xk must be [B, H, N, D]")
    B, Hq, N, D = xq.shape
    _require(xk.shape[0] == B and xk.shape[2] == N and xk.shape[3] == D, "xk must be [B, Hk, N, D] matching xq")
    _require(freqs_cis.dtype == torch.complex64, "freqs_cis must be complex64")
    f = freqs_cis if freqs_cis.dim() == 3 else freqs_cis.unsqueeze(0)
    _require(f.dim() == 3 and f.shape[1:] == (N, D // 2) and f.shape[0] in (1, B),
             "freqs_cis must be [N, D/2] or [B or 1, N, D/2]")
    _require(f.stride(-1) == 1 and xq.stride(-1) == 1 and xk.stride(-1) == 1, "last dims must be contiguous")
    fb = f.stride(0) if f.shape[0] == B and B > 1 else 0
    qo, ko = torch.empty_like(xq, memory_format=torch.contiguous_format), torch.empty_like(
        xk, memory_format=torch.contiguous_format)
    if xq.numel() + xk.numel() == 0:
        return qo, ko
    st = lambda t: _lib.i64_array([t.stride(0), t.stride(1), t.stride(2)])  # noqa: E731
    lib = _lib.load()
    fn = lib.rldx_rope_interleaved_bf16 if dt == BF16 else lib.rldx_rope_interleaved_f32
    fr = torch.view_as_real(f)
    _lib.check(fn(xq.data_ptr(), st(xq), qo.data_ptr(), st(qo), xk.data_ptr(), st(xk), ko.data_ptr(), st(ko), B, Hq,
                  xk.shape[1], N, D, fr.data_ptr(), _lib.i64_array([fb, f.stride(1)]), _stream_ptr(xq)),
               "rldx_rope_interleaved")
    return qo, ko


# ---------------------------------------------------------------------------
# MSAT multi-stream QKV gather + QK-RMSNorm + interleaved RoPE
# ---------------------------------------------------------------------------
class StreamSpec:
    """One stream of the MSAT joint sequence: packed QKV rows + norm weights + optional tables."""

    __slots__ = ("qkv", "q_w", "k_w", "cos", "sin")

    def __init__(self, qkv: torch.Tensor, q_w: torch.Tensor, k_w: torch.Tensor,
                 cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None):
        self.qkv, self.q_w, self.k_w, self.cos, self.sin = qkv, q_w, k_w, cos, sin


def _rope_tables(s: StreamSpec, rows: int, head_dim: int, keep: list):
    """(cos, sin, row stride) of a stream's fp32 RoPE tables [>= rows, head_dim/2], or (None, None, 0)."""
    if s.cos is None:
        _require(s.sin is None, "cos and sin go together")
        return None, None, 0
    _require(s.sin is not None, "cos and sin go together")
    c = s.cos.to(F32).contiguous() if s.cos.dtype != F32 or not s.cos.is_contiguous() else s.cos
    sn = s.sin.to(F32).contiguous() if s.sin.dtype != F32 or not s.sin.is_contiguous() else s.sin
    _require(c.dim() == 2 and c.shape == sn.shape and c.shape[0] >= rows and c.shape[1] == head_dim // 2,
             "rope tables must be [>= rows, head_dim/2]")
    keep += [c, sn]
    return c.data_ptr(), sn.data_ptr(), c.stride(0)


def _check_kvp_out(kvp: torch.Tensor, num_heads: int, M: int, head_dim: int) -> None:
    _require(kvp.dtype == BF16 and kvp.dim() == 2 and kvp.shape[0] == num_heads and
             kvp.shape[1] >= kv_packed_elems(M, head_dim) and kvp.stride(1) == 1,
             "kvp out must be (H, >= kv_packed_elems(M, D)) bf16")


def msat_qkv_norm_rope(streams: Sequence[StreamSpec], num_heads: int, head_dim: int, eps: float = 1e-6,
                       out: Optional[tuple] = None, kv_packed: bool = False, batch: int = 1,
                       batch_rows: Optional[Sequence[int]] = None):
    """Gather Q/K/V of 1-3 streams into (H, M, D) bf16 with per-stream QK RMSNorm
    (one rounding) and interleaved RoPE on the streams that carry tables.

    Returns (q, k, v).  With `kv_packed`, returns (q, kvp) instead: K and V are
    written as the packed K/V tiles `attention_packed` reads, kvp of shape
    (H, kv_packed_elems(M, D)) bf16.  `out` gives the output tensors in the
    same form.  batch > 1 (rldx_msat_qkv_norm_rope_batch_bf16, one launch):
    each StreamSpec's qkv holds the rows of batch entry 0 and entry b's start
    batch_rows[i] rows further on in the same buffer (the rows of entry b may
    run into entry b + 1's); the outputs gain a leading batch dimension
    (B, H, M, D) / (B, H, kv_packed_elems(M, D)).

    rmsnorm_rope_ds.py:11-231 / rmsnorm_rope_ds_3way.py:22-386 fused layout,
    eager semantics of norms.py:18-22 and action_model/ops.py:48-67."""
    _require(1 <= len(streams) <= 3, "between 1 and 3 streams")
    _require(batch >= 1 and (batch == 1 or (batch_rows is not None and len(batch_rows) == len(streams))),
             "batch > 1 needs one batch_rows entry per stream")
    inner = num_heads * head_dim
    descs = (_lib.MsatStream * len(streams))()
    M = 0
    dev = streams[0].qkv.device
    keep = []
    for i, s in enumerate(streams):
        _on_gpu(s.qkv, s.q_w, s.k_w, s.cos, s.sin)
        _require(s.qkv.device == dev, "all streams on one device")
        _require(s.qkv.dtype == BF16 and s.qkv.dim() == 2 and s.qkv.stride(1) == 1, "qkv must be 2-D bf16 rows")
        _require(s.qkv.shape[1] >= 3 * inner, "qkv rows must hold Q|K|V of num_heads*head_dim each")
        _require(s.q_w.dtype == BF16 and s.k_w.dtype == BF16 and s.q_w.numel() == head_dim and
                 s.k_w.numel() == head_dim and s.q_w.is_contiguous() and s.k_w.is_contiguous(),
                 "norm weights must be contiguous bf16 [head_dim]")
        n = s.qkv.shape[0]
        if batch > 1 and n > 0:  # the last entry's rows must lie inside the qkv buffer
            last = s.qkv.storage_offset() + ((batch - 1) * int(batch_rows[i]) + n - 1) * s.qkv.stride(0) + 3 * inner
            _require(batch_rows[i] >= 0 and last * s.qkv.element_size() <= s.qkv.untyped_storage().nbytes(),
                     "the batch's rows of a stream run past its qkv buffer")
        cos_p, sin_p, rope_ld = _rope_tables(s, n, head_dim, keep)
        descs[i] = _lib.MsatStream(s.qkv.data_ptr(), s.qkv.stride(0), n, s.q_w.data_ptr(), s.k_w.data_ptr(),
                                   cos_p, sin_p, rope_ld)
        M += n
    lead = (batch,) if batch > 1 else ()
    if out is None:
        q = torch.empty((*lead, num_heads, M, head_dim), dtype=BF16, device=dev)
        rest = ((torch.empty((*lead, num_heads, kv_packed_elems(M, head_dim)), dtype=BF16, device=dev),)
                if kv_packed else (torch.empty_like(q), torch.empty_like(q)))
    else:
        q, *rest = out
        _require(q.shape == (*lead, num_heads, M, head_dim), "q out must be (H, M, D), or (B, H, M, D) for a batch")
        if kv_packed:
            _require(len(rest) == 1, "packed mode takes out=(q, kvp)")
            if batch > 1:
                _require(rest[0].shape[0] == batch, "kvp out must be (B, H, >= kv_packed_elems(M, D)) for a batch")
                _check_kvp_out(rest[0][0], num_heads, M, head_dim)
            else:
                _check_kvp_out(rest[0], num_heads, M, head_dim)
        else:
            _require(len(rest) == 2, "out=(q, k, v)")
            for t in rest:
                _require(t.shape == q.shape and t.stride() == q.stride(), "k/v out tensors must match q")
    if M == 0:
        return (q, *rest)
    lib = _lib.load()
    h_ax = 1 if batch > 1 else 0
    if batch > 1:
        kvp = rest[0] if kv_packed else None
        k, v = (None, None) if kv_packed else rest
        _lib.check(lib.rldx_msat_qkv_norm_rope_batch_bf16(
            descs, len(streams), batch, _lib.i64_array(batch_rows), num_heads, head_dim, q.data_ptr(),
            None if kv_packed else k.data_ptr(), None if kv_packed else v.data_ptr(), q.stride(0), q.stride(1),
            q.stride(2), kvp.data_ptr() if kv_packed else None, kvp.stride(0) if kv_packed else 0,
            kvp.stride(1) if kv_packed else 0, float(eps), _stream_ptr(q)), "rldx_msat_qkv_norm_rope_batch_bf16")
    elif kv_packed:
        kvp = rest[0]
        _lib.check(lib.rldx_msat_qkv_norm_rope_bf16(descs, len(streams), num_heads, head_dim, q.data_ptr(), None, None,
                                                    q.stride(h_ax), q.stride(h_ax + 1), kvp.data_ptr(), kvp.stride(0),
                                                    float(eps), _stream_ptr(q)), "rldx_msat_qkv_norm_rope_bf16")
    else:
        k, v = rest
        _lib.check(lib.rldx_msat_qkv_norm_rope_bf16(descs, len(streams), num_heads, head_dim, q.data_ptr(),
                                                    k.data_ptr(), v.data_ptr(), q.stride(h_ax), q.stride(h_ax + 1),
                                                    None, 0, float(eps), _stream_ptr(q)), "rldx_msat_qkv_norm_rope_bf16")
    return (q, *rest)


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
def _bhs_strides(t: torch.Tensor, layout: str):
    if layout == "bhsd":
        return [t.stride(0), t.stride(1), t.stride(2)]
    if layout == "bshd":
        return [t.stride(0), t.stride(2), t.stride(1)]
    raise ValueError(f"unknown layout {layout}")


def _key_bias_args(key_bias: Optional[torch.Tensor], B: int, Sk: int):
    if key_bias is None:
        return None, 0
    _require(key_bias.dtype == F32 and key_bias.stride(-1) == 1, "key_bias must be fp32 with contiguous keys")
    if key_bias.dim() == 1:
        _require(key_bias.shape[0] == Sk, "key_bias must have seq_k entries")
        return key_bias.data_ptr(), 0
    _require(key_bias.dim() == 2 and key_bias.shape[1] == Sk and key_bias.shape[0] in (1, B), "key_bias must be [B, Sk]")
    return key_bias.data_ptr(), (key_bias.stride(0) if key_bias.shape[0] == B and B > 1 else 0)


def _attn_dims(q, k, layout):
    for t, n in ((q, "q"), (k, "k")):
        _require(t.dtype == BF16 and t.dim() == 4 and t.stride(-1) == 1, f"{n} must be 4-D bf16, last dim contiguous")
    if layout == "bhsd":
        B, Hq, Sq, D = q.shape
        _, Hkv, Sk, _ = k.shape
    else:
        B, Sq, Hq, D = q.shape
        _, Sk, Hkv, _ = k.shape
    _require(D in (64, 128), "head_dim must be 64 or 128")
    _require(k.shape[0] == B and k.shape[3] == D, "k batch/head_dim must match q")
    _require(Hkv > 0 and Hq % Hkv == 0, "q heads must be a multiple of kv heads")
    return B, Hq, Hkv, Sq, Sk, D


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, key_bias: Optional[torch.Tensor] = None,
              causal: bool = False, scale: Optional[float] = None, layout: str = "bhsd",
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(Q K^T * scale + key_bias (+ causal)) V with GQA, bf16.

    layout "bhsd": tensors [B, H, S, D]; "bshd": [B, S, H, D].  key_bias: fp32
    [B, Sk] or [Sk] additive (0 / -inf).  scale defaults to 1/sqrt(D)."""
    _on_gpu(q, k, v, key_bias, out)
    B, Hq, Hkv, Sq, Sk, D = _attn_dims(q, k, layout)
    _require(v.dtype == BF16 and k.shape == v.shape and v.stride(-1) == 1, "v must match k")
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    _require(out.shape == q.shape and out.dtype == BF16 and out.stride(-1) == 1, "out must match q")
    kb_ptr, kb_stride = _key_bias_args(key_bias, B, Sk)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    lib = _lib.load()
    ws_bytes = int(lib.rldx_attention_workspace_bytes(B, Hkv, Sk, D))
    ws = torch.empty(max(ws_bytes // 2, 8), dtype=BF16, device=q.device)
    _lib.check(lib.rldx_attention_fwd_bf16(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, Hq, Hkv, Sq, Sk,
                                           D, _lib.i64_array(_bhs_strides(q, layout)),
                                           _lib.i64_array(_bhs_strides(k, layout)),
                                           _lib.i64_array(_bhs_strides(v, layout)),
                                           _lib.i64_array(_bhs_strides(out, layout)), kb_ptr, kb_stride, float(scale),
                                           int(bool(causal)), ws.data_ptr(), ws.numel() * 2, _stream_ptr(q)),
               "rldx_attention_fwd_bf16")
    return out


def kv_packed_elems(seq_k: int, head_dim: int) -> int:
    """bf16 elements of the packed K/V tiles of one (batch, kv head): ceil(Sk/32) * 64 * D."""
    return (seq_k + 31) // 32 * 64 * head_dim


def kv_pack(k: torch.Tensor, v: torch.Tensor, layout: str = "bhsd") -> torch.Tensor:
    """K, V [B, H, S, D] (or [B, S, H, D]) -> packed K/V tiles [B, H, kv_packed_elems(S, D)]
    (32 keys per tile; every MFMA operand of the attention kernel is one 1 KB block)."""
    _on_gpu(k, v)
    for t in (k, v):
        _require(t.dtype == BF16 and t.dim() == 4 and t.stride(-1) == 1, "k/v must be 4-D bf16, last dim contiguous")
    _require(k.shape == v.shape, "k and v must have one shape")
    if layout == "bhsd":
        B, H, S, D = k.shape
    else:
        B, S, H, D = k.shape
    kvp = torch.empty((B, H, kv_packed_elems(S, D)), dtype=BF16, device=k.device)
    lib = _lib.load()
    _lib.check(lib.rldx_attention_kv_pack_bf16(k.data_ptr(), _lib.i64_array(_bhs_strides(k, layout)), v.data_ptr(),
                                               _lib.i64_array(_bhs_strides(v, layout)), kvp.data_ptr(),
                                               _lib.i64_array([kvp.stride(0), kvp.stride(1)]), B, H, S, D,
                                               _stream_ptr(k)), "rldx_attention_kv_pack_bf16")
    return kvp


def attention_packed(q: torch.Tensor, kvp: torch.Tensor, seq_k: int, *, key_bias: Optional[torch.Tensor] = None,
                     causal: bool = False, scale: Optional[float] = None, layout: str = "bhsd",
                     out=None, warm: Optional[Sequence[torch.Tensor]] = None,
                     segments: Optional[Sequence[tuple]] = None):
    """Attention with K/V given as packed tiles [B, Hkv, >= kv_packed_elems(seq_k, D)]
    (see kv_pack; the MSAT QKV kernel writes them directly).  `out` may be a
    PackedAct [Sq, Hq*D] (batch 1), or a column view of a wider one: O is then
    written in the grouped GEMM's packed activation order.  segments (with a
    PackedAct out, any batch): 1-3 (first query row, rows, first packed row)
    triples; query row r of batch entry b inside a segment goes to packed row
    first + b * rows + (r - first query row), rows outside every segment are
    not stored (rldx_attention_packed_segments_fwd_bf16).  warm: up to three
    tensors (e.g. the packed weights of a later GEMM) whose memory extra
    workgroups of the launch read into the memory-side cache while it runs
    (rldx_attention_packed_fwd_warm_bf16; the attention result is unchanged)."""
    _on_gpu(q, kvp, key_bias)
    _require(q.dtype == BF16 and q.dim() == 4 and q.stride(-1) == 1, "q must be 4-D bf16, last dim contiguous")
    if layout == "bhsd":
        B, Hq, Sq, D = q.shape
    elif layout == "bshd":
        B, Sq, Hq, D = q.shape
    else:
        raise ValueError(f"unknown layout {layout}")
    _require(D in (64, 128), "head_dim must be 64 or 128")
    _require(kvp.dtype == BF16 and kvp.dim() == 3 and kvp.shape[0] == B and kvp.stride(2) == 1 and
             kvp.shape[2] >= kv_packed_elems(seq_k, D), "kvp must be [B, Hkv, >= kv_packed_elems(seq_k, D)] bf16")
    Hkv = kvp.shape[1]
    _require(Hkv > 0 and Hq % Hkv == 0, "q heads must be a multiple of kv heads")
    packed_out = isinstance(out, PackedAct)
    if segments is not None:
        _require(packed_out and not warm, "segments need a PackedAct out (and no warm ranges)")
        segments = [tuple(int(v) for v in sg) for sg in segments]
        _require(1 <= len(segments) <= 3 and all(len(sg) == 3 for sg in segments),
                 "segments: 1-3 (first query row, rows, first packed row) triples")
        end = 0
        for off, rows, base in segments:
            _require(off >= end and rows >= 0 and base >= 0 and off + rows <= Sq and base + B * rows <= out.m,
                     "segments must be ascending, disjoint, inside the queries and inside the packed out")
            end = off + rows
    if packed_out:
        _on_gpu(out.data)
        _require(out.k == Hq * D and (segments is not None or (B == 1 and out.m == Sq)),
                 "packed out must be a PackedAct [Sq, Hq*D] (or a column view of that width), batch 1, "
                 "unless row segments map the batch into it")
        o_ptr, o_strides = out.data.data_ptr(), [0, 0, 0]
    else:
        if out is None:
            out = torch.empty_like(q, memory_format=torch.contiguous_format)
        _on_gpu(out)
        _require(out.shape == q.shape and out.dtype == BF16 and out.stride(-1) == 1, "out must match q")
        o_ptr, o_strides = out.data_ptr(), _bhs_strides(out, layout)
    kb_ptr, kb_stride = _key_bias_args(key_bias, B, seq_k)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    lib = _lib.load()
    args = (q.data_ptr(), kvp.data_ptr(), _lib.i64_array([kvp.stride(0), kvp.stride(1)]), o_ptr,
            (out.ld if out.ld != out.k else 1) if packed_out else 0, B, Hq, Hkv, Sq, seq_k, D,
            _lib.i64_array(_bhs_strides(q, layout)), _lib.i64_array(o_strides), kb_ptr, kb_stride, float(scale),
            int(bool(causal)))
    if segments is not None:
        seg = _lib.i64_array([v for sg in segments for v in sg])
        _lib.check(lib.rldx_attention_packed_segments_fwd_bf16(
            q.data_ptr(), kvp.data_ptr(), _lib.i64_array([kvp.stride(0), kvp.stride(1)]), o_ptr,
            out.ld if out.ld != out.k else 1, seg, len(segments), B, Hq, Hkv, Sq, seq_k, D,
            _lib.i64_array(_bhs_strides(q, layout)), kb_ptr, kb_stride, float(scale), int(bool(causal)),
            _stream_ptr(q)), "rldx_attention_packed_segments_fwd_bf16")
    elif warm:
        ptrs, nbytes, count = _warm_args(warm, q.device)
        _lib.check(lib.rldx_attention_packed_fwd_warm_bf16(*args, ptrs, nbytes, count, _stream_ptr(q)),
                   "rldx_attention_packed_fwd_warm_bf16")
    else:
        _lib.check(lib.rldx_attention_packed_fwd_bf16(*args, _stream_ptr(q)), "rldx_attention_packed_fwd_bf16")
    return out


def llm_fused_attention(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, cos: torch.Tensor,
                        sin: torch.Tensor, num_heads: int, num_kv_heads: int, head_dim: int, *,
                        sin_is_signed: bool = True, eps: float = 1e-6,
                        out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Packed QKV (M, (Hq + 2*Hkv)*D) -> (M, Hq*D): q_norm/k_norm + rotate-half RoPE +
    causal GQA attention (rldx_backbone::fused_attention semantics)."""
    _on_gpu(qkv, q_norm_w, k_norm_w, cos, sin, out)
    M = qkv.shape[0]
    Hq, Hkv, D = num_heads, num_kv_heads, head_dim
    _require(qkv.dtype == BF16 and qkv.dim() == 2 and qkv.stride(1) == 1, "qkv must be 2-D bf16 rows")
    _require(qkv.shape[1] >= (Hq + 2 * Hkv) * D, f"qkv rows must hold (Hq + 2*Hkv)*D = {(Hq + 2 * Hkv) * D} columns")
    for t, n in ((q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w")):
        _require(t.dtype == BF16 and t.is_contiguous() and t.numel() == D, f"{n} must be contiguous bf16 [D]")
    _require(cos.dtype == BF16 and sin.dtype == BF16 and cos.shape == (M, D) and sin.shape == (M, D),
             "cos / sin must be bf16 [M, D]")
    _require(cos.stride(1) == 1 and sin.stride() == cos.stride(), "cos / sin must share a row-major layout")
    if out is None:
        out = torch.empty((M, Hq * D), dtype=BF16, device=qkv.device)
    _require(out.dtype == BF16 and out.shape == (M, Hq * D) and out.stride(1) == 1, "out must be bf16 (M, Hq*D)")
    lib = _lib.load()
    ws_bytes = int(lib.rldx_llm_fused_attention_workspace_bytes(M, Hkv, D))
    ws = torch.empty(max(ws_bytes // 2, 8), dtype=BF16, device=qkv.device)
    _lib.check(lib.rldx_llm_fused_attention_bf16(qkv.data_ptr(), qkv.stride(0), q_norm_w.data_ptr(), k_norm_w.data_ptr(),
                                                 cos.data_ptr(), sin.data_ptr(), cos.stride(0), int(bool(sin_is_signed)),
                                                 out.data_ptr(), out.stride(0), M, Hq, Hkv, D, float(eps), ws.data_ptr(),
                                                 ws.numel() * 2, _stream_ptr(qkv)), "rldx_llm_fused_attention_bf16")
    return out


def vision_attention_workspace_bytes(total_tokens: int, num_seqs: int, num_heads: int, head_dim: int) -> int:
    n = int(_lib.load().rldx_vision_attention_workspace_bytes(total_tokens, num_seqs, num_heads, head_dim))
    _require(n >= 0, f"vision attention: unsupported head_dim {head_dim} (multiple of 8 in [8, 128])")
    return n


def vision_attention(qkv: torch.Tensor, rope_cos: torch.Tensor, rope_sin: torch.Tensor, cu_seqlens: torch.Tensor,
                     scaling: float, num_heads: int, head_dim: int, *, out: Optional[torch.Tensor] = None,
                     workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused QKV (M, 3*H*D) bf16 -> (M, H*D) bf16: rotate-half RoPE with the
    baked fp32 tables (sin's first half negated) on Q and K, then non-causal
    attention within each cu_seqlens segment (rldx_backbone::vision_attention
    semantics).  `workspace` (uint8, >= vision_attention_workspace_bytes) may
    be passed in to keep the call allocation-free."""
    _on_gpu(qkv, rope_cos, rope_sin, cu_seqlens, out, workspace)
    H, D = int(num_heads), int(head_dim)
    _require(qkv.dtype == BF16 and qkv.dim() == 2 and qkv.is_contiguous() and qkv.shape[1] == 3 * H * D,
             f"qkv must be contiguous bf16 (M, 3*H*D = {3 * H * D})")
    M = qkv.shape[0]
    if rope_cos.dtype != F32:
        rope_cos = rope_cos.float()
    if rope_sin.dtype != F32:
        rope_sin = rope_sin.float()
    rope_cos, rope_sin = rope_cos.contiguous(), rope_sin.contiguous()
    _require(rope_cos.shape == (M, D) and rope_sin.shape == (M, D), f"rope_cos / rope_sin must be (M, D) = ({M}, {D})")
    _require(cu_seqlens.dtype == torch.int32 and cu_seqlens.dim() == 1 and cu_seqlens.numel() >= 2 and
             cu_seqlens.is_contiguous(), "cu_seqlens must be contiguous int32 (num_seqs + 1,)")
    S = cu_seqlens.numel() - 1
    if out is None:
        out = torch.empty((M, H * D), dtype=BF16, device=qkv.device)
    _require(out.dtype == BF16 and out.shape == (M, H * D) and out.is_contiguous(), "out must be contiguous bf16 (M, H*D)")
    need = vision_attention_workspace_bytes(M, S, H, D)
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=qkv.device)
    _require(workspace.dtype == torch.uint8 and workspace.is_contiguous() and workspace.numel() >= need,
             f"workspace must be contiguous uint8 with >= {need} bytes")
    lib = _lib.load()
    _lib.check(lib.rldx_vision_attention_bf16(qkv.data_ptr(), rope_cos.data_ptr(), rope_sin.data_ptr(),
                                              cu_seqlens.data_ptr(), S, out.data_ptr(), M, H, D, float(scaling),
                                              workspace.data_ptr(), workspace.numel(), _stream_ptr(qkv)),
               "rldx_vision_attention_bf16")
    return out


def memory_attention(qkv: torch.Tensor, cos: torch.Tensor, signed_sin: torch.Tensor, num_heads: int,
                     head_dim: int, block_attn_size: int, *, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused QKV (M, 3*H*D) bf16 -> (M, H*D) bf16: bf16 rotate-half RoPE on Q and K
    (cos / signed_sin (M, D) bf16), then block-causal attention (query i sees key j
    iff j // block_attn_size <= i // block_attn_size); mem::fused_attention semantics."""
    _on_gpu(qkv, cos, signed_sin, out)
    H, D = int(num_heads), int(head_dim)
    _require(D in (64, 128, 256), f"memory attention: head_dim {D} not in (64, 128, 256)")
    _require(int(block_attn_size) >= 1, "block_attn_size must be >= 1")
    _require(qkv.dtype == BF16 and qkv.dim() == 2 and qkv.is_contiguous() and qkv.shape[1] == 3 * H * D,
             f"qkv must be contiguous bf16 (M, 3*H*D = {3 * H * D})")
    M = qkv.shape[0]
    for t, n in ((cos, "cos"), (signed_sin, "signed_sin")):
        _require(t.dtype == BF16 and t.is_contiguous() and t.shape == (M, D), f"{n} must be contiguous bf16 (M, D)")
    if out is None:
        out = torch.empty((M, H * D), dtype=BF16, device=qkv.device)
    _require(out.dtype == BF16 and out.shape == (M, H * D) and out.is_contiguous(), "out must be contiguous bf16 (M, H*D)")
    _lib.check(_lib.load().rldx_memory_attention_bf16(qkv.data_ptr(), cos.data_ptr(), signed_sin.data_ptr(),
                                                      out.data_ptr(), M, H, D, int(block_attn_size), _stream_ptr(qkv)),
               "rldx_memory_attention_bf16")
    return out


# ---------------------------------------------------------------------------
# grouped GEMM (MSAT block linears)
# ---------------------------------------------------------------------------
class PackedWeight:
    """A weight W [n, k] bf16 packed once into the grouped GEMM's operand order,
    with its fp32 row sums s[j] = sum_k W[j][k] (original row order), which a
    GEMM with the LayerNorm fold needs."""

    __slots__ = ("data", "n", "k", "swiglu_pairs", "row_sums")

    def __init__(self, data: torch.Tensor, n: int, k: int, swiglu_pairs: bool, row_sums: Optional[torch.Tensor] = None):
        self.data, self.n, self.k, self.swiglu_pairs, self.row_sums = data, n, k, swiglu_pairs, row_sums


def pack_weight(w: torch.Tensor, swiglu_pairs: bool = False) -> PackedWeight:
    """nn.Linear weight [out_features, in_features] bf16 -> PackedWeight.  With
    swiglu_pairs, w = [gate; up] and the GEMM's SwiGLU epilogue can be used."""
    _on_gpu(w)
    _require(w.dtype == BF16 and w.dim() == 2 and w.stride(1) == 1, "weight must be 2-D bf16, rows contiguous")
    n, k = w.shape
    _require(n % (64 if swiglu_pairs else 32) == 0 and k % 16 == 0, "weight shape not tileable")
    out = torch.empty(n * k, dtype=BF16, device=w.device)
    lib = _lib.load()
    _lib.check(lib.rldx_gemm_pack_weight_bf16(w.data_ptr(), w.stride(0), n, k, int(swiglu_pairs), out.data_ptr(),
                                              _stream_ptr(w)), "rldx_gemm_pack_weight_bf16")
    return PackedWeight(out, n, k, swiglu_pairs, w.float().sum(dim=1).contiguous())


class PackedAct:
    """Activations [m, k] bf16 in the grouped GEMM's packed operand order
    (32-row x 16-column chunks, rows padded to a multiple of 32).  A column
    view (`cols`) covers columns of a wider packed matrix `ld` columns wide."""

    __slots__ = ("data", "m", "k", "ld")

    def __init__(self, data: torch.Tensor, m: int, k: int, ld: Optional[int] = None):
        self.data, self.m, self.k = data, m, k
        self.ld = k if ld is None else ld

    @staticmethod
    def empty(m: int, k: int, device) -> "PackedAct":
        return PackedAct(torch.empty((m + 31) // 32 * 32 * k, dtype=BF16, device=device), m, k)

    def rows(self, start: int, stop: int) -> "PackedAct":
        """Rows [start, stop) as a PackedAct view; start must be a multiple of 32."""
        _require(start % 32 == 0 and 0 <= start <= stop <= self.m, "row range must start on a 32-row boundary")
        return PackedAct(self.data[start * self.ld:], stop - start, self.k, self.ld)

    def cols(self, start: int, stop: int) -> "PackedAct":
        """Columns [start, stop) as an output view (a write target of the packed
        GEMM epilogues and the attention kernel); start must be a multiple of 16."""
        _require(self.k == self.ld, "column view of a column view")
        _require(start % 16 == 0 and 0 <= start < stop <= self.k, "column range must start on a 16-column chunk")
        return PackedAct(self.data[start // 16 * 512:], self.m, stop - start, self.ld)

    def unpack(self) -> torch.Tensor:
        """Row-major copy (for tests and debugging)."""
        _require(self.k == self.ld, "unpack a whole packed matrix")
        m, k = self.m, self.k
        mp = (m + 31) // 32
        t = self.data[: mp * 32 * k].view(mp, k // 16, 2, 32, 8)  # mb, kb, half, row, i
        return t.permute(0, 3, 1, 2, 4).reshape(mp * 32, k)[:m]


def ln_stats_empty(m: int, k: int, device) -> torch.Tensor:
    """LayerNorm statistics of m rows of width k for a LayerNorm-folding GEMM:
    fp32 [k / 64, m, 2], (sum, sum of squares) per 64-column slot, slot-major."""
    _require(k % 64 == 0, "k must be a multiple of 64")
    return torch.empty(k // 64, m, 2, dtype=F32, device=device)


def _check_stats(st: torch.Tensor, m: int, k: int) -> None:
    _on_gpu(st)
    _require(st.dtype == F32 and tuple(st.shape) == (k // 64, m, 2) and st.is_contiguous(),
             "LayerNorm statistics must be contiguous fp32 [k / 64, m, 2]")


def pack_act(x: torch.Tensor, out: Optional[PackedAct] = None, stats: Optional[torch.Tensor] = None) -> PackedAct:
    """Row-major x [m, k] -> PackedAct; with `stats` ([k / 64, m, 2] fp32) also the
    rows' LayerNorm statistics (rldx_act_pack_stats_bf16)."""
    _on_gpu(x)
    _require(x.dtype == BF16 and x.dim() == 2 and x.stride(1) == 1, "x must be 2-D bf16, rows contiguous")
    m, k = x.shape
    out = PackedAct.empty(m, k, x.device) if out is None else out
    _require(out.m == m and out.k == k, "out shape mismatch")
    lib = _lib.load()
    if stats is not None:
        _check_stats(stats, m, k)
        _lib.check(lib.rldx_act_pack_stats_bf16(x.data_ptr(), x.stride(0), m, k, out.data.data_ptr(),
                                                stats.data_ptr(), _stream_ptr(x)), "rldx_act_pack_stats_bf16")
        return out
    _lib.check(lib.rldx_act_pack_bf16(x.data_ptr(), x.stride(0), m, k, out.data.data_ptr(), _stream_ptr(x)),
               "rldx_act_pack_bf16")
    return out


def _check_pack_target(out: PackedAct, m: int, k: int) -> None:
    _require(isinstance(out, PackedAct) and out.m == m and out.k == k, "out shape mismatch")
    _require(out.ld == out.k, "out must be a whole packed matrix, not a column view")
    _require(out.data.dtype == BF16 and out.data.numel() >= (m + 31) // 32 * 32 * k, "out buffer too small")
    _on_gpu(out.data)


def layernorm_pack(x: torch.Tensor, eps: float = 1e-6, out: Optional[PackedAct] = None) -> PackedAct:
    """LayerNorm without affine parameters over the last dim of x [m, k], packed."""
    _on_gpu(x)
    _require(x.dtype == BF16 and x.dim() == 2 and x.stride(1) == 1, "x must be 2-D bf16, rows contiguous")
    m, k = x.shape
    out = PackedAct.empty(m, k, x.device) if out is None else out
    _check_pack_target(out, m, k)
    lib = _lib.load()
    _lib.check(lib.rldx_layernorm_pack_bf16(x.data_ptr(), x.stride(0), m, k, float(eps), out.data.data_ptr(),
                                            _stream_ptr(x)), "rldx_layernorm_pack_bf16")
    return out


def layernorm_pack_many(pairs: Sequence[tuple], eps: float = 1e-6) -> None:
    """layernorm_pack of up to 4 (x [m, k], out PackedAct) pairs in one launch
    (rldx_layernorm_pack_many_bf16): the pre-norms of a block's streams."""
    _require(1 <= len(pairs) <= 4, "between 1 and 4 matrices")
    rows = (_lib.Rows * len(pairs))()
    for i, (x, out) in enumerate(pairs):
        _on_gpu(x)
        _require(x.dtype == BF16 and x.dim() == 2 and x.stride(1) == 1, "x must be 2-D bf16, rows contiguous")
        _check_pack_target(out, x.shape[0], x.shape[1])
        _require(x.device == pairs[0][0].device and out.data.device == x.device, "all matrices on one device")
        rows[i] = _lib.Rows(x.data_ptr(), x.stride(0), x.shape[0], x.shape[1], out.data.data_ptr())
    _lib.check(_lib.load().rldx_layernorm_pack_many_bf16(rows, len(pairs), float(eps), _stream_ptr(pairs[0][0])),
               "rldx_layernorm_pack_many_bf16")


def _bf16_rows(t: torch.Tensor, shape: tuple, what: str) -> None:
    _on_gpu(t)
    _require(t.dtype == BF16 and tuple(t.shape) == shape and t.is_contiguous(), f"{what} must be contiguous bf16 {shape}")


def action_encode_pack(act: torch.Tensor, w_in: torch.Tensor, b_in: torch.Tensor, temb: torch.Tensor,
                       pos: torch.Tensor, out: PackedAct, stats: torch.Tensor,
                       others: Sequence[tuple] = ()) -> None:
    """One launch (rldx_action_encode_pack_bf16): out = the packed rows
    bf16(bf16(bf16(act W_in^T + b_in) + temb) + pos) with their LayerNorm
    statistics `stats` ([hidden / 64, n, 2]), and each (x [m, hidden], out
    PackedAct, stats) of `others` (up to 3) packed with its statistics."""
    n, adim = act.shape
    hidden = w_in.shape[0]
    _bf16_rows(act, (n, adim), "act")
    _bf16_rows(w_in, (hidden, adim), "w_in")
    _bf16_rows(b_in, (hidden,), "b_in")
    _bf16_rows(temb.reshape(-1), (hidden,), "temb")
    _bf16_rows(pos, (n, hidden), "pos")
    _check_pack_target(out, n, hidden)
    _check_stats(stats, n, hidden)
    _require(len(others) <= 3, "at most 3 more matrices")
    rows = (_lib.Rows * max(1, len(others)))()
    sts = (ctypes.c_void_p * max(1, len(others)))()
    for i, (x, o, st) in enumerate(others):
        _on_gpu(x)
        _require(x.dtype == BF16 and x.dim() == 2 and x.shape[1] == hidden and x.stride(1) == 1,
                 "x must be 2-D bf16 [m, hidden], rows contiguous")
        _check_pack_target(o, x.shape[0], hidden)
        _check_stats(st, x.shape[0], hidden)
        rows[i] = _lib.Rows(x.data_ptr(), x.stride(0), x.shape[0], hidden, o.data.data_ptr())
        sts[i] = st.data_ptr()
    _lib.check(_lib.load().rldx_action_encode_pack_bf16(act.data_ptr(), n, adim, w_in.data_ptr(), b_in.data_ptr(),
                                                        temb.data_ptr(), pos.data_ptr(), hidden, out.data.data_ptr(),
                                                        stats.data_ptr(), rows, sts, len(others), _stream_ptr(act)),
               "rldx_action_encode_pack_bf16")


def action_decode_euler(x: PackedAct, w_out: torch.Tensor, b_out: torch.Tensor, act: torch.Tensor, dt: float,
                        eps: float = 1e-6) -> None:
    """act += dt * (LN(x) W_out^T + b_out), in place, one launch
    (rldx_action_decode_euler_bf16; each of the eager chain's roundings)."""
    n, adim = act.shape
    hidden = w_out.shape[1]
    _require(isinstance(x, PackedAct) and x.m == n and x.k == hidden and x.ld == x.k, "x must be a PackedAct [n, hidden]")
    _on_gpu(x.data)
    _bf16_rows(w_out, (adim, hidden), "w_out")
    _bf16_rows(b_out, (adim,), "b_out")
    _bf16_rows(act, (n, adim), "act")
    _lib.check(_lib.load().rldx_action_decode_euler_bf16(x.data.data_ptr(), n, hidden, float(eps), w_out.data_ptr(),
                                                         b_out.data_ptr(), adim, float(dt), act.data_ptr(),
                                                         _stream_ptr(act)), "rldx_action_decode_euler_bf16")


class GemmWorkspace:
    """Device scratch of the split-K grouped GEMM: per-tile arrival counters and
    fp32 partial tiles.  Zero-filled once here; every launch leaves its counters
    at zero again, so one workspace serves any number of grouped_gemm calls that
    run one after another on one stream (calls that overlap in time need their own)."""

    __slots__ = ("data",)

    COUNTER_BYTES = 65536  # the tile counters; the fp32 partials follow and need no initial value

    def __init__(self, nbytes: int, device):
        self.data = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        self.data[: self.COUNTER_BYTES].zero_()


_GEMM_EPI = {"bias": _lib.GEMM_EPI_BIAS, "residual": _lib.GEMM_EPI_RESIDUAL, "swiglu": _lib.GEMM_EPI_SWIGLU,
             "swiglu_packed": _lib.GEMM_EPI_SWIGLU_PACKED, "bias_packed": _lib.GEMM_EPI_BIAS_PACKED,
             "residual_packed": _lib.GEMM_EPI_RESIDUAL_PACKED}
_PACKED_EPI = (_lib.GEMM_EPI_SWIGLU_PACKED, _lib.GEMM_EPI_BIAS_PACKED, _lib.GEMM_EPI_RESIDUAL_PACKED)


def _mixed(items: Sequence[tuple]) -> bool:
    """Groups of different weight shapes (a launch of rldx_grouped_gemm_mixed_bf16)."""
    return any((it[1].n, it[1].k) != (items[0][1].n, items[0][1].k) for it in items)


def _gemm_groups(items: Sequence[tuple], epi: int, pack: bool):
    _require(1 <= len(items) <= 3, "between 1 and 3 groups")
    groups = (_lib.GemmGroup * len(items))()
    keep = []
    for i, (a, w, bias, out, res) in enumerate(items):
        n, k = w.n, w.k
        if not isinstance(a, PackedAct):
            _require(isinstance(a, torch.Tensor) and a.dim() == 2, "a must be a PackedAct or a 2-D tensor")
            if not pack:  # shape-only query
                a = PackedAct(a, a.shape[0], a.shape[1])
            else:
                a = pack_act(a)
                keep.append(a)
        _on_gpu(a.data, w.data, bias, res if isinstance(res, torch.Tensor) else None)
        _require(a.k == k and a.ld == k, "a must be a PackedAct [m, k] of the weight's k")
        swiglu = epi in (_lib.GEMM_EPI_SWIGLU, _lib.GEMM_EPI_SWIGLU_PACKED)
        _require(not swiglu or w.swiglu_pairs, "SwiGLU epilogue needs a swiglu_pairs weight")
        m = a.m
        n_out = n // 2 if swiglu else n
        if epi in _PACKED_EPI:
            _require(isinstance(out, PackedAct) and out.m == m and out.k == n_out,
                     "out must be a PackedAct [m, n_out] (or a column view of that width)")
            out_ptr, ldo = out.data.data_ptr(), (0 if out.ld == out.k else out.ld)
        else:
            _require(out.dtype == BF16 and out.dim() == 2 and out.stride(1) == 1 and tuple(out.shape) == (m, n_out),
                     "out must be [m, n_out] bf16")
            out_ptr, ldo = out.data_ptr(), out.stride(0)
        if bias is not None:
            _require(bias.dtype == BF16 and bias.is_contiguous() and bias.numel() == n, "bias must be [n] bf16")
        res_ptr, ldr = None, 0
        if epi == _lib.GEMM_EPI_RESIDUAL:
            _require(res is not None and res.dtype == BF16 and res.dim() == 2 and res.stride(1) == 1 and
                     tuple(res.shape) == (m, n), "residual must be [m, n] bf16")
            res_ptr, ldr = res.data_ptr(), res.stride(0)
        elif epi == _lib.GEMM_EPI_RESIDUAL_PACKED:
            _require(isinstance(res, PackedAct) and res.m == m and res.k == n, "residual must be a PackedAct [m, n]")
            _on_gpu(res.data)
            res_ptr, ldr = res.data.data_ptr(), (0 if res.ld == res.k else res.ld)
        groups[i] = _lib.GemmGroup(a.data.data_ptr(), m, w.data.data_ptr(), _ptr(bias), out_ptr, ldo, res_ptr, ldr)
    return groups, items[0][1].n, items[0][1].k, keep, w.data


def _shape_arrays(items: Sequence[tuple], split_k):
    """Per-group n, k (and split) arrays for the mixed-shape entry points."""
    ns = _lib.i64_array([it[1].n for it in items])
    ks = _lib.i64_array([it[1].k for it in items])
    sp = [int(split_k)] * len(items) if isinstance(split_k, int) else [int(x) for x in split_k]
    _require(len(sp) == len(items) and all(1 <= x <= 64 for x in sp), "one split factor in [1, 64] per group")
    return ns, ks, (ctypes.c_int32 * len(items))(*sp), max(sp) > 1


def grouped_gemm_workspace_bytes(items: Sequence[tuple], epilogue: str = "bias", split_k: int = 1,
                                 wide_tiles: bool = False) -> int:
    """Workspace bytes grouped_gemm(items, epilogue, split_k, workspace, wide_tiles) needs (0: no split)."""
    epi = _GEMM_EPI[epilogue]
    groups, n, k, _, _ = _gemm_groups(items, epi, pack=False)
    flags = _lib.GEMM_WIDE_TILES if wide_tiles else 0
    if _mixed(items) or not isinstance(split_k, int):
        ns, ks, sp, _ = _shape_arrays(items, split_k)
        r = _lib.load().rldx_grouped_gemm_mixed_workspace_bytes(groups, ns, ks, sp, len(items), epi, flags)
    else:
        r = _lib.load().rldx_grouped_gemm_ex_workspace_bytes(groups, len(items), n, k, epi, int(split_k), flags)
    _require(r >= 0, "grouped GEMM shape not supported")
    return int(r)


def _row_sums_array(items: Sequence[tuple]):
    sums = (ctypes.c_void_p * len(items))()
    for i, it in enumerate(items):
        w = it[1]
        _require(w.row_sums is not None and w.row_sums.dtype == F32 and w.row_sums.numel() == w.n,
                 "the LayerNorm fold needs the weight's fp32 row sums")
        _on_gpu(w.row_sums)
        sums[i] = w.row_sums.data_ptr()
    return sums


def _stats_array(items: Sequence[tuple], stats: Sequence[torch.Tensor], width: Optional[int]):
    """Pointers to one statistics tensor per group, width columns (None: the group's own n)."""
    _require(len(stats) == len(items), "one statistics tensor per group")
    arr = (ctypes.c_void_p * len(items))()
    for i, (it, st) in enumerate(zip(items, stats)):
        a = it[0]
        _check_stats(st, a.m if isinstance(a, PackedAct) else a.shape[0], it[1].n if width is None else width)
        arr[i] = st.data_ptr()
    return arr


def grouped_gemm(items: Sequence[tuple], epilogue: str = "bias", split_k=1,
                 workspace: Optional[GemmWorkspace] = None, wide_tiles: bool = False,
                 splits_across_xcds: bool = False, ln_eps: Optional[float] = None,
                 ln_stats: Optional[Sequence[torch.Tensor]] = None,
                 stats_out: Optional[Sequence[torch.Tensor]] = None) -> None:
    """One launch of y_s = a_s W_s^T + bias_s for up to 3 streams sharing n and k.
    items: (a PackedAct [m, k] or row-major tensor (packed first), PackedWeight,
    bias [n] or None, out, residual or None).  epilogue: "bias" (out = y),
    "residual" (out = residual + y, residual may be out), "swiglu" (out [m, n/2] =
    swiglu(y)), "swiglu_packed" or "bias_packed" (out a PackedAct, or a column view
    of a wider one: PackedAct.cols).  split_k > 1 splits the K
    range of every stream over that many workgroups (partials summed in a fixed
    order: deterministic); it needs a workspace of grouped_gemm_workspace_bytes(...)
    bytes.  wide_tiles: 64 x 128 / 32 x 128 tiles for the streams below the 128 x
    128 threshold (RLDX_GEMM_WIDE_TILES; the same results, faster or slower by
    shape).  splits_across_xcds: the splits of each tile on different XCDs
    (RLDX_GEMM_SPLITS_ACROSS_XCDS; the same results, for tests).
    ln_eps, ln_stats: the LayerNorm fold (rldx_grouped_gemm_ln_bf16): each a is
    the un-normalised rows x, ln_stats[i] their statistics ([k / 64, m, 2], from
    a `stats_out` or pack_act(..., stats=)), and the result is LN(x) W^T (+ bias
    ...), LN without affine parameters with this eps; epilogues "bias" and
    "swiglu_packed", no split-K; the weights' row sums come from pack_weight.
    stats_out: the residual epilogues also write the statistics of the rows
    they store, stats_out[i] [n / 64, m, 2] (rldx_grouped_gemm_stats_bf16).
    Groups whose weights differ in shape (or split_k given per group) go to
    rldx_grouped_gemm_mixed_bf16: one launch, each group its own n, k, split."""
    epi = _GEMM_EPI[epilogue]
    groups, n, k, keep, wt = _gemm_groups(items, epi, pack=True)
    lib = _lib.load()
    if _mixed(items) or not isinstance(split_k, int):
        _require(ln_eps is None, "the LayerNorm fold takes groups of one shape")
        ns, ks, sp, split = _shape_arrays(items, split_k)
        _require(not split or workspace is not None, "split factors > 1 need a GemmWorkspace")
        if split:
            _on_gpu(workspace.data)
        ws_ptr, ws_n = (workspace.data.data_ptr(), workspace.data.numel()) if split else (None, 0)
        outs = None
        if stats_out is not None:
            _require(epilogue in ("residual", "residual_packed"), "stats_out needs a residual epilogue")
            outs = _stats_array(items, stats_out, None)
        flags = (_lib.GEMM_WIDE_TILES if wide_tiles else 0) | (_lib.GEMM_SPLITS_ACROSS_XCDS if splits_across_xcds else 0)
        _lib.check(lib.rldx_grouped_gemm_mixed_bf16(groups, ns, ks, sp, outs, len(items), epi, flags, ws_ptr, ws_n,
                                                    _stream_ptr(wt)), "rldx_grouped_gemm_mixed_bf16")
        return
    if ln_eps is not None:
        _require(split_k <= 1 and not splits_across_xcds, "the LayerNorm fold does not split K")
        _require(ln_stats is not None and stats_out is None, "the LayerNorm fold needs ln_stats")
        sums = _row_sums_array(items)
        stats = _stats_array(items, ln_stats, k)
        _lib.check(lib.rldx_grouped_gemm_ln_bf16(groups, sums, stats, len(items), n, k, epi,
                                                 _lib.GEMM_WIDE_TILES if wide_tiles else 0, float(ln_eps),
                                                 _stream_ptr(wt)), "rldx_grouped_gemm_ln_bf16")
        return
    if stats_out is not None:
        _require(epilogue in ("residual", "residual_packed"), "stats_out needs a residual epilogue")
        outs = _stats_array(items, stats_out, n)
        _require(split_k <= 1 or workspace is not None, "split_k > 1 needs a GemmWorkspace")
        ws_ptr, ws_n = (workspace.data.data_ptr(), workspace.data.numel()) if split_k > 1 else (None, 0)
        flags = (_lib.GEMM_WIDE_TILES if wide_tiles else 0) | (_lib.GEMM_SPLITS_ACROSS_XCDS if splits_across_xcds else 0)
        _lib.check(lib.rldx_grouped_gemm_stats_bf16(groups, outs, len(items), n, k, epi, int(split_k), flags, ws_ptr,
                                                    ws_n, _stream_ptr(wt)), "rldx_grouped_gemm_stats_bf16")
        return
    flags = (_lib.GEMM_WIDE_TILES if wide_tiles else 0) | (_lib.GEMM_SPLITS_ACROSS_XCDS if splits_across_xcds else 0)
    if flags:
        _require(split_k <= 1 or workspace is not None, "split_k > 1 needs a GemmWorkspace")
        ws_ptr, ws_n = (workspace.data.data_ptr(), workspace.data.numel()) if split_k > 1 else (None, 0)
        if split_k > 1:
            _on_gpu(workspace.data)
        _lib.check(lib.rldx_grouped_gemm_ex_bf16(groups, len(items), n, k, epi, int(split_k), flags,
                                                 ws_ptr, ws_n, _stream_ptr(wt)), "rldx_grouped_gemm_ex_bf16")
    elif split_k <= 1:
        _lib.check(lib.rldx_grouped_gemm_bf16(groups, len(items), n, k, epi, _stream_ptr(wt)), "rldx_grouped_gemm_bf16")
    else:
        _require(workspace is not None, "split_k > 1 needs a GemmWorkspace")
        _on_gpu(workspace.data)
        _lib.check(lib.rldx_grouped_gemm_ws_bf16(groups, len(items), n, k, epi, int(split_k), workspace.data.data_ptr(),
                                                 workspace.data.numel(), _stream_ptr(wt)), "rldx_grouped_gemm_ws_bf16")


def _warm_args(warm: Sequence[torch.Tensor], device):
    _require(len(warm) <= 3, "at most three warm-up ranges")
    _on_gpu(*warm)
    _require(all(t.is_contiguous() and t.device == device for t in warm), "warm-up tensors: contiguous, one device")
    ptrs = (ctypes.c_void_p * max(1, len(warm)))(*[t.data_ptr() for t in warm])
    return ptrs, _lib.i64_array([t.numel() * t.element_size() for t in warm] or [0]), len(warm)


def grouped_gemm_qkv_norm_rope(items: Sequence[tuple], norms: Sequence[StreamSpec], num_heads: int,
                               head_dim: int, eps: float = 1e-6, out: Optional[tuple] = None,
                               ln_eps: Optional[float] = None, ln_stats: Optional[Sequence[torch.Tensor]] = None):
    """The QKV linears of 1-3 streams (joint-sequence order) with the QK RMSNorm +
    RoPE + K/V tiling of `msat_qkv_norm_rope` in the GEMM epilogue: one launch,
    the same bits as grouped_gemm(items, "bias") followed by
    msat_qkv_norm_rope(..., kv_packed=True).  items: (a PackedAct [m, k],
    PackedWeight [3 H D, k], bias [3 H D] or None); norms: one StreamSpec per item
    (norm weights and tables; its qkv is not read, pass None).  Each stream
    starts a 32-row block of the joint sequence: a stream before the last with
    rows % 32 != 0 is followed by zero padding keys (its padding Q rows are not
    written).  Returns (q (H, M, D), kvp (H, kv_packed_elems(M, D))) with M the
    joint rows; `out` gives them.  head_dim 128, or 64 with an even head count.  Items
    may differ in K (streams of different widths, rldx_grouped_gemm_qkv_norm_rope_mixed_bf16).
    ln_eps, ln_stats: with the LayerNorm fold (each a the un-normalised rows,
    ln_stats their statistics; rldx_grouped_gemm_qkv_norm_rope_ln_bf16; one K)."""
    _require(1 <= len(items) <= 3 and len(norms) == len(items), "1-3 groups, one StreamSpec each")
    _require(head_dim == 128 or (head_dim == 64 and num_heads % 2 == 0),
             "the fused QKV epilogue needs head_dim 128, or 64 with an even head count")
    inner = num_heads * head_dim
    n, k = 3 * inner, items[0][1].k
    ks = [it[1].k for it in items]
    groups = (_lib.GemmGroup * len(items))()
    descs = (_lib.MsatStream * len(items))()
    keep, M = [], 0  # joint rows: each non-empty stream starts a 32-row (32-key) block
    for i, ((a, w, bias), s) in enumerate(zip(items, norms)):
        _require(isinstance(a, PackedAct) and a.ld == a.k, "a must be a PackedAct")
        _on_gpu(a.data, w.data, bias, s.q_w, s.k_w, s.cos, s.sin)
        _require(w.n == n and a.k == w.k and not w.swiglu_pairs, "weights must be [3 H D, k] with a [m, k]")
        if bias is not None:
            _require(bias.dtype == BF16 and bias.is_contiguous() and bias.numel() == n, "bias must be [n] bf16")
        _require(s.q_w.dtype == BF16 and s.k_w.dtype == BF16 and s.q_w.numel() == head_dim and
                 s.k_w.numel() == head_dim and s.q_w.is_contiguous() and s.k_w.is_contiguous(),
                 "norm weights must be contiguous bf16 [head_dim]")
        cos_p, sin_p, rope_ld = _rope_tables(s, a.m, head_dim, keep)
        groups[i] = _lib.GemmGroup(a.data.data_ptr(), a.m, w.data.data_ptr(), _ptr(bias), None, 0, None, 0)
        descs[i] = _lib.MsatStream(None, 0, a.m, s.q_w.data_ptr(), s.k_w.data_ptr(), cos_p, sin_p, rope_ld)
        if a.m:
            M = (M + 31) // 32 * 32 + a.m
    dev = items[0][0].data.device
    if out is None:
        q = torch.empty((num_heads, M, head_dim), dtype=BF16, device=dev)
        kvp = torch.empty((num_heads, kv_packed_elems(M, head_dim)), dtype=BF16, device=dev)
    else:
        q, kvp = out
        _require(q.dtype == BF16 and q.shape == (num_heads, M, head_dim) and q.stride(2) == 1, "q out must be (H, M, D)")
        _check_kvp_out(kvp, num_heads, M, head_dim)
    _on_gpu(q, kvp)
    if ln_eps is not None:
        _require(ln_stats is not None, "the LayerNorm fold needs ln_stats")
        _require(all(x == k for x in ks), "the LayerNorm fold takes groups of one K")
        sums = _row_sums_array(items)
        stats = _stats_array(items, ln_stats, k)
        _lib.check(_lib.load().rldx_grouped_gemm_qkv_norm_rope_ln_bf16(
            groups, descs, sums, stats, len(items), num_heads, head_dim, k, q.data_ptr(), q.stride(0), q.stride(1),
            kvp.data_ptr(), kvp.stride(0), float(eps), float(ln_eps), _stream_ptr(q)),
            "rldx_grouped_gemm_qkv_norm_rope_ln_bf16")
        return q, kvp
    if any(x != k for x in ks):
        _lib.check(_lib.load().rldx_grouped_gemm_qkv_norm_rope_mixed_bf16(
            groups, descs, len(items), num_heads, head_dim, _lib.i64_array(ks), q.data_ptr(), q.stride(0), q.stride(1),
            kvp.data_ptr(), kvp.stride(0), float(eps), _stream_ptr(q)), "rldx_grouped_gemm_qkv_norm_rope_mixed_bf16")
        return q, kvp
    _lib.check(_lib.load().rldx_grouped_gemm_qkv_norm_rope_bf16(
        groups, descs, len(items), num_heads, head_dim, k, q.data_ptr(), q.stride(0), q.stride(1), kvp.data_ptr(),
        kvp.stride(0), float(eps), _stream_ptr(q)), "rldx_grouped_gemm_qkv_norm_rope_bf16")
    return q, kvp


# ---------------------------------------------------------------------------
# Residual-add + norm epilogues (block boundaries)
# ---------------------------------------------------------------------------
def _rows_of(t: torch.Tensor, m: int, d: int, what: str, reshape: bool = False) -> torch.Tensor:
    """t as contiguous [m, d] bf16 rows: the reference launchers' `.view(M, DIM)`
    (contiguous input required), or with reshape=True their `.reshape(M, D)`
    (a strided input is first copied on the device)."""
    _require(t.dtype == BF16, f"{what} must be bfloat16")
    _require(t.numel() == m * d, f"{what} must hold {m} x {d} elements")
    if reshape:
        return t.reshape(m, d).contiguous()
    _require(t.is_contiguous(), f"{what} must be contiguous")
    return t.view(m, d)


def _vec_of(t: torch.Tensor, d: int, what: str) -> torch.Tensor:
    _require(t.dtype == BF16 and t.dim() == 1 and t.shape[0] == d and t.is_contiguous(),
             f"{what} must be a contiguous bf16 [{d}] vector")
    return t


def _out_rows(out: Optional[torch.Tensor], m: int, d: int, like: torch.Tensor, what: str) -> torch.Tensor:
    if out is None:
        return torch.empty((1, m, d), dtype=BF16, device=like.device)
    _on_gpu(out, like)
    _rows_of(out, m, d, what)
    return out


def _lead_rows(t: torch.Tensor):
    return t.shape[1] if t.dim() == 3 else t.shape[0]


def fused_grouped_res_ln(sa_residual: torch.Tensor, sa_proj_bias: torch.Tensor, sa_proj_out: torch.Tensor,
                         vl_residual: torch.Tensor, vl_proj_bias: torch.Tensor, vl_proj_out: torch.Tensor,
                         M_sa: Optional[int] = None, M_vl: Optional[int] = None, SA_DIM: Optional[int] = None,
                         VL_DIM: Optional[int] = None, eps: float = 1e-6):
    """Per stream: LayerNorm(residual + proj_out + proj_bias), fp32 sum, no affine.

    Mirrors fused_grouped_res_ln, rldx/inference/action_model/double_stream/engine/
    kernels/grouped_res_ln.py:151-211 (eps 1e-6 there, fixed).  Returns
    (sa_out [1, M_sa, SA_DIM], vl_out [1, M_vl, VL_DIM])."""
    _on_gpu(sa_residual, sa_proj_bias, sa_proj_out, vl_residual, vl_proj_bias, vl_proj_out)
    M_sa = _lead_rows(sa_residual) if M_sa is None else M_sa
    M_vl = _lead_rows(vl_residual) if M_vl is None else M_vl
    SA_DIM = sa_residual.shape[-1] if SA_DIM is None else SA_DIM
    VL_DIM = vl_residual.shape[-1] if VL_DIM is None else VL_DIM
    sr = _rows_of(sa_residual, M_sa, SA_DIM, "sa_residual")
    sp = _rows_of(sa_proj_out, M_sa, SA_DIM, "sa_proj_out")
    sb = _vec_of(sa_proj_bias, SA_DIM, "sa_proj_bias")
    vr = _rows_of(vl_residual, M_vl, VL_DIM, "vl_residual")
    vp = _rows_of(vl_proj_out, M_vl, VL_DIM, "vl_proj_out")
    vb = _vec_of(vl_proj_bias, VL_DIM, "vl_proj_bias")
    sa_out = torch.empty((1, M_sa, SA_DIM), dtype=BF16, device=sr.device)
    vl_out = torch.empty((1, M_vl, VL_DIM), dtype=BF16, device=sr.device)
    lib = _lib.load()
    _lib.check(lib.rldx_grouped_res_ln_bf16(sr.data_ptr(), sb.data_ptr(), sp.data_ptr(), sa_out.data_ptr(),
                                            vr.data_ptr(), vb.data_ptr(), vp.data_ptr(), vl_out.data_ptr(),
                                            M_sa, M_vl, SA_DIM, VL_DIM, eps, _stream_ptr(sr)),
               "rldx_grouped_res_ln_bf16")
    return sa_out, vl_out


def fused_vl_epilogue_ln(vl_residual: torch.Tensor, proj_bias: torch.Tensor, w3_bias: torch.Tensor,
                         w3_out: torch.Tensor, M: Optional[int] = None, DIM: Optional[int] = None,
                         new_vl_out: Optional[torch.Tensor] = None, ln_vl_out: Optional[torch.Tensor] = None,
                         eps: float = 1e-6):
    """new_vl = ((residual + proj_bias) + w3_bias) + w3_out (bf16 adds); ln_vl = LayerNorm(new_vl).

    Mirrors fused_vl_epilogue_ln, rldx/inference/action_model/double_stream/engine/
    kernels/vl_epilogue_ln.py:128-183, including the static `new_vl_out` /
    `ln_vl_out` buffers.  Returns (new_vl, ln_vl), both [1, M, DIM]."""
    _on_gpu(vl_residual, proj_bias, w3_bias, w3_out)
    M = _lead_rows(vl_residual) if M is None else M
    DIM = vl_residual.shape[-1] if DIM is None else DIM
    r = _rows_of(vl_residual, M, DIM, "vl_residual")
    w3 = _rows_of(w3_out, M, DIM, "w3_out")
    pb = _vec_of(proj_bias, DIM, "proj_bias")
    wb = _vec_of(w3_bias, DIM, "w3_bias")
    new_vl = _out_rows(new_vl_out, M, DIM, r, "new_vl_out")
    ln_vl = _out_rows(ln_vl_out, M, DIM, r, "ln_vl_out")
    lib = _lib.load()
    _lib.check(lib.rldx_vl_epilogue_ln_bf16(r.data_ptr(), pb.data_ptr(), wb.data_ptr(), w3.data_ptr(),
                                            new_vl.data_ptr(), ln_vl.data_ptr(), M, DIM, eps, _stream_ptr(r)),
               "rldx_vl_epilogue_ln_bf16")
    return new_vl, ln_vl


def fused_ss_epilogue_ln(hidden: torch.Tensor, M: Optional[int] = None, DIM: Optional[int] = None,
                         residual: Optional[torch.Tensor] = None, new_hidden_out: Optional[torch.Tensor] = None,
                         ln_out_out: Optional[torch.Tensor] = None, eps: float = 1e-6):
    """With residual: new_hidden = hidden + residual (bf16), ln = LayerNorm(new_hidden);
    without: new_hidden = hidden (no copy), ln = LayerNorm(hidden).

    Mirrors fused_ss_epilogue_ln, rldx/inference/action_model/single_stream/engine/
    kernels/ss_epilogue_ln.py:146-205.  Returns (new_hidden [1, M, DIM], ln [1, M, DIM])."""
    _on_gpu(hidden, residual)
    M = _lead_rows(hidden) if M is None else M
    DIM = hidden.shape[-1] if DIM is None else DIM
    h = _rows_of(hidden, M, DIM, "hidden")
    if residual is not None:
        r = _rows_of(residual, M, DIM, "residual")
        new_hidden = _out_rows(new_hidden_out, M, DIM, h, "new_hidden_out")
        r_ptr, n_ptr = r.data_ptr(), new_hidden.data_ptr()
    else:
        new_hidden = hidden if hidden.dim() == 3 else hidden.view(1, M, DIM)
        r_ptr, n_ptr = None, None
    ln = _out_rows(ln_out_out, M, DIM, h, "ln_out_out")
    lib = _lib.load()
    _lib.check(lib.rldx_ss_epilogue_ln_bf16(h.data_ptr(), r_ptr, n_ptr, ln.data_ptr(), M, DIM, eps, _stream_ptr(h)),
               "rldx_ss_epilogue_ln_bf16")
    return new_hidden, ln


def fused_add_rmsnorm(hidden: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                      deepstack: Optional[torch.Tensor] = None, eps: float = 1e-6):
    """new_hidden = hidden + residual [+ deepstack] (bf16 adds, in that order);
    normed = Qwen3VLTextRMSNorm(new_hidden) = bf16(weight * bf16(x * rsqrt(mean(x^2) + eps))).

    The `forward` of rldx/inference/backbone/llm/engine/kernels/fused_add2_rmsnorm.py:86-115
    (deepstack=None) and fused_add3_rmsnorm.py (with deepstack), with the eager
    rounding of modeling_qwen3_vl.py:366-371.  Returns (new_hidden, normed) shaped like hidden."""
    _on_gpu(hidden, residual, weight, deepstack)
    shape = hidden.shape
    D = shape[-1]
    M = hidden.numel() // D if D else 0
    h = _rows_of(hidden, M, D, "hidden", reshape=True)
    r = _rows_of(residual, M, D, "residual", reshape=True)
    ds = None if deepstack is None else _rows_of(deepstack, M, D, "deepstack", reshape=True)
    w = _vec_of(weight, D, "weight")
    new_hidden = torch.empty_like(h)
    normed = torch.empty_like(h)
    lib = _lib.load()
    _lib.check(lib.rldx_add_rmsnorm_bf16(h.data_ptr(), r.data_ptr(), _ptr(ds), w.data_ptr(), new_hidden.data_ptr(),
                                         normed.data_ptr(), M, D, eps, _stream_ptr(h)),
               "rldx_add_rmsnorm_bf16")
    return new_hidden.view(shape), normed.view(shape)


def fused_add2_rmsnorm(hidden: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor):
    """fused_add2_rmsnorm.forward(hidden, residual, weight) (fused_add2_rmsnorm.py:86-115)."""
    return fused_add_rmsnorm(hidden, residual, weight)


def fused_add3_rmsnorm(hidden: torch.Tensor, residual: torch.Tensor, deepstack: torch.Tensor, weight: torch.Tensor):
    """fused_add3_rmsnorm.forward(hidden, residual, deepstack, weight) (fused_add3_rmsnorm.py:86-117)."""
    return fused_add_rmsnorm(hidden, residual, weight, deepstack)


def mask_to_key_bias(kv_mask: torch.Tensor) -> torch.Tensor:
    """1 = visible / 0 = masked (the eager encoder_attention_mask convention,
    blocks.py:843-864) -> fp32 additive bias 0 / -inf."""
    m = kv_mask if kv_mask.dim() == 2 else kv_mask.unsqueeze(0)
    return torch.where(m == 0, torch.tensor(float("-inf"), device=m.device),
                       torch.tensor(0.0, device=m.device)).to(F32).contiguous()


def host_swiglu_bf16_bits(g_bits, u_bits):
    """Run the device SwiGLU element function on the CPU (numpy uint16 arrays)."""
    import numpy as np

    g = np.ascontiguousarray(g_bits, dtype=np.uint16)
    u = np.ascontiguousarray(u_bits, dtype=np.uint16)
    y = np.empty_like(g)
    lib = _lib.load()
    rc = lib.rldx_host_swiglu_bf16(g.ctypes.data_as(ctypes.c_void_p), u.ctypes.data_as(ctypes.c_void_p),
                                   y.ctypes.data_as(ctypes.c_void_p), g.size)
    _require(rc == 0, "rldx_host_swiglu_bf16 failed")
    return y
