"""Mirror of the RoPE and FFN utilities of rldx/model/modules/action_model/
ops.py on the rldx_amd kernels: precompute_freqs_cis (:11-25),
apply_rotary_emb (:48-67, interleaved RoPE through rldx_rope_interleaved_*) and
SwiGLUFFN (:137-161, the grouped GEMM with its packed SwiGLU epilogue, then the
bias epilogue).  CUDA tensors only (no CPU path)."""

from __future__ import annotations

from typing import Callable, Optional

import torch
import torch.nn as nn

from rldx_amd import functional as Fn
from rldx_amd import workloads as _W

__all__ = ["precompute_freqs_cis", "apply_rotary_emb", "SwiGLUFFN"]


def precompute_freqs_cis(dim: int, end: int, theta: float = 10000.0) -> torch.Tensor:
    """(end, dim / 2) complex64 RoPE frequencies, the reference's fp32 recipe."""
    return _W.msat_freqs_cis(dim, end, theta)


def apply_rotary_emb(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor):
    """xq [B, H, N, D], xk [B, H, N, D] rotated pairwise by freqs_cis ([N, D/2],
    [1, N, D/2] or [B, N, D/2] complex64) in fp32, returned in the input type."""
    return Fn.rope_interleaved(xq, xk, freqs_cis)


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


class SwiGLUFFN(nn.Module):
    """w3(silu(x W12_gate^T + b_gate) * (x W12_up^T + b_up)) + b3 with the
    reference's parameters (`w12` [2 hidden, in], `w3` [out, hidden]).  The
    weights are packed into the GEMM operand order on the first call and again
    whenever a weight tensor is replaced or updated in place; a hidden width
    that is not a multiple of 128 is padded with zero rows / columns (silu(0) *
    0 = 0).  Needs bf16 weights and input, in_features % 128 == 0 and
    out_features % 64 == 0.  Rounding as eager bf16: each linear rounds its fp32
    sum + bias once, SwiGLU rounds after silu and after the product."""

    def __init__(self, in_features: int, hidden_features: Optional[int] = None,
                 out_features: Optional[int] = None, act_layer: Optional[Callable[..., nn.Module]] = None,
                 drop: float = 0.0, bias: bool = True) -> None:
        super().__init__()
        out_features = out_features or in_features
        hidden_features = hidden_features or in_features
        self.w12 = nn.Linear(in_features, 2 * hidden_features, bias=bias)
        self.w3 = nn.Linear(hidden_features, out_features, bias=bias)
        self._packed = None

    def _pack(self):
        ws = [self.w12.weight, self.w3.weight] + [b for b in (self.w12.bias, self.w3.bias) if b is not None]
        key = tuple((t.data_ptr(), t._version) for t in ws)
        if self._packed is not None and self._packed[0] == key:
            return self._packed[1:]
        w12, w3 = self.w12.weight.detach(), self.w3.weight.detach()
        Fn._require(w12.dtype == torch.bfloat16 and w3.dtype == torch.bfloat16, "SwiGLUFFN: bf16 weights")
        h, k = w12.shape[0] // 2, w12.shape[1]
        n = w3.shape[0]
        Fn._require(k % 128 == 0 and n % 64 == 0, "SwiGLUFFN: in_features % 128 == 0 and out_features % 64 == 0")
        hp = _round_up(h, 128)
        dev = w12.device
        g = torch.zeros(2 * hp, k, dtype=torch.bfloat16, device=dev)
        g[:h], g[hp:hp + h] = w12[:h], w12[h:]
        w3p = torch.zeros(n, hp, dtype=torch.bfloat16, device=dev)
        w3p[:, :h] = w3
        b12 = None
        if self.w12.bias is not None:
            b = self.w12.bias.detach()
            b12 = torch.zeros(2 * hp, dtype=torch.bfloat16, device=dev)
            b12[:h], b12[hp:hp + h] = b[:h], b[h:]
        b3 = None if self.w3.bias is None else self.w3.bias.detach().contiguous()
        self._packed = (key, Fn.pack_weight(g, swiglu_pairs=True), b12, Fn.pack_weight(w3p), b3, hp)
        return self._packed[1:]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        pw12, b12, pw3, b3, hp = self._pack()
        Fn._require(x.dtype == torch.bfloat16, "SwiGLUFFN: bf16 input")
        lead = x.shape[:-1]
        a = x.reshape(-1, x.shape[-1])
        m = a.shape[0]
        out = torch.empty(m, self.w3.weight.shape[0], dtype=torch.bfloat16, device=x.device)
        if m:
            gl = Fn.PackedAct.empty(m, hp, x.device)
            Fn.grouped_gemm([(a, pw12, b12, gl, None)], "swiglu_packed")
            Fn.grouped_gemm([(gl, pw3, b3, out, None)], "bias")
        return out.reshape(*lead, out.shape[-1])
