"""fused_grouped_swiglu of rldx/inference/action_model/double_stream/engine/kernels/
grouped_swiglu.py:213-257, on rldx_grouped_swiglu_bf16."""

from rldx_amd import functional as Fn

__all__ = ["fused_grouped_swiglu"]


def fused_grouped_swiglu(sa_w12_out, sa_bias, vl_w12_out, vl_bias, M_sa=None, M_vl=None, N_half_sa=None,
                         N_half_vl=None):
    """SA and VL bias + SwiGLU in one launch: (sa_out (M_sa, N_half_sa), vl_out
    (M_vl, N_half_vl)) bf16.  Row counts default to the inputs' rows, N_half to
    half their widths, as in the reference launcher."""
    M_sa = sa_w12_out.shape[0] if M_sa is None else M_sa
    N_half_sa = sa_w12_out.shape[1] // 2 if N_half_sa is None else N_half_sa
    M_vl = vl_w12_out.shape[0] if M_vl is None else M_vl
    N_half_vl = vl_w12_out.shape[1] // 2 if N_half_vl is None else N_half_vl
    return Fn.grouped_swiglu(sa_w12_out, sa_bias, vl_w12_out, vl_bias, M_sa, M_vl, N_half_sa, N_half_vl)
