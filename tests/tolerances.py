"""Parity tolerances (fp32 max-abs 1e-5; bf16 max-abs 2e-2 and relative L2 1e-2)."""

import torch

FP32_MAX_ABS = 1e-5
BF16_MAX_ABS = 2e-2
BF16_REL_L2 = 1e-2


def stats(out: torch.Tensor, ref: torch.Tensor) -> dict:
    o = out.detach().float().cpu()
    r = ref.detach().float().cpu()
    diff = (o - r).abs()
    finite = torch.isfinite(r)
    max_abs = float(diff[finite].max()) if finite.any() else 0.0
    rel_l2 = float((o - r)[finite].norm() / r[finite].norm().clamp_min(1e-30))
    return {"max_abs": max_abs, "rel_l2": rel_l2, "nonfinite_mismatch": int((torch.isfinite(o) != finite).sum())}


def assert_bf16_close(out, ref, what=""):
    s = stats(out, ref)
    assert s["nonfinite_mismatch"] == 0, f"{what}: non-finite pattern differs {s}"
    assert s["max_abs"] <= BF16_MAX_ABS and s["rel_l2"] <= BF16_REL_L2, f"{what}: {s}"
    return s


def assert_fp32_close(out, ref, what=""):
    s = stats(out, ref)
    assert s["nonfinite_mismatch"] == 0, f"{what}: non-finite pattern differs {s}"
    assert s["max_abs"] <= FP32_MAX_ABS, f"{what}: {s}"
    return s
