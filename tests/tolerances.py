"""Tolerance protocol for kernel parity (mirrors the reference's two levels,
tests/triton_utils.py:1-27 in the reference):

- fp32 inputs with TOL_F32: only reduction-order drift is tolerated, so any
  indexing/mask/boundary error fails.
- bf16 inputs with the north-star tolerances: activations within 2e-2
  relative (RMSNorm, RoPE, attention, fp32 accumulate); quantised GEMM within
  1e-2 relative (norm-wise) of the float64 dequantised matmul.
"""
import torch

TOL_F32 = dict(rtol=1e-5, atol=1e-5)
TOL_BF16 = dict(rtol=2e-2, atol=2e-2)
GEMM_REL = 1e-2


def max_abs_diff(a: torch.Tensor, b: torch.Tensor) -> float:
    assert a.shape == b.shape
    if a.numel() == 0:
        return 0.0
    return (a.double().cpu() - b.double().cpu()).abs().max().item()


def rel_err(out: torch.Tensor, ref: torch.Tensor) -> float:
    """Norm-wise relative error ||out - ref|| / ||ref||."""
    o, r = out.double().cpu(), ref.double().cpu()
    return ((o - r).norm() / r.norm().clamp_min(1e-30)).item()
