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


def ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Per-element distance in units in the last place of a 16-bit float dtype
    (bf16 / fp16): the difference of the order-preserving integer keys."""
    assert a.dtype == b.dtype and a.dtype in (torch.bfloat16, torch.float16)
    ia = a.cpu().view(torch.int16).to(torch.int32)
    ib = b.cpu().view(torch.int16).to(torch.int32)
    ka = torch.where(ia < 0, -(ia & 0x7FFF), ia)      # sign-magnitude -> monotone
    kb = torch.where(ib < 0, -(ib & 0x7FFF), ib)
    return (ka - kb).abs()


# Bitwise bar for the 16-bit norm / RoPE outputs: the oracle rounds the same
# fp32 chain once; the kernels differ from it only in the fp32 reduction
# order of mean(x^2) and in the hardware rsqrt, so an output may land one
# ulp away where the fp32 value sits on a rounding boundary. Asserted: no
# element more than 1 ulp away, and at most this fraction 1 ulp away.
MAX_ONE_ULP_FRACTION = 1e-3
