"""K1: fused residual add + RMSNorm on the GPU.

Drop-in for acorninfer/ops/rmsnorm.py:39-71 (`fused_add_rmsnorm`); the kernel
is csrc/rmsnorm.hip (acorn_fused_add_rmsnorm).
"""
from __future__ import annotations

import torch

from acorninfer_amd._lib import check, dtype_code, lib, ptr, require_gpu, stream_ptr


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor,
                      eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(normed, residual_new) with the reference's contract (rmsnorm.py:39-56):

    - residual is None: residual_new = x (a new tensor), normed = rmsnorm(x)
    - otherwise:        residual_new = round(residual + x), normed = rmsnorm(residual_new)

    The add happens in fp32 and is rounded to x.dtype; the norm is computed in
    fp32 on the rounded residual and cast back. x: [..., H] of any leading
    shape (non-contiguous input is copied), residual: None or like x,
    weight: [H]. Both outputs are new tensors; x and residual are never written.
    """
    require_gpu(x, residual, weight)
    *lead, H = x.shape
    rows = x.numel() // H if H else 0
    x2 = x.reshape(rows, H).contiguous()
    r2 = None
    if residual is not None:
        assert residual.shape == x.shape and residual.dtype == x.dtype, \
            "residual must match x in shape and dtype"
        r2 = residual.reshape(rows, H).contiguous()
    w = weight.contiguous()
    assert w.numel() == H, "weight must be [H]"
    normed = torch.empty_like(x2)
    res_out = torch.empty_like(x2)
    rc = lib().acorn_fused_add_rmsnorm(
        ptr(x2), ptr(r2), ptr(res_out), ptr(w), ptr(normed), rows, H, float(eps),
        dtype_code(x2), dtype_code(w), stream_ptr(x.device))
    check(rc, "fused_add_rmsnorm")
    return normed.view(*lead, H), res_out.view(*lead, H)


def fused_add_rmsnorm_partials(part: torch.Tensor, residual: torch.Tensor | None,
                               weight: torch.Tensor, eps: float, *,
                               normed: torch.Tensor, residual_out: torch.Tensor,
                               x_out: torch.Tensor | None = None) -> None:
    """K1 fed by fp32 split-K partials part[S, rows, H] of the preceding
    projection: x = round(sum_s part[s]) then fused_add_rmsnorm(x, residual).
    Writes into the caller's buffers (decode-step form, no allocation)."""
    S, rows, H = part.shape
    assert part.dtype == torch.float32 and part.is_contiguous()
    assert normed.is_contiguous() and residual_out.is_contiguous()
    rc = lib().acorn_fused_add_rmsnorm_partials(
        ptr(part), S, ptr(residual), ptr(residual_out), ptr(weight), ptr(normed), ptr(x_out),
        rows, H, float(eps), dtype_code(normed), dtype_code(weight), stream_ptr(part.device))
    check(rc, "fused_add_rmsnorm_partials")


def fused_add_rmsnorm_ref(x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor,
                          eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Plain torch statement of the K1 contract, exported because the
    reference module exports one (acorninfer/ops/rmsnorm.py:74-82) and its
    callers' tests import it from here. Device-agnostic; the GPU op above never
    calls it. The residual add is in x's dtype; the norm is fp32 then cast."""
    res = x if residual is None else residual + x
    f = res.float()
    scale = torch.rsqrt(f.square().mean(dim=-1, keepdim=True) + eps)
    return (f * scale * weight.float()).to(x.dtype), res.to(x.dtype)
