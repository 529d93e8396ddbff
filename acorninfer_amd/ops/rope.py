"""K2: RoPE and fused per-head qk-RMSNorm + RoPE on the GPU.

`fused_rope_inplace` is a drop-in for acorninfer/ops/rope.py:91-113;
`qknorm_rope_inplace` adds the per-head RMSNorm the reference leaves in torch
(models/qwen3.py:184-185). Kernels: csrc/rope.hip.
"""
from __future__ import annotations

import torch

from acorninfer_amd._lib import check, dtype_code, lib, ptr, require_gpu, stream_ptr


def _rope_args(q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor):
    B, H, s, D = q.shape
    assert s == 1 and D % 2 == 0 and (D & (D - 1)) == 0, "s==1 and D power-of-2 required"
    assert q.is_contiguous() and k.is_contiguous()
    assert k.dtype == q.dtype and k.device == q.device
    assert k.shape[0] == B and k.shape[2] == s and k.shape[3] == D
    pos = positions.to(device=q.device)
    if pos.dtype not in (torch.int32, torch.int64):
        pos = pos.long()
    return B, H, D, pos.contiguous()


def fused_rope_inplace(q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor,
                       inv_freq: torch.Tensor) -> None:
    """In-place half-rotate RoPE on q [B,H,1,D] and k [B,KV,1,D] (contiguous).

    positions [B] int; inv_freq [D/2] (any float dtype, used as fp32 — the
    reference's `inv_freq.float()`). Rounding follows the torch path: cos/sin
    rounded to the activation dtype, each product rounded, then the sum.
    """
    require_gpu(q, k)
    B, H, D, pos = _rope_args(q, k, positions)
    inv = inv_freq.to(device=q.device, dtype=torch.float32).contiguous()
    st = stream_ptr(q.device)
    is64 = int(pos.dtype == torch.int64)
    for t in (q, k):
        rc = lib().acorn_rope_inplace(ptr(t), B, t.shape[1], D, ptr(pos), is64, ptr(inv),
                                      dtype_code(t), st)
        check(rc, "fused_rope_inplace")


def qknorm_rope_inplace(q: torch.Tensor, k: torch.Tensor, q_w: torch.Tensor,
                        k_w: torch.Tensor, eps: float, positions: torch.Tensor,
                        inv_freq: torch.Tensor) -> None:
    """In place: q = rope(rmsnorm_D(q) * q_w), k = rope(rmsnorm_D(k) * k_w).

    Same layouts as fused_rope_inplace; q_w/k_w are the [D] q_norm/k_norm
    weights; the norm is computed in fp32 and rounded to q.dtype before the
    rotation (models/qwen3.py:50-60 followed by rope.py's rounding chain).
    """
    require_gpu(q, k, q_w, k_w)
    B, H, D, pos = _rope_args(q, k, positions)
    assert q_w.numel() == D and k_w.numel() == D and q_w.dtype == k_w.dtype
    inv = inv_freq.to(device=q.device, dtype=torch.float32).contiguous()
    rc = lib().acorn_qknorm_rope_inplace(
        ptr(q), ptr(k), B, H, k.shape[1], D, ptr(q_w.contiguous()), ptr(k_w.contiguous()),
        float(eps), ptr(pos), int(pos.dtype == torch.int64), ptr(inv), dtype_code(q),
        dtype_code(q_w), stream_ptr(q.device))
    check(rc, "qknorm_rope_inplace")


def fused_rope_ref(x: torch.Tensor, positions: torch.Tensor,
                   inv_freq: torch.Tensor) -> torch.Tensor:
    """Plain torch statement of the RoPE contract on x [B, H, 1, D], exported
    because the reference module exports one (acorninfer/ops/rope.py:116-125).
    Angles pos * inv_freq in fp32; cos and sin are rounded to x.dtype; the
    rotate-half products and their sum are in x.dtype. The GPU op above never
    calls it."""
    ang = positions.to(device=x.device, dtype=torch.float32)[:, None] * \
        inv_freq.to(device=x.device, dtype=torch.float32)[None, :]
    ang = torch.cat([ang, ang], dim=-1)                        # [B, D]
    cos = ang.cos().to(x.dtype).view(x.shape[0], 1, 1, -1)
    sin = ang.sin().to(x.dtype).view(x.shape[0], 1, 1, -1)
    half = x.shape[-1] // 2
    rotated = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * cos + rotated * sin
