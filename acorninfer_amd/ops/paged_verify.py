"""Speculative-verify attention over the paged cache.

Drop-in for acorninfer/ops/paged_verify.py (`paged_verify_attention`,
:96-123): the m = spec_num + 1 window positions of each sequence are scored
together, each with causal visibility inside the window. Row (b, j) sees
seq_lens[b] - (m - 1 - j) tokens (its history plus the window's first j + 1
tokens); seq_lens counts the whole window, and the window's k/v are already in
the pages (`PagedKVCache.scatter_verify`).

On this build the rows are K3 rows (csrc/paged_attention.hip through
`acorn_paged_attention`): the window is flattened to B*m query rows, row
(b, j) carries sequence b's block table and its own visible length, and the
same split/combine kernels as decode run over them. Nothing about K3 changes:
decode is the m = 1 case. Like the reference this path is eager (a verify
step is not graph-captured there); the per-row tables and lengths are built
on the device each call.
"""
from __future__ import annotations

import torch

from acorninfer_amd._lib import require_gpu
from acorninfer_amd.ops.paged_attention import paged_decode_attention

__all__ = ["paged_verify_attention"]


def paged_verify_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                           tables: torch.Tensor, seq_lens: torch.Tensor,
                           num_splits: int) -> torch.Tensor:
    """q [B, m, H, D] (normed + roped, positions len .. len+m-1); k/v_pages
    [NB, P, KV, D] (read only); tables [B, MP] int32; seq_lens [B] int32 =
    len + m. Returns [B, m, H, D] in q.dtype: row j is the window-causal
    attention output at position len + j. Shape contracts raise
    AssertionError as the reference's do (paged_verify.py:110-118)."""
    require_gpu(q, k_pages, v_pages, tables, seq_lens)
    B, M, H, D = q.shape
    NB, P, KV, _ = k_pages.shape
    assert M >= 1, "verify window must be non-empty"
    assert D & (D - 1) == 0 and P & (P - 1) == 0, "D and P must be power-of-2"
    assert H % KV == 0, "GQA requires H divisible by KV"
    assert num_splits >= 1
    assert v_pages.shape == k_pages.shape
    assert tables.shape[0] == B and seq_lens.shape[0] == B
    assert k_pages.is_contiguous() and v_pages.is_contiguous()
    assert tables.is_contiguous() and seq_lens.is_contiguous()
    assert tables.dtype == torch.int32 and seq_lens.dtype == torch.int32
    # row (b, j): sequence b's table, length seq_lens[b] - (m - 1 - j)
    row_tables = tables.repeat_interleave(M, dim=0)
    back = torch.arange(M - 1, -1, -1, device=seq_lens.device, dtype=torch.int32)
    row_lens = (seq_lens[:, None] - back[None, :]).reshape(-1).contiguous()
    out = paged_decode_attention(q.reshape(B * M, H, D), k_pages, v_pages, row_tables,
                                 row_lens, num_splits)
    return out.view(B, M, H, D)
