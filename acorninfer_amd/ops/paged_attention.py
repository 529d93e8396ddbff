"""K3: paged flash-decoding attention on the GPU, plus block-table helpers.

Drop-in for acorninfer/ops/paged_attention.py: `paged_decode_attention`
(:125-152), `num_splits_for` (:155-158) and `build_tables` (:161-189). The
kernel is csrc/paged_attention.hip (acorn_paged_attention): one workgroup per
(split, kv head, sequence) whose waves divide the split's pages and serve
every query head of the kv head.

`plan_splits` is this build's split heuristic for MI355X (256 CUs); the
reference's `num_splits_for` is kept with its exact semantics for callers that
use it.
"""
from __future__ import annotations

import torch

from acorninfer_amd._lib import check, dtype_code, lib, ptr, require_gpu, stream_ptr

_SM_COUNT = 128          # the reference's fixed heuristic constant (num_splits_for)
MI355X_CUS = 256


def paged_decode_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                           tables: torch.Tensor, seq_lens: torch.Tensor,
                           num_splits: int, *, out: torch.Tensor | None = None,
                           workspace: tuple[torch.Tensor, torch.Tensor] | None = None
                           ) -> torch.Tensor:
    """q [B,H,D] (normed + roped); k/v_pages [NB,P,KV,D]; tables [B,MP] int32;
    seq_lens [B] int32 (including the current token, >= 1). Returns [B,H,D] in
    q.dtype. q head j reads kv head j // (H//KV). `num_splits` page-aligned
    splits per sequence; empty splits contribute nothing.

    `out` / `workspace` (fp32 acc [B*H*S*D], fp32 m|l [2*B*H*S]) let a caller
    pass address-stable buffers (graph capture); by default they are
    allocated per call like the reference's.
    """
    require_gpu(q, k_pages, v_pages, tables, seq_lens)
    B, H, D = q.shape
    NB, P, KV, _ = k_pages.shape
    S = int(num_splits)
    assert D & (D - 1) == 0 and P & (P - 1) == 0, "D and P must be power-of-2"
    assert H % KV == 0, "GQA requires H divisible by KV"
    assert S >= 1
    assert v_pages.shape == k_pages.shape and k_pages.shape[3] == D
    assert tables.shape[0] == B and seq_lens.shape[0] == B
    assert k_pages.is_contiguous() and v_pages.is_contiguous()
    assert tables.is_contiguous() and seq_lens.is_contiguous()
    assert tables.dtype == torch.int32 and seq_lens.dtype == torch.int32
    assert k_pages.dtype == q.dtype == v_pages.dtype
    # a sequence holds >= 1 token, so its table row holds >= 1 page (the
    # width passed below is raised to 1 only for an empty batch)
    assert B == 0 or tables.shape[1] >= 1, "tables must hold at least one page per sequence"
    q2 = q.contiguous()
    if out is None:
        out = torch.empty((B, H, D), dtype=q.dtype, device=q.device)
    _check_out(out, (B, H, D), q)
    if workspace is None and S > 1:
        workspace = (torch.empty(B * H * S * D, dtype=torch.float32, device=q.device),
                     torch.empty(2 * B * H * S, dtype=torch.float32, device=q.device))
    acc, ml = workspace if workspace is not None else (None, None)
    rc = lib().acorn_paged_attention(
        ptr(q2), ptr(k_pages), ptr(v_pages), ptr(tables), ptr(seq_lens), ptr(out), ptr(acc),
        ptr(ml), B, H, KV, D, P, NB, max(1, tables.shape[1]), S, float(D ** -0.5),
        dtype_code(q2), stream_ptr(q.device))
    check(rc, "paged_decode_attention")
    return out


def _check_out(out: torch.Tensor, shape: tuple, q: torch.Tensor) -> None:
    """A caller-supplied output is written through its raw pointer: it must
    be exactly the result's shape, dtype and device, and contiguous."""
    assert tuple(out.shape) == tuple(shape), f"out must be {tuple(shape)}, not {tuple(out.shape)}"
    assert out.dtype == q.dtype, f"out dtype {out.dtype} != q dtype {q.dtype}"
    assert out.device == q.device and out.is_contiguous(), "out must be contiguous on q's device"


def prefill_supported(dtype: torch.dtype, head_dim: int, page_size: int, num_heads: int,
                      kv_heads: int) -> bool:
    """Shapes acorn_paged_prefill_attention is built for."""
    return (dtype in (torch.bfloat16, torch.float16) and head_dim in (64, 128)
            and page_size % 16 == 0 and (page_size & (page_size - 1)) == 0
            and num_heads % kv_heads == 0 and num_heads // kv_heads in (1, 2, 4, 8))


def paged_prefill_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                            tables: torch.Tensor, seq_row0: torch.Tensor,
                            seq_pos0: torch.Tensor, seq_nq: torch.Tensor, max_nq: int, *,
                            out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal prefill attention over the paged cache (acorn_paged_prefill_attention).

    q [R,H,D]: the prompt rows of N sequences, packed; sequence n's rows
    q[seq_row0[n] : seq_row0[n] + seq_nq[n]] sit at positions seq_pos0[n] +
    j and attend to the sequence's tokens 0 .. their own position, whose K/V
    (the new rows' included) are already in k/v_pages through tables[n].
    Returns [R,H,D] in q.dtype (rows not covered by a sequence are left as
    they were in `out`)."""
    require_gpu(q, k_pages, v_pages, tables, seq_row0, seq_pos0, seq_nq)
    R, H, D = q.shape
    NB, P, KV, _ = k_pages.shape
    N = seq_row0.shape[0]
    assert H % KV == 0 and P % 16 == 0 and D in (64, 128)
    assert v_pages.shape == k_pages.shape and k_pages.shape[3] == D
    assert tables.shape[0] == N and seq_pos0.shape[0] == N and seq_nq.shape[0] == N
    for t in (tables, seq_row0, seq_pos0, seq_nq):
        assert t.dtype == torch.int32 and t.is_contiguous()
    assert k_pages.is_contiguous() and v_pages.is_contiguous()
    assert q.dtype == k_pages.dtype == v_pages.dtype
    assert N == 0 or tables.shape[1] >= 1, "tables must hold at least one page per sequence"
    q2 = q.contiguous()
    if out is None:
        out = torch.empty_like(q2)
    _check_out(out, (R, H, D), q)
    rc = lib().acorn_paged_prefill_attention(
        ptr(q2), ptr(k_pages), ptr(v_pages), ptr(tables), ptr(seq_row0), ptr(seq_pos0),
        ptr(seq_nq), ptr(out), N, R, int(max_nq), H, KV, D, P, NB, max(1, tables.shape[1]),
        float(D ** -0.5), dtype_code(q2), stream_ptr(q.device))
    check(rc, "paged_prefill_attention")
    return out


def num_splits_for(B: int, num_heads: int, *, sm_count: int = _SM_COUNT,
                   max_splits: int = 8) -> int:
    """The reference's split heuristic (paged_attention.py:155-158), unchanged:
    enough (b, q-head, split) programs to cover `sm_count` SMs, capped."""
    return max(1, min(max_splits, -(-sm_count // (B * num_heads))))


def plan_splits(B: int, kv_heads: int, max_pages: int, **kw) -> int:
    """Split count for the MI355X kernel (models.qwen3.attention_splits):
    splits of a few pages each, up to a bound on the workspace."""
    from acorninfer_amd.models.qwen3 import attention_splits
    return attention_splits(B, kv_heads, max_pages, **kw)


def build_tables(views, page_size: int, device, *, lens_override=None,
                 out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Block tables -> ([B, max_pages] int32 zero-padded, [B] int32 lengths).

    Same contract as the reference (paged_attention.py:161-189): lengths come
    from `lens_override` or each view's `seq_len`; row i holds the first
    ceil(L_i / page_size) entries of `views[i].table`. With `out` (a CPU
    buffer, e.g. a pinned mirror) the first B rows are zeroed and filled in
    place and (out[:B], CPU lens) is returned with no device transfer.
    """
    if lens_override is not None:
        lens = [int(L) for L in lens_override]
    else:
        lens = [int(v.seq_len) for v in views]
    npages = [-(-L // page_size) for L in lens]
    max_pages = max([1, *npages])
    if out is not None:
        assert out.shape[0] >= len(views) and out.shape[1] >= max_pages, \
            "out buffer must be at least [B, max_pages]"
        t = out[: len(views)]
        t.zero_()
    else:
        t = torch.zeros((len(views), max_pages), dtype=torch.int32)
    for i, v in enumerate(views):
        n = npages[i]
        if n:
            t[i, :n] = torch.tensor(list(v.table[:n]), dtype=torch.int32)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    if out is not None:
        return t, lens_t
    return t.to(device), lens_t.to(device)


def paged_decode_attention_ref(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                               tables: torch.Tensor, seq_lens: torch.Tensor) -> torch.Tensor:
    """Plain torch statement of K3's contract, exported because the reference
    module exports one (acorninfer/ops/paged_attention.py:192-216): for each
    sequence, gather tokens 0..L-1 from (tables[b, t // P], t % P), map q head
    h to kv head h // (H / KV), softmax(q.K^T * D^-0.5) V in fp32, cast to
    q.dtype. Device-agnostic; the GPU op above never calls it."""
    B, H, D = q.shape
    P, KV = k_pages.shape[1], k_pages.shape[2]
    group = H // KV
    out = torch.empty_like(q)
    for b in range(B):
        L = int(seq_lens[b])
        t = torch.arange(L, device=k_pages.device)
        blocks = tables[b].to(k_pages.device).long()[t // P]
        k = k_pages[blocks, t % P].float()                     # [L, KV, D]
        v = v_pages[blocks, t % P].float()
        k = k.permute(1, 0, 2).repeat_interleave(group, dim=0)  # [H, L, D]
        v = v.permute(1, 0, 2).repeat_interleave(group, dim=0)
        scores = torch.bmm(k, q[b].float().unsqueeze(-1)).squeeze(-1) * D ** -0.5   # [H, L]
        p = torch.softmax(scores, dim=-1)
        out[b] = torch.bmm(p.unsqueeze(1), v).squeeze(1).to(q.dtype)
    return out
