"""Restatements of the reference's op oracles (torch, CPU, fp32 semantics).

Pins (tests/test_oracle_ops.py):
- fused_add_rmsnorm_ref: float64 closed form; residual=None identity case;
  scale invariance rmsnorm(c*x) == rmsnorm(x).
- rope_ref: the reference's known answer test_qwen3_model.py:64-82
  (inv_freq[0] == 1 so the first pair rotates by exactly `pos` radians);
  position 0 is the identity; norm preservation in fp32; float64 rotation.
- paged_attention_ref: float64 brute-force per-token softmax; L=1 -> v0;
  q=0 -> mean of V; output invariant under relabelling the pool's blocks.
- build_tables_ref: the reference's known answers
  test_ops_paged_attention.py:157-191.
- paged_verify_ref: a window of 1 equals paged_attention_ref; a float64
  brute force over an explicit causal mask; k = 0 gives the exact mean of
  each row's visible v.
"""
from __future__ import annotations

import torch


def inv_freq_ref(head_dim: int, theta: float) -> torch.Tensor:
    """models/qwen3.py:68-74: 1 / theta^(2i/D), fp32."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))


def rmsnorm_ref(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """models/qwen3.py:56-60: fp32 norm, times fp32 weight, cast to x.dtype."""
    dtype = x.dtype
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * weight.float()).to(dtype)


def fused_add_rmsnorm_ref(x, residual, weight, eps):
    """ops/rmsnorm.py:74-82: res = x or residual + x (input-dtype add);
    normed = fp32 rmsnorm(res) cast back. Returns (normed, res)."""
    res = x if residual is None else residual + x
    xf = res.float()
    normed = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * weight.float()).to(x.dtype)
    return normed, res.to(x.dtype)


def rope_ref(x: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor) -> torch.Tensor:
    """ops/rope.py:116-125 (= qwen3.py:76-95 per row): x [B,H,1,D] ->
    x*cos + rotate_half(x)*sin with cos/sin computed in fp32 and cast to x.dtype."""
    pos = positions.to(dtype=torch.float32)
    freqs = torch.outer(pos, inv_freq.float())
    emb = torch.cat((freqs, freqs), dim=-1)
    cos = emb.cos().to(x.dtype)[:, None, None, :]
    sin = emb.sin().to(x.dtype)[:, None, None, :]
    x1, x2 = x.chunk(2, dim=-1)
    rot = torch.cat((-x2, x1), dim=-1)
    return x * cos + rot * sin


def qknorm_rope_ref(q, k, q_w, k_w, eps, positions, inv_freq):
    """qwen3.py:184-195: q_norm/k_norm (RMSNorm over D) then RoPE."""
    return (rope_ref(rmsnorm_ref(q, q_w, eps), positions, inv_freq),
            rope_ref(rmsnorm_ref(k, k_w, eps), positions, inv_freq))


def paged_attention_ref(q, k_pages, v_pages, tables, seq_lens):
    """ops/paged_attention.py:192-216: per sequence gather tokens
    (table[t//P], t%P), repeat kv heads (head j <- kv j // (H/KV)), fp32
    softmax(q.k * D^-0.5) @ v, cast to q.dtype."""
    B, H, D = q.shape
    NB, P, KV, _ = k_pages.shape
    rep = H // KV
    outs = []
    for b in range(B):
        L = int(seq_lens[b])
        n_pages = -(-L // P)
        idx = tables[b, :n_pages].long()
        kf = k_pages[idx].reshape(-1, KV, D)[:L].permute(1, 0, 2)
        vf = v_pages[idx].reshape(-1, KV, D)[:L].permute(1, 0, 2)
        kf = kf.repeat_interleave(rep, 0).float()
        vf = vf.repeat_interleave(rep, 0).float()
        s = torch.einsum("hd,hld->hl", q[b].float(), kf) * (D ** -0.5)
        p = torch.softmax(s, dim=-1)
        outs.append(torch.einsum("hl,hld->hd", p, vf).to(q.dtype))
    return torch.stack(outs, dim=0)


def paged_attention_brute(q, k_pages, v_pages, tables, seq_lens):
    """Independent float64 brute force: explicit per-(b,h,t) loops over the
    block table. Small shapes only."""
    B, H, D = q.shape
    NB, P, KV, _ = k_pages.shape
    rep = H // KV
    out = torch.zeros(B, H, D, dtype=torch.float64)
    for b in range(B):
        L = int(seq_lens[b])
        for h in range(H):
            kv = h // rep
            qs = q[b, h].double()
            scores = []
            for t in range(L):
                page = int(tables[b, t // P])
                scores.append(float(qs @ k_pages[page, t % P, kv].double()) / D ** 0.5)
            m = max(scores)
            w = [pow(2.718281828459045, s - m) for s in scores]
            z = sum(w)
            for t in range(L):
                page = int(tables[b, t // P])
                out[b, h] += (w[t] / z) * v_pages[page, t % P, kv].double()
    return out


def paged_verify_ref(q, k_pages, v_pages, tables, seq_lens):
    """ops/paged_verify.py:96-123 (and the dense reference of
    tests/test_paged_verify.py:35-58): q [B, m, H, D]; seq_lens[b] = len + m
    counts the whole window. Row (b, j) attends to tokens 0 .. seq_lens[b] -
    (m - 1 - j) - 1 of sequence b (its history and the window's first j + 1
    tokens), with the decode oracle's gather, GQA map and fp32 softmax; the
    result is cast to q.dtype."""
    B, M, H, D = q.shape
    rows = []
    for b in range(B):
        for j in range(M):
            Lj = int(seq_lens[b]) - (M - 1 - j)
            rows.append(paged_attention_ref(q[b, j][None], k_pages, v_pages, tables[b][None],
                                            torch.tensor([Lj]))[0])
    return torch.stack(rows, 0).view(B, M, H, D)


def paged_verify_brute(q, k_pages, v_pages, tables, seq_lens):
    """Independent float64 brute force: the whole window's keys gathered once
    per sequence, scores over all seq_lens[b] tokens, future positions masked
    with an explicit [m, L] causal mask before a row-wise softmax."""
    B, M, H, D = q.shape
    NB, P, KV, _ = k_pages.shape
    rep = H // KV
    out = torch.zeros(B, M, H, D, dtype=torch.float64)
    for b in range(B):
        L = int(seq_lens[b])
        pos = torch.arange(L)
        k = torch.stack([k_pages[int(tables[b, t // P]), t % P] for t in range(L)]).double()
        v = torch.stack([v_pages[int(tables[b, t // P]), t % P] for t in range(L)]).double()
        limit = torch.tensor([L - (M - 1 - j) for j in range(M)])
        visible = pos[None, :] < limit[:, None]                       # [m, L]
        for h in range(H):
            s = q[b, :, h].double() @ k[:, h // rep].T * (D ** -0.5)   # [m, L]
            s = s.masked_fill(~visible, float("-inf"))
            out[b, :, h] = torch.softmax(s, dim=-1) @ v[:, h // rep]
    return out


def num_splits_ref(B: int, num_heads: int, sm_count: int = 128, max_splits: int = 8) -> int:
    """ops/paged_attention.py:155-158."""
    return max(1, min(max_splits, -(-sm_count // (B * num_heads))))


def build_tables_ref(tables_lists, lens, page_size):
    """ops/paged_attention.py:161-189 (default path): zero-padded
    [B, max(1, max ceil(L/P))] int32 + lens int32."""
    npages = [-(-int(L) // page_size) for L in lens]
    width = max([1, *npages])
    t = torch.zeros(len(lens), width, dtype=torch.int32)
    for i, tb in enumerate(tables_lists):
        t[i, : npages[i]] = torch.tensor(list(tb[: npages[i]]), dtype=torch.int32)
    return t, torch.tensor([int(L) for L in lens], dtype=torch.int32)
