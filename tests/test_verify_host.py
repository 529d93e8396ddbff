"""Speculative verify, host side and oracle (CPU).

- The verify oracle (oracle.ops_ref.paged_verify_ref, restating
  acorninfer/ops/paged_verify.py:96-123) is pinned three ways: a window of
  one is the decode oracle; a float64 brute force over an explicit causal
  mask agrees; with k = 0 every row is exactly the mean of its visible v.
- The window bookkeeping of cache/pager.py:211-244: ensure_append_capacity_n
  (n = 1 equals ensure_append_capacity; blocks only where a page starts;
  BlockExhausted keeps the blocks already taken and commits no length) and
  set_lens (rollback only; ValueError forward).
"""
import pytest
import torch

from acorninfer_amd.cache.pager import (BlockAllocator, BlockExhausted, PagedCacheView,
                                        PagedKVCache)
from oracle.ops_ref import paged_attention_ref, paged_verify_brute, paged_verify_ref


def _case(B, M, hist, H=4, KV=2, D=16, P=16, seed=0):
    g = torch.Generator().manual_seed(seed)
    lens = [hist + b + M for b in range(B)]
    mp = max(-(-n // P) for n in lens)
    nb = B * mp + 2
    q = torch.randn(B, M, H, D, generator=g)
    kp = torch.randn(nb, P, KV, D, generator=g)
    vp = torch.randn(nb, P, KV, D, generator=g)
    perm = torch.randperm(nb, generator=g)
    tables = torch.zeros(B, mp, dtype=torch.int32)
    for b in range(B):
        tables[b] = perm[b * mp:(b + 1) * mp]
    return q, kp, vp, tables, torch.tensor(lens, dtype=torch.int32)


@pytest.mark.parametrize("B,M,hist", [(1, 2, 1), (3, 5, 15), (2, 5, 16), (4, 2, 17), (2, 3, 48)])
def test_verify_oracle_against_brute_force(B, M, hist):
    q, kp, vp, tables, lens = _case(B, M, hist, seed=B * 100 + M * 10 + hist)
    ref = paged_verify_ref(q, kp, vp, tables, lens)
    brute = paged_verify_brute(q, kp, vp, tables, lens)
    torch.testing.assert_close(ref.double(), brute, rtol=1e-5, atol=1e-5)


def test_verify_oracle_window_of_one_is_decode():
    q, kp, vp, tables, lens = _case(3, 1, 20, seed=7)
    assert torch.equal(paged_verify_ref(q, kp, vp, tables, lens)[:, 0],
                       paged_attention_ref(q[:, 0], kp, vp, tables, lens))


def test_verify_oracle_zero_keys_give_the_visible_mean():
    B, M, hist, KV, H = 2, 4, 9, 2, 4
    q, kp, vp, tables, lens = _case(B, M, hist, H=H, KV=KV, seed=3)
    kp.zero_()
    out = paged_verify_ref(q, kp, vp, tables, lens)
    P = kp.shape[1]
    for b in range(B):
        for j in range(M):
            L = int(lens[b]) - (M - 1 - j)
            rows = torch.stack([vp[int(tables[b, t // P]), t % P] for t in range(L)])
            for h in range(H):
                torch.testing.assert_close(out[b, j, h], rows[:, h // (H // KV)].mean(0),
                                           rtol=1e-5, atol=1e-6)


def _view(num_blocks, P=16):
    cache = PagedKVCache(1, 2, 16, P, BlockAllocator(num_blocks), "cpu", torch.float32)
    return cache, PagedCacheView(cache)


def test_ensure_capacity_n_positions_and_allocation():
    cache, view = _view(8)
    assert view.ensure_append_capacity_n(0, 1) == [view.ensure_append_capacity(0)]
    view._lens[0] = 13
    got = view.ensure_append_capacity_n(0, 5)          # 13..17 crosses into a second page
    assert len(view.table) == 2
    assert got == [(view.table[0], s) for s in (13, 14, 15)] + [(view.table[1], 0),
                                                               (view.table[1], 1)]
    assert view.seq_len == 13                          # no length committed
    assert view.ensure_append_capacity_n(0, 3) == got[:3]   # nothing new allocated
    assert len(view.table) == 2


def test_ensure_capacity_n_exhaustion_keeps_taken_blocks():
    cache, view = _view(2)
    view._lens[0] = 10
    with pytest.raises(BlockExhausted):
        view.ensure_append_capacity_n(0, 40)           # needs 4 blocks, 2 exist
    assert len(view.table) == 2 and cache.allocator.num_free == 0
    assert view.seq_len == 10


def test_set_lens_is_rollback_only():
    cache, view = _view(4)
    view._lens[0] = 18
    view.set_lens(0, 16)
    assert view.seq_len == 16
    with pytest.raises(ValueError, match="only move a length back"):
        view.set_lens(0, 17)
    view.set_lens(0, 16)                               # same length is allowed
