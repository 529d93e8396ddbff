"""Paged-cache host logic (cache/pager.py) and the HIP KV scatter.

CPU: the reference's allocator semantics (tests/test_pager.py: LIFO reuse,
exhaustion, double free, leak guard) and the block-table contract of
`ensure_append_capacity` / `build_tables` (ops/paged_attention.py:161-189,
known answer [[3,4,5],[7,0,0]] from the reference's
tests/test_ops_paged_attention.py:101-136).
GPU: `scatter_decode` through acorn_kv_scatter is bit-exact against
element-wise indexing (the reference pins scatter_decode == per-view write,
tests/test_pager.py:205), and out-of-pool targets are skipped.
"""
from types import SimpleNamespace

import pytest
import torch

from acorninfer_amd.cache.pager import (BlockAllocator, BlockExhausted, PagedCacheView,
                                        PagedKVCache)
from acorninfer_amd.ops.paged_attention import build_tables


def test_allocator_lifo_exhaustion_and_guards():
    a = BlockAllocator(3)
    assert [a.allocate() for _ in range(3)] == [0, 1, 2]
    with pytest.raises(BlockExhausted):
        a.allocate()
    a.free(1)
    a.free(2)
    assert a.allocate() == 2          # last freed comes back first
    with pytest.raises(ValueError):
        a.free(1)                     # not live
    with pytest.raises(AssertionError):
        a.assert_balanced()
    for b in (0, 2):
        a.free(b)
    a.assert_balanced()
    assert a.num_free == a.total == 3


def test_ensure_append_capacity_allocates_exactly_at_page_starts():
    a = BlockAllocator(8)
    cache = SimpleNamespace(page_size=4, allocator=a)
    v = PagedCacheView(cache)
    seen = []
    for n in range(10):
        v._lens[0] = n
        seen.append(v.ensure_append_capacity(0))
    assert [s for _, s in seen] == [0, 1, 2, 3] * 2 + [0, 1]
    assert v.table == [0, 1, 2] and a.num_live == 3
    assert [p for p, _ in seen] == [0] * 4 + [1] * 4 + [2] * 2


def test_build_tables_known_answer_and_out_buffer():
    views = [SimpleNamespace(seq_len=40, table=[3, 4, 5]), SimpleNamespace(seq_len=9, table=[7, 1])]
    t, lens = build_tables(views, 16, "cpu")
    assert t.tolist() == [[3, 4, 5], [7, 0, 0]] and t.dtype == torch.int32
    assert lens.tolist() == [40, 9]
    out = torch.full((4, 6), 99, dtype=torch.int32)
    t2, lens2 = build_tables(views, 16, "cpu", lens_override=[41, 17], out=out)
    assert t2.tolist() == [[3, 4, 5, 0, 0, 0], [7, 1, 0, 0, 0, 0]]
    assert out[2:].eq(99).all() and lens2.tolist() == [41, 17]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_scatter_decode_bit_exact(dtype):
    alloc = BlockAllocator(10)
    cache = PagedKVCache(2, 8, 128, 16, alloc, "cuda", dtype)
    views = [PagedCacheView(cache) for _ in range(3)]
    for v, n in zip(views, (5, 16, 33)):
        for li in range(2):
            v._lens[li] = n
    targets = [v.ensure_append_capacity(1) for v in views]
    pages = torch.tensor([p for p, _ in targets], device="cuda")
    slots = torch.tensor([s for _, s in targets], device="cuda")
    k = torch.randn(4, 8, 1, 128, device="cuda").to(dtype)
    v = torch.randn(4, 8, 1, 128, device="cuda").to(dtype)
    before_k = cache.k_pages[1].clone()
    # a host-side target outside the pool is an IndexError, as the reference's
    # indexing raises (targets on the device are never read back: the kernel
    # skips such a row, checked below)
    with pytest.raises(IndexError):
        cache.scatter_decode(views + [PagedCacheView(cache)], 1, k, v,
                             torch.cat([pages, pages.new_tensor([10**6])]).cpu(),
                             torch.cat([slots, slots.new_tensor([0])]).cpu())
    with pytest.raises(AssertionError):            # kv heads of another pool
        cache.scatter_decode(views, 1, k[:3, :4], v[:3, :4], pages, slots)
    assert torch.equal(cache.k_pages[1], before_k) and [vw._lens[1] for vw in views] == [5, 16, 33]
    cache.scatter_decode(views, 1, k[:3], v[:3], pages, slots)
    want_k, want_v = before_k.clone(), cache.v_pages[1].clone() * 0
    for b, (p, s) in enumerate(targets):
        want_k[p, s] = k[b, :, 0]
        want_v[p, s] = v[b, :, 0]
    assert torch.equal(cache.k_pages[1], want_k)
    assert torch.equal(cache.v_pages[1], want_v)
    assert [vw._lens[1] for vw in views] == [6, 17, 34]
    # the kernel itself skips a row whose (page, slot) lies outside the pool
    from acorninfer_amd._lib import dtype_code, lib, ptr, stream_ptr
    kk = k[3:].reshape(1, 8, 128).contiguous()
    for bad_page, bad_slot in ((10**6, 0), (-1, 0), (pages[0].item(), 16)):
        pg = torch.tensor([bad_page], device="cuda")
        sl = torch.tensor([bad_slot], device="cuda")
        assert lib().acorn_kv_scatter(ptr(kk), ptr(kk), ptr(cache.k_pages[1]),
                                      ptr(cache.v_pages[1]), ptr(pg), ptr(sl), 1, 8, 128, 16,
                                      cache.num_blocks, dtype_code(kk), stream_ptr("cuda")) == 0
    torch.cuda.synchronize()
    assert torch.equal(cache.k_pages[1], want_k) and torch.equal(cache.v_pages[1], want_v)
