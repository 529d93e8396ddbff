"""Paged KV cache: block allocator, per-layer page pool and per-sequence views.

Mirrors acorninfer/cache/pager.py so an AcornInfer-style engine can swap it
in:

- `BlockAllocator` (pager.py:16-55): LIFO free list of physical block ids;
  `allocate` raises `BlockExhausted` when empty, `free` rejects a block that
  is not live, `assert_balanced` raises when blocks leak.
- `PagedKVCache` (pager.py:58-113): k/v pages of shape
  [num_blocks, page_size, kv_heads, head_dim] per layer. Here every layer's
  pages are slices of ONE contiguous HBM allocation [layers, NB, P, KV, D]
  per K and V (one allocation for the whole pool; layer l's pages stay the
  reference's per-layer tensors as views). `scatter_decode` is the HIP
  kernel acorn_kv_scatter.
- Speculative verify (pager.py:115-148, 211-244): `scatter_verify` writes an
  m-token window per sequence with the same scatter kernel,
  `ensure_append_capacity_n` reserves the window, `set_lens` rolls a length
  back after a partial accept.
- `PagedCacheView` (pager.py:151-259): the block table is a `list[int]`
  shared with the caller; written length is tracked per layer; token t of a
  sequence lives at (table[t // P], t % P). `ensure_append_capacity`
  allocates a new block exactly when the append position starts a page.

`write`/`update`/`_gather` are the reference's prefill/oracle-side plumbing
(torch indexing on the pool); the decode hot path never calls them.
"""
from __future__ import annotations

import torch

from acorninfer_amd._lib import check, dtype_code, lib, ptr, stream_ptr


class BlockExhausted(Exception):
    """No free physical KV block; the scheduler queues or preempts."""


class BlockAllocator:
    """LIFO free list of physical KV block ids 0..num_blocks-1."""

    def __init__(self, num_blocks: int):
        self._free: list[int] = list(range(num_blocks - 1, -1, -1))
        self._live: set[int] = set()

    @property
    def num_free(self) -> int:
        return len(self._free)

    @property
    def num_live(self) -> int:
        return len(self._live)

    @property
    def total(self) -> int:
        return len(self._free) + len(self._live)

    def allocate(self) -> int:
        if not self._free:
            raise BlockExhausted(f"all {self.total} KV blocks are in use")
        block = self._free.pop()
        self._live.add(block)
        return block

    def free(self, block: int) -> None:
        if block not in self._live:
            raise ValueError(f"free({block}): that block is not allocated")
        self._live.remove(block)
        self._free.append(block)

    def assert_balanced(self) -> None:
        """Raise (also under `python -O`) if any block is still live."""
        if self._live:
            raise AssertionError(f"KV leak: {len(self._live)} block(s) still allocated: "
                                 f"{sorted(self._live)}")


class PagedKVCache:
    """Physical page storage for every layer, one contiguous pool per K / V."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, page_size: int,
                 allocator: BlockAllocator, device, dtype: torch.dtype):
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self.allocator = allocator
        self.device = torch.device(device)
        self.dtype = dtype
        self.num_blocks = allocator.total
        shape = (num_layers, self.num_blocks, page_size, num_kv_heads, head_dim)
        self.k_pool = torch.zeros(shape, device=self.device, dtype=dtype)
        self.v_pool = torch.zeros(shape, device=self.device, dtype=dtype)
        self.k_pages = [self.k_pool[i] for i in range(num_layers)]
        self.v_pages = [self.v_pool[i] for i in range(num_layers)]

    @property
    def layer_stride(self) -> int:
        """Elements between layer l and l+1 of the pool."""
        return self.num_blocks * self.page_size * self.num_kv_heads * self.head_dim

    def _check_rows(self, k, v, pages, slots) -> None:
        """The kernel indexes k/v with the pool's kv-head count and head size,
        and writes (page, slot) into the pool: reject what does not fit. With
        pages/slots on the host an out-of-range target raises IndexError, as
        the reference's torch indexing does. Targets already on the GPU are
        not read back (that would synchronise the stream and break graph
        capture): the scatter kernel skips a row whose (page, slot) lies
        outside the pool and writes nothing for it."""
        for name, t in (("k", k), ("v", v)):
            assert t.dim() == 4 and t.shape[1] == self.num_kv_heads and \
                t.shape[3] == self.head_dim, \
                f"{name} is {tuple(t.shape)}; the pool holds {self.num_kv_heads} kv heads " \
                f"of {self.head_dim}"
        if pages.numel() == 0 or pages.is_cuda or slots.is_cuda:
            return
        bad = ((pages < 0) | (pages >= self.num_blocks)).any() | \
              ((slots < 0) | (slots >= self.page_size)).any()
        if bool(bad):
            raise IndexError(f"(page, slot) outside the pool of {self.num_blocks} blocks x "
                             f"{self.page_size} slots")

    def scatter_decode(self, views: list["PagedCacheView"], layer_idx: int, k: torch.Tensor,
                       v: torch.Tensor, pages: torch.Tensor, slots: torch.Tensor) -> None:
        """Decode-step batched write (pager.py:87-113): k_pages[l][pages[b], slots[b]] =
        k[b, :, 0, :] (same for v), then each view's layer length grows by one.

        k/v [B, KV, 1, D]; pages/slots [B] int64 from ensure_append_capacity.
        """
        B = len(views)
        assert k.shape[2] == 1 and v.shape[2] == 1, "scatter_decode writes one token per row"
        assert B == k.shape[0] == v.shape[0] == pages.shape[0] == slots.shape[0]
        self._check_rows(k, v, pages, slots)
        kc = k.to(self.dtype).contiguous()
        vc = v.to(self.dtype).contiguous()
        pg = pages.to(device=self.device, dtype=torch.int64).contiguous()
        sl = slots.to(device=self.device, dtype=torch.int64).contiguous()
        rc = lib().acorn_kv_scatter(
            ptr(kc), ptr(vc), ptr(self.k_pages[layer_idx]), ptr(self.v_pages[layer_idx]),
            ptr(pg), ptr(sl), B, self.num_kv_heads, self.head_dim, self.page_size,
            self.num_blocks, dtype_code(kc), stream_ptr(self.device))
        check(rc, "scatter_decode")
        for view in views:
            view._lens[layer_idx] = view._lens.get(layer_idx, 0) + 1

    def scatter_verify(self, views: list["PagedCacheView"], layer_idx: int, k: torch.Tensor,
                       v: torch.Tensor, pages: torch.Tensor, slots: torch.Tensor) -> None:
        """Verify-step write of an m-token window per sequence (pager.py:115-148):
        k_pages[l][pages[b, j], slots[b, j]] = k[b, :, j, :] (same for v), then
        each view's layer length grows by m. k/v [B, KV, m, D]; pages/slots
        [B, m] int64 from ensure_append_capacity_n. The window is flattened to
        B*m rows in (b, j) order and written by the decode scatter kernel
        (m = 1 is scatter_decode). Capacity was reserved beforehand, so this
        never raises BlockExhausted."""
        B = len(views)
        m = k.shape[2]
        assert m == v.shape[2], "k and v must hold windows of the same length"
        assert B == k.shape[0] == v.shape[0] == pages.shape[0] == slots.shape[0]
        assert pages.shape[1] == slots.shape[1] == m, "one (page, slot) per window token"
        self._check_rows(k, v, pages, slots)
        kc = k.permute(0, 2, 1, 3).reshape(B * m, k.shape[1], k.shape[3]).to(self.dtype).contiguous()
        vc = v.permute(0, 2, 1, 3).reshape(B * m, v.shape[1], v.shape[3]).to(self.dtype).contiguous()
        pg = pages.reshape(-1).to(device=self.device, dtype=torch.int64).contiguous()
        sl = slots.reshape(-1).to(device=self.device, dtype=torch.int64).contiguous()
        rc = lib().acorn_kv_scatter(
            ptr(kc), ptr(vc), ptr(self.k_pages[layer_idx]), ptr(self.v_pages[layer_idx]),
            ptr(pg), ptr(sl), B * m, self.num_kv_heads, self.head_dim, self.page_size,
            self.num_blocks, dtype_code(kc), stream_ptr(self.device))
        check(rc, "scatter_verify")
        for view in views:
            view._lens[layer_idx] = view._lens.get(layer_idx, 0) + m


class PagedCacheView:
    """Per-sequence view: a block table (shared list) and per-layer lengths."""

    def __init__(self, cache: PagedKVCache, table: list[int] | None = None):
        self.cache = cache
        self.table: list[int] = table if table is not None else []
        self._lens: dict[int, int] = {}

    @property
    def seq_len(self) -> int:
        """Written length of layer 0 (layers advance in lock step)."""
        return self._lens.get(0, 0)

    def _grow_to(self, needed_blocks: int) -> None:
        while len(self.table) < needed_blocks:
            self.table.append(self.cache.allocator.allocate())

    def write(self, layer_idx: int, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """Append s tokens k_new/v_new [1, KV, s, D]: blocks are allocated first
        (a BlockExhausted leaves no partial write and no length change)."""
        c = self.cache
        s = k_new.shape[2]
        base = self._lens.get(layer_idx, 0)
        self._grow_to((base + s + c.page_size - 1) // c.page_size)
        positions = range(base, base + s)
        rows = torch.tensor([self.table[p // c.page_size] for p in positions],
                            device=c.device, dtype=torch.long)
        slots = torch.tensor([p % c.page_size for p in positions],
                             device=c.device, dtype=torch.long)
        c.k_pages[layer_idx][rows, slots] = k_new[0].permute(1, 0, 2).to(c.dtype)
        c.v_pages[layer_idx][rows, slots] = v_new[0].permute(1, 0, 2).to(c.dtype)
        self._lens[layer_idx] = base + s

    def reserve(self, n: int) -> list[tuple[int, int]]:
        """Make room for n more tokens after layer 0's length; return each
        one's (block id, slot) in position order. Like `write`, it allocates
        before anything is written; lengths are not advanced."""
        base, page = self.seq_len, self.cache.page_size
        self._grow_to((base + n + page - 1) // page)
        return [(self.table[p // page], p % page) for p in range(base, base + n)]

    def ensure_append_capacity(self, layer_idx: int) -> tuple[int, int]:
        """Make room for one more token at layer `layer_idx`; return its
        (block id, slot). Allocates only when the append position starts a page."""
        base = self._lens.get(layer_idx, 0)
        page = self.cache.page_size
        self._grow_to(base // page + 1)
        return self.table[base // page], base % page

    def ensure_append_capacity_n(self, layer_idx: int, n: int) -> list[tuple[int, int]]:
        """Room for n more tokens at layer `layer_idx` (pager.py:211-227): the
        table grows to ceil((len + n) / P) blocks as `write` would, then each
        position's (block id, slot) in order. A BlockExhausted part-way keeps
        the blocks already taken in the table; lengths are not advanced
        (scatter_verify commits them). n = 1 is ensure_append_capacity."""
        base = self._lens.get(layer_idx, 0)
        page = self.cache.page_size
        self._grow_to((base + n + page - 1) // page)
        return [(self.table[p // page], p % page) for p in range(base, base + n)]

    def set_lens(self, layer_idx: int, new_len: int) -> None:
        """Roll layer `layer_idx` back to `new_len` written tokens after a
        verify step accepted fewer than it wrote (pager.py:229-244). Blocks stay
        in the table (the dead slots are rewritten by the next window); moving
        forward is a ValueError (only writes advance a length)."""
        cur = self._lens.get(layer_idx, 0)
        if new_len > cur:
            raise ValueError(f"set_lens can only move a length back: asked for {new_len}, "
                             f"{cur} written")
        self._lens[layer_idx] = new_len

    def update(self, layer_idx: int, k_new: torch.Tensor, v_new: torch.Tensor
               ) -> tuple[torch.Tensor, torch.Tensor]:
        """write + gather the full [1, KV, seq_len, D] K and V."""
        self.write(layer_idx, k_new, v_new)
        return (self._gather(layer_idx, self.cache.k_pages),
                self._gather(layer_idx, self.cache.v_pages))

    def _gather(self, layer_idx: int, pages: list[torch.Tensor]) -> torch.Tensor:
        c = self.cache
        idx = torch.tensor(self.table, device=c.device, dtype=torch.long)
        t = pages[layer_idx][idx].reshape(-1, c.num_kv_heads, c.head_dim)
        return t[: self._lens.get(layer_idx, 0)].permute(1, 0, 2)[None]
