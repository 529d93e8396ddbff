"""Helpers shared by the decode-model tests."""
import torch

from acorninfer_amd.cache.pager import BlockAllocator, PagedCacheView, PagedKVCache


def new_cache(model, num_blocks, page_size=16, dtype=None):
    cfg = model.cfg
    alloc = BlockAllocator(num_blocks)
    cache = PagedKVCache(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim,
                         page_size, alloc, model.device, dtype or model.dtype)
    return alloc, cache


def feed_prompt(model, view, prompt):
    """Run the prompt through the decode step one token at a time (causal
    attention over the cache, mathematically the prefill of generate.py).
    Returns the fp32 logits of the last prompt position."""
    logits = None
    for t in prompt:
        ids = torch.tensor([[int(t)]], device=model.device)
        logits = model.forward_decode(ids, [view])[0]
    return logits


def release(alloc, views):
    for v in views:
        for b in v.table:
            alloc.free(b)
        v.table.clear()
