"""Restatement of acorninfer/sampler.py:38-68 (torch, CPU) — TEST INFRASTRUCTURE ONLY.

process_ref: temperature -> top-k -> top-p in HF warper order (sampler.py:38-55).
The ascending sort of the top-p step is stable (torch.sort(stable=True)): among
equal values the lower vocabulary index comes first, so at a tie straddling
the top-p boundary the higher indices are kept. (The reference calls
torch.sort without `stable`; on ties its order is implementation-defined.)
draw_ref: the inverse-CDF draw of a uniform u over the kept tokens in
vocabulary order, and the logprob under the processed distribution
(sampler.py:57-68 with multinomial replaced by an explicit uniform).

Pins (tests/test_oracle_sampler.py): the reference's known answers
(tests/test_sampler.py:10-39 in the reference) and HF transformers'
TemperatureLogitsWarper / TopKLogitsWarper / TopPLogitsWarper (the reference's
own oracle, tests/test_sampler.py:41-67) on random vocab-size rows.
"""
from __future__ import annotations

import torch


def process_ref(logits: torch.Tensor, temperature: float, top_k: int, top_p: float) -> torch.Tensor:
    x = logits.float().clone()
    if not torch.isfinite(x).all():
        raise ValueError("logits contain NaN/inf; model forward is broken")
    x = x / temperature
    if top_k > 0:
        k = min(top_k, x.size(-1))
        kth = torch.topk(x, k).values[-1]
        x[x < kth] = float("-inf")
    if top_p < 1.0:
        sorted_x, idx = torch.sort(x, descending=False, stable=True)
        cum = sorted_x.softmax(dim=-1).cumsum(dim=-1)
        remove = cum <= (1.0 - top_p)
        remove[-1] = False
        mask = torch.zeros_like(remove).scatter(0, idx, remove)
        x[mask] = float("-inf")
    return x


def draw_ref(processed: torch.Tensor, u: float) -> tuple[int, float]:
    """First vocabulary index whose running kept mass exceeds u * total."""
    p = torch.softmax(processed.double(), dim=-1)
    cum = torch.cumsum(p, dim=-1)
    idx = int(torch.searchsorted(cum, torch.tensor([u], dtype=torch.float64), right=True)[0])
    idx = min(idx, processed.numel() - 1)
    while not torch.isfinite(processed[idx]):
        idx -= 1
    return idx, float(torch.log_softmax(processed.double(), dim=-1)[idx])
