"""Sampling on the GPU: temperature -> top-k -> top-p -> draw.

Drop-in for acorninfer/sampler.py: `SamplingParams` (:18-22) and
`Sampler(params, generator)` with `.process(logits)` (:38-55) and
`.sample(logits) -> (token, logprob)` (:57-68), same argument checks and
errors. The work is csrc/sampler.hip (acorn_sample): the row is never
sorted; top-k and top-p are radix selects over the fp32 order keys (top-p on
fixed-point softmax mass, so results are deterministic), ties at the top-p
boundary resolved in the stable ascending order HF sorts in.

The draw takes a uniform u from the caller's generator and picks the
inverse-CDF token over the kept set in vocabulary order (the reference's
torch.multinomial stream is not reproducible across implementations; the
processed distribution and the logprob are). `sample_batch` is the
graph-capturable batched form for the decode step: it never synchronises.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from acorninfer_amd._lib import check, dtype_code, lib, ptr, require_gpu, stream_ptr


@dataclass(frozen=True)
class SamplingParams:
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0  # 0 = disabled


def sample_batch(logits: torch.Tensor, temperature: torch.Tensor, top_k: torch.Tensor,
                 top_p: torch.Tensor, uniform: torch.Tensor, *,
                 token: torch.Tensor | None = None, logprob: torch.Tensor | None = None,
                 status: torch.Tensor | None = None,
                 processed: torch.Tensor | None = None):
    """logits [B, V] (fp32/bf16/fp16 on the GPU); per-row fp32 temperature
    (0 = greedy), int32 top_k (0 = off), fp32 top_p (1 = off), fp32 uniform.
    Returns (token int64 [B], logprob fp32 [B], status int32 [B]); status 1
    marks a row holding NaN/inf. No host synchronisation."""
    require_gpu(logits, temperature, top_k, top_p, uniform)
    B, V = logits.shape
    dev = logits.device
    lg = logits.contiguous()
    token = torch.empty(B, dtype=torch.int64, device=dev) if token is None else token
    logprob = torch.empty(B, dtype=torch.float32, device=dev) if logprob is None else logprob
    status = torch.empty(B, dtype=torch.int32, device=dev) if status is None else status
    # the kernel reads and writes element r of each of these for every row r < B
    for name, t, dt in (("temperature", temperature, torch.float32),
                        ("top_k", top_k, torch.int32), ("top_p", top_p, torch.float32),
                        ("uniform", uniform, torch.float32), ("token", token, torch.int64),
                        ("logprob", logprob, torch.float32), ("status", status, torch.int32)):
        assert t.dtype == dt, f"sample_batch: {name} must be {dt}, got {t.dtype}"
        assert t.device == dev, f"sample_batch: {name} is on {t.device}, logits on {dev}"
        assert t.is_contiguous() and t.numel() >= B, \
            f"sample_batch: {name} needs {B} contiguous elements, has {t.numel()}"
    if processed is not None:
        assert processed.shape == (B, V) and processed.dtype == torch.float32
        assert processed.device == dev and processed.is_contiguous()
    rc = lib().acorn_sample(ptr(lg), B, V, dtype_code(lg), ptr(temperature), ptr(top_k),
                            ptr(top_p), ptr(uniform), ptr(token), ptr(logprob), ptr(processed),
                            ptr(status), stream_ptr(dev))
    check(rc, "sample")
    return token, logprob, status


class Sampler:
    def __init__(self, params: SamplingParams, generator: torch.Generator | None = None):
        """`generator` must live on the logits' device and must not be shared
        between sequences (one stream of uniforms per request)."""
        if params.temperature <= 0:
            raise ValueError("temperature must be > 0")
        if not (0.0 < params.top_p <= 1.0):
            raise ValueError("top_p must be in (0, 1]")
        if params.top_k < 0:
            raise ValueError("top_k must be >= 0 (0 disables)")
        self.params = params
        self.generator = generator

    def _run(self, logits: torch.Tensor, uniform: float, want_processed: bool):
        row = logits.reshape(1, -1)
        dev = row.device
        p = self.params
        processed = (torch.empty(row.shape, dtype=torch.float32, device=dev)
                     if want_processed else None)
        tok, lp, st = sample_batch(
            row, torch.tensor([p.temperature], dtype=torch.float32, device=dev),
            torch.tensor([min(p.top_k, 2**31 - 1)], dtype=torch.int32, device=dev),
            torch.tensor([p.top_p], dtype=torch.float32, device=dev),
            torch.tensor([uniform], dtype=torch.float32, device=dev), processed=processed)
        if int(st[0]) != 0:
            raise ValueError("logits contain NaN/inf; model forward is broken")
        return tok, lp, processed

    def process(self, logits: torch.Tensor) -> torch.Tensor:
        """temperature -> top-k -> top-p; returns the processed fp32 [vocab]
        logits (-inf where removed)."""
        _, _, processed = self._run(logits, 0.0, True)
        return processed[0]

    def sample(self, logits: torch.Tensor) -> tuple[int, float]:
        """(token, its logprob under the processed distribution)."""
        u = float(torch.rand(1, generator=self.generator, device=logits.device))
        tok, lp, _ = self._run(logits, u, False)
        return int(tok[0]), float(lp[0])
