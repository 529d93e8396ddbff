"""Request lifecycle and the step loop on the MI355X decode path: the
reference's Engine (acorninfer/engine/engine.py:30-378) without TP,
speculative decoding, the tokenizer and the server, with the same
submit / step / drop / has_pending / assert_balanced contract.

A step runs the scheduler, then
- every prefill chunk of the step in one Qwen3DecodeModel.forward_extend
  launch sequence (new and recomputed sequences start from an empty view,
  continuations extend theirs); a chunk that completes its sequence's ids
  yields the next token: argmax at temperature 0, else the GPU sampler;
- every decode-level sequence in one graph-replayed DecodeGraphRunner step
  (sampled rows are drawn inside the graph),
and retires finished sequences (their blocks go back to the allocator) even
when a forward raises.
"""
from __future__ import annotations

import time
from dataclasses import dataclass

import torch

from acorninfer_amd.cache.pager import BlockAllocator, PagedCacheView, PagedKVCache
from acorninfer_amd.engine.graph_runner import BUCKETS, DecodeGraphRunner
from acorninfer_amd.engine.scheduler import Scheduler
from acorninfer_amd.engine.sequence import RequestStatus, Sequence
from acorninfer_amd.models.qwen3 import Qwen3DecodeModel
from acorninfer_amd.sampler import Sampler, SamplingParams

QWEN3_EOS_IDS = frozenset({151643, 151645})  # <|endoftext|>, <|im_end|>


@dataclass
class TokenOutput:
    seq_id: int
    token_id: int
    finished: bool
    stop_reason: str | None = None


class Engine:
    def __init__(self, model: Qwen3DecodeModel, *, num_blocks: int = 1024, page_size: int = 16,
                 max_running: int = 8, watermark_blocks: int = 8,
                 chunked_budget: int | None = None, max_model_len: int = 4096,
                 capture: bool = True, seed: int = 0):
        if watermark_blocks >= num_blocks:
            raise ValueError(f"watermark_blocks ({watermark_blocks}) must be < num_blocks "
                             f"({num_blocks})")
        if max_running > BUCKETS[-1]:
            raise ValueError(f"max_running {max_running} exceeds the largest decode bucket "
                             f"{BUCKETS[-1]}")
        cfg = model.cfg
        self.model = model
        self.page_size = page_size
        self.allocator = BlockAllocator(num_blocks)
        self.cache = PagedKVCache(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim,
                                  page_size, self.allocator, model.device, model.dtype)
        self.scheduler = Scheduler(self.allocator, page_size, max_running, watermark_blocks,
                                   chunked_budget)
        # the runner keeps one resident block (the padding rows' KV target)
        top = min(b for b in BUCKETS if b >= max_running)
        self.graph_runner = DecodeGraphRunner(
            model, self.cache, self.allocator, max_model_len=max_model_len,
            buckets=tuple(b for b in BUCKETS if b <= top), capture=capture, seed=seed)
        self.max_model_len = max_model_len
        self.seqs: dict[int, Sequence] = {}
        self._views: dict[int, PagedCacheView] = {}
        self._next_id = 0
        self._gen = torch.Generator(device=model.device).manual_seed(seed + 1)

    def submit(self, prompt_ids: list[int], sampling: SamplingParams, *, max_tokens: int,
               eos_ids: frozenset[int] | None = None) -> int:
        if not prompt_ids:
            raise ValueError("prompt_ids must be non-empty")
        if max_tokens < 1:
            raise ValueError("max_tokens must be >= 1")
        if len(prompt_ids) + max_tokens > self.max_model_len:
            raise ValueError(f"prompt + max_tokens ({len(prompt_ids) + max_tokens}) exceeds "
                             f"max_model_len ({self.max_model_len})")
        # a prompt beyond the schedulable capacity (blocks minus watermark and
        # the runner's resident block) would wait at the head of the queue forever
        capacity = self.allocator.total - self.scheduler.watermark - 1
        if -(-len(prompt_ids) // self.page_size) > capacity:
            raise ValueError(f"prompt needs more KV blocks than the schedulable capacity "
                             f"({capacity}); it could never be admitted")
        seq = Sequence(seq_id=self._next_id, prompt_ids=list(prompt_ids), sampling=sampling,
                       max_tokens=max_tokens,
                       eos_ids=frozenset(eos_ids) if eos_ids is not None else QWEN3_EOS_IDS)
        self._next_id += 1
        self.seqs[seq.seq_id] = seq
        self.scheduler.add(seq)
        return seq.seq_id

    def _sample(self, seq: Sequence, logits: torch.Tensor) -> int:
        if seq.sampling.temperature == 0:
            return int(logits.argmax())
        return Sampler(seq.sampling, self._gen).sample(logits)[0]

    def _prefill(self, chunks, outputs: list[TokenOutput]) -> None:
        views, starts, lens, rows = [], [], [], []
        for seq, start, n in chunks:
            if start == 0:
                # a new or recomputed sequence starts from a fresh view over
                # its (shared, emptied) block table
                view = PagedCacheView(self.cache, seq.block_table)
                self._views[seq.seq_id] = view
            else:
                view = self._views[seq.seq_id]
            views.append(view)
            starts.append(start)
            lens.append(n)
            rows.append(seq.all_ids[start:start + n])
        ids = torch.zeros(len(rows), max(lens), dtype=torch.int64)
        for i, r in enumerate(rows):
            ids[i, :len(r)] = torch.tensor(r, dtype=torch.int64)
        logits = self.model.forward_extend(ids.to(self.model.device), views, starts=starts,
                                           chunk_lens=lens)
        for i, (seq, start, n) in enumerate(chunks):
            seq.num_pages = len(views[i].table)
            seq.prefill_cursor = start + n
            if start + n == len(seq.all_ids):
                self._record(seq, self._sample(seq, logits[i]), outputs)

    @torch.inference_mode()
    def step(self) -> list[TokenOutput]:
        chunks, decodes = self.scheduler.schedule()
        outputs: list[TokenOutput] = []
        try:
            if chunks:
                self._prefill(chunks, outputs)
            if decodes:
                views = [self._views[s.seq_id] for s in decodes]
                tokens = self.graph_runner.decode_batch(decodes, views)
                for seq, view, token in zip(decodes, views, tokens):
                    seq.num_pages = len(view.table)
                    self._record(seq, token, outputs)
        finally:
            # retire even when a forward raised: a finished sequence must not
            # be decoded again
            for seq in [s for s in self.scheduler.running if s.is_finished]:
                self.scheduler.running.remove(seq)
                self._views.pop(seq.seq_id, None)
                for b in seq.block_table:
                    self.allocator.free(b)
                seq.block_table.clear()
                seq.num_pages = 0
        return outputs

    def _record(self, seq: Sequence, token_id: int, outputs: list[TokenOutput]) -> None:
        seq.generated_ids.append(token_id)
        now = time.perf_counter()
        if seq.first_token_at is None:
            seq.first_token_at = now
        seq.last_token_at = now
        reason = None
        if token_id in seq.eos_ids:
            reason = "stop"
        elif len(seq.generated_ids) >= seq.max_tokens:
            reason = "length"
        if reason is not None:
            seq.stop_reason = reason
            seq.status = RequestStatus.FINISHED
        outputs.append(TokenOutput(seq.seq_id, token_id, reason is not None, reason))

    def drop(self, seq_id: int) -> None:
        """Forget a finished sequence's record (the caller consumed its output)."""
        seq = self.seqs.get(seq_id)
        if seq is not None and not seq.is_finished:
            raise ValueError(f"seq {seq_id} is still pending; cannot drop")
        self.seqs.pop(seq_id, None)

    def has_pending(self) -> bool:
        return bool(self.scheduler.waiting or self.scheduler.running)

    def assert_balanced(self) -> None:
        """After draining: exactly the runner's resident block is live."""
        if self.allocator.num_live != 1:
            raise AssertionError(f"expected exactly 1 live block (graph runner scratch), "
                                 f"got {self.allocator.num_live}")
