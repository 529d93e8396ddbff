"""FCFS scheduler with a block watermark, preemption of the oldest running
sequence (recompute) and an optional per-step prefill budget: the policy of
acorninfer/engine/scheduler.py:14-160, restated.

Each step, schedule() returns (chunks, decodes):
- chunks: (sequence, start, length) prefill pieces, at most one per
  sequence; start is the sequence's prefill cursor (0 for a new or
  recomputed sequence);
- decodes: the running sequences that take one decode step.

Block accounting (page = P tokens):
- a running sequence at decode level whose tokens no longer fit its pages
  (num_tokens > num_pages * P) takes one block inside this step; a
  mid-prefill sequence takes ceil((cursor + length) / P) - num_pages blocks
  for its chunk. Those blocks are the step's reserve;
- while the free blocks cannot cover the reserve, the oldest running sequence
  is preempted: its blocks are freed, its cursor reset, and it goes back to
  the front of the queue (it is not readmitted in the same step);
- admission is FCFS while fewer than max_running run and the free blocks
  minus what this step already admitted, the reserve and the watermark cover
  the candidate's whole need, ceil(num_tokens / P) - num_pages. A recomputed
  sequence (it has generated tokens) is prefilled whole, outside the budget;
  a new one gets at most the remaining budget (None = its whole prompt).

Retirement is the engine's: it removes finished sequences from `running` and
frees their blocks.
"""
from __future__ import annotations

from collections import deque

from acorninfer_amd.cache.pager import BlockAllocator
from acorninfer_amd.engine.sequence import RequestStatus, Sequence


def _pages(tokens: int, page: int) -> int:
    return -(-tokens // page)


class Scheduler:
    def __init__(self, allocator: BlockAllocator, page_size: int, max_running: int = 8,
                 watermark_blocks: int = 0, chunked_budget: int | None = None):
        if chunked_budget is not None and chunked_budget < 1:
            raise ValueError(f"chunked_budget must be >= 1, got {chunked_budget}")
        self.allocator = allocator
        self.page_size = page_size
        self.max_running = max_running
        self.watermark = watermark_blocks
        self.chunked_budget = chunked_budget
        self.waiting: deque[Sequence] = deque()
        self.running: list[Sequence] = []

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    @staticmethod
    def _mid_prefill(seq: Sequence) -> bool:
        return not seq.generated_ids and seq.prefill_cursor < len(seq.prompt_ids)

    def _release(self, seq: Sequence) -> None:
        for b in seq.block_table:
            self.allocator.free(b)
        seq.block_table.clear()
        seq.num_pages = 0
        seq.prefill_cursor = 0

    def _running_chunks(self):
        """Chunks of the running mid-prefill sequences (running order), the
        blocks they add this step, and the budget left after them."""
        chunks, add_pages, left = [], 0, self.chunked_budget
        for seq in self.running:
            if not self._mid_prefill(seq):
                continue
            n = len(seq.prompt_ids) - seq.prefill_cursor
            if left is not None:
                n = min(n, left)
            if n <= 0:
                continue                     # budget spent: this sequence waits a step
            if left is not None:
                left -= n
            add_pages += max(_pages(seq.prefill_cursor + n, self.page_size) - seq.num_pages, 0)
            chunks.append((seq, seq.prefill_cursor, n))
        return chunks, add_pages, left

    def _decode_deficit(self) -> int:
        return sum(1 for s in self.running
                   if not self._mid_prefill(s) and s.num_tokens > s.num_pages * self.page_size)

    def schedule(self) -> tuple[list[tuple[Sequence, int, int]], list[Sequence]]:
        preempted: set[int] = set()
        while True:
            chunks, add_pages, left = self._running_chunks()
            reserve = self._decode_deficit() + add_pages
            if self.allocator.num_free >= reserve:
                break
            victim = self.running.pop(0)     # the oldest
            victim.status = RequestStatus.WAITING
            self._release(victim)
            self.waiting.appendleft(victim)
            preempted.add(victim.seq_id)

        admitted_pages = 0                   # blocks the admitted sequences will take
        while self.waiting and len(self.running) < self.max_running:
            cand = self.waiting[0]
            if cand.seq_id in preempted:
                break
            need = _pages(cand.num_tokens, self.page_size) - cand.num_pages
            if self.allocator.num_free - admitted_pages - reserve - self.watermark < need:
                break
            if cand.generated_ids:
                start, n = 0, len(cand.all_ids)   # recompute: whole, outside the budget
            else:
                start = cand.prefill_cursor
                n = len(cand.prompt_ids) - start
                if left is not None:
                    n = min(n, left)
                if n <= 0:
                    break                    # budget spent: the head of the queue waits
                if left is not None:
                    left -= n
            self.waiting.popleft()
            admitted_pages += need
            cand.status = RequestStatus.RUNNING
            self.running.append(cand)
            chunks.append((cand, start, n))

        in_chunks = {s.seq_id for s, _, _ in chunks}
        return chunks, [s for s in self.running if s.seq_id not in in_chunks]
