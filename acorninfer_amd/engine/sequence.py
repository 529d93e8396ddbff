"""Request state of the engine: the reference's Sequence record
(acorninfer/engine/sequence.py:12-46), same fields and meaning, so the
scheduler policy and its tests carry over."""
from __future__ import annotations

import enum
import time
from dataclasses import dataclass, field

from acorninfer_amd.sampler import SamplingParams


class RequestStatus(enum.Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"


@dataclass
class Sequence:
    seq_id: int
    prompt_ids: list[int]
    sampling: SamplingParams
    max_tokens: int
    eos_ids: frozenset[int]
    generated_ids: list[int] = field(default_factory=list)
    block_table: list[int] = field(default_factory=list)  # shared with its PagedCacheView
    num_pages: int = 0                                     # synced by the engine after a forward
    status: RequestStatus = RequestStatus.WAITING
    stop_reason: str | None = None
    created_at: float = field(default_factory=time.perf_counter)
    first_token_at: float | None = None
    last_token_at: float | None = None
    prefill_cursor: int = 0                                # prompt tokens already in the cache

    @property
    def num_tokens(self) -> int:
        return len(self.prompt_ids) + len(self.generated_ids)

    @property
    def all_ids(self) -> list[int]:
        """prompt + generated: the prefill input of a recomputed (preempted) sequence."""
        return self.prompt_ids + self.generated_ids

    @property
    def is_finished(self) -> bool:
        return self.status is RequestStatus.FINISHED
