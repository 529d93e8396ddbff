"""Scheduler policy (acorninfer/engine/scheduler.py:14-160) on the CPU:
FCFS admission, max_running, the watermark, the in-step block reserve of
page-full decodes, preemption of the oldest running sequence with recompute,
and the per-step prefill budget. Pages of 4 tokens throughout."""
import pytest

from acorninfer_amd.cache.pager import BlockAllocator
from acorninfer_amd.engine.scheduler import Scheduler
from acorninfer_amd.engine.sequence import RequestStatus, Sequence
from acorninfer_amd.sampler import SamplingParams

P = 4


def seq(sid, n_prompt, n_gen=0):
    s = Sequence(seq_id=sid, prompt_ids=list(range(sid * 1000, sid * 1000 + n_prompt)),
                 sampling=SamplingParams(temperature=0.0), max_tokens=100,
                 eos_ids=frozenset({-1}))
    s.generated_ids = [7] * n_gen
    return s


def hold(alloc, s, pages):
    """The engine's side of a prefill: s holds `pages` blocks, prompt done."""
    s.status = RequestStatus.RUNNING
    s.block_table = [alloc.allocate() for _ in range(pages)]
    s.num_pages = pages
    s.prefill_cursor = len(s.prompt_ids)


def plan(chunks):
    return [(s.seq_id, start, n) for s, start, n in chunks]


@pytest.mark.parametrize("bad", [0, -3])
def test_budget_must_be_positive(bad):
    with pytest.raises(ValueError, match="chunked_budget"):
        Scheduler(BlockAllocator(4), P, chunked_budget=bad)


def test_fcfs_whole_prompts():
    sch = Scheduler(BlockAllocator(16), P)
    for i in range(3):
        sch.add(seq(i, 6))
    chunks, decodes = sch.schedule()
    assert plan(chunks) == [(0, 0, 6), (1, 0, 6), (2, 0, 6)] and decodes == []
    assert all(s.status is RequestStatus.RUNNING for s in sch.running)


def test_max_running():
    sch = Scheduler(BlockAllocator(64), P, max_running=2)
    for i in range(3):
        sch.add(seq(i, 6))
    chunks, _ = sch.schedule()
    assert plan(chunks) == [(0, 0, 6), (1, 0, 6)]
    assert [s.seq_id for s in sch.waiting] == [2]


def test_watermark_holds_back_admission():
    alloc = BlockAllocator(8)
    sch = Scheduler(alloc, P, max_running=8, watermark_blocks=3)
    for i in range(3):
        sch.add(seq(i, 6))                     # 2 pages each
    chunks, _ = sch.schedule()
    assert [s for s, _, _ in plan(chunks)] == [0, 1]   # 8-2-2 = 4, minus 3 < 2
    for s in list(sch.running):
        hold(alloc, s, 2)
        s.generated_ids.append(5)              # 7 tokens: still within 2 pages
    assert sch.schedule() == ([], sch.running)
    sch.watermark = 0
    chunks, decodes = sch.schedule()
    assert plan(chunks) == [(2, 0, 6)] and [s.seq_id for s in decodes] == [0, 1]


def test_page_full_decode_is_reserved():
    alloc = BlockAllocator(3)
    sch = Scheduler(alloc, P)
    a = seq(0, 3, n_gen=1)                     # 4 tokens in the cache: one full page
    sch.add(a)
    sch.schedule()
    hold(alloc, a, 1)
    a.generated_ids.append(9)                  # 5 tokens: this step's decode needs a block
    b = seq(1, 8)                              # needs 2 blocks; 2 free but 1 is reserved
    sch.add(b)
    chunks, decodes = sch.schedule()
    assert chunks == [] and [s.seq_id for s in decodes] == [0]
    assert sch.waiting[0] is b


def test_preempt_oldest_and_recompute():
    alloc = BlockAllocator(3)
    sch = Scheduler(alloc, P)
    a, b = seq(0, 3, n_gen=1), seq(1, 3, n_gen=1)
    sch.add(a)
    sch.add(b)
    sch.schedule()
    for s in (a, b):
        hold(alloc, s, 1)
        s.generated_ids.append(9)              # both overflow their page
    chunks, decodes = sch.schedule()           # deficit 2 > free 1: a goes
    assert a.status is RequestStatus.WAITING and sch.waiting[0] is a
    assert a.block_table == [] and a.num_pages == 0 and a.prefill_cursor == 0
    assert chunks == [] and [s.seq_id for s in decodes] == [1]   # not readmitted this step
    assert alloc.num_free == 2
    sch.running.remove(b)                      # b finishes; the engine frees its block
    for blk in b.block_table:
        alloc.free(blk)
    b.block_table.clear()
    chunks, decodes = sch.schedule()
    assert plan(chunks) == [(0, 0, 5)]         # recompute: all ids, whole
    assert decodes == []


def test_budget_orders_running_chunks_first_and_splits_new_prompts():
    alloc = BlockAllocator(64)
    sch = Scheduler(alloc, P, chunked_budget=8)
    a = seq(0, 10)
    sch.add(a)
    assert plan(sch.schedule()[0]) == [(0, 0, 8)]
    a.block_table = [alloc.allocate() for _ in range(2)]
    a.num_pages, a.prefill_cursor = 2, 8
    b = seq(1, 9)
    sch.add(b)
    chunks, decodes = sch.schedule()
    assert plan(chunks) == [(0, 8, 2), (1, 0, 6)]   # a's rest first, b gets what is left
    assert decodes == []


def test_budget_spent_leaves_head_waiting_and_recompute_is_exempt():
    alloc = BlockAllocator(64)
    sch = Scheduler(alloc, P, chunked_budget=4)
    a = seq(0, 4)
    c = seq(2, 3, n_gen=2)                     # a preempted sequence waiting to recompute
    sch.add(a)
    sch.add(seq(1, 4))
    chunks, _ = sch.schedule()
    assert plan(chunks) == [(0, 0, 4)]        # budget spent: seq 1 waits at the head
    sch.waiting.appendleft(c)
    hold(alloc, a, 1)
    a.generated_ids.append(3)
    chunks, decodes = sch.schedule()
    assert plan(chunks)[0] == (2, 0, 5)        # whole all_ids, outside the budget
    assert (1, 0, 4) in plan(chunks) and [s.seq_id for s in decodes] == [0]


def test_one_chunk_per_sequence_and_mid_prefill_is_not_decoded():
    alloc = BlockAllocator(64)
    sch = Scheduler(alloc, P, chunked_budget=3)
    a = seq(0, 10)
    sch.add(a)
    chunks, decodes = sch.schedule()
    assert plan(chunks) == [(0, 0, 3)] and decodes == []
    a.block_table = [alloc.allocate()]
    a.num_pages, a.prefill_cursor = 1, 3
    chunks, decodes = sch.schedule()
    assert plan(chunks) == [(0, 3, 3)] and decodes == []


def test_preempting_mid_prefill_resets_its_cursor():
    alloc = BlockAllocator(3)
    sch = Scheduler(alloc, P, chunked_budget=8)
    a, b = seq(0, 3, n_gen=1), seq(1, 12)
    sch.add(a)
    sch.schedule()
    hold(alloc, a, 1)
    sch.add(b)
    sch.waiting.clear()
    sch.running.append(b)                     # b running mid-prefill: 8 of 12 written
    b.status = RequestStatus.RUNNING
    b.block_table = [alloc.allocate(), alloc.allocate()]
    b.num_pages, b.prefill_cursor = 2, 8
    a.generated_ids.append(9)                 # a now needs a block, b its third page
    chunks, decodes = sch.schedule()          # reserve 2 > free 0: a goes; then 1 <= 1
    assert a.status is RequestStatus.WAITING and a.prefill_cursor == 0
    assert plan(chunks) == [(1, 8, 4)] and decodes == []
