"""hipGraph decode runner (engine/graph_runner.py) — the reference's
tests/test_graph_runner.py:51-114 scenarios on the HIP step:

- graph replay equals the same runner un-captured, bitwise, step by step,
  while the batch shrinks inside a bucket (4 -> 3), a retired sequence's
  blocks are reused (LIFO) and the bucket switches (4 -> 2);
- replay matches eager `forward_decode` (tokens equal, logits within bf16
  tolerance: the bucket's split count differs from the eager batch's);
- per-layer lengths advance on the host; after draining, exactly the scratch
  block stays live;
- `decode_loop` (device-fed ids) yields the same tokens as step-by-step
  `decode_batch`.
"""
from types import SimpleNamespace

import pytest
import torch

from acorninfer_amd.cache.pager import PagedCacheView
from acorninfer_amd.config import Qwen3Config
from acorninfer_amd.engine.graph_runner import DecodeGraphRunner
from acorninfer_amd.models.qwen3 import Qwen3DecodeModel, random_state_dict
from model_utils import feed_prompt, new_cache, release

CFG = Qwen3Config.qwen3_0_6b().with_layers(2)
LENS = [11, 23, 47, 5]
STEPS = 6


@pytest.fixture(scope="module")
def model():
    sd = random_state_dict(CFG, seed=7, std=0.02, dtype=torch.bfloat16)
    return Qwen3DecodeModel.from_state_dict(CFG, sd, device="cuda")


def _prompts():
    g = torch.Generator().manual_seed(3)
    return [torch.randint(0, CFG.vocab_size, (n,), generator=g).tolist() for n in LENS]


def _schedule():
    """(active rows, fed ids) per step: 4 rows, then row 3 retires (B=3), then
    rows 1 and 2 only (bucket 2)."""
    g = torch.Generator().manual_seed(4)
    sched = []
    for t in range(STEPS):
        rows = [0, 1, 2, 3] if t < 2 else [0, 1, 2] if t < 4 else [1, 2]
        sched.append((rows, torch.randint(0, CFG.vocab_size, (len(rows),), generator=g).tolist()))
    return sched


def _run(model, mode):
    alloc, cache = new_cache(model, 64)
    views = [PagedCacheView(cache) for _ in LENS]
    for v, p in zip(views, _prompts()):
        feed_prompt(model, v, p)
    runner = None
    if mode != "eager":
        runner = DecodeGraphRunner(model, cache, alloc, max_model_len=256,
                                   capture=(mode == "graph"))
    out = []
    retired = False
    for rows, ids in _schedule():
        if len(rows) == 3 and not retired:      # row 3 retires: its blocks go back (LIFO reuse)
            release(alloc, [views[3]])
            retired = True
        vs = [views[r] for r in rows]
        if runner is None:
            logits = model.forward_decode(torch.tensor(ids, device="cuda")[:, None], vs)
            out.append((logits.argmax(1).tolist(), logits.cpu()))
        else:
            seqs = [SimpleNamespace(generated_ids=[i]) for i in ids]
            toks = runner.decode_batch(seqs, vs)
            out.append((toks, runner.last_logits[:len(rows)].float().cpu()))
    for v in views[:3]:
        assert all(v._lens[li] == v.seq_len for li in range(CFG.num_hidden_layers))
    release(alloc, views[:3])
    if runner is not None:
        assert alloc.num_live == 1          # the resident scratch block
        alloc.free(runner.scratch)
    alloc.assert_balanced()
    return out, [v.seq_len for v in views]


@pytest.mark.gpu
def test_graph_replay_bitwise_equals_uncaptured(model):
    g, lens_g = _run(model, "graph")
    u, lens_u = _run(model, "uncaptured")
    assert lens_g == lens_u
    for (tg, lg), (tu, lu) in zip(g, u):
        assert tg == tu
        assert torch.equal(lg, lu)


@pytest.mark.gpu
def test_graph_replay_matches_eager(model):
    g, _ = _run(model, "graph")
    e, _ = _run(model, "eager")
    for (tg, lg), (te, le) in zip(g, e):
        torch.testing.assert_close(lg, le, rtol=2e-2, atol=2e-2)
        top2 = le.topk(2, dim=1).values
        for r in range(len(tg)):
            if (top2[r, 0] - top2[r, 1]).item() >= 0.05:
                assert tg[r] == te[r]


@pytest.mark.gpu
def test_decode_loop_matches_decode_batch(model):
    prompts = _prompts()[:3]

    def setup():
        alloc, cache = new_cache(model, 64)
        views = [PagedCacheView(cache) for _ in prompts]
        firsts = [int(feed_prompt(model, v, p).argmax()) for v, p in zip(views, prompts)]
        return alloc, cache, views, firsts

    alloc, cache, views, firsts = setup()
    runner = DecodeGraphRunner(model, cache, alloc, max_model_len=256)
    log = runner.decode_loop(views, firsts, 5)          # [5, 3]
    alloc2, cache2, views2, firsts2 = setup()
    assert firsts2 == firsts
    runner2 = DecodeGraphRunner(model, cache2, alloc2, max_model_len=256)
    cur = firsts2
    for t in range(5):
        cur = runner2.decode_batch([SimpleNamespace(generated_ids=[i]) for i in cur], views2)
        assert log[t].tolist() == cur
    assert [v.seq_len for v in views] == [v.seq_len for v in views2]


@pytest.mark.gpu
def test_sampled_rows_inside_the_graph(model):
    """Rows with temperature > 0 are sampled inside the captured step (the
    reference falls back to eager for them): greedy rows take the argmax of
    the step's logits; sampled rows take the oracle's processed distribution
    and inverse-CDF draw for the runner's seeded uniform."""
    from acorninfer_amd.sampler import SamplingParams
    from oracle.sampler_ref import draw_ref, process_ref
    prompts = _prompts()[:3]
    alloc, cache = new_cache(model, 64)
    views = [PagedCacheView(cache) for _ in prompts]
    ids = [int(feed_prompt(model, v, p).argmax()) for v, p in zip(views, prompts)]
    runner = DecodeGraphRunner(model, cache, alloc, max_model_len=256, seed=5)
    rng = torch.Generator().manual_seed(5)
    sps = [SamplingParams(temperature=0.7, top_p=0.95, top_k=20), None,
           SamplingParams(temperature=1.0, top_p=0.9, top_k=50)]
    for step in range(4):
        seqs = [SimpleNamespace(generated_ids=[ids[i]], sampling=sps[i]) for i in range(3)]
        toks = runner.decode_batch(seqs, views)
        u = torch.rand(3, generator=rng)
        logits = runner.last_logits[:3].float().cpu()
        for i, sp in enumerate(sps):
            if sp is None:
                assert toks[i] == int(logits[i].argmax())
            else:
                want = process_ref(logits[i], sp.temperature, sp.top_k, sp.top_p)
                assert toks[i] == draw_ref(want, float(u[i]))[0]
        ids = toks
    # a greedy-only step after sampled ones resets the device sampling block
    seqs = [SimpleNamespace(generated_ids=[i]) for i in ids]
    toks = runner.decode_batch(seqs, views)
    assert toks == runner.last_logits[:3].float().argmax(1).tolist()
