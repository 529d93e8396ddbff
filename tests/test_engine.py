"""Engine (acorninfer/engine/engine.py:30-378 contract: submit / step /
drop / has_pending / assert_balanced) on the GPU: continuous batching of
requests of different lengths through prefill (forward_extend) and the
graph-captured decode step, against the CPU oracle's greedy generation of
each request alone (oracle/qwen3_ref.py, fp32, so the ids must be equal).
Also with a block pool small enough to force preemption (recompute), with a
per-step prefill budget, and with sampled requests."""
import pytest
import torch

from acorninfer_amd.config import Qwen3Config
from acorninfer_amd.engine.engine import Engine
from acorninfer_amd.models.qwen3 import Qwen3DecodeModel, random_state_dict
from acorninfer_amd.sampler import SamplingParams
from oracle.qwen3_ref import Qwen3Ref, generate_greedy

SEED = 20261111
NO_EOS = frozenset({-1})
GREEDY = SamplingParams(temperature=0.0)


@pytest.fixture(scope="module")
def models():
    cfg = Qwen3Config.qwen3_0_6b().with_layers(2)
    sd = random_state_dict(cfg, seed=SEED, std=0.02, dtype=torch.float32)
    ref = Qwen3Ref(cfg, sd, torch.float32)
    model = Qwen3DecodeModel.from_state_dict(cfg, sd, dtype=torch.float32, device="cuda")
    return cfg, ref, model


def _requests(cfg, lens, new):
    g = torch.Generator().manual_seed(SEED + 1)
    return [(torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist(), m)
            for n, m in zip(lens, new)]


def _run(engine, reqs, sampling=GREEDY, max_steps=500):
    ids = [engine.submit(p, sampling, max_tokens=m, eos_ids=NO_EOS) for p, m in reqs]
    steps = 0
    while engine.has_pending():
        engine.step()
        steps += 1
        assert steps < max_steps
    out = [list(engine.seqs[i].generated_ids) for i in ids]
    for i in ids:
        assert engine.seqs[i].stop_reason == "length"
        engine.drop(i)
    engine.assert_balanced()
    return out


def _oracle(ref, reqs):
    return [generate_greedy(ref, p, m)[0] for p, m in reqs]


@pytest.mark.gpu
def test_continuous_batching_matches_oracle(models):
    cfg, ref, model = models
    reqs = _requests(cfg, [5, 37, 16, 23, 2], [9, 4, 12, 1, 7])
    print("\n[engine: 5 requests, max_running 3]", flush=True)
    got = _run(Engine(model, num_blocks=64, max_running=3, watermark_blocks=2,
                      max_model_len=128), reqs)
    assert got == _oracle(ref, reqs)


@pytest.mark.gpu
def test_preemption_recompute_matches_oracle(models):
    cfg, ref, model = models
    reqs = _requests(cfg, [15, 15, 15], [20, 20, 20])
    eng = Engine(model, num_blocks=6, max_running=3, watermark_blocks=0, max_model_len=64)
    seen_waiting = []
    ids = [eng.submit(p, GREEDY, max_tokens=m, eos_ids=NO_EOS) for p, m in reqs]
    steps = 0
    while eng.has_pending():
        eng.step()
        seen_waiting.append(len(eng.scheduler.waiting))
        steps += 1
        assert steps < 500
    assert max(seen_waiting[3:]) >= 1          # someone was preempted after admission
    got = [list(eng.seqs[i].generated_ids) for i in ids]
    eng.assert_balanced()
    assert got == _oracle(ref, reqs)


@pytest.mark.gpu
def test_chunked_prefill_budget_matches_oracle(models):
    cfg, ref, model = models
    reqs = _requests(cfg, [40, 9, 33], [5, 6, 4])
    got = _run(Engine(model, num_blocks=64, max_running=4, watermark_blocks=1,
                      chunked_budget=12, max_model_len=128), reqs)
    assert got == _oracle(ref, reqs)


@pytest.mark.gpu
def test_sampled_requests_finish_and_validate(models):
    cfg, _, model = models
    eng = Engine(model, num_blocks=64, max_running=4, watermark_blocks=1, max_model_len=128)
    with pytest.raises(ValueError):
        eng.submit([], GREEDY, max_tokens=4)
    with pytest.raises(ValueError):
        eng.submit([1, 2], GREEDY, max_tokens=0)
    reqs = _requests(cfg, [7, 12], [6, 9])
    out = _run(eng, reqs, sampling=SamplingParams(temperature=0.7, top_k=20, top_p=0.9))
    assert [len(o) for o in out] == [6, 9]
    assert all(0 <= t < cfg.vocab_size for o in out for t in o)
