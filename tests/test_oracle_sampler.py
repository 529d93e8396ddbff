"""Pins the sampler oracle (oracle/sampler_ref.py) on the CPU: the reference's
known answers (its tests/test_sampler.py:10-39) and HF's warpers, the
reference's own oracle (tests/test_sampler.py:41-67)."""
import pytest
import torch

from oracle.sampler_ref import draw_ref, process_ref

LOGITS = torch.tensor([2.0, 1.0, 0.5, -1.0])


def test_known_answers():
    assert torch.equal(process_ref(LOGITS, 2.0, 0, 1.0), LOGITS / 2.0)
    p = process_ref(LOGITS, 1.0, 2, 1.0)
    assert p[:2].isfinite().all() and p[2:].isinf().all()
    p = process_ref(LOGITS, 1.0, 0, 0.6)       # ascending tail mass 0.391 <= 0.4
    assert p[0].isfinite() and p[1:].isinf().all()
    tok, lp = draw_ref(process_ref(LOGITS, 1.0, 1, 1.0), 0.5)
    assert tok == 0 and lp == pytest.approx(0.0, abs=1e-9)
    with pytest.raises(ValueError, match="NaN/inf"):
        process_ref(torch.tensor([1.0, float("nan")]), 1.0, 0, 1.0)


def test_matches_hf_warpers():
    lp = pytest.importorskip("transformers.generation.logits_process")
    g = torch.Generator().manual_seed(7)
    for t, k, p in [(0.7, 20, 0.95), (1.0, 0, 0.9), (0.6, 50, 1.0), (1.3, 0, 0.5)]:
        warpers = [lp.TemperatureLogitsWarper(temperature=t)]
        if k:
            warpers.append(lp.TopKLogitsWarper(top_k=k, min_tokens_to_keep=1))
        if p < 1.0:
            warpers.append(lp.TopPLogitsWarper(top_p=p, min_tokens_to_keep=1))
        for _ in range(5):
            logits = torch.randn(151936, generator=g)
            hf = logits[None]
            for w in warpers:
                hf = w(torch.zeros(1, 1, dtype=torch.long), hf)
            assert torch.equal(process_ref(logits, t, k, p), hf[0])


def test_draw_is_inverse_cdf():
    x = torch.tensor([0.0, float("-inf"), 1.0, 0.5])
    probs = torch.softmax(x, 0)
    assert draw_ref(x, 0.0)[0] == 0
    assert draw_ref(x, float(probs[0]) + 1e-6)[0] == 2
    assert draw_ref(x, 0.999999)[0] == 3
