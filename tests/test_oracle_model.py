"""Pins the CPU model oracle (oracle/qwen3_ref.py) before it is trusted.

- Against HF transformers' Qwen3ForCausalLM, the reference's own golden
  oracle (its tests/test_golden_m0.py compares to HF), on identical weights:
  full-sequence logits agree to fp32 rounding.
- Prefill of a prompt then one decode step equals the full-sequence forward
  at the last position (the reference's invariant,
  tests/test_forward_decode.py:32-48 and tests/test_paged_forward.py).
- A planted mistake in the oracle (a dropped qk-norm) is caught by the HF pin.
"""
import pytest
import torch

from acorninfer_amd.config import Qwen3Config
from acorninfer_amd.models.qwen3 import random_state_dict
from oracle.qwen3_ref import Qwen3Ref, generate_greedy

CFG = Qwen3Config.tiny()


def _hf_model(cfg, sd):
    transformers = pytest.importorskip("transformers")
    hc = transformers.Qwen3Config(
        vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
        intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
        num_attention_heads=cfg.num_attention_heads, num_key_value_heads=cfg.num_key_value_heads,
        head_dim=cfg.head_dim, rms_norm_eps=cfg.rms_norm_eps, rope_theta=cfg.rope_theta,
        tie_word_embeddings=False, attention_bias=False, max_position_embeddings=4096)
    m = transformers.Qwen3ForCausalLM(hc).float().eval()
    hsd = {("lm_head.weight" if k == "lm_head.weight" else "model." + k): v.float()
           for k, v in sd.items()}
    missing, unexpected = m.load_state_dict(hsd, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return m


def _sd(seed=0, std=0.2):
    # a larger std than 0.02 makes attention non-uniform, so mistakes show
    return random_state_dict(CFG, seed=seed, std=std, dtype=torch.float32)


def test_oracle_matches_hf_qwen3_fp32():
    sd = _sd()
    hf = _hf_model(CFG, sd)
    ref = Qwen3Ref(CFG, sd, torch.float32)
    ids = torch.randint(0, CFG.vocab_size, (2, 11), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        want = hf(ids).logits.float()
    got = ref.forward(ids)
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-4)


def test_planted_mistake_is_caught_by_hf_pin():
    sd = _sd()
    hf = _hf_model(CFG, sd)
    ref = Qwen3Ref(CFG, sd, torch.float32)
    for i in range(CFG.num_hidden_layers):   # plant: a q_norm weight the model does not hold
        ref.w[f"layers.{i}.self_attn.q_norm.weight"] = torch.full((CFG.head_dim,), 3.0)
    ids = torch.randint(0, CFG.vocab_size, (1, 9), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        want = hf(ids).logits.float()
    assert not torch.allclose(ref.forward(ids), want, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prefill_then_decode_equals_full_forward(dtype):
    sd = _sd(seed=3)
    ref = Qwen3Ref(CFG, sd, dtype)
    ids = torch.randint(0, CFG.vocab_size, (1, 13), generator=torch.Generator().manual_seed(4))
    full = ref.forward(ids)[0]
    cache = ref.new_cache()
    ref.forward(ids[:, :7], cache)
    steps = [ref.forward(ids[:, t:t + 1], cache)[0, 0] for t in range(7, 13)]
    tol = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=3e-2, atol=3e-2)
    torch.testing.assert_close(torch.stack(steps), full[7:13], **tol)


def test_generate_greedy_forced_stream_and_eos():
    sd = _sd(seed=5)
    ref = Qwen3Ref(CFG, sd, torch.float32)
    prompt = [3, 1, 4, 1, 5]
    ids, logits = generate_greedy(ref, prompt, 8)
    assert len(ids) == 8 and all(int(l.argmax()) == t for l, t in zip(logits, ids))
    forced = [7] * 8
    ids2, _ = generate_greedy(ref, prompt, 8, forced=forced)
    assert ids2 == forced
    # the chosen EOS is appended, then generation stops (generate.py:104-105)
    ids3, _ = generate_greedy(ref, prompt, 8, eos_ids=frozenset({ids[2]}))
    assert ids3 == ids[:3]


def test_decode_ragged_equals_per_sequence_forward():
    """The batched ragged decode step equals one forward([[id]], cache) per
    sequence (different cache lengths, one empty), and grows each cache by one
    token; a planted per-row position mistake (every row at position 0) is
    caught."""
    sd = _sd(seed=6)
    ref = Qwen3Ref(CFG, sd, torch.float32)
    g = torch.Generator().manual_seed(7)
    hist = [5, 0, 17, 2]
    caches, solo = [], []
    for n in hist:
        c, s = ref.new_cache(), ref.new_cache()
        if n:
            ids = torch.randint(0, CFG.vocab_size, (1, n), generator=g)
            ref.forward(ids, c)
            ref.forward(ids, s)
        caches.append(c)
        solo.append(s)
    for step in range(3):
        ids = torch.randint(0, CFG.vocab_size, (len(hist),), generator=g).tolist()
        got = ref.decode_ragged(ids, caches)
        want = torch.stack([ref.forward(torch.tensor([[t]]), s)[0, -1] for t, s in zip(ids, solo)])
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    assert [c[0][0].shape[2] for c in caches] == [n + 3 for n in hist]
    # planted mistake: the positions of every row forced to 0
    bad = Qwen3Ref(CFG, sd, torch.float32)
    bad._rope = lambda positions, f=bad._rope: f(torch.zeros_like(positions))
    c2 = [[[x.clone() for x in layer] for layer in c] for c in caches]
    ids = [1, 2, 3, 4]
    assert not torch.allclose(bad.decode_ragged(ids, c2), ref.decode_ragged(ids, caches),
                              rtol=1e-3, atol=1e-3)


def test_weight_dtype_keeps_projection_weights_and_rounds_activations():
    """Qwen3Ref(dtype=bf16, weight_dtype=fp32): the projection and lm_head
    weights stay fp32 (a dequantised int4 / int8 weight stays exact), every
    activation is rounded to bf16 as in the bf16 path. With weight_dtype ==
    dtype it is the plain oracle bit for bit; with fp32 copies of bf16
    weights it gives the bf16 path's logits up to fp32 accumulation order;
    with weights that bf16 cannot hold it differs from the bf16 path (the
    weights were not rounded)."""
    sd = {k: v.to(torch.bfloat16) for k, v in _sd(seed=9, std=0.05).items()}
    ids = torch.randint(0, CFG.vocab_size, (1, 11), generator=torch.Generator().manual_seed(10))
    plain = Qwen3Ref(CFG, sd, torch.bfloat16)
    same = Qwen3Ref(CFG, sd, torch.bfloat16, weight_dtype=torch.bfloat16)
    assert torch.equal(plain.forward(ids), same.forward(ids))
    wide = Qwen3Ref(CFG, sd, torch.bfloat16, weight_dtype=torch.float32)
    assert wide.w["lm_head.weight"].dtype == torch.float32
    assert wide.w["layers.0.mlp.down_proj.weight"].dtype == torch.float32
    assert wide.w["layers.0.input_layernorm.weight"].dtype == torch.bfloat16
    assert wide.w["embed_tokens.weight"].dtype == torch.bfloat16
    a, b = plain.forward(ids), wide.forward(ids)
    assert b.dtype == torch.float32
    torch.testing.assert_close(b, a, rtol=2e-2, atol=2e-2)
    # weights off the bf16 grid: the fp32-weight oracle keeps them, so its
    # logits move away from the all-bf16 oracle's
    off = {k: (v.float() * (1 + 2 ** -10) if k.endswith("_proj.weight") else v)
           for k, v in sd.items()}
    assert not torch.equal(Qwen3Ref(CFG, off, torch.bfloat16, weight_dtype=torch.float32)
                           .forward(ids), b)
