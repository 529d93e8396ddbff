"""The HIP decode step (Qwen3DecodeModel) against the CPU oracle of the
reference's SDPA path (oracle/qwen3_ref.py, itself pinned against HF Qwen3).

- fp32, BASELINE config 1 (Qwen3-0.6B shape, N(0, 0.02) weights, 32 seeded
  prompt ids, 32 greedy tokens, page 16): the greedy token ids are identical
  and every step's logits agree to fp32 reduction-order drift.
- bf16 / W8A16 / W4A16: forced-token streams (the reference's protocol,
  tests/test_forward_decode.py:86-140: both sides are fed the same ids, so a
  bf16 near-tie cannot make them compare different contexts); logits within
  a norm-relative tolerance, argmax equal wherever the oracle's top-2 margin
  is at least MARGIN (tests/test_quant_wiring.py:297-343's margin gate).
- The GPU side consumes the prompt through the decode step itself, one token
  at a time (equal to the reference's prefill: causal attention over the
  cache).
"""
import pytest
import torch

from acorninfer_amd.cache.pager import PagedCacheView
from acorninfer_amd.config import Qwen3Config
from acorninfer_amd.models.qwen3 import Qwen3DecodeModel, random_state_dict
from model_utils import feed_prompt, new_cache, release
from oracle.qwen3_ref import Qwen3Ref, generate_greedy

SEED = 20261027
MARGIN = 0.05


def _prompt(n, vocab, seed=SEED):
    return torch.randint(0, vocab, (n,), generator=torch.Generator().manual_seed(seed)).tolist()


def _gpu_stream(model, prompt, feed, n):
    """GPU logits for n steps; feed[t] is the id fed after step t (None = greedy)."""
    alloc, cache = new_cache(model, -(-(len(prompt) + n + 1) // 16) + 2)
    view = PagedCacheView(cache)
    logits = feed_prompt(model, view, prompt)
    out_ids, out_logits = [], []
    for t in range(n):
        out_logits.append(logits.cpu())
        nxt = int(logits.argmax()) if feed is None else int(feed[t])
        out_ids.append(nxt)
        logits = model.forward_decode(torch.tensor([[nxt]], device=model.device), [view])[0]
    release(alloc, [view])
    alloc.assert_balanced()
    return out_ids, out_logits


@pytest.mark.gpu
def test_config1_fp32_greedy_ids_identical_to_oracle():
    cfg = Qwen3Config.qwen3_0_6b()
    sd = random_state_dict(cfg, seed=SEED, std=0.02, dtype=torch.float32)
    prompt = _prompt(32, cfg.vocab_size)
    print(f"\n[config1 fp32: 28 layers, prompt 32, 32 new]", flush=True)
    ref = Qwen3Ref(cfg, sd, torch.float32)
    want_ids, want_logits = generate_greedy(ref, prompt, 32)
    model = Qwen3DecodeModel.from_state_dict(cfg, sd, dtype=torch.float32, device="cuda")
    del sd
    got_ids, got_logits = _gpu_stream(model, prompt, None, 32)
    worst = max((g - w).abs().max().item() for g, w in zip(got_logits, want_logits))
    print(f"[config1 fp32 max|dlogit| = {worst:.3g}; ids {got_ids[:8]}...]")
    assert got_ids == want_ids
    for g, w in zip(got_logits, want_logits):
        torch.testing.assert_close(g, w, rtol=1e-3, atol=1e-3)


def _forced_compare(cfg, weight_format, n_steps, rel_tol, seed=SEED, std=0.02):
    sd = random_state_dict(cfg, seed=seed, std=std, dtype=torch.bfloat16)
    prompt = _prompt(9, cfg.vocab_size, seed + 1)
    model = Qwen3DecodeModel.from_state_dict(cfg, sd, weight_format=weight_format,
                                             device="cuda")
    if weight_format == "bf16":
        ref = Qwen3Ref(cfg, sd, torch.bfloat16)
    else:
        # the oracle runs the dequantised weights of the same quantised model
        ref_sd = dict(sd)
        for i, L in enumerate(model.layers):
            p = f"layers.{i}."
            qkv, gu = L.qkv.dense().cpu(), L.gate_up.dense().cpu()
            nq = cfg.num_attention_heads * cfg.head_dim
            nkv = cfg.num_key_value_heads * cfg.head_dim
            ref_sd[p + "self_attn.q_proj.weight"] = qkv[:nq]
            ref_sd[p + "self_attn.k_proj.weight"] = qkv[nq:nq + nkv]
            ref_sd[p + "self_attn.v_proj.weight"] = qkv[nq + nkv:]
            ref_sd[p + "self_attn.o_proj.weight"] = L.o.dense().cpu()
            ref_sd[p + "mlp.gate_proj.weight"] = gu[:cfg.intermediate_size]
            ref_sd[p + "mlp.up_proj.weight"] = gu[cfg.intermediate_size:]
            ref_sd[p + "mlp.down_proj.weight"] = L.down.dense().cpu()
        ref_sd["lm_head.weight"] = model.lm_head.dense().cpu()
        ref = Qwen3Ref(cfg, ref_sd, torch.float32)
    feed = _prompt(n_steps, cfg.vocab_size, seed + 2)
    _, want = generate_greedy(ref, prompt, n_steps, forced=feed)
    _, got = _gpu_stream(model, prompt, feed, n_steps)
    gated = flips = 0
    worst = 0.0
    for g, w in zip(got, want):
        rel = ((g.double() - w.double()).norm() / w.double().norm()).item()
        worst = max(worst, rel)
        top2 = w.topk(2).values
        if (top2[0] - top2[1]).item() >= MARGIN:
            gated += 1
            flips += int(g.argmax() != w.argmax())
    print(f"\n[{weight_format} forced stream: worst rel err {worst:.3g}, "
          f"margin-gated steps {gated}/{n_steps}, flips {flips}]")
    assert worst < rel_tol
    assert flips == 0


@pytest.mark.gpu
@pytest.mark.parametrize("weight_format,rel_tol", [("bf16", 3e-2), ("w8a16", 3e-2),
                                                    ("w4a16", 3e-2)])
def test_forced_stream_matches_oracle(weight_format, rel_tol):
    """Qwen3-0.6B shape with 4 layers (keeps the CPU oracle to seconds)."""
    cfg = Qwen3Config.qwen3_0_6b().with_layers(4)
    _forced_compare(cfg, weight_format, 12, rel_tol)


@pytest.mark.gpu
def test_tiny_config_bf16_forced_stream():
    _forced_compare(Qwen3Config.tiny(), "bf16", 8, 3e-2, std=0.2)
