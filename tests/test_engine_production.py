"""The Engine (acorninfer/engine/engine.py:167-262) on the production kernels:
the Qwen3-8B layer shapes (hidden 4096, 32/8 heads, D 128, intermediate
12288, vocab 151936) cut to 2 layers, in bf16 and in W4A16, so every step
runs the MFMA GEMMs (bf16 streaming, int4 direct kernel with the fused
SwiGLU), the fused K3 + qkv epilogue, the batched prefill and the in-graph
sampler. As the reference's own Engine tests (tests/test_engine.py:152-230):

- graph vs eager: the same submits through an Engine that replays captured
  decode steps and one that launches them uncaptured give bitwise the same
  token streams, greedy and sampled rows mixed in one batch;
- EOS retirement shrinks the batch across buckets (8 -> 4 -> 2): each trap
  id comes from an earlier run with the same batch history up to it, the
  graph and eager runs with them agree bitwise and stop exactly where the
  traps say;
- C=8 requests of 512-token prompts, greedy: the token streams against the
  oracle (oracle/qwen3_ref.py with bf16 activations; for W4A16 the
  dequantised weights kept exact in fp32) fed the same streams: wherever the
  oracle's top-2 margin is at least the gate, the engine's token is the
  oracle's argmax (the reference's margin gate, tests/test_quant_wiring.py:
  297-343). The reference's 0.05 is set for its mini model, whose logits are
  small; at this shape the top logit sits near 4-8, where one bf16 step is
  1/32, and both sides round their logits to bf16: the final rounding alone
  moves a top-2 margin by up to 2 steps (half a step on each of two logits, on
  each side). The gate is therefore max(MARGIN, 3 bf16 steps of the top
  logit): the rounding plus one step for the bf16 activations upstream.
"""
import math

import pytest
import torch

from acorninfer_amd.config import Qwen3Config
from acorninfer_amd.engine.engine import Engine
from acorninfer_amd.models.qwen3 import Qwen3DecodeModel, random_state_dict
from acorninfer_amd.sampler import SamplingParams

CFG8 = Qwen3Config.qwen3_8b().with_layers(2)
SEED = 20261203
MARGIN = 0.05
GATE_ULPS = 3


def _bf16_step(v: float) -> float:
    """Spacing of bf16 values at |v| (8 significant bits)."""
    return 2.0 ** (math.floor(math.log2(abs(v))) - 7) if v else 2.0 ** -133


def _gate(top1: float) -> float:
    return max(MARGIN, GATE_ULPS * _bf16_step(top1))
GREEDY = SamplingParams(temperature=0.0)
SAMPLED = SamplingParams(temperature=0.6, top_k=20, top_p=0.95)
NO_EOS = frozenset({-1})


def _ids(n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, CFG8.vocab_size, (n,), generator=g).tolist()


@pytest.fixture(scope="module")
def sd8():
    print("\n[engine production: drawing the 2-layer Qwen3-8B-shaped weights]", flush=True)
    return random_state_dict(CFG8, seed=SEED, std=0.02, dtype=torch.bfloat16)


@pytest.fixture(scope="module")
def models(sd8):
    out = {}
    for fmt in ("bf16", "w4a16"):
        m = Qwen3DecodeModel.from_state_dict(CFG8, sd8, weight_format=fmt, device="cuda")
        m.tune(8)                       # the bench's load-time tilings at bucket 8
        out[fmt] = m
    return out


def _engine(model, capture, max_model_len=640, num_blocks=400):
    return Engine(model, num_blocks=num_blocks, max_running=8, watermark_blocks=1,
                  max_model_len=max_model_len, capture=capture, seed=SEED)


def _run(engine, reqs):
    """reqs: (prompt, sampling, max_tokens, eos_ids) -> each request's token
    stream; checks retirement and the allocator balance."""
    ids = [engine.submit(p, sp, max_tokens=m, eos_ids=e) for p, sp, m, e in reqs]
    steps = 0
    while engine.has_pending():
        engine.step()
        steps += 1
        assert steps < 500
    out = [list(engine.seqs[i].generated_ids) for i in ids]
    for i in ids:
        engine.drop(i)
    engine.assert_balanced()
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["bf16", "w4a16"])
def test_engine_graph_equals_eager_mixed_sampling(models, fmt):
    model = models[fmt]
    lens = [33, 70, 100, 17, 64, 128, 5, 90]
    reqs = [(_ids(n, SEED + i), SAMPLED if i in (2, 5) else GREEDY, 12, NO_EOS)
            for i, n in enumerate(lens)]
    streams = {}
    for capture in (False, True):
        eng = _engine(model, capture)
        streams[capture] = _run(eng, reqs)
        captured = [bk for bk, st in eng.graph_runner.states.items() if st.graph is not None]
        assert bool(captured) == capture and (8 in eng.graph_runner.states)
        print(f"\n[{fmt} engine capture={capture}: buckets {sorted(eng.graph_runner.states)}]",
              flush=True)
    assert streams[True] == streams[False]
    assert all(len(s) == 12 for s in streams[True])
    assert all(0 <= t < CFG8.vocab_size for s in streams[True] for t in s)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["bf16", "w4a16"])
def test_engine_eos_shrinks_batch_across_buckets(models, fmt):
    """The trap ids are each taken from a run with the same batch history as
    the run they stop (the reference's two-phase traps,
    tests/test_engine.py:185-226): a row's tokens are the same bits only
    while the batch, and so the bucket's tilings and split-K summation
    order, is the same."""
    model = models[fmt]
    prompts = [_ids(n, SEED + 40 + i) for i, n in enumerate([20, 41, 9, 63, 30, 52, 11, 77])]

    def reqs(traps):
        return [(p, GREEDY, 10, frozenset({traps[i]}) if i in traps else NO_EOS)
                for i, p in enumerate(prompts)]

    # requests 0-3 stop on their first decode token (batch 8 -> 4), taken
    # from the untrapped run (the first decode step runs all 8 rows in both)
    full = _run(_engine(model, False), reqs({}))
    traps = {i: full[i][1] for i in range(4)}
    # 4-5 on their third (4 -> 2), taken from a run with 0-3 trapped
    mid = _run(_engine(model, False), reqs(traps))
    assert [s[:2] for s in mid[:4]] == [s[:2] for s in full[:4]]
    traps.update({i: mid[i][3] for i in (4, 5)})
    want_len = [mid[i].index(traps[i]) + 1 if i in traps else 10 for i in range(8)]
    runs = {}
    for capture in (False, True):
        eng = _engine(model, capture)
        runs[capture] = _run(eng, reqs(traps))
        if capture:
            used = sorted(eng.graph_runner.states)
            assert {8, 4, 2} <= set(used), used
            assert all(eng.graph_runner.states[b].graph is not None for b in (8, 4, 2))
    assert runs[True] == runs[False]
    assert [len(s) for s in runs[True]] == want_len
    assert [s[:n] for s, n in zip(mid[:6], want_len[:6])] == runs[True][:6]
    print(f"\n[{fmt} engine EOS: lengths {want_len}, buckets 8 -> 4 -> 2]", flush=True)


def _oracle_for(fmt, model, sd8):
    from oracle.qwen3_ref import Qwen3Ref
    if fmt == "bf16":
        return Qwen3Ref(CFG8, sd8, torch.bfloat16)
    cfg = model.cfg
    sd = dict(sd8)
    nq = cfg.num_attention_heads * cfg.head_dim
    nkv = cfg.num_key_value_heads * cfg.head_dim
    for i, L in enumerate(model.layers):
        p = f"layers.{i}."
        qkv, gu = L.qkv.dense().cpu(), L.gate_up.dense().cpu()
        sd[p + "self_attn.q_proj.weight"] = qkv[:nq]
        sd[p + "self_attn.k_proj.weight"] = qkv[nq:nq + nkv]
        sd[p + "self_attn.v_proj.weight"] = qkv[nq + nkv:]
        sd[p + "self_attn.o_proj.weight"] = L.o.dense().cpu()
        sd[p + "mlp.gate_proj.weight"] = gu[:cfg.intermediate_size]
        sd[p + "mlp.up_proj.weight"] = gu[cfg.intermediate_size:]
        sd[p + "mlp.down_proj.weight"] = L.down.dense().cpu()
    sd["lm_head.weight"] = model.lm_head.dense().cpu()
    # the GPU's numeric domain: activations rounded to bf16 where the bf16
    # path rounds them, the dequantised weights exact
    return Qwen3Ref(CFG8, sd, torch.bfloat16, weight_dtype=torch.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["bf16", "w4a16"])
def test_engine_c8_prompts_512_greedy_against_oracle(models, sd8, fmt):
    model = models[fmt]
    C, L, new = 8, 512, 6
    prompts = [_ids(L, SEED + 100 + i) for i in range(C)]
    got = _run(_engine(model, True), [(p, GREEDY, new, NO_EOS) for p in prompts])
    print(f"\n[{fmt} engine C={C} x {L}: oracle forced streams]", flush=True)
    ref = _oracle_for(fmt, model, sd8)
    caches = [ref.new_cache() for _ in range(C)]
    logits = torch.stack([ref.forward(torch.tensor([p]), c, num_logits_to_keep=1)[0, -1]
                          for p, c in zip(prompts, caches)])
    gated = flips = 0
    for t in range(new):
        for b in range(C):
            w = logits[b].double()
            top2 = w.topk(2).values
            top1, margin = top2[0].item(), (top2[0] - top2[1]).item()
            if margin >= _gate(top1):
                gated += 1
                if got[b][t] != int(w.argmax()):
                    flips += 1
                    print(f"[flip: step {t} row {b}: engine {got[b][t]} oracle "
                          f"{int(w.argmax())} top1 {top1:.3f} margin {margin:.3f}]")
            elif got[b][t] != int(w.argmax()):
                print(f"[ungated disagreement: step {t} row {b}: top1 {top1:.3f} "
                      f"margin {margin:.3f} gate {_gate(top1):.3f}]")
        if t + 1 < new:
            logits = ref.decode_ragged([s[t] for s in got], caches)
    print(f"[{fmt}: margin-gated tokens {gated}/{C * new}, flips {flips}]", flush=True)
    assert gated >= C * new // 2
    assert flips == 0
