"""BASELINE configurations 4 and 5 on the production kernels, at the
Qwen3-8B layer shapes (hidden 4096, 32/8 heads, D 128, intermediate 12288,
vocab 151936) cut to 2 layers so that the CPU oracle stays cheap.

The bf16 model is compared with the oracle in bf16 (the reference's own
precision: each op rounded where its torch path rounds), the W4A16 model
with the oracle in fp32 on the dequantised weights. Everything runs through
the same code as the benchmark: prefill through
`forward_prefill_batch` / `forward_extend`, decode through
`DecodeGraphRunner` (hipGraph-captured step, bf16 MFMA GEMMs, the fused K3,
the in-graph sampler). Checks, each against oracle/qwen3_ref.py
(pinned against HF Qwen3) on the same seeded weights and ids:

- configuration 4 (bf16): C=8 real prompts of 512 ids; prefill logits and
  the KV pages the prefill wrote; then forced-token decode steps in the
  graph at bucket 8 with the load-time tuned tilings;
- buckets 1, 4, 16, 32, 64 over ragged 512-token histories: logits against
  the oracle, graph replay bitwise equal to the same runner uncaptured, and
  the greedy tokens equal to the first maximum of the step's logits;
- configuration 5 (W4A16, the oracle runs the dequantised weights): prompt
  lengths from U[1024, 8192] (table width 516 pages, the 64-split cap,
  multi-page splits), one whole real prompt plus real 128-token chunks on
  top of synthetic histories, then sampled decode (T 0.6, top-k 20,
  top-p 0.95) at C=8 and C=64: every sampled token equals the oracle
  sampler's processing and inverse-CDF draw on that step's logits, and the
  logits match the oracle fed the same tokens.

Logits: norm-relative error below REL_TOL and, wherever the oracle's top-2
margin is at least MARGIN, the oracle's argmax is a maximum of the GPU's
logits (bf16 logits tie; argmax then takes the first) (the reference's margin gate,
tests/test_quant_wiring.py:297-343; forced streams as in
tests/test_forward_decode.py:86-140).
"""
from types import SimpleNamespace

import pytest
import torch

from acorninfer_amd.cache.pager import BlockAllocator, PagedCacheView, PagedKVCache
from acorninfer_amd.config import Qwen3Config
from acorninfer_amd.engine.graph_runner import DecodeGraphRunner
from acorninfer_amd.models.qwen3 import Qwen3DecodeModel, random_state_dict

CFG8 = Qwen3Config.qwen3_8b().with_layers(2)
SEED = 20261202
REL_TOL = 3e-2
MARGIN = 0.05
PAGE = 16


def _ids(n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, CFG8.vocab_size, (n,), generator=g).tolist()


def _check_rows(got, want, what):
    """got/want fp32 [B, vocab]: per-row norm-relative error and the margin gate."""
    worst, gated, flips = 0.0, 0, 0
    for g, w in zip(got.double(), want.double()):
        worst = max(worst, ((g - w).norm() / w.norm()).item())
        top2 = w.topk(2).values
        if (top2[0] - top2[1]).item() >= MARGIN:
            gated += 1
            # bf16 logits tie often (spacing 1/32 near 5): the oracle's choice
            # must be a maximum of ours, which argmax may resolve to a lower index
            if g[w.argmax()] < g.max():
                flips += 1
                print(f"[{what}: flip: oracle top-2 {w.topk(2)}, got at those "
                      f"{g[w.topk(2).indices]}, got top-2 {g.topk(2)}]", flush=True)
    print(f"[{what}: worst rel err {worst:.3g}, margin-gated rows {gated}/{len(got)}, "
          f"flips {flips}]", flush=True)
    assert worst < REL_TOL, f"{what}: rel err {worst}"
    assert flips == 0, f"{what}: {flips} argmax flips above the margin"


def _oracle(sd, dtype=torch.float32):
    from oracle.qwen3_ref import Qwen3Ref
    return Qwen3Ref(CFG8, sd, dtype)


def _dequant_sd(model, sd):
    """The reference-named state dict of a quantised model's dequantised weights."""
    cfg = model.cfg
    out = dict(sd)
    nq = cfg.num_attention_heads * cfg.head_dim
    nkv = cfg.num_key_value_heads * cfg.head_dim
    for i, L in enumerate(model.layers):
        p = f"layers.{i}."
        qkv, gu = L.qkv.dense().cpu(), L.gate_up.dense().cpu()
        out[p + "self_attn.q_proj.weight"] = qkv[:nq]
        out[p + "self_attn.k_proj.weight"] = qkv[nq:nq + nkv]
        out[p + "self_attn.v_proj.weight"] = qkv[nq + nkv:]
        out[p + "self_attn.o_proj.weight"] = L.o.dense().cpu()
        out[p + "mlp.gate_proj.weight"] = gu[:cfg.intermediate_size]
        out[p + "mlp.up_proj.weight"] = gu[cfg.intermediate_size:]
        out[p + "mlp.down_proj.weight"] = L.down.dense().cpu()
    out["lm_head.weight"] = model.lm_head.dense().cpu()
    return out


@pytest.fixture(scope="module")
def sd8():
    print("\n[config45: drawing the 2-layer Qwen3-8B-shaped weights]", flush=True)
    return random_state_dict(CFG8, seed=SEED, std=0.02, dtype=torch.bfloat16)


@pytest.fixture(scope="module")
def bf16_model(sd8):
    return Qwen3DecodeModel.from_state_dict(CFG8, sd8, device="cuda")


@pytest.fixture(scope="module")
def bf16_ref(sd8):
    # the reference's bf16 path: the same weights, every op rounded to bf16
    return _oracle(sd8, torch.bfloat16)


class _Caches:
    """GPU paged caches (any number of identical copies, each with its own
    allocator) and oracle caches holding the same per-sequence history."""

    def __init__(self, model, lens, copies=1, seed=SEED, spare_tokens=64,
                 ref_dtype=torch.bfloat16, final_lens=None):
        final_lens = lens if final_lens is None else final_lens
        blocks = sum(-(-(n + spare_tokens) // PAGE) for n in final_lens) + 4
        self.pairs = []
        for _ in range(copies):
            alloc = BlockAllocator(blocks)
            cache = PagedKVCache(CFG8.num_hidden_layers, CFG8.num_key_value_heads,
                                 CFG8.head_dim, PAGE, alloc, model.device, model.dtype)
            self.pairs.append((alloc, cache, [PagedCacheView(cache) for _ in lens]))
        self.ref = [[[None, None] for _ in range(CFG8.num_hidden_layers)] for _ in lens]
        # synthetic post-RoPE keys and values ~ N(0, 1), drawn on the GPU
        g = torch.Generator(device=model.device).manual_seed(seed)
        shape_kv = (CFG8.num_key_value_heads, CFG8.head_dim)
        for b, n in enumerate(lens):
            if n == 0:
                continue
            for li in range(CFG8.num_hidden_layers):
                k = torch.randn(1, shape_kv[0], n, shape_kv[1], generator=g,
                                device=model.device).to(model.dtype)
                v = torch.randn(1, shape_kv[0], n, shape_kv[1], generator=g,
                                device=model.device).to(model.dtype)
                for _, _, views in self.pairs:
                    views[b].write(li, k, v)
                self.ref[b][li] = [k.cpu().to(ref_dtype), v.cpu().to(ref_dtype)]

    def views(self, i=0):
        return self.pairs[i][2]


def _seqs(ids, sampling=None):
    return [SimpleNamespace(generated_ids=[int(i)], sampling=sampling) for i in ids]


# --------------------------------------------------------------- configuration 4 --

@pytest.mark.gpu
def test_config4_bf16_prefill512_then_graph_decode_c8(bf16_model, bf16_ref):
    model, ref = bf16_model, bf16_ref
    C, L, steps = 8, 512, 4
    prompts = [_ids(L, SEED + 10 + i) for i in range(C)]
    caches = _Caches(model, [0] * C, spare_tokens=L + 64)
    alloc, cache, views = caches.pairs[0]
    print(f"\n[config4 bf16 C={C}: prefill {C}x{L} on the GPU]", flush=True)
    got = model.forward_prefill_batch(torch.tensor(prompts, device="cuda"), views,
                                      real_lens=[L] * C).cpu()
    print("[config4: oracle prefill]", flush=True)
    want = torch.stack([ref.forward(torch.tensor([p]), c, num_logits_to_keep=1)[0, -1]
                        for p, c in zip(prompts, caches.ref)])
    _check_rows(got, want, "config4 prefill logits")
    # the KV pages the prefill wrote hold the oracle's post-RoPE k and its v
    for b in (0, C - 1):
        for li in range(CFG8.num_hidden_layers):
            for j, pages in enumerate((cache.k_pages, cache.v_pages)):
                g_kv = views[b]._gather(li, pages).float().cpu()
                w_kv = caches.ref[b][li][j]
                rel = ((g_kv - w_kv).norm() / w_kv.norm()).item()
                assert rel < REL_TOL, f"prefill KV seq {b} layer {li} {'kv'[j]}: {rel}"
    # graph decode at bucket 8 with tuned tilings, forced ids
    model.tune(8)
    runner = DecodeGraphRunner(model, cache, alloc, max_model_len=L + 64)
    for t in range(steps):
        feed = _ids(C, SEED + 100 + t)
        toks = runner.decode_batch(_seqs(feed), views)
        g_logits = runner.last_logits[:C].float().cpu()
        assert toks == g_logits.argmax(1).tolist()
        _check_rows(g_logits, ref.decode_ragged(feed, caches.ref), f"config4 C=8 step {t}")


@pytest.mark.gpu
@pytest.mark.parametrize("C", [1, 4, 16, 32, 64])
def test_config4_bf16_buckets_graph_equals_uncaptured_and_oracle(bf16_model, bf16_ref, C):
    model, ref = bf16_model, bf16_ref
    g = torch.Generator().manual_seed(SEED + C)
    lens = torch.randint(448, 577, (C,), generator=g).tolist()
    caches = _Caches(model, lens, copies=2, seed=SEED + C)
    print(f"\n[config4 bf16 bucket {C}: histories {min(lens)}..{max(lens)}]", flush=True)
    runners = [DecodeGraphRunner(model, cache, alloc, max_model_len=640, capture=(i == 0))
               for i, (alloc, cache, _) in enumerate(caches.pairs)]
    for t in range(3):
        feed = _ids(C, SEED + 200 + 7 * C + t)
        toks, logits = [], []
        for r, (_, _, views) in zip(runners, caches.pairs):
            toks.append(r.decode_batch(_seqs(feed), views))
            logits.append(r.last_logits[:C].clone())
        assert toks[0] == toks[1]
        assert torch.equal(logits[0], logits[1]), f"bucket {C} step {t}: replay != uncaptured"
        g_logits = logits[0].float().cpu()
        assert toks[0] == g_logits.argmax(1).tolist()
        _check_rows(g_logits, ref.decode_ragged(feed, caches.ref), f"bucket {C} step {t}")
    for alloc, cache, views in caches.pairs:
        assert all(v.seq_len == n + 3 for v, n in zip(views, lens))


# --------------------------------------------------------------- configuration 5 --

@pytest.fixture(scope="module")
def w4_pair(sd8):
    model = Qwen3DecodeModel.from_state_dict(CFG8, sd8, weight_format="w4a16", device="cuda")
    return model, _oracle(_dequant_sd(model, sd8))


def _sampled_steps(model, ref, runner, caches, views, C, steps, seed, what):
    from acorninfer_amd.sampler import SamplingParams
    from oracle.sampler_ref import draw_ref, process_ref
    sp = SamplingParams(temperature=0.6, top_p=0.95, top_k=20)
    rng = torch.Generator().manual_seed(seed)       # the runner's uniform stream
    feed = _ids(C, seed + 1)
    for t in range(steps):
        toks = runner.decode_batch(_seqs(feed, sp), views)
        u = torch.rand(C, generator=rng)
        g_logits = runner.last_logits[:C].float().cpu()
        for i in range(C):
            want = process_ref(g_logits[i], sp.temperature, sp.top_k, sp.top_p)
            assert toks[i] == draw_ref(want, float(u[i]))[0], f"{what} step {t} row {i}"
        _check_rows(g_logits, ref.decode_ragged(feed, caches.ref), f"{what} step {t}")
        feed = toks


@pytest.mark.gpu
def test_config5_w4a16_long_prompts_sampled_c8(w4_pair):
    model, ref = w4_pair
    C, chunk = 8, 128
    g = torch.Generator().manual_seed(SEED + 5)
    lens = torch.randint(1024, 8193, (C,), generator=g).tolist()
    lens[1] = 8192                                   # table width 512: the 64-split cap
    # sequence 0 prefills its whole prompt; the others a real chunk on a synthetic history
    hist = [0] + [n - chunk for n in lens[1:]]
    caches = _Caches(model, hist, seed=SEED + 5, ref_dtype=torch.float32, final_lens=lens)
    alloc, cache, views = caches.pairs[0]
    prompts = [_ids(lens[0], SEED + 50)] + [_ids(chunk, SEED + 50 + i) for i in range(1, C)]
    n_new = [len(p) for p in prompts]
    padded = torch.zeros(C, max(n_new), dtype=torch.int64)
    for i, p in enumerate(prompts):
        padded[i, :len(p)] = torch.tensor(p)
    print(f"\n[config5 w4a16 C={C}: lens {lens}; extend rows {sum(n_new)}]", flush=True)
    got = model.forward_extend(padded.cuda(), views, starts=hist, chunk_lens=n_new).cpu()
    print("[config5: oracle prefill]", flush=True)
    want = torch.stack([ref.forward(torch.tensor([p]), c, num_logits_to_keep=1)[0, -1]
                        for p, c in zip(prompts, caches.ref)])
    _check_rows(got, want, "config5 prefill logits")
    assert [v.seq_len for v in views] == lens
    model.tune(8)
    runner = DecodeGraphRunner(model, cache, alloc, max_model_len=8192 + 64, seed=SEED)
    _sampled_steps(model, ref, runner, caches, views, C, 4, SEED, "config5 C=8")
    st = runner.states[8]
    assert st.buf.num_splits == 64 and st.buf.max_pages == 516


@pytest.mark.gpu
def test_config5_w4a16_sampled_c64(w4_pair):
    model, ref = w4_pair
    C = 64
    g = torch.Generator().manual_seed(SEED + 64)
    lens = torch.randint(1024, 8193, (C,), generator=g).tolist()
    caches = _Caches(model, lens, seed=SEED + 64, ref_dtype=torch.float32)
    alloc, cache, views = caches.pairs[0]
    print(f"\n[config5 w4a16 C={C}: mean history {sum(lens) / C:.0f}]", flush=True)
    model.tune(C)          # the bench's choice at this bucket (tiled or wide int4 kernel)
    print(f"  tilings {model.tilings[C]}", flush=True)
    runner = DecodeGraphRunner(model, cache, alloc, max_model_len=8192 + 64, seed=SEED + 1)
    _sampled_steps(model, ref, runner, caches, views, C, 3, SEED + 1, "config5 C=64")
    st = runner.states[64]
    assert st.buf.num_splits == 33 and st.buf.max_pages == 516   # 16-page K3 splits
