"""Prefill and chunked prefill (forward_prefill_batch, forward_extend;
acorninfer/models/qwen3.py:597-686): the decode step's kernels with one row
per token and, for bf16 / fp16, the query-tiled prefill attention kernel,
against the CPU oracle of the reference's SDPA path (oracle/qwen3_ref.py:
a whole-prompt forward, pinned against HF Qwen3) and against the GPU's own
token-by-token decode of the same prompt.

- fp32: the last prompt position's logits equal the oracle's within fp32
  reduction drift, and greedy decoding continued on the prefilled cache gives
  the oracle's ids; the KV pages equal those of the token-by-token path.
- bf16: a ragged batch of three prompts, each row's last logits within the
  decode tests' norm-relative tolerance of the oracle's (argmax equal where
  the top-2 margin is at least 0.05); two chunks through forward_extend equal
  the one-shot prefill; the tiled prefill attention and K3 with one row per
  token give the same logits and KV on a ragged batch and on an
  8192-token prompt that crosses the launch-block boundary.
"""
import pytest
import torch

from acorninfer_amd.cache.pager import PagedCacheView
from acorninfer_amd.config import Qwen3Config
from acorninfer_amd.models.qwen3 import Qwen3DecodeModel, random_state_dict
from model_utils import feed_prompt, new_cache, release
from oracle.qwen3_ref import Qwen3Ref, generate_greedy

SEED = 20261101
MARGIN = 0.05


def _ids(n, vocab, seed):
    return torch.randint(0, vocab, (n,), generator=torch.Generator().manual_seed(seed)).tolist()


def _padded(prompts, device):
    L = max(len(p) for p in prompts)
    x = torch.zeros(len(prompts), L, dtype=torch.int64)
    for i, p in enumerate(prompts):
        x[i, :len(p)] = torch.tensor(p)
    return x.to(device)


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


@pytest.mark.gpu
def test_prefill_fp32_matches_oracle_and_decode_continues():
    cfg = Qwen3Config.qwen3_0_6b().with_layers(4)
    sd = random_state_dict(cfg, seed=SEED, std=0.02, dtype=torch.float32)
    prompt = _ids(37, cfg.vocab_size, SEED + 1)       # 2 pages and a 5-token tail
    ref = Qwen3Ref(cfg, sd, torch.float32)
    want_ids, want_logits = generate_greedy(ref, prompt, 12)
    model = Qwen3DecodeModel.from_state_dict(cfg, sd, dtype=torch.float32, device="cuda")
    print("\n[fp32 prefill: 4 layers, prompt 37, 12 new]", flush=True)
    alloc, cache = new_cache(model, 12)
    view = PagedCacheView(cache)
    logits = model.forward_prefill_batch(_padded([prompt], model.device), [view],
                                         real_lens=[len(prompt)])[0]
    assert view.seq_len == len(prompt)
    got = []
    for t in range(12):
        torch.testing.assert_close(logits.cpu(), want_logits[t], rtol=1e-3, atol=1e-3)
        got.append(int(logits.argmax()))
        logits = model.forward_decode(torch.tensor([[got[-1]]], device=model.device), [view])[0]
    assert got == want_ids
    # the KV pages equal the token-by-token path's
    alloc2, cache2 = new_cache(model, 12)
    view2 = PagedCacheView(cache2)
    feed_prompt(model, view2, prompt)
    n = len(prompt)
    for li in range(cfg.num_hidden_layers):
        for pages, pages2 in ((cache.k_pages, cache2.k_pages), (cache.v_pages, cache2.v_pages)):
            a = pages[li][torch.tensor(view.table)].reshape(-1, *pages[li].shape[2:])[:n]
            b = pages2[li][torch.tensor(view2.table)].reshape(-1, *pages2[li].shape[2:])[:n]
            torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-5)
    release(alloc, [view])
    release(alloc2, [view2])
    alloc.assert_balanced()


@pytest.mark.gpu
def test_prefill_batch_ragged_bf16_matches_oracle():
    cfg = Qwen3Config.qwen3_0_6b().with_layers(4)
    sd = random_state_dict(cfg, seed=SEED + 2, std=0.02, dtype=torch.bfloat16)
    prompts = [_ids(n, cfg.vocab_size, SEED + 10 + n) for n in (5, 33, 17)]
    ref = Qwen3Ref(cfg, sd, torch.bfloat16)
    model = Qwen3DecodeModel.from_state_dict(cfg, sd, weight_format="bf16", device="cuda")
    alloc, cache = new_cache(model, 16)
    views = [PagedCacheView(cache) for _ in prompts]
    got = model.forward_prefill_batch(_padded(prompts, model.device), views,
                                      real_lens=[len(p) for p in prompts]).cpu()
    for i, p in enumerate(prompts):
        want = ref.forward(torch.tensor([p]), num_logits_to_keep=1)[0, -1]
        rel = _rel(got[i], want)
        top2 = want.topk(2).values
        print(f"\n[bf16 prefill row {i} (len {len(p)}): rel err {rel:.3g}]", flush=True)
        assert rel < 3e-2
        if (top2[0] - top2[1]).item() >= MARGIN:
            assert int(got[i].argmax()) == int(want.argmax())
        assert views[i].seq_len == len(p)
    release(alloc, views)
    alloc.assert_balanced()


@pytest.mark.gpu
def test_extend_in_chunks_equals_one_shot_bf16():
    cfg = Qwen3Config.qwen3_0_6b().with_layers(4)
    sd = random_state_dict(cfg, seed=SEED + 3, std=0.02, dtype=torch.bfloat16)
    model = Qwen3DecodeModel.from_state_dict(cfg, sd, weight_format="bf16", device="cuda")
    prompt = _ids(41, cfg.vocab_size, SEED + 4)
    alloc, cache = new_cache(model, 16)
    one, two = PagedCacheView(cache), PagedCacheView(cache)
    whole = model.forward_prefill_batch(_padded([prompt], model.device), [one],
                                        real_lens=[41])[0].cpu()
    model.forward_prefill_batch(_padded([prompt[:20]], model.device), [two], real_lens=[20])
    part = model.forward_extend(_padded([prompt[20:]], model.device), [two], starts=[20],
                                chunk_lens=[21])[0].cpu()
    assert two.seq_len == 41
    assert _rel(part, whole) < 3e-2
    for li in range(cfg.num_hidden_layers):
        a = cache.k_pages[li][torch.tensor(one.table)].reshape(-1, cfg.num_key_value_heads,
                                                              cfg.head_dim)[:41].float()
        b = cache.k_pages[li][torch.tensor(two.table)].reshape(-1, cfg.num_key_value_heads,
                                                              cfg.head_dim)[:41].float()
        assert _rel(b, a) < 3e-2
    with pytest.raises(ValueError):
        model.forward_extend(_padded([prompt[:4]], model.device), [two], starts=[40],
                             chunk_lens=[4])
    release(alloc, [one, two])
    alloc.assert_balanced()


@pytest.mark.gpu
@pytest.mark.parametrize("lens", [(600, 500), (200, 100)])
def test_prefill_at_dense_gemm_sizes_bf16_matches_oracle(lens):
    """>= DENSE_M_MIN (256) rows: the bf16 projections run on the large-M
    GEMM kernel with the planner's default split. 300 rows take its 8-16
    K-split plans through the qkv epilogue, K1 and silu_mul (no SwiGLU
    epilogue below 512 rows); 1100 rows the SwiGLU epilogue."""
    from acorninfer_amd.models.qwen3 import DENSE_M_MIN, DENSE_RT, PREFILL_SWIGLU_M
    cfg = Qwen3Config.qwen3_0_6b().with_layers(2)
    sd = random_state_dict(cfg, seed=SEED + 5, std=0.02, dtype=torch.bfloat16)
    prompts = [_ids(n, cfg.vocab_size, SEED + 20 + n) for n in lens]
    rows = sum(len(p) for p in prompts)
    assert rows >= DENSE_M_MIN
    ref = Qwen3Ref(cfg, sd, torch.bfloat16)
    model = Qwen3DecodeModel.from_state_dict(cfg, sd, weight_format="bf16", device="cuda")
    for lin in (model.layers[0].qkv, model.layers[0].o, model.layers[0].down):
        assert lin.plan(rows)[0][0] == DENSE_RT
    assert model.prefill_swiglu(rows) == (rows >= PREFILL_SWIGLU_M)
    alloc, cache = new_cache(model, 80)
    views = [PagedCacheView(cache) for _ in prompts]
    got = model.forward_prefill_batch(_padded(prompts, model.device), views,
                                      real_lens=[len(p) for p in prompts]).cpu()
    for i, p in enumerate(prompts):
        want = ref.forward(torch.tensor([p]), num_logits_to_keep=1)[0, -1]
        rel = _rel(got[i], want)
        print(f"\n[bf16 prefill {len(p)} tokens in an {sum(map(len, prompts))}-row launch: "
              f"rel err {rel:.3g}]", flush=True)
        assert rel < 3e-2
    release(alloc, views)
    alloc.assert_balanced()


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["bf16", "w4a16"])
def test_prefill_direct_outputs_equal_partials(fmt):
    """Prefill blocks whose qkv / o / down run in one split on the large-M
    kernel write them in bf16 and the qkv epilogue / K1 read that; the same
    prefill through fp32 planes gives the same logits and KV bits. 1500 rows:
    the dense kernel (bf16 from 512 rows, int4 dequantised from 1024) with
    the SwiGLU epilogue."""
    from acorninfer_amd.models.qwen3 import DENSE_RT, DEQUANT_RT, PREFILL_DIRECT_M
    from acorninfer_amd.ops.quant_gemm import Tiling
    cfg = Qwen3Config.qwen3_0_6b().with_layers(2)
    sd = random_state_dict(cfg, seed=SEED + 9, std=0.02, dtype=torch.bfloat16)
    model = Qwen3DecodeModel.from_state_dict(cfg, sd, weight_format=fmt, device="cuda")
    prompts = [_ids(n, cfg.vocab_size, SEED + 60 + n) for n in (700, 400, 400)]
    rows = sum(map(len, prompts))
    assert rows >= PREFILL_DIRECT_M
    # one split each (this small model's planner would split K to fill the CUs)
    t = Tiling(DENSE_RT if fmt == "bf16" else DEQUANT_RT, 256, 128, 1, 4)
    model.tilings[rows] = {"qkv": t, "o": t, "down": t}
    got = {}
    for direct in (True, False):
        model.prefill_direct = direct
        alloc, cache = new_cache(model, 120)
        views = [PagedCacheView(cache) for _ in prompts]
        logits = model.forward_prefill_batch(_padded(prompts, model.device), views,
                                             real_lens=[len(p) for p in prompts])
        assert model._extend_buf[1].direct == direct
        got[direct] = (logits.cpu(), cache.k_pool.clone(), cache.v_pool.clone())
        release(alloc, views)
    model.prefill_direct = True
    for a, b in zip(got[True], got[False]):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b)
    del model.tilings[rows]
    print(f"\n[{fmt} prefill {rows} rows: direct outputs == fp32 planes]")


@pytest.mark.gpu
def test_prefill_w4a16_dequant_route_matches_oracle():
    """int4 weights at >= 2048 rows: every projection dequantises into the step
    workspace and runs on the large-M bf16 kernel; the last-row logits stay
    within the decode tests' tolerance of the oracle on the dequantised
    weights, as with the int4 kernels below that size."""
    from acorninfer_amd.models.qwen3 import DEQUANT_M_MIN, DEQUANT_RT
    cfg = Qwen3Config.qwen3_0_6b().with_layers(2)
    sd = random_state_dict(cfg, seed=SEED + 7, std=0.02, dtype=torch.bfloat16)
    model = Qwen3DecodeModel.from_state_dict(cfg, sd, weight_format="w4a16", device="cuda")
    prompts = [_ids(n, cfg.vocab_size, SEED + 40 + n) for n in (1500, 700)]
    assert sum(len(p) for p in prompts) >= DEQUANT_M_MIN
    dq = dict(sd)
    nq, nkv = cfg.num_attention_heads * cfg.head_dim, cfg.num_key_value_heads * cfg.head_dim
    for i, L in enumerate(model.layers):
        p = f"layers.{i}."
        qkv, gu = L.qkv.dense().cpu(), L.gate_up.dense().cpu()
        dq[p + "self_attn.q_proj.weight"] = qkv[:nq]
        dq[p + "self_attn.k_proj.weight"] = qkv[nq:nq + nkv]
        dq[p + "self_attn.v_proj.weight"] = qkv[nq + nkv:]
        dq[p + "self_attn.o_proj.weight"] = L.o.dense().cpu()
        dq[p + "mlp.gate_proj.weight"] = gu[:cfg.intermediate_size]
        dq[p + "mlp.up_proj.weight"] = gu[cfg.intermediate_size:]
        dq[p + "mlp.down_proj.weight"] = L.down.dense().cpu()
    dq["lm_head.weight"] = model.lm_head.dense().cpu()
    ref = Qwen3Ref(cfg, dq, torch.float32)
    alloc, cache = new_cache(model, 160)
    views = [PagedCacheView(cache) for _ in prompts]
    got = model.forward_prefill_batch(_padded(prompts, model.device), views,
                                      real_lens=[len(p) for p in prompts]).cpu()
    buf = model._extend_buf[1]
    assert all(buf.cfgs[n].rt == DEQUANT_RT for n in ("qkv", "o", "gate_up", "down"))
    assert buf.wtmp.numel() == 2 * cfg.intermediate_size * cfg.hidden_size
    for i, p in enumerate(prompts):
        want = ref.forward(torch.tensor([p]), num_logits_to_keep=1)[0, -1]
        rel = _rel(got[i], want)
        print(f"\n[w4a16 prefill {len(p)} tokens in a {sum(map(len, prompts))}-row launch: "
              f"rel err {rel:.3g}]", flush=True)
        assert rel < 3e-2
    release(alloc, views)
    alloc.assert_balanced()


@pytest.mark.gpu
@pytest.mark.parametrize("lens", [(5, 33, 17, 200), (8300,)])
def test_tiled_prefill_attention_equals_k3_rows_bf16(lens):
    """The model's prefill with the query-tiled attention kernel against the
    same prefill with K3 (one decode row per token): last-row logits and
    every layer's KV. 8300 tokens is two launch blocks (8192 rows each), so
    the second block's tiles read the first block's KV from the pool."""
    cfg = Qwen3Config.qwen3_0_6b().with_layers(2)
    sd = random_state_dict(cfg, seed=SEED + 6, std=0.02, dtype=torch.bfloat16)
    model = Qwen3DecodeModel.from_state_dict(cfg, sd, weight_format="bf16", device="cuda")
    prompts = [_ids(n, cfg.vocab_size, SEED + 30 + n) for n in lens]
    pages = sum(-(-n // 16) for n in lens) + 4
    got = {}
    for tiled in (True, False):
        print(f"\n[prefill {lens} tokens, tiled attention {tiled}]", flush=True)
        model.tiled_prefill = tiled
        alloc, cache = new_cache(model, pages)
        views = [PagedCacheView(cache) for _ in prompts]
        logits = model.forward_prefill_batch(_padded(prompts, model.device), views,
                                             real_lens=list(lens)).cpu()
        # the last layer's k (layer 0's k/v are computed before any attention)
        kv = [cache.k_pages[-1][torch.tensor(v.table)].reshape(-1, cfg.num_key_value_heads,
                                                             cfg.head_dim)[:n].float().cpu()
              for v, n in zip(views, lens)]
        got[tiled] = (logits, kv)
        release(alloc, views)
    model.tiled_prefill = True
    for i in range(len(lens)):
        rel = _rel(got[True][0][i], got[False][0][i])
        print(f"\n[row {i} ({lens[i]} tokens): tiled vs K3 rows rel err {rel:.3g}]", flush=True)
        assert rel < 3e-2
        assert _rel(got[True][1][i], got[False][1][i]) < 3e-2
