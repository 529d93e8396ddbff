"""Decode throughput of the Qwen3-8B-shaped hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--format bf16|w4a16|w8a16]
                    [--batch C] [--prompt-len L] [--no-extra] [--no-kernels]
                    [--no-cpu-baseline]

A step is one hipGraph-replayed decode step of C sequences (BASELINE
configuration 4: Qwen3-8B shape, 36 layers, random-init weights N(0, 0.02),
greedy, page 16, prompts of L=512 tokens). The prompts' KV is synthetic
(random bf16 written straight into the paged pool; prefill is not part of
the measured path), the first ids are random, every later id is the greedy
choice of the previous step (fed back on the device). `value` is decode
tokens per second over the K timed steps: C*K / elapsed.

The JSON line also carries:
- roofline: the dominant kernel (the weight-streaming GEMM) timed with HIP
  events on its own stream: a hipGraph of one step's GEMM launches (36 x
  {qkv, o, gate|up, down} + lm_head, the step's own weights and buffers) is
  replayed and timed; achieved = algorithmic bytes of those launches / time.
  `in_step` is the same launches' time inside the captured step, read from
  the committed rocprofv3 summary of that step; `traffic` the HBM bytes from
  the committed FETCH_SIZE / WRITE_SIZE summary.
- extra (unless --no-extra): the reference's decode_batch protocol (one
  host copy per step) at the headline size, other batch sizes and formats
  (W4A16 and W8A16 at C=8 with their own GEMM rooflines, configuration 5),
  the batched prefill (C x 512, and one 8192-token prompt) and
  configuration 4 end to end through the Engine.
- decode: the metric's figures in one object (bf16 / W4A16 tok/s at C=1 and
  C=8, W8A16 at C=8, each format's GEMM fraction of peak in a graph of the
  step's GEMM launches and inside the step, K3's fraction at configurations
  2 and 5); the run's last stderr lines restate them.
- extra.kernels (unless --no-kernels): the isolated kernels at
  configurations 2 (K3, K1, K2), 5 (K3 + combine over one layer's pages at
  C=8 and C=64; prefill attention over an 8192-token prompt and 8 x 512
  against K3 with one row per token) and 3 (int4 / int8 GEMM at every shape
  and M = 1/8/64/256, HBM and MFMA fractions; the bf16 large-M GEMM at
  M = 512/2048/8192 against hipBLASLt).
- cpu_baseline: BASELINE configuration 1 run whole on the CPU oracle of the
  reference's path (oracle/qwen3_ref.py, fp32 torch on the host cores),
  the CPU oracles of the kernels at configuration 2/3 shapes, and the GPU
  path on the same configuration-1 workload.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0     # dense bf16 MFMA (the int4 / int8 paths compute in bf16)


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _release() -> None:
    """Drop the tensors nothing refers to any more, keeping their memory in
    torch's cache rather than handing it back to the driver: memory a process
    gets from the driver again after freeing it streamed ~5% slower in the
    decode step on this part (bf16 C=8 3.28 against 3.13 ms, every model built
    after the first) than its first allocations or blocks torch's cache hands
    out again (3.13-3.14 ms), so every leg after the first reuses the cache.
    torch still empties the cache itself when an allocation would fail."""
    import gc
    gc.collect()


def _gemm_bytes(lin, M: int) -> int:
    """Algorithmic bytes of one projection launch: weights (+ scales) once,
    activations in and bf16 results out."""
    return lin.nbytes() + 2 * M * lin.K + 2 * M * lin.N


def measured_traffic(fmt: str, batch: int):
    """HBM bytes per step of the GEMM launches from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary for this workload (scaled by the copy
    calibration), or None when no such summary exists."""
    path = os.path.join(ROOT, "profiles", f"gemm_traffic_{fmt}_C{batch}.txt")
    try:
        with open(path) as fh:
            for line in fh:
                if line.startswith("traffic_bytes_per_step:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def k3_profile_split() -> dict:
    """K3's main kernel and its split combine, each alone, from the committed
    rocprofv3 kernel-trace summaries (profiles/k3_config{2,5}_kernel_stats.txt):
    {config: {main_us, combine_us, main_frac, source}}; configurations whose
    summary is missing are left out. This run's own K3 timings (main +
    combine as one captured launch pair) are the K3_* entries of `kernels`."""
    out = {}
    for cfgs, name in ((("config2",), "k3_config2_kernel_stats.txt"),
                       (("config5_C8", "config5_C64"), "k3_config5_kernel_stats.txt")):
        path = os.path.join(ROOT, "profiles", name)
        try:
            lines = open(path).read().splitlines()
        except OSError:
            continue
        blocks, cur = [], None
        for ln in lines:
            if ln.startswith("## configuration"):
                cur = {}
                blocks.append(cur)
            elif cur is not None and ln.strip().startswith(("main ", "combine ")):
                cur[ln.split()[0]] = float(ln.split()[2])
            elif cur is not None and "algorithmic bytes" in ln:
                cur["bytes"] = int(ln.split()[0])
        for c, b in zip(cfgs, blocks):
            if {"main", "combine", "bytes"} <= set(b):
                out[c] = {"main_us": b["main"], "combine_us": b["combine"],
                          "main_frac": round(b["bytes"] / b["main"] / 1e3 / HBM_PEAK_GBS, 4),
                          "source": f"profiles/{name}"}
    return out


def in_step_gemm(fmt: str, batch: int, nbytes: int):
    """The GEMM launches' time inside the captured step, from the committed
    rocprofv3 kernel-trace summary of that step (the line's `achieved` times
    them back to back in a graph of their own): µs per step and the same
    bytes' fraction of peak, or None when no such summary exists."""
    path = os.path.join(ROOT, "profiles", f"decode_{fmt}_C{batch}_step_breakdown.txt")
    try:
        with open(path) as fh:
            for line in fh:
                if line.startswith("gemm_in_step_us_per_step:"):
                    us = float(line.split(":", 1)[1])
                    return {"us_per_step": us, "frac": round(nbytes / (us * 1e-6) / 1e9 /
                                                             HBM_PEAK_GBS, 4),
                            "source": os.path.relpath(path, ROOT)}
    except OSError:
        pass
    return None


def build_workload(cfg, fmt: str, batch: int, prompt_len: int, total_steps: int, seed: int,
                   tune: bool = True, prompt_lens: list[int] | None = None,
                   tilings: dict | None = None):
    import torch

    from acorninfer_amd.cache.pager import BlockAllocator, PagedCacheView, PagedKVCache
    from acorninfer_amd.engine.graph_runner import DecodeGraphRunner
    from acorninfer_amd.models.qwen3 import Qwen3DecodeModel

    t0 = time.perf_counter()
    model = Qwen3DecodeModel.random_init(cfg, weight_format=fmt, seed=seed, device="cuda")
    torch.cuda.synchronize()
    _log(f"model {fmt}: {model.weight_bytes() / 1e9:.3f} GB weights in "
         f"{time.perf_counter() - t0:.1f} s")
    report = {}
    if tilings is not None:
        # a fixed choice (e.g. an unprofiled run's, for a profiled one)
        from acorninfer_amd.ops.quant_gemm import Tiling
        model.tilings[batch] = {k: Tiling(*v) for k, v in tilings.items()
                                if k not in ("swiglu", "fold")}
        model.swiglu_choice[batch] = bool(tilings.get("swiglu", True))
        model.fold_choice[batch] = bool(tilings.get("fold", True))
        report = {k: {"tiling": tuple(v), "us": float("nan"), "bytes": 1}
                  for k, v in model.tilings[batch].items()}
    elif tune:
        t0 = time.perf_counter()
        report = model.tune(batch)
        _log(f"tuned {fmt} C={batch} in {time.perf_counter() - t0:.1f} s "
             f"(fold {report.get('fold')})")
    P = 16
    lens = prompt_lens if prompt_lens is not None else [prompt_len] * batch
    max_len = max(lens) + total_steps + 1
    per_seq = -(-max_len // P)
    alloc = BlockAllocator(sum(-(-(n + total_steps + 1) // P) for n in lens) + 2)
    cache = PagedKVCache(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim, P, alloc,
                         "cuda", torch.bfloat16)
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    cache.k_pool.normal_(generator=g)
    cache.v_pool.normal_(generator=g)
    views = []
    for n in lens:
        v = PagedCacheView(cache)
        for _t in range(-(-n // P)):
            v.table.append(alloc.allocate())
        for li in range(cfg.num_hidden_layers):
            v._lens[li] = n
        views.append(v)
    runner = DecodeGraphRunner(model, cache, alloc, max_model_len=max_len, buckets=(batch,))
    first = torch.randint(0, cfg.vocab_size, (batch,), generator=torch.Generator().manual_seed(
        seed + 2)).tolist()
    model.tune_report = report
    return model, cache, runner, views, first


def time_decode(runner, views, first, steps: int, warmup: int, sampling=None):
    import torch
    log = runner.decode_loop(views, first, warmup, sampling) if warmup else None
    nxt = log[-1].tolist() if warmup else first
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    log = runner.decode_loop(views, nxt, steps, sampling)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return dt, log


def time_decode_batch(runner, views, first, steps: int):
    """The reference's step protocol (DecodeGraphRunner.decode_batch: the
    step's tokens come back to the host after every step) over `steps`
    steps; seconds."""
    import torch
    from types import SimpleNamespace
    seqs = [SimpleNamespace(generated_ids=[t]) for t in first]
    runner.decode_batch(seqs, views)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        toks = runner.decode_batch(seqs, views)
        for s_, t in zip(seqs, toks):
            s_.generated_ids.append(t)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def prefill_benchmark(model, cfg, batch: int, prompt_len: int, seed: int, reps: int = 3):
    """Batched prefill (forward_prefill_batch) of `batch` prompts of
    `prompt_len` random ids into a fresh cache: ms per call (wall clock around
    synchronised calls, after one warm-up call) and prompt tok/s."""
    import torch

    from acorninfer_amd.cache.pager import BlockAllocator, PagedCacheView, PagedKVCache

    P = 16
    per = -(-prompt_len // P)
    alloc = BlockAllocator(batch * per + 1)
    cache = PagedKVCache(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim, P, alloc,
                         "cuda", model.dtype)
    ids = torch.randint(0, cfg.vocab_size, (batch, prompt_len),
                        generator=torch.Generator().manual_seed(seed)).cuda()
    times = []
    for r in range(reps + 1):
        views = [PagedCacheView(cache) for _ in range(batch)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        model.forward_prefill_batch(ids, views, real_lens=[prompt_len] * batch)
        torch.cuda.synchronize()
        if r:
            times.append(time.perf_counter() - t0)
        for v in views:
            for blk in v.table:
                alloc.free(blk)
    ms = 1e3 * sorted(times)[len(times) // 2]
    return ms, batch * prompt_len / ms * 1e3


def engine_benchmark(model, cfg, concurrency: int, prompt_len, new_tokens: int, seed: int,
                     sampling=None, warm_len: int | None = None):
    """Configurations 4 and 5 end to end: `concurrency` requests of random ids
    (prompt_len: one length, or a list of one per request) and `new_tokens`
    generated tokens each, submitted at once to the Engine (continuous
    batching: batched prefill, then the graph-captured decode step); greedy
    unless `sampling` (a SamplingParams) is given. A warm-up run with prompts
    of `warm_len` tokens (default: the same lengths) captures the decode graph
    first. Returns (generated tok/s over the wall time of the whole run, mean
    time to first token in ms)."""
    import torch

    from acorninfer_amd.engine.engine import Engine
    from acorninfer_amd.sampler import SamplingParams

    P = 16
    lens = list(prompt_len) if isinstance(prompt_len, (list, tuple)) else [prompt_len] * concurrency
    longest = max(lens)
    blocks = sum(-(-(n + new_tokens + 1) // P) for n in lens) + 8
    eng = Engine(model, num_blocks=blocks, max_running=concurrency, watermark_blocks=1,
                 max_model_len=longest + new_tokens + 1, seed=seed)
    g = torch.Generator().manual_seed(seed)
    sp = sampling if sampling is not None else SamplingParams(temperature=0.0)
    never = frozenset({-1})

    def run(n_new, plens):
        ids = [eng.submit(torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist(),
                          sp, max_tokens=n_new, eos_ids=never) for n in plens]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while eng.has_pending():
            eng.step()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        ttft = [1e3 * (eng.seqs[i].first_token_at - t0) for i in ids]
        for i in ids:
            eng.drop(i)
        return dt, sum(ttft) / len(ttft)

    run(4, [warm_len] * concurrency if warm_len else lens)   # warm-up: captures the decode graph
    dt, ttft = run(new_tokens, lens)
    eng.assert_balanced()
    return concurrency * new_tokens / dt, ttft


def gemm_step_bytes(model, batch: int) -> int:
    """Algorithmic bytes of one decode step's GEMM launches."""
    lins = [lin for lw in model.layers for lin in (lw.qkv, lw.o, lw.gate_up, lw.down)]
    return sum(_gemm_bytes(lin, batch) for lin in lins + [model.lm_head])


def gemm_roofline(model, runner, batch: int, reps: int = 5):
    """Time one step's GEMM launches (hipGraph on a private stream, HIP events
    on that stream): the forms the step runs, the folded ones (normalise on
    load, residual epilogue) where it folds the RMSNorms, on copies of the
    residual and its sums. Returns (achieved GB/s, per-step bytes, per-step
    µs, launches per step)."""
    import torch
    st = runner._state(batch)
    buf = st.buf
    s = torch.cuda.Stream()
    launches = []
    for lw in model.layers:
        launches += [("qkv", lw.qkv, buf.normed, buf.part_qkv, lw.input_norm),
                     ("o", lw.o, buf.attn, buf.part_o, None),
                     ("gate_up", lw.gate_up, buf.normed,
                      "swiglu" if buf.swiglu else buf.part_gu, lw.post_norm),
                     ("down", lw.down, buf.act, buf.part_down, None)]
    launches.append(("lm_head", model.lm_head, buf.normed, None, None))
    nbytes = sum(_gemm_bytes(lin, batch) for _, lin, *_ in launches)
    eps = float(model.cfg.rms_norm_eps)
    if buf.fold:
        res = buf.res.clone()
        xw = buf.normed.clone()
        ss = buf.ss_dn.clone()

    def body():
        sp = s.cuda_stream
        for name, lin, x, part, nw in launches:
            c = buf.cfgs[name]
            if part is None:
                lin.launch(x, batch, c, out=buf.logits, part=buf.ws_lm, stream=sp)
            elif buf.fold and nw is not None:
                kw = {"act": buf.act} if isinstance(part, str) else {"part": part}
                lin.launch_norm(xw, batch, c, ss=ss, eps=eps, stream=sp, **kw)
            elif buf.fold:
                lin.launch_resid(x, batch, c, res=res, res_out=res, ss=ss,
                                 norm_w=model.layers[0].input_norm, xw=xw, stream=sp)
            elif isinstance(part, str):
                lin.launch_swiglu(x, batch, c, buf.act, sp)
            else:
                lin.launch(x, batch, c, part=part, stream=sp)

    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            body()
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            g.replay()
        e1.record(s)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    return nbytes / (us * 1e-6) / 1e9, nbytes, us, len(launches)


def _time_graph(body, reps: int = 10) -> float:
    """µs per replay of a hipGraph of `body`, HIP events on its stream. Bodies
    hold many launches so the graph's own launch cost is amortised."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            body(s)
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            g.replay()
        e1.record(s)
    e1.synchronize()
    torch.cuda.current_stream().wait_stream(s)
    return e0.elapsed_time(e1) * 1e3 / reps


def kernel_benchmarks(seed: int = 23, only_attention: bool = False,
                      attn_splits: list[int] | None = None, gemm_ms=(1, 8, 64, 256),
                      with_attention: bool = True) -> dict:
    """Isolated kernels at BASELINE configurations 2, 3 and 5 (algorithmic
    bytes / time, HIP events around hipGraph replays)."""
    out = {}
    if with_attention or only_attention:
        out.update(attention_benchmarks(seed, attn_splits))
        # K3's two launches apart (main kernel, split combine) from the committed profile
        for k, v in k3_profile_split().items():
            if f"K3_{k}" in out:
                out[f"K3_{k}"]["profile_main_us"] = v["main_us"]
                out[f"K3_{k}"]["profile_combine_us"] = v["combine_us"]
                out[f"K3_{k}"]["profile_main_frac"] = v["main_frac"]
    if only_attention:
        return out
    if with_attention:
        out.update(norm_benchmarks(seed))
    out.update(gemm_benchmarks(seed, gemm_ms))
    out.update(dense_gemm_benchmarks(seed))
    return out


def attention_benchmarks(seed: int, attn_splits: list[int] | None = None) -> dict:
    """K3 (+ combine) at configuration 2 and at configuration 5's contexts."""
    import torch

    from acorninfer_amd import _lib
    from acorninfer_amd._lib import lib, ptr
    from acorninfer_amd.models.qwen3 import attention_splits

    out = {}
    g = torch.Generator(device="cuda").manual_seed(seed)
    # ---- K3, configuration 2 --------------------------------------------
    B, H, KV, D, P, NB = 8, 32, 8, 128, 16, 4096
    lens = torch.randint(512, 4097, (B,), generator=torch.Generator().manual_seed(seed))
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(seed + 1))
    mp = -(-int(lens.max()) // P)
    tables = torch.zeros(B, 256, dtype=torch.int32)
    o = 0
    for b in range(B):
        n = -(-int(lens[b]) // P)
        tables[b, :n] = perm[o:o + n].to(torch.int32)
        o += n
    # rotate 4 pools so the 256 MB MALL cannot hold the one being read
    pools = [(torch.randn(NB, P, KV, D, device="cuda", generator=g).bfloat16(),
              torch.randn(NB, P, KV, D, device="cuda", generator=g).bfloat16()) for _ in range(4)]
    q = torch.randn(B, H, D, device="cuda", generator=g).bfloat16()
    attn_out = torch.empty_like(q)
    tb, ln = tables.cuda(), lens.to(torch.int32).cuda()
    S = attention_splits(B, KV, 256)
    smax = max([S] + list(attn_splits or []))
    ws_acc = torch.empty(B * H * smax * D, device="cuda")
    ws_ml = torch.empty(2 * B * H * smax, device="cuda")
    st_code = _lib.BF16

    def k3_us(nsplit):
        def k3(st):
            for kp, vp in pools * 16:
                _lib.check(lib().acorn_paged_attention(
                    ptr(q), ptr(kp), ptr(vp), ptr(tb), ptr(ln), ptr(attn_out), ptr(ws_acc),
                    ptr(ws_ml), B, H, KV, D, P, NB, 256, nsplit, D ** -0.5, st_code,
                    st.cuda_stream), "K3")
        return _time_graph(k3) / (16 * len(pools))

    us = k3_us(S)
    nbytes = int(lens.sum()) * KV * D * 2 * 2 + 2 * B * H * D * 2 + 4 * sum(
        -(-int(L) // P) for L in lens) + 4 * B
    if attn_splits:
        out["K3_config2_split_sweep_us"] = {n: round(k3_us(n), 2) for n in attn_splits}
    out["K3_config2"] = {"us": round(us, 2), "bytes": nbytes,
                         "GBps": round(nbytes / us / 1e3, 1),
                         "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "splits": S,
                         "mean_ctx": round(float(lens.float().mean()), 1)}
    del pools
    # ---- K3 (+ combine) at configuration 5's long contexts: one layer's pages
    # for C sequences of U[1024, 8192] tokens (the decode step's split rule)
    for C in (8, 64):
        clens = torch.randint(1024, 8193, (C,), generator=torch.Generator().manual_seed(seed + 5))
        npg = [-(-int(L) // P) for L in clens]
        nb5 = sum(npg) + 1
        w5 = -(-8193 // P)
        perm5 = torch.randperm(nb5, generator=torch.Generator().manual_seed(seed + 6))
        tb5 = torch.zeros(C, w5, dtype=torch.int32)
        o = 0
        for b in range(C):
            tb5[b, :npg[b]] = perm5[o:o + npg[b]].to(torch.int32)
            o += npg[b]
        kp5 = torch.empty(nb5, P, KV, D, device="cuda", dtype=torch.bfloat16).normal_(generator=g)
        vp5 = torch.empty_like(kp5).normal_(generator=g)
        q5 = torch.randn(C, H, D, device="cuda", generator=g).bfloat16()
        o5 = torch.empty_like(q5)
        S5 = attention_splits(C, KV, w5)
        acc5 = torch.empty(C * H * S5 * D, device="cuda")
        ml5 = torch.empty(2 * C * H * S5, device="cuda")
        tb5c, ln5 = tb5.cuda(), clens.to(torch.int32).cuda()

        def k3c5(st):
            for _ in range(4):
                _lib.check(lib().acorn_paged_attention(
                    ptr(q5), ptr(kp5), ptr(vp5), ptr(tb5c), ptr(ln5), ptr(o5), ptr(acc5),
                    ptr(ml5), C, H, KV, D, P, nb5, w5, S5, D ** -0.5, st_code, st.cuda_stream),
                    "K3")
        us5 = _time_graph(k3c5, 5) / 4
        nb = int(clens.sum()) * KV * D * 2 * 2 + 2 * C * H * D * 2 + 4 * sum(npg) + 4 * C
        if attn_splits:
            sweep = {}
            for n in attn_splits:
                acc5 = torch.empty(C * H * n * D, device="cuda")
                ml5 = torch.empty(2 * C * H * n, device="cuda")

                def k3n(st, n=n, acc5=acc5, ml5=ml5):
                    for _ in range(4):
                        _lib.check(lib().acorn_paged_attention(
                            ptr(q5), ptr(kp5), ptr(vp5), ptr(tb5c), ptr(ln5), ptr(o5),
                            ptr(acc5), ptr(ml5), C, H, KV, D, P, nb5, w5, n, D ** -0.5,
                            st_code, st.cuda_stream), "K3")
                sweep[n] = round(_time_graph(k3n, 5) / 4, 2)
            out[f"K3_config5_C{C}_split_sweep_us"] = sweep
        out[f"K3_config5_C{C}"] = {"us": round(us5, 2), "bytes": nb,
                                   "GBps": round(nb / us5 / 1e3, 1),
                                   "frac": round(nb / us5 / 1e3 / HBM_PEAK_GBS, 4), "splits": S5,
                                   "mean_ctx": round(float(clens.float().mean()), 1)}
        del kp5, vp5, acc5, ml5
        _release()
    out.update(prefill_attention_benchmarks(seed))
    return out


def prefill_attention_benchmarks(seed: int) -> dict:
    """Prefill attention of one layer, Qwen3-8B heads: one 8192-token prompt
    (configuration 5's longest) and 8 prompts of 512 (configuration 4's), the
    query-tiled kernel against K3 with one decode row per token. FLOPs are the
    causal algorithmic count 4 * H * D * sum over rows of (position + 1)."""
    import torch

    from acorninfer_amd import _lib
    from acorninfer_amd._lib import lib, ptr

    out = {}
    H, KV, D, P = 32, 8, 128, 16
    g = torch.Generator(device="cuda").manual_seed(seed + 11)
    for n, L in ((1, 8192), (8, 512)):
        R, per = n * L, L // P
        nb = n * per + 1
        kp = torch.empty(nb, P, KV, D, device="cuda", dtype=torch.bfloat16).normal_(generator=g)
        vp = torch.empty_like(kp).normal_(generator=g)
        q = torch.randn(R, H, D, device="cuda", generator=g).bfloat16()
        o = torch.empty_like(q)
        perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed + 12))
        tabs = perm[:n * per].view(n, per).to(torch.int32).cuda()
        row0 = torch.arange(n, dtype=torch.int32, device="cuda") * L
        pos0 = torch.zeros(n, dtype=torch.int32, device="cuda")
        nq = torch.full((n,), L, dtype=torch.int32, device="cuda")
        # K3 rows: one decode row per token, length position + 1
        rtabs = tabs.repeat_interleave(L, 0).contiguous()
        rlens = torch.arange(1, L + 1, dtype=torch.int32, device="cuda").repeat(n)
        S = 4
        acc = torch.empty(R * H * S * D, device="cuda")
        ml = torch.empty(2 * R * H * S, device="cuda")

        def tiled(st):
            _lib.check(lib().acorn_paged_prefill_attention(
                ptr(q), ptr(kp), ptr(vp), ptr(tabs), ptr(row0), ptr(pos0), ptr(nq), ptr(o),
                n, R, L, H, KV, D, P, nb, per, D ** -0.5, _lib.BF16, st.cuda_stream),
                "prefill attention")

        def rows(st):
            _lib.check(lib().acorn_paged_attention(
                ptr(q), ptr(kp), ptr(vp), ptr(rtabs), ptr(rlens), ptr(o), ptr(acc), ptr(ml),
                R, H, KV, D, P, nb, per, S, D ** -0.5, _lib.BF16, st.cuda_stream), "K3")

        us = _time_graph(tiled, 10)
        us_rows = _time_graph(rows, 2)
        flops = 4.0 * H * D * n * L * (L + 1) / 2
        out[f"prefill_attention_{n}x{L}"] = {
            "us": round(us, 1), "TFLOPs": round(flops / us / 1e6, 1),
            "frac_mfma": round(flops / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4),
            "k3_rows_us": round(us_rows, 1), "speedup_vs_k3_rows": round(us_rows / us, 2)}
        del kp, vp, acc, ml
        _release()
    return out


def norm_benchmarks(seed: int) -> dict:
    """K1 and K2 at configuration-2 sizes (latency-bound: µs per call)."""
    import torch

    from acorninfer_amd import _lib
    from acorninfer_amd._lib import lib, ptr

    out = {}
    g = torch.Generator(device="cuda").manual_seed(seed + 2)
    lens = torch.randint(512, 4097, (8,), generator=torch.Generator().manual_seed(seed))
    # ---- K1 / K2 at configuration-2 sizes (latency-bound: µs) ----------
    x = torch.randn(8, 4096, device="cuda", generator=g).bfloat16()
    res = torch.randn(8, 4096, device="cuda", generator=g).bfloat16()
    w = torch.ones(4096, device="cuda").bfloat16()
    normed, res_out = torch.empty_like(x), torch.empty_like(x)

    def k1(st):
        for _ in range(100):
            _lib.check(lib().acorn_fused_add_rmsnorm(ptr(x), ptr(res), ptr(res_out), ptr(w),
                                                     ptr(normed), 8, 4096, 1e-6, _lib.BF16,
                                                     _lib.BF16, st.cuda_stream), "K1")
    out["K1_8x4096_us"] = round(_time_graph(k1, 5) / 100, 2)
    qq = torch.randn(8, 32, 128, device="cuda", generator=g).bfloat16()
    kk = torch.randn(8, 8, 128, device="cuda", generator=g).bfloat16()
    wq = torch.ones(128, device="cuda").bfloat16()
    pos = (lens - 1).cuda()
    invf = (1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).cuda()

    def k2(st):
        for _ in range(100):
            _lib.check(lib().acorn_qknorm_rope_inplace(
                ptr(qq), ptr(kk), 8, 32, 8, 128, ptr(wq), ptr(wq), 1e-6, ptr(pos), 1,
                ptr(invf), _lib.BF16, _lib.BF16, st.cuda_stream), "K2")
    out["K2_qknorm_rope_us"] = round(_time_graph(k2, 5) / 100, 2)
    return out


def dense_gemm_benchmarks(seed: int) -> dict:
    """bf16 projections at prefill M (configuration 3's shapes): this
    library's large-M kernel (its planner's tiling) on the model's weight
    layout (BF16B blocks) against torch.mm (hipBLASLt) on natural rows, fp32
    output as the prefill step consumes it; TFLOP/s and the fraction of the
    2.5 PFLOP/s dense bf16 peak."""
    import torch

    from acorninfer_amd import _lib
    from acorninfer_amd._lib import lib, ptr
    from acorninfer_amd.ops.quant_gemm import plan
    from acorninfer_amd.quant.quantize import to_bf16b

    out = {}
    g = torch.Generator(device="cuda").manual_seed(seed + 21)
    shapes = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (24576, 4096),
              "down": (4096, 12288)}
    for M in (512, 2048, 8192):
        for name, (n, k) in shapes.items():
            x = torch.randn(M, k, device="cuda", generator=g).bfloat16()
            w = (0.02 * torch.randn(n, k, device="cuda", generator=g)).bfloat16()
            wb = to_bf16b(w)
            t, _ = plan(M, n, k, _lib.WFMT_BF16B)
            part = torch.empty(t.ksplit, M, n, device="cuda")
            arr = (ctypes.c_int * 6)(*t, 0)

            def own(st):
                for _ in range(4):
                    _lib.check(lib().acorn_quant_gemm(ptr(x), ptr(wb), None, None, None,
                                                      ptr(part), M, n, k, _lib.WFMT_BF16B, arr,
                                                      st.cuda_stream), "dense GEMM")

            def library(st):
                for _ in range(4):
                    torch.ops.aten.mm.dtype_out(x, w.t(), torch.float32, out=part[0])

            fl = 2.0 * M * n * k
            us, us_lib = _time_graph(own, 3) / 4, _time_graph(library, 3) / 4
            out[f"dense_gemm_{name}_M{M}"] = {
                "us": round(us, 1),
                "frac_mfma": round(fl / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4),
                "hipblaslt_us": round(us_lib, 1)}
            del x, w, wb, part
    _release()
    return out


def gemm_benchmarks(seed: int, gemm_ms=(1, 8, 64, 256), fixed: dict | None = None) -> dict:
    """The int4 / int8 GEMM at configuration 3's shapes and M. `fixed` maps
    "{w4|w8}_{shape}_M{M}" to a tiling to time instead of searching (a
    profiled run takes an unprofiled run's choice)."""
    import torch

    from acorninfer_amd import _lib
    from acorninfer_amd.models.qwen3 import QLinear
    from acorninfer_amd.ops.quant_gemm import Tiling, candidates

    out = {}
    g = torch.Generator(device="cuda").manual_seed(seed + 3)
    # ---- quant GEMM, configuration 3 -------------------------------------
    # int4 and int8 in the decode model's block layouts; every
    # candidate tiling is timed once (one graph of 16 launches over distinct
    # weights), the fastest four again with 64 launches x 3 replays
    shapes = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (24576, 4096),
              "down": (4096, 12288)}
    for fmt_name, wf in (("w4", _lib.WFMT_W4), ("w8", _lib.WFMT_W8)):
        for name, (n, k) in shapes.items():
            nsets = max(2, -(-1_200_000_000 // (n * k // (2 if wf == _lib.WFMT_W4 else 1))))
            lins = []
            for _ in range(nsets):
                if wf == _lib.WFMT_W4:
                    wq4 = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device="cuda",
                                        generator=g)
                    sc = (0.005 + 0.015 * torch.rand(n, k // 128, device="cuda",
                                                     generator=g)).half()
                    lins.append(QLinear(wf, wq4, n, k, sc).blocked())   # the model's layout
                else:
                    wq8 = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda",
                                        generator=g)
                    sc = (0.005 + 0.015 * torch.rand(n, device="cuda", generator=g)).half()
                    lins.append(QLinear(wf, wq8, n, k, sc).blocked())   # the model's layout
            for M in gemm_ms:
                xm = torch.randn(M, k, device="cuda", generator=g).bfloat16()

                def timed(t, nl, reps):
                    part = torch.empty(t.ksplit, M, n, device="cuda")
                    ob = torch.empty(M, n, device="cuda").bfloat16()

                    def gemm(st):
                        for i in range(nl):
                            lins[i % len(lins)].launch(xm, M, t, out=ob, part=part,
                                                       stream=st.cuda_stream)
                    return _time_graph(gemm, reps) / nl

                key = f"{fmt_name}_{name}_M{M}"
                if fixed is not None:
                    if key not in fixed:
                        continue
                    first = [(0.0, Tiling(*fixed[key]))]
                else:
                    first = sorted((timed(lins[0].plan(M, c)[0], 16, 1), c)
                                   for c in candidates(M, n, k, lins[0].fmt))
                best = min((timed(lins[0].plan(M, c)[0], 64, 3), c) for _, c in first[:4])
                t = lins[0].plan(M, best[1])[0]
                nb = lins[0].nbytes() + 2 * M * k + 2 * M * n
                flops = 2 * M * n * k
                out[f"gemm_{key}"] = {
                    "us": round(best[0], 2),
                    "frac_hbm": round(nb / best[0] / 1e3 / HBM_PEAK_GBS, 4),
                    "frac_mfma": round(flops / best[0] / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4),
                    "tiling": ",".join(map(str, t))}
            del lins
            _release()
    return out


def cpu_baseline(seed: int = 20261027, new_tokens: int = 32, prompt_len: int = 32) -> dict:
    """BASELINE configuration 1 on the CPU oracle of the reference's path
    (oracle/qwen3_ref.py: the SDPA decode path and greedy loop of
    generate.py:55-110, fp32 torch on the host cores): the Qwen3-0.6B-shaped
    model (28 layers, fp32 weights N(0, 0.02), norms 1), batch 1, a prompt of
    `prompt_len` random ids, `new_tokens` greedy tokens, EOS disabled. tok/s
    is the reference's formula (bench.py:68-99): generated tokens / (time of
    the last token - submit), prefill included; decode-only tok/s beside it.
    Also the CPU oracles of the kernels at configuration 2 / 3 shapes (µs per
    call, median of a few calls): K3 paged attention, K1, K2, and the
    dequantise + matmul GEMM anchors at M = 8."""
    import numpy as np
    import torch

    from acorninfer_amd.config import Qwen3Config
    from acorninfer_amd.models.qwen3 import random_state_dict
    from oracle import ops_ref, quant_ref
    from oracle.qwen3_ref import Qwen3Ref

    threads = torch.get_num_threads()
    t_all = time.perf_counter()
    cfg = Qwen3Config.qwen3_0_6b()
    sd = random_state_dict(cfg, seed=seed, std=0.02, dtype=torch.float32)
    ref = Qwen3Ref(cfg, sd, torch.float32)
    del sd
    prompt = torch.randint(0, cfg.vocab_size, (prompt_len,),
                           generator=torch.Generator().manual_seed(seed + 3)).tolist()
    with torch.no_grad():
        cache = ref.new_cache()
        t0 = time.perf_counter()
        last = ref.forward(torch.tensor([prompt]), cache, num_logits_to_keep=1)[0, -1]
        t_first = time.perf_counter()
        ids = [int(last.argmax())]
        for _ in range(new_tokens - 1):
            last = ref.forward(torch.tensor([[ids[-1]]]), cache)[0, -1]
            ids.append(int(last.argmax()))
        t_last = time.perf_counter()
    del ref, cache

    def med_us(fn, reps=3):
        fn()
        ts = []
        for _ in range(reps):
            a = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - a)
        return round(1e6 * sorted(ts)[len(ts) // 2], 1)

    kernels = {}
    g = torch.Generator().manual_seed(seed + 4)
    # K3 at configuration 2
    B, H, KV, D, P, NB = 8, 32, 8, 128, 16, 4096
    lens = torch.randint(512, 4097, (B,), generator=g)
    perm = torch.randperm(NB, generator=g)
    tables = torch.zeros(B, 256, dtype=torch.int32)
    o = 0
    for b in range(B):
        n = -(-int(lens[b]) // P)
        tables[b, :n] = perm[o:o + n].to(torch.int32)
        o += n
    kp = torch.randn(NB, P, KV, D, generator=g).bfloat16()
    vp = torch.randn(NB, P, KV, D, generator=g).bfloat16()
    q = torch.randn(B, H, D, generator=g).bfloat16()
    kernels["K3_config2_us"] = med_us(lambda: ops_ref.paged_attention_ref(q, kp, vp, tables, lens))
    del kp, vp
    x = torch.randn(8, 4096, generator=g).bfloat16()
    r = torch.randn(8, 4096, generator=g).bfloat16()
    w = torch.ones(4096).bfloat16()
    kernels["K1_8x4096_us"] = med_us(lambda: ops_ref.fused_add_rmsnorm_ref(x, r, w, 1e-6), 10)
    kk = torch.randn(8, 8, 1, 128, generator=g).bfloat16()
    qq = torch.randn(8, 32, 1, 128, generator=g).bfloat16()
    wq = torch.ones(128).bfloat16()
    invf = ops_ref.inv_freq_ref(128, 1e6)
    pos = (lens - 1).long()
    kernels["K2_qknorm_rope_us"] = med_us(
        lambda: ops_ref.qknorm_rope_ref(qq, kk, wq, wq, 1e-6, pos, invf), 10)
    # GEMM anchors at configuration 3, M = 8: dequantise (numpy) + fp32 matmul
    rng = np.random.default_rng(seed + 5)
    xm = torch.randn(8, 12288, generator=g)
    for name, (n, k) in {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (24576, 4096),
                         "down": (4096, 12288)}.items():
        u = rng.integers(0, 16, (n, k), dtype=np.uint8)
        s4 = (0.005 + 0.015 * rng.random((n, k // 128))).astype(np.float16)
        xs = xm[:, :k]
        kernels[f"gemm_w4_{name}_M8_us"] = med_us(
            lambda: xs @ torch.from_numpy(quant_ref.dequant_w4_sym_ref(u, s4)).T, 1)
        q8 = rng.integers(-127, 128, (n, k), dtype=np.int8)
        s8 = (0.005 + 0.015 * rng.random(n)).astype(np.float16)
        kernels[f"gemm_w8_{name}_M8_us"] = med_us(
            lambda: xs @ torch.from_numpy(quant_ref.dequant_w8_ref(q8, s8)).T, 1)
        del u, q8
    return {
        "value": round(new_tokens / (t_last - t0), 3),
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"BASELINE configuration 1 whole: oracle/qwen3_ref.py (the reference's SDPA "
                   f"decode path) fp32 on {threads} host threads, Qwen3-0.6B shape (28 layers), "
                   f"batch 1, prompt {prompt_len} random ids, {new_tokens} greedy tokens; "
                   f"tok/s = tokens / (last token - submit), prefill included"),
        "decode_only_tok_s": round((new_tokens - 1) / (t_last - t_first), 3),
        "ttft_ms": round(1e3 * (t_first - t0), 1),
        "kernels_us": kernels,
        "wall_s": round(time.perf_counter() - t_all, 1),
    }


def gpu_config1(seed: int = 20261027, new_tokens: int = 32, prompt_len: int = 32) -> dict:
    """The same configuration-1 run on the GPU path (fp32 parity kernels and
    the bf16 production kernels): prefill of the prompt, then the
    graph-captured step for the remaining tokens; tok/s with the CPU
    baseline's formula."""
    import torch

    from acorninfer_amd.cache.pager import BlockAllocator, PagedCacheView, PagedKVCache
    from acorninfer_amd.config import Qwen3Config
    from acorninfer_amd.engine.graph_runner import DecodeGraphRunner
    from acorninfer_amd.models.qwen3 import Qwen3DecodeModel, random_state_dict
    from types import SimpleNamespace

    cfg = Qwen3Config.qwen3_0_6b()
    prompt = torch.randint(0, cfg.vocab_size, (prompt_len,),
                           generator=torch.Generator().manual_seed(seed + 3)).tolist()
    out = {}
    for dtype, tag in ((torch.float32, "fp32"), (torch.bfloat16, "bf16")):
        sd = random_state_dict(cfg, seed=seed, std=0.02, dtype=dtype, device="cuda")
        model = Qwen3DecodeModel.from_state_dict(cfg, sd, dtype=dtype, device="cuda")
        del sd
        alloc = BlockAllocator(16)
        cache = PagedKVCache(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim, 16,
                             alloc, "cuda", dtype)
        runner = DecodeGraphRunner(model, cache, alloc, max_model_len=prompt_len + new_tokens + 8,
                                   buckets=(1,))
        times = []
        for rep in range(2):                     # the first run captures the graph
            view = PagedCacheView(cache)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            logits = model.forward_prefill_batch(torch.tensor([prompt], device="cuda"), [view],
                                                 real_lens=[prompt_len])
            ids = [int(logits[0].argmax())]
            for _ in range(new_tokens - 1):
                ids.append(runner.decode_batch([SimpleNamespace(generated_ids=ids)], [view])[0])
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
            for blk in view.table:
                alloc.free(blk)
        out[f"config1_{tag}_tok_s"] = round(new_tokens / times[-1], 2)
        del model, runner, cache
        _release()
    return out


def decode_summary(tok_s, ms, gbs, nbytes, args, extra) -> dict:
    """The metric's decode figures in one place: tok/s of bf16 / W4A16 at
    C=1 and C=8 and W8A16 at C=8, each format's GEMM fraction of the 8 TB/s
    peak (timed as a graph of the step's GEMM launches, and inside the
    captured step from the committed profile), and K3's fraction at
    configurations 2 and 5. Figures a --no-extra / --no-kernels run skips
    are None."""
    head = f"{args.format}_C{args.batch}"
    out = {f"{head}_tok_s": round(tok_s, 2), f"{head}_ms_per_step": round(ms, 4)}
    for k in ("bf16_C1", "w4a16_C8", "w4a16_C1", "w8a16_C8"):
        if k != head:
            out[f"{k}_tok_s"] = extra.get(f"{k}_tok_s")
            out[f"{k}_ms_per_step"] = extra.get(f"{k}_ms_per_step")
    ins = in_step_gemm(args.format, args.batch, nbytes)
    graph = {head: round(gbs / HBM_PEAK_GBS, 4)}
    in_step = {head: ins["frac"] if ins else None}
    for fmt in ("w4a16", "w8a16"):
        r = extra.get(f"{fmt}_C8_gemm_roofline")
        if r:
            graph[f"{fmt}_C8"] = r["frac"]
            in_step[f"{fmt}_C8"] = r["in_step"]["frac"] if r.get("in_step") else None
    out["gemm_frac_graph"] = graph
    out["gemm_frac_in_step"] = in_step
    kern = extra.get("kernels", {})
    out["K3_frac"] = {k: kern[f"K3_{k}"]["frac"] for k in ("config2", "config5_C8", "config5_C64")
                      if f"K3_{k}" in kern}
    # the main kernel alone (the combine is its own launch), from the committed profile
    out["K3_main_frac"] = {k: v["main_frac"] for k, v in k3_profile_split().items()}
    return out


def summary_lines(line: dict) -> list[str]:
    """A few short lines that restate the decode figures at the end of the
    run's output (a reader of the last lines sees the whole metric)."""
    d = line["decode"]

    def f(v, nd=1):
        return "n/a" if v is None else f"{v:.{nd}f}"

    toks = " | ".join(f"{k[:-6].replace('_', ' ')} {f(v)}" for k, v in d.items()
                      if k.endswith("_tok_s"))
    gemm = " | ".join(f"{k} {f(v, 3)}/{f(d['gemm_frac_in_step'].get(k), 3)}"
                      for k, v in d["gemm_frac_graph"].items())
    k3 = " | ".join(f"{k} {f(v, 3)}/{f(d['K3_main_frac'].get(k), 3)}"
                    for k, v in d["K3_frac"].items()) or "n/a"
    cpu = line.get("cpu_baseline")
    out = [f"summary decode tok/s: {toks}",
           f"summary GEMM frac of 8 TB/s (graph/in-step): {gemm}",
           f"summary K3 frac of 8 TB/s (main + combine / main alone): {k3}",
           f"summary value {line['value']} {line['unit']} at {line['ms_per_step']} ms/step; "
           f"roofline frac {line['roofline']['frac']}"]
    if cpu:
        out.append(f"summary cpu baseline: {cpu['value']} {cpu['unit']} on {cpu['cores']} "
                   f"threads ({cpu['kind']})")
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--format", default="bf16", choices=["bf16", "w8a16", "w4a16"])
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--prompt-len", type=int, default=512)
    ap.add_argument("--layers", type=int, default=0, help="override layer count (debug only)")
    ap.add_argument("--extra", action="store_true",
                    help="(default) also measure C=1, C=32, W4A16 at C=1/8 and configuration 5 "
                         "(reported under 'extra')")
    ap.add_argument("--no-extra", action="store_true", help="only the C=8 bf16 headline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-tune", action="store_true", help="use the planner's default tilings")
    ap.add_argument("--tilings", default="",
                    help="JSON {projection: [rt, upw, nw, ksplit, tpw], 'swiglu': bool} for the "
                         "headline workload instead of tuning (a profiled run takes an "
                         "unprofiled run's choice: the profiler distorts the tuner's timings)")
    ap.add_argument("--no-kernels", action="store_true",
                    help="skip the isolated kernels at configurations 2, 3 and 5")
    ap.add_argument("--splits", default="",
                    help="with --mode attention: comma-separated K3 split counts to time")
    ap.add_argument("--mode", default="full",
                    choices=["full", "step", "attention", "kernels", "copy", "prefill", "dense"],
                    help="profiling workloads: 'step' = decode steps only (no JSON line), "
                         "'prefill' = --batch prompts of --prompt-len random ids prefilled "
                         "(one warm-up call, --steps timed calls; no JSON line), 'dense' = "
                         "the large-M bf16 GEMMs at M = 512 / 2048 / 8192 against hipBLASLt, "
                         "'attention' = K3 at configuration 2 only, 'kernels' = the isolated "
                         "kernels only (configurations 2, 3, 5), 'copy' = the 1 GiB "
                         "copy that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--gemm-m", default="",
                    help="with --mode kernels: comma-separated M of the configuration-3 GEMMs "
                         "only (no attention / norm kernels)")
    ap.add_argument("--gemm-tilings", default="",
                    help="with --mode kernels --gemm-m: JSON {'{w4|w8}_{shape}_M{M}': tiling} "
                         "timed instead of searched")
    ap.add_argument("--seed", type=int, default=20261027)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the decode step is sized for one MI355X; see the sharding notes).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from acorninfer_amd.config import Qwen3Config

    if args.mode == "copy":
        a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        _log("copied 1 GiB x 5")
        return
    if args.mode == "kernels":
        ms = tuple(int(m) for m in args.gemm_m.split(",")) if args.gemm_m else (1, 8, 64, 256)
        if args.gemm_tilings:
            print(json.dumps(gemm_benchmarks(23, ms, json.loads(args.gemm_tilings))), flush=True)
        else:
            print(json.dumps(kernel_benchmarks(gemm_ms=ms, with_attention=not args.gemm_m)),
                  flush=True)
        return
    if args.mode == "dense":
        print(json.dumps(dense_gemm_benchmarks(23)), flush=True)
        return
    if args.mode == "attention":
        sweep = [int(x) for x in args.splits.split(",")] if args.splits else None
        _log(f"K3 configuration 2: {kernel_benchmarks(only_attention=True, attn_splits=sweep)}")
        return
    cfg = Qwen3Config.qwen3_8b()
    if args.layers:
        cfg = cfg.with_layers(args.layers)
    if args.mode == "prefill":
        from acorninfer_amd.models.qwen3 import Qwen3DecodeModel
        model = Qwen3DecodeModel.random_init(cfg, weight_format=args.format, device="cuda:0")
        ms_p, tps = prefill_benchmark(model, cfg, args.batch, args.prompt_len, args.seed,
                                      reps=args.steps)
        _log(f"{args.format} prefill {args.batch} x {args.prompt_len}: {ms_p:.2f} ms "
             f"({tps:.0f} prompt tok/s)")
        return
    total = args.warmup + args.steps
    # room for the decode_batch protocol's steps after the timed decode_loop ones
    model, cache, runner, views, first = build_workload(
        cfg, args.format, args.batch, args.prompt_len, total + args.steps + 2, args.seed,
        tune=not args.no_tune,
        tilings=json.loads(args.tilings) if args.tilings else None)
    tilings_arg = json.dumps({**{k: list(v) for k, v in model.tilings.get(args.batch, {}).items()},
                              "swiglu": model.fused_swiglu(args.batch),
                              "fold": model.fold_possible(args.batch)}, separators=(",", ":"))
    _log(f"tilings of this run (--tilings): {tilings_arg}")
    _log(f"graph captured for C={args.batch}; warmup {args.warmup}, timed {args.steps}")
    dt, log = time_decode(runner, views, first, args.steps, args.warmup)
    tok_s = args.batch * args.steps / dt
    ms = dt * 1e3 / args.steps
    _log(f"decode: {tok_s:.1f} tok/s, {ms:.3f} ms/step; last tokens {log[-1].tolist()}")
    if args.mode == "step":
        _log(f"GEMM algorithmic bytes per step: {gemm_step_bytes(model, args.batch)}")
        return
    dtb = time_decode_batch(runner, views, log[-1].tolist(), args.steps)
    gbs, nbytes, us, nl = gemm_roofline(model, runner, args.batch)
    _log(f"GEMM: {nl} launches/step, {nbytes / 1e9:.3f} GB, {us:.1f} us -> {gbs:.0f} GB/s")
    step_bytes = model.weight_bytes() + sum(
        v.seq_len for v in views) * cfg.num_hidden_layers * cfg.num_key_value_heads * \
        cfg.head_dim * 2 * 2
    extra = {"step_hbm_bound_ms": round(step_bytes / (HBM_PEAK_GBS * 1e9) * 1e3, 4),
             "step_roofline_frac": round(step_bytes / (HBM_PEAK_GBS * 1e9) / (dt / args.steps), 4),
             "gemm_us_per_step": round(us, 2), "gemm_launches_per_step": nl,
             f"{args.format}_C{args.batch}_decode_batch_tok_s": round(args.batch * args.steps / dtb, 2),
             "tilings_arg": tilings_arg,
             "tuned": {k: {"tiling": v["tiling"], "us": v["us"],
                           "GBps": round(v["bytes"] / v["us"] / 1e3, 1)}
                       for k, v in model.tune_report.items() if k != "fold"},
             "fold": model.tune_report.get("fold")}
    if not args.no_extra:
        # configuration 4's prompts: prefill of C x 512 random ids (TTFT of a batch)
        for c in (1, args.batch):
            ms_p, tps = prefill_benchmark(model, cfg, c, args.prompt_len, args.seed + 7)
            extra[f"bf16_prefill_C{c}_ms"] = round(ms_p, 3)
            extra[f"bf16_prefill_C{c}_tok_s"] = round(tps, 1)
            _log(f"bf16 prefill C={c} x {args.prompt_len}: {ms_p:.2f} ms ({tps:.0f} tok/s)")
        # configuration 5's longest prompt: one 8192-token prefill (the
        # projections on this library's large-M kernel; its GEMMs against
        # hipBLASLt are in kernels.dense_gemm_*)
        ms_p, tps = prefill_benchmark(model, cfg, 1, 8192, args.seed + 8, reps=2)
        extra["bf16_prefill_1x8192_ms"] = round(ms_p, 3)
        extra["bf16_prefill_1x8192_tok_s"] = round(tps, 1)
        _log(f"bf16 prefill 1 x 8192: {ms_p:.2f} ms ({tps:.0f} tok/s)")
        model._extend_buf = None
        # configuration 4 end to end through the Engine (prefill + decode)
        del cache, runner, views
        _release()
        e2e, ttft = engine_benchmark(model, cfg, args.batch, args.prompt_len, 256, args.seed + 9)
        extra[f"bf16_engine_C{args.batch}_tok_s"] = round(e2e, 1)
        extra[f"bf16_engine_C{args.batch}_ttft_ms"] = round(ttft, 2)
        _log(f"bf16 engine C={args.batch}, {args.prompt_len} + 256 tokens: {e2e:.1f} tok/s "
             f"end to end, TTFT {ttft:.1f} ms")
        del model
        _release()
        for fmt, c in (("bf16", 1), ("w4a16", 8), ("w4a16", 1), ("w8a16", 8)):
            m2, c2, r2, v2, f2 = build_workload(cfg, fmt, c, args.prompt_len, total, args.seed,
                                                tune=not args.no_tune)
            dt2, _ = time_decode(r2, v2, f2, args.steps, args.warmup)
            extra[f"{fmt}_C{c}_tok_s"] = round(c * args.steps / dt2, 2)
            extra[f"{fmt}_C{c}_ms_per_step"] = round(dt2 * 1e3 / args.steps, 4)
            if m2.tune_report.get("fold"):
                extra[f"{fmt}_C{c}_fold"] = m2.tune_report["fold"]
            _log(f"{fmt} C={c}: {c * args.steps / dt2:.1f} tok/s "
                 f"(fold {m2.tune_report.get('fold')})")
            if c == 8 and fmt != "bf16":
                # the quantised formats' own GEMM roofline (the line's is bf16's)
                g2, nb2, us2, nl2 = gemm_roofline(m2, r2, c)
                extra[f"{fmt}_C8_gemm_roofline"] = {
                    "achieved_GBps": round(g2, 1), "frac": round(g2 / HBM_PEAK_GBS, 4),
                    "bytes_per_step": nb2, "us_per_step": round(us2, 2), "launches": nl2,
                    "traffic": measured_traffic(fmt, c), "in_step": in_step_gemm(fmt, c, nb2),
                    "tilings_arg": json.dumps(
                        {**{k: list(v) for k, v in m2.tilings.get(c, {}).items()},
                         "swiglu": m2.fused_swiglu(c), "fold": m2.fold_possible(c)},
                        separators=(",", ":"))}
                _log(f"{fmt} C=8 GEMM: {nb2 / 1e9:.3f} GB in {us2:.1f} us -> {g2:.0f} GB/s")
            del m2, c2, r2, v2, f2
            _release()
        # configuration 4's largest concurrency: C=32, bf16, prompts of 512
        m2, c2, r2, v2, f2 = build_workload(cfg, "bf16", 32, args.prompt_len, total, args.seed,
                                            tune=not args.no_tune)
        dt2, _ = time_decode(r2, v2, f2, args.steps, args.warmup)
        extra["bf16_C32_tok_s"] = round(32 * args.steps / dt2, 2)
        extra["bf16_C32_ms_per_step"] = round(dt2 * 1e3 / args.steps, 4)
        _log(f"bf16 C=32: {32 * args.steps / dt2:.1f} tok/s")
        del m2, c2, r2, v2, f2
        _release()
        # configuration 5: W4A16, prompts U[1024, 8192], sampled, C=8 and C=64
        from acorninfer_amd.sampler import SamplingParams
        for c in (8, 64):
            plens = torch.randint(1024, 8193, (c,), generator=torch.Generator().manual_seed(
                args.seed + 5)).tolist()
            m2, c2, r2, v2, f2 = build_workload(cfg, "w4a16", c, 0, total, args.seed,
                                                tune=not args.no_tune, prompt_lens=plens)
            sp = [SamplingParams(temperature=0.6, top_p=0.95, top_k=20)] * c
            dt2, _ = time_decode(r2, v2, f2, args.steps, args.warmup, sampling=sp)
            extra[f"w4a16_C{c}_long_sampled_tok_s"] = round(c * args.steps / dt2, 2)
            extra[f"w4a16_C{c}_long_sampled_ms_per_step"] = round(dt2 * 1e3 / args.steps, 4)
            extra[f"w4a16_C{c}_long_sampled_mean_ctx"] = round(sum(plens) / c, 1)
            _log(f"w4a16 C={c} long sampled (mean ctx {sum(plens) / c:.0f}): "
                 f"{c * args.steps / dt2:.1f} tok/s")
            if c == 64:
                # configuration 5 end to end through the Engine: the same 64
                # prompt lengths prefilled, then 128 sampled tokens each
                del c2, r2, v2, f2
                _release()
                e2e, ttft = engine_benchmark(m2, cfg, c, plens, 128, args.seed + 11,
                                             sampling=SamplingParams(temperature=0.6, top_p=0.95,
                                                                     top_k=20),
                                             warm_len=64)
                extra["w4a16_engine_C64_long_tok_s"] = round(e2e, 1)
                extra["w4a16_engine_C64_long_ttft_ms"] = round(ttft, 1)
                _log(f"w4a16 engine C=64, prompts U[1024, 8192] + 128 sampled tokens: "
                     f"{e2e:.1f} tok/s end to end, mean TTFT {ttft:.0f} ms")
                del m2
                _release()
                continue
            if c == 8:
                # configuration 5's longest prompt in W4A16: one 8192-token
                # prefill, int4 projections dequantised onto the bf16 kernel
                # ("own") and on the int4 kernels themselves
                del c2, r2, v2, f2
                _release()
                for how in ("own", "int4"):
                    m2.prefill_gemm = how
                    ms_p, tps = prefill_benchmark(m2, cfg, 1, 8192, args.seed + 8, reps=2)
                    sfx = "" if how == "own" else "_int4_gemm"
                    extra[f"w4a16_prefill_1x8192{sfx}_ms"] = round(ms_p, 3)
                    extra[f"w4a16_prefill_1x8192{sfx}_tok_s"] = round(tps, 1)
                    _log(f"w4a16 prefill 1 x 8192 ({how}): {ms_p:.2f} ms ({tps:.0f} tok/s)")
                m2._extend_buf = None
                del m2
                _release()
                continue
            del m2, c2, r2, v2, f2
            _release()
    if not args.no_kernels:
        t0 = time.perf_counter()
        extra["kernels"] = kernel_benchmarks()
        _log(f"kernel benchmarks in {time.perf_counter() - t0:.1f} s")
    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        cpu = cpu_baseline()
        cpu["gpu_same_workload"] = gpu_config1()
        _log(f"cpu baseline (configuration 1) {cpu['value']} tok/s in "
             f"{time.perf_counter() - t0:.1f} s")
    line = {
        "metric": "decode tok/s Qwen3-8B C=1/8 (bf16, W4A16); kernel HBM GB/s vs 8 TB/s peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.format == "bf16" else f"bf16 activations, {args.format} weights",
        "data": "synthetic: random-init weights N(0,0.02), random prompt KV, greedy ids",
        "config": {"workload": f"Qwen3-8B-shaped decode, C={args.batch}, prompt "
                               f"{args.prompt_len}, {args.format}, hipGraph step, page 16",
                   "batch": args.batch, "prompt_len": args.prompt_len,
                   "layers": cfg.num_hidden_layers, "weights": args.format},
        "decode": decode_summary(tok_s, ms, gbs, nbytes, args, extra),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(args.format, args.batch),
                     "kernel": "weight-streaming GEMMs (all projections of one step)",
                     "bytes_per_step": nbytes, "us_per_step": round(us, 2),
                     "in_step": in_step_gemm(args.format, args.batch, nbytes)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line, separators=(",", ":")), flush=True)
    for msg in summary_lines(line):
        _log(msg)


if __name__ == "__main__":
    main()
