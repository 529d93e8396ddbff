"""Decode throughput of the Qwen3-8B-shaped hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--format bf16|w4a16|w8a16]
                    [--batch C] [--prompt-len L] [--extra] [--no-cpu-baseline]

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
- extra (unless --no-extra): other batch sizes and formats, and the batched
  prefill (forward_prefill_batch) of C prompts of L random ids: ms per call
  and prompt tokens per second.
- cpu_baseline: the CPU oracle of the reference's path (oracle/qwen3_ref.py,
  fp32 torch on the host cores) on a bounded sample of the same workload
  (C sequences at context L, a few decode steps of a few layers plus the
  lm_head), scaled to the 36-layer step.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


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


def build_workload(cfg, fmt: str, batch: int, prompt_len: int, total_steps: int, seed: int,
                   tune: bool = True, prompt_lens: list[int] | None = None):
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
    if tune:
        t0 = time.perf_counter()
        report = model.tune(batch)
        _log(f"tuned C={batch} in {time.perf_counter() - t0:.1f} s: " + ", ".join(
            f"{k} {v['tiling']} {v['us']:.1f}us {v['bytes'] / v['us'] / 1e3:.0f}GB/s"
            for k, v in report.items()))
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


def engine_benchmark(model, cfg, concurrency: int, prompt_len: int, new_tokens: int,
                     seed: int):
    """Configuration 4 end to end: `concurrency` greedy requests of
    `prompt_len` random ids and `new_tokens` generated tokens each, submitted
    at once to the Engine (continuous batching: batched prefill, then the
    graph-captured decode step). Returns (generated tok/s over the wall time
    of the whole run, mean time to first token in ms)."""
    import torch

    from acorninfer_amd.engine.engine import Engine
    from acorninfer_amd.sampler import SamplingParams

    P = 16
    blocks = concurrency * -(-(prompt_len + new_tokens + 1) // P) + 8
    eng = Engine(model, num_blocks=blocks, max_running=concurrency, watermark_blocks=1,
                 max_model_len=prompt_len + new_tokens + 1, seed=seed)
    g = torch.Generator().manual_seed(seed)
    greedy = SamplingParams(temperature=0.0)
    never = frozenset({-1})

    def run(n_new):
        ids = [eng.submit(torch.randint(0, cfg.vocab_size, (prompt_len,), generator=g).tolist(),
                          greedy, max_tokens=n_new, eos_ids=never) for _ in range(concurrency)]
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

    run(4)                                    # warm-up: captures the decode graph
    dt, ttft = run(new_tokens)
    eng.assert_balanced()
    return concurrency * new_tokens / dt, ttft


def gemm_roofline(model, runner, batch: int, reps: int = 5):
    """Time one step's GEMM launches (hipGraph on a private stream, HIP events
    on that stream). Returns (achieved GB/s, per-step bytes, per-step µs,
    launches per step)."""
    import torch
    st = runner._state(batch)
    buf = st.buf
    s = torch.cuda.Stream()
    launches = []
    for lw in model.layers:
        launches += [("qkv", lw.qkv, buf.normed, buf.part_qkv), ("o", lw.o, buf.attn, buf.part_o),
                     ("gate_up", lw.gate_up, buf.normed, "swiglu" if buf.swiglu else buf.part_gu),
                     ("down", lw.down, buf.act, buf.part_down)]
    launches.append(("lm_head", model.lm_head, buf.normed, None))
    nbytes = sum(_gemm_bytes(lin, batch) for _, lin, *_ in launches)

    def body():
        sp = s.cuda_stream
        for name, lin, x, part in launches:
            if part is None:
                lin.launch(x, batch, buf.cfgs[name], out=buf.logits, part=buf.ws_lm, stream=sp)
            elif isinstance(part, str):
                lin.launch_swiglu(x, batch, buf.cfgs[name], buf.act, sp)
            else:
                lin.launch(x, batch, buf.cfgs[name], part=part, stream=sp)

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
                      attn_splits: list[int] | None = None) -> dict:
    """Isolated kernels at BASELINE configurations 2 and 3 (algorithmic bytes
    / time, HIP events around hipGraph replays)."""
    import torch

    from acorninfer_amd import _lib
    from acorninfer_amd._lib import lib, ptr
    from acorninfer_amd.models.qwen3 import QLinear, attention_splits
    from acorninfer_amd.ops.quant_gemm import candidates

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
    if only_attention:
        return out
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
    # ---- quant GEMM, configuration 3 -------------------------------------
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
                    lins.append(QLinear(wf, wq8, n, k, sc))
            for M in (1, 8, 64, 256):
                xm = torch.randn(M, k, device="cuda", generator=g).bfloat16()
                best = None
                cands = candidates(M, n, k, lins[0].fmt)
                for c in cands:
                    t = lins[0].plan(M, c)[0]
                    part = torch.empty(t.ksplit, M, n, device="cuda")
                    ob = torch.empty(M, n, device="cuda").bfloat16()

                    nl = max(64, len(lins))

                    def gemm(st, t=t, part=part, ob=ob, nl=nl):
                        for i in range(nl):
                            lins[i % len(lins)].launch(xm, M, t, out=ob, part=part,
                                                       stream=st.cuda_stream)
                    us = _time_graph(gemm, 3) / nl
                    if best is None or us < best[0]:
                        best = (us, t)
                nb = lins[0].nbytes() + 2 * M * k + 2 * M * n
                flops = 2 * M * n * k
                out[f"gemm_{fmt_name}_{name}_M{M}"] = {
                    "us": round(best[0], 2), "GBps": round(nb / best[0] / 1e3, 1),
                    "frac_hbm": round(nb / best[0] / 1e3 / HBM_PEAK_GBS, 4),
                    "TFLOPs": round(flops / best[0] / 1e6, 2), "tiling": tuple(best[1])}
            del lins
            torch.cuda.empty_cache()
    return out


def cpu_baseline(cfg, batch: int, prompt_len: int, layers: int = 2, steps: int = 2):
    """The CPU oracle (fp32 torch) on a bounded sample of the same step:
    `layers` of the 36 layers plus the lm_head, `steps` decode steps of
    `batch` sequences at context `prompt_len`; the per-step time is scaled to
    36 layers."""
    import torch

    from acorninfer_amd.models.qwen3 import random_state_dict
    from oracle.qwen3_ref import Qwen3Ref

    threads = torch.get_num_threads()
    sub = cfg.with_layers(layers)
    sd = random_state_dict(sub, seed=5, std=0.02, dtype=torch.float32)
    ref = Qwen3Ref(sub, sd, torch.float32)
    del sd
    g = torch.Generator().manual_seed(6)
    shape = (batch, cfg.num_key_value_heads, prompt_len, cfg.head_dim)
    cache = [[torch.randn(*shape, generator=g), torch.randn(*shape, generator=g)]
             for _ in range(layers)]
    ids = torch.randint(0, cfg.vocab_size, (batch, 1), generator=g)
    # split the step into the layer part and the lm_head part
    t_total = 0.0
    for _ in range(steps):
        t0 = time.perf_counter()
        ref.forward(ids, cache)
        t_total += time.perf_counter() - t0
    per_step_sample = t_total / steps
    h = torch.randn(batch, 1, cfg.hidden_size, generator=g)
    t0 = time.perf_counter()
    for _ in range(steps):
        ref._linear(h, "lm_head")
    t_head = (time.perf_counter() - t0) / steps
    t_layers = max(per_step_sample - t_head, 0.0)
    t_step = t_layers * cfg.num_hidden_layers / layers + t_head
    return {
        "value": round(batch / t_step, 4),
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle/qwen3_ref.py fp32 on {threads} host threads: {steps} decode steps "
                   f"of {batch} sequences at context {prompt_len}, {layers} of "
                   f"{cfg.num_hidden_layers} layers + lm_head, scaled to "
                   f"{cfg.num_hidden_layers} layers ({t_step:.2f} s/step)"),
    }


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
    ap.add_argument("--kernels", action="store_true",
                    help="also time the isolated kernels at configurations 2 and 3")
    ap.add_argument("--splits", default="",
                    help="with --mode attention: comma-separated K3 split counts to time")
    ap.add_argument("--mode", default="full", choices=["full", "step", "attention", "copy"],
                    help="profiling workloads: 'step' = decode steps only (no JSON line), "
                         "'attention' = K3 at configuration 2 only, 'copy' = the 1 GiB "
                         "copy that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE")
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
    if args.mode == "attention":
        sweep = [int(x) for x in args.splits.split(",")] if args.splits else None
        _log(f"K3 configuration 2: {kernel_benchmarks(only_attention=True, attn_splits=sweep)}")
        return
    cfg = Qwen3Config.qwen3_8b()
    if args.layers:
        cfg = cfg.with_layers(args.layers)
    total = args.warmup + args.steps
    model, cache, runner, views, first = build_workload(cfg, args.format, args.batch,
                                                        args.prompt_len, total, args.seed,
                                                        tune=not args.no_tune)
    _log(f"graph captured for C={args.batch}; warmup {args.warmup}, timed {args.steps}")
    dt, log = time_decode(runner, views, first, args.steps, args.warmup)
    tok_s = args.batch * args.steps / dt
    ms = dt * 1e3 / args.steps
    _log(f"decode: {tok_s:.1f} tok/s, {ms:.3f} ms/step; last tokens {log[-1].tolist()}")
    if args.mode == "step":
        return
    gbs, nbytes, us, nl = gemm_roofline(model, runner, args.batch)
    _log(f"GEMM: {nl} launches/step, {nbytes / 1e9:.3f} GB, {us:.1f} us -> {gbs:.0f} GB/s")
    step_bytes = model.weight_bytes() + sum(
        v.seq_len for v in views) * cfg.num_hidden_layers * cfg.num_key_value_heads * \
        cfg.head_dim * 2 * 2
    extra = {"step_hbm_bound_ms": round(step_bytes / (HBM_PEAK_GBS * 1e9) * 1e3, 4),
             "step_roofline_frac": round(step_bytes / (HBM_PEAK_GBS * 1e9) / (dt / args.steps), 4),
             "gemm_us_per_step": round(us, 2), "gemm_launches_per_step": nl,
             "tuned": {k: {"tiling": v["tiling"], "us": v["us"],
                           "GBps": round(v["bytes"] / v["us"] / 1e3, 1)}
                       for k, v in model.tune_report.items()}}
    if not args.no_extra:
        # configuration 4's prompts: prefill of C x 512 random ids (TTFT of a batch)
        for c in (1, args.batch):
            ms_p, tps = prefill_benchmark(model, cfg, c, args.prompt_len, args.seed + 7)
            extra[f"bf16_prefill_C{c}_ms"] = round(ms_p, 3)
            extra[f"bf16_prefill_C{c}_tok_s"] = round(tps, 1)
            _log(f"bf16 prefill C={c} x {args.prompt_len}: {ms_p:.2f} ms ({tps:.0f} tok/s)")
        # configuration 4 end to end through the Engine (prefill + decode)
        del cache, runner
        torch.cuda.empty_cache()
        e2e, ttft = engine_benchmark(model, cfg, args.batch, args.prompt_len, 256, args.seed + 9)
        extra[f"bf16_engine_C{args.batch}_tok_s"] = round(e2e, 1)
        extra[f"bf16_engine_C{args.batch}_ttft_ms"] = round(ttft, 2)
        _log(f"bf16 engine C={args.batch}, {args.prompt_len} + 256 tokens: {e2e:.1f} tok/s "
             f"end to end, TTFT {ttft:.1f} ms")
        del model
        torch.cuda.empty_cache()
        for fmt, c in (("bf16", 1), ("w4a16", 8), ("w4a16", 1)):
            m2, c2, r2, v2, f2 = build_workload(cfg, fmt, c, args.prompt_len, total, args.seed,
                                                tune=not args.no_tune)
            dt2, _ = time_decode(r2, v2, f2, args.steps, args.warmup)
            extra[f"{fmt}_C{c}_tok_s"] = round(c * args.steps / dt2, 2)
            extra[f"{fmt}_C{c}_ms_per_step"] = round(dt2 * 1e3 / args.steps, 4)
            _log(f"{fmt} C={c}: {c * args.steps / dt2:.1f} tok/s")
            del m2, c2, r2
            torch.cuda.empty_cache()
        # configuration 4's largest concurrency: C=32, bf16, prompts of 512
        m2, c2, r2, v2, f2 = build_workload(cfg, "bf16", 32, args.prompt_len, total, args.seed,
                                            tune=not args.no_tune)
        dt2, _ = time_decode(r2, v2, f2, args.steps, args.warmup)
        extra["bf16_C32_tok_s"] = round(32 * args.steps / dt2, 2)
        extra["bf16_C32_ms_per_step"] = round(dt2 * 1e3 / args.steps, 4)
        _log(f"bf16 C=32: {32 * args.steps / dt2:.1f} tok/s")
        del m2, c2, r2
        torch.cuda.empty_cache()
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
            del m2, c2, r2
            torch.cuda.empty_cache()
    if args.kernels:
        t0 = time.perf_counter()
        extra["kernels"] = kernel_benchmarks()
        _log(f"kernel benchmarks in {time.perf_counter() - t0:.1f} s: {extra['kernels']}")
    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        cpu = cpu_baseline(cfg, args.batch, args.prompt_len)
        _log(f"cpu baseline {cpu['value']} tok/s in {time.perf_counter() - t0:.1f} s")
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
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(args.format, args.batch),
                     "kernel": "wgemm_kernel (all projections of one step)",
                     "bytes_per_step": nbytes, "us_per_step": round(us, 2)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
