"""hipGraph decode runner: one captured decode step per batch bucket.

Protocol of acorninfer/engine/graph_runner.py:61-184 (`DecodeGraphRunner`),
re-designed for MI355X serving sizes:

- one graph per bucket (BUCKETS up to 64, the reference stops at 8); the
  graph body is `Qwen3DecodeModel.step` over that bucket's `StepBuffers`;
- the host fills pinned mirrors (ids | positions | pages | slots as one
  int64 block, lens | tables as one int32 block) and issues one H2D copy per
  block before the replay; tables are [bucket, max_pages] with max_pages =
  ceil(max_model_len / page) (the reference uses the whole pool as width);
- padding rows write their K/V to a resident scratch block, read one token
  of it, and their outputs are ignored; the scratch block is allocated at
  construction and never freed (so a drained engine holds exactly one live
  block, as in the reference);
- per-layer lengths are committed on the host, outside the graph
  (`_commit_lens`);
- `decode_batch` returns the greedy tokens with one device-to-host copy per
  step (the reference's contract); `decode_loop` keeps the greedy tokens on
  the device (the graph ends by copying them into the next step's ids) and
  copies the whole token log back once, so host preparation of step t+1
  overlaps the GPU's step t.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from acorninfer_amd.models.qwen3 import Qwen3DecodeModel, StepBuffers

BUCKETS = (1, 2, 4, 8, 16, 32, 64)
WARMUP_STEPS = 3
MIRRORS = 4          # pinned mirror ring per bucket (host runs ahead of the GPU)


@dataclass
class _Bucket:
    bucket: int
    buf: StepBuffers
    graph: torch.cuda.CUDAGraph | None
    pin: list[torch.Tensor]           # ring of pinned byte mirrors of buf.meta
    pin_i64: list[torch.Tensor]       # their int64 ids|positions|pages|slots
    pin_i32: list[torch.Tensor]       # their int32 lens|tables
    pin_f32: list[torch.Tensor]       # their f32 temperature|top_p|uniform|top_k
    done: list[torch.cuda.Event | None]
    turn: int = 0
    sampled: bool = False             # the device block holds sampling rows


class DecodeGraphRunner:
    def __init__(self, model: Qwen3DecodeModel, cache, allocator, *, max_model_len: int,
                 buckets: tuple[int, ...] = BUCKETS, capture: bool = True, seed: int = 0):
        self.model = model
        self.cache = cache
        self.allocator = allocator
        self.num_layers = model.cfg.num_hidden_layers
        self.page_size = cache.page_size
        self.max_pages = -(-max_model_len // cache.page_size)
        self.device = model.device
        self.scratch = allocator.allocate()      # resident; padding rows' KV target
        self.buckets = tuple(sorted(buckets))
        self.states: dict[int, _Bucket] = {}
        self.capture = capture
        self.last_logits: torch.Tensor | None = None
        self.last_logprobs: torch.Tensor | None = None
        self.rng = torch.Generator().manual_seed(seed)   # uniforms of sampled rows

    # ------------------------------------------------------------- construction --
    def _state(self, B: int) -> _Bucket:
        bk = min(b for b in self.buckets if b >= B)
        st = self.states.get(bk)
        if st is None:
            st = self._build(bk)
            self.states[bk] = st
        return st

    def _build(self, bk: int) -> _Bucket:
        buf = self.model.buffers(bk, self.max_pages)
        W = self.max_pages
        e64, e32, ef = buf.meta_ends
        pin, pin_i64, pin_i32, pin_f32 = [], [], [], []
        for _ in range(MIRRORS):
            m = torch.zeros(ef, dtype=torch.uint8, pin_memory=True)
            a, b, f = m[:e64].view(torch.int64), m[e64:e32].view(torch.int32), m[e32:].view(
                torch.float32)
            f[bk:2 * bk] = 1.0                       # top_p off
            a[2 * bk:3 * bk] = self.scratch          # pages of padding rows
            b[0:bk] = 1                              # lens of padding rows
            b[bk:].view(bk, W)[:, 0] = self.scratch  # their table points at scratch
            pin.append(m)
            pin_i64.append(a)
            pin_i32.append(b)
            pin_f32.append(f)
        # device side starts from the same "all padding" state
        buf.meta.copy_(pin[0].to(self.device))
        st = _Bucket(bk, buf, None, pin, pin_i64, pin_i32, pin_f32, [None] * MIRRORS)
        if self.capture:
            self._capture(st)
        return st

    def _body(self, st: _Bucket) -> None:
        c = self.cache
        # the sampler writes the next ids over buf.ids (device-fed decode_loop)
        self.model.step(st.buf, c.k_pool, c.v_pool, c.num_blocks, c.page_size)

    def _capture(self, st: _Bucket) -> None:
        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            for _ in range(WARMUP_STEPS):
                self._body(st)
        torch.cuda.current_stream(self.device).wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._body(st)
        st.graph = g

    def _run(self, st: _Bucket) -> None:
        if st.graph is not None:
            st.graph.replay()
        else:
            self._body(st)

    # -------------------------------------------------------------- per step --
    def _prepare(self, st: _Bucket, views, ids: list[int] | None, sampling=None) -> list[int]:
        """Fill the next pinned mirror and copy it to the step's buffers.
        `sampling`: None (all greedy) or one SamplingParams-like (temperature,
        top_k, top_p) per row; each sampled row draws a fresh uniform from the
        runner's generator. Returns the new lengths (pre-write + 1)."""
        from acorninfer_amd.ops.paged_attention import build_tables
        B, bk = len(views), st.bucket
        j = st.turn % MIRRORS
        st.turn += 1
        if st.done[j] is not None:
            st.done[j].synchronize()                 # the copy that read this mirror is done
        a, b = st.pin_i64[j], st.pin_i32[j]
        targets = [v.ensure_append_capacity(0) for v in views]
        pre = [int(v.seq_len) for v in views]
        new_len = [p + 1 for p in pre]
        if ids is not None:
            a[0:B] = torch.tensor(ids, dtype=torch.int64)
        a[bk:bk + B] = torch.tensor(pre, dtype=torch.int64)
        a[2 * bk:2 * bk + B] = torch.tensor([p for p, _ in targets], dtype=torch.int64)
        a[3 * bk:3 * bk + B] = torch.tensor([s for _, s in targets], dtype=torch.int64)
        a[2 * bk + B:3 * bk] = self.scratch          # padding rows back onto scratch
        a[3 * bk + B:4 * bk] = 0
        b[0:B] = torch.tensor(new_len, dtype=torch.int32)
        b[B:bk] = 1
        tables = b[bk:].view(bk, self.max_pages)
        build_tables(views, self.page_size, self.device, lens_override=new_len, out=tables)
        tables[B:].zero_()
        tables[B:, 0] = self.scratch
        buf = st.buf
        f = st.pin_f32[j]
        send_f32 = sampling is not None or st.sampled
        if send_f32:
            f.zero_()
            f[bk:2 * bk] = 1.0
            st.sampled = False
            if sampling is not None:
                u = torch.rand(B, generator=self.rng)
                for i, sp in enumerate(sampling):
                    if sp is None or sp.temperature == 0:
                        continue
                    f[i] = sp.temperature
                    f[bk + i] = sp.top_p
                    f[2 * bk + i] = u[i]
                    f[3 * bk:4 * bk].view(torch.int32)[i] = sp.top_k
                    st.sampled = True
        # one copy: ids (when given) .. tables (.. the sampling block)
        _, e32, ef = buf.meta_ends
        lo = 0 if ids is not None else 8 * bk
        hi = ef if send_f32 else e32
        buf.meta[lo:hi].copy_(st.pin[j][lo:hi], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        st.done[j] = ev
        self._commit_lens(views, new_len)
        return new_len

    def _commit_lens(self, views, new_len) -> None:
        for v, n in zip(views, new_len):
            for li in range(self.num_layers):
                v._lens[li] = n

    def decode_batch(self, seqs, views) -> list[int]:
        """One decode step for `views` (ids = each seq's last generated id).
        Same arguments and result as the reference's runner; rows whose
        `seq.sampling` has temperature > 0 are sampled inside the graph (the
        reference routes them to eager decoding)."""
        B = len(views)
        assert 1 <= B <= self.buckets[-1], f"batch {B} exceeds the largest bucket"
        assert len(seqs) == B, "seqs and views must correspond"
        st = self._state(B)
        sampling = [getattr(s, "sampling", None) for s in seqs]
        if all(sp is None or sp.temperature == 0 for sp in sampling):
            sampling = None
        self._prepare(st, views, [int(s.generated_ids[-1]) for s in seqs], sampling)
        self._run(st)
        self.last_logits = st.buf.logits
        self.last_logprobs = st.buf.logprob
        toks = st.buf.next_ids[:B].tolist()
        if sampling is not None and int(st.buf.status[:B].max()) != 0:
            raise ValueError("logits contain NaN/inf; model forward is broken")
        return toks

    def decode_loop(self, views, first_ids: list[int], steps: int, sampling=None
                    ) -> torch.Tensor:
        """`steps` decode steps starting from `first_ids` (greedy, or per-row
        `sampling` params), tokens fed back on the device. Returns the int64
        token log [steps, B] (one D2H copy)."""
        B = len(views)
        st = self._state(B)
        log = torch.empty(steps, st.bucket, dtype=torch.int64, device=self.device)
        for t in range(steps):
            self._prepare(st, views, first_ids if t == 0 else None, sampling)
            self._run(st)
            log[t].copy_(st.buf.ids)               # = this step's greedy tokens
        self.last_logits = st.buf.logits
        return log[:, :B].cpu()
