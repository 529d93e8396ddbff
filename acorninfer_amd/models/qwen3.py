"""Qwen3 dense decode step on the MI355X kernels.

Mirrors the decode half of acorninfer/models/qwen3.py:
`Qwen3ForCausalLM.forward_decode` (:520-595) with its fused branch
(`Qwen3Block.forward_decode` :412-439, `Qwen3Attention.forward_decode`
:154-233 with attention_backend="triton" and fused_ops=True) and
`dispatch_linear` (:21-47).

The step is a fixed sequence of libacorn_hip.so launches over static
buffers (`StepBuffers`), so it can be recorded once into a hipGraph:

    embed ─► per layer:
      K1  fused_add_rmsnorm(x | partials, residual)        (layer 0: no residual)
      GEMM qkv (fused [q;k;v] rows)  ─► fp32 split-K partials
      K2  qkv_epilogue: reduce partials, q/k RMSNorm, RoPE, scatter k/v into the pool
      K3  paged attention (split-K over pages, GQA reuse)
      GEMM o ─► partials ─► K1 (reduce + residual add + RMSNorm)
      GEMM gate|up ─► partials ─► silu_mul ─► GEMM down ─► partials
    final K1 (reduce + residual + norm) ─► lm_head GEMM (bf16 logits) ─► argmax

Numerics are the reference's: every bf16 op of the torch path is rounded at
the same place (projection outputs, residual adds, norm outputs, RoPE steps,
SwiGLU steps); reductions accumulate in fp32. The fused qkv / gate|up
projections compute exactly the per-projection dot products of the
reference's separate q/k/v and gate/up Linear layers.

Weight formats (`QLinear.fmt`): dense bf16 (the reference's F.linear path),
W8 per-channel (the reference's w8a16) and W4 group-128 symmetric (W4A16).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field

import torch

from acorninfer_amd import _lib
from acorninfer_amd._lib import (BF16, WFMT_BF16, WFMT_W4, WFMT_W8, check, dtype_code, lib,
                                 ptr, stream_ptr)
from acorninfer_amd.config import Qwen3Config
from acorninfer_amd.quant import quantize as Q

MI355X_CUS = 256
FORMATS = {"bf16": WFMT_BF16, "w8a16": WFMT_W8, "w4a16": WFMT_W4}


# --------------------------------------------------------------------------- weights --

@dataclass
class QLinear:
    """One projection y = x @ W^T in a decode weight format.

    bf16: w [N,K] bf16.  w8a16: w int8 [N,K], scale fp16 [N].
    w4a16: w uint8 [N,K/2] (low nibble = even k), scale fp16 [N,K/128], zero
    None (symmetric) or fp16 [N,K/128].
    """
    fmt: int
    w: torch.Tensor
    N: int
    K: int
    scale: torch.Tensor | None = None
    zero: torch.Tensor | None = None

    @classmethod
    def from_dense(cls, w: torch.Tensor, fmt: int) -> "QLinear":
        N, K = w.shape
        if fmt == WFMT_BF16:
            return cls(fmt, w.to(torch.bfloat16).contiguous(), N, K)
        if fmt == WFMT_W8:
            q, s = Q.quantize_w8(w)
            return cls(fmt, q.contiguous(), N, K, s.contiguous())
        if fmt == WFMT_W4:
            u, s = Q.quantize_w4_sym(w)
            return cls(fmt, Q.pack_w4(u).contiguous(), N, K, s.contiguous())
        raise ValueError(f"unknown weight format {fmt}")

    def dense(self) -> torch.Tensor:
        """fp32 dequantised weight [N, K] (test/inspection helper)."""
        if self.fmt in (WFMT_BF16, _lib.WFMT_F32):
            return self.w.float()
        if self.fmt == WFMT_W8:
            return Q.dequant_w8(self.w, self.scale)
        u = Q.unpack_w4(self.w)
        zero = self.zero if self.zero is not None else Q.sym_zero(self.scale)
        return Q.dequant_w4(u, self.scale, zero)

    def nbytes(self) -> int:
        n = self.w.numel() * self.w.element_size()
        for t in (self.scale, self.zero):
            if t is not None:
                n += t.numel() * t.element_size()
        return n

    def plan(self, M: int, partials: bool) -> tuple[int, int, int]:
        rt, nw, ks = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        rc = lib().acorn_gemm_plan(M, self.N, self.K, self.fmt, int(partials),
                                   ctypes.byref(rt), ctypes.byref(nw), ctypes.byref(ks))
        check(rc, "gemm_plan")
        return rt.value, nw.value, ks.value

    def launch(self, x: torch.Tensor, M: int, cfg: tuple[int, int, int], *,
               out: torch.Tensor | None = None, part: torch.Tensor | None = None,
               stream: int) -> None:
        rt, nw, ks = cfg
        if self.fmt == _lib.WFMT_F32 and part is None:
            part = out      # fp32 results come back through the partials pointer
        rc = lib().acorn_quant_gemm(ptr(x), ptr(self.w), ptr(self.scale), ptr(self.zero),
                                    None if part is not None else ptr(out), ptr(part),
                                    M, self.N, self.K, self.fmt, rt, nw, ks, stream)
        check(rc, "quant_gemm")


@dataclass
class LayerWeights:
    input_norm: torch.Tensor      # [hidden]
    qkv: QLinear                  # rows [q (H*D); k (KV*D); v (KV*D)]
    q_norm: torch.Tensor          # [D]
    k_norm: torch.Tensor          # [D]
    o: QLinear
    post_norm: torch.Tensor       # [hidden]
    gate_up: QLinear              # rows [gate (I); up (I)]
    down: QLinear


# HF / reference module names of one layer's tensors (models/qwen3.py:100-112, 385-405)
_LAYER_KEYS = ("input_layernorm", "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
               "self_attn.o_proj", "self_attn.q_norm", "self_attn.k_norm",
               "post_attention_layernorm", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def random_state_dict(cfg: Qwen3Config, *, seed: int, std: float = 0.02,
                      dtype: torch.dtype = torch.bfloat16, device="cpu",
                      layer_range: range | None = None, with_globals: bool = True
                      ) -> dict[str, torch.Tensor]:
    """Seeded by-name init: every projection and the embedding ~ N(0, std),
    every RMSNorm weight = 1 (the benchmark configurations' init). Tensors are
    drawn in a fixed order from one generator on `device`, so the CPU oracle
    and the GPU model built from the same seed hold identical weights."""
    g = torch.Generator(device=device).manual_seed(seed)
    H, D = cfg.hidden_size, cfg.head_dim
    nq, nkv, inter = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.intermediate_size

    def normal(*shape):
        return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std
                ).to(dtype)

    def ones(n):
        return torch.ones(n, device=device, dtype=dtype)

    sd: dict[str, torch.Tensor] = {}
    if with_globals:
        sd["embed_tokens.weight"] = normal(cfg.vocab_size, H)
    for i in (layer_range if layer_range is not None else range(cfg.num_hidden_layers)):
        p = f"layers.{i}."
        sd[p + "input_layernorm.weight"] = ones(H)
        sd[p + "self_attn.q_proj.weight"] = normal(nq * D, H)
        sd[p + "self_attn.k_proj.weight"] = normal(nkv * D, H)
        sd[p + "self_attn.v_proj.weight"] = normal(nkv * D, H)
        sd[p + "self_attn.o_proj.weight"] = normal(H, nq * D)
        sd[p + "self_attn.q_norm.weight"] = ones(D)
        sd[p + "self_attn.k_norm.weight"] = ones(D)
        sd[p + "post_attention_layernorm.weight"] = ones(H)
        sd[p + "mlp.gate_proj.weight"] = normal(inter, H)
        sd[p + "mlp.up_proj.weight"] = normal(inter, H)
        sd[p + "mlp.down_proj.weight"] = normal(H, inter)
    if with_globals:
        sd["norm.weight"] = ones(H)
        sd["lm_head.weight"] = normal(cfg.vocab_size, H)
    return sd


class Qwen3DecodeModel:
    """Weights in decode layouts + the kernel sequence of one decode step."""

    def __init__(self, cfg: Qwen3Config, *, embed: torch.Tensor, layers: list[LayerWeights],
                 norm: torch.Tensor, lm_head: QLinear, dtype: torch.dtype):
        self.cfg = cfg
        self.dtype = dtype
        self.embed = embed
        self.layers = layers
        self.norm = norm
        self.lm_head = lm_head
        self.device = embed.device
        D = cfg.head_dim
        self.inv_freq = (1.0 / (cfg.rope_theta ** (
            torch.arange(0, D, 2, dtype=torch.float32) / D))).to(self.device)
        self.scale = D ** -0.5
        # Switches with the reference's names (qwen3.py:487-489).
        self.attention_backend = "hip"
        self.fused_ops = True

    # ---------------------------------------------------------------- building --
    @classmethod
    def from_state_dict(cls, cfg: Qwen3Config, sd: dict[str, torch.Tensor], *,
                        weight_format: str = "bf16", device="cuda",
                        dtype: torch.dtype = torch.bfloat16) -> "Qwen3DecodeModel":
        """Build from reference-named tensors (any device; moved to `device`)."""
        fmt = FORMATS[weight_format]
        dev = torch.device(device)

        def t(name):
            return sd[name].to(device=dev)

        layers = []
        for i in range(cfg.num_hidden_layers):
            layers.append(cls._layer(cfg, lambda k, i=i: t(f"layers.{i}.{k}.weight"), fmt, dtype))
        return cls(cfg, embed=t("embed_tokens.weight").to(dtype).contiguous(), layers=layers,
                   norm=t("norm.weight").to(dtype).contiguous(),
                   lm_head=QLinear.from_dense(t("lm_head.weight"), fmt)
                   if dtype == torch.bfloat16 else _dense_linear(t("lm_head.weight"), dtype),
                   dtype=dtype)

    @staticmethod
    def _layer(cfg, get, fmt: int, dtype) -> LayerWeights:
        def lin(w):
            return QLinear.from_dense(w, fmt) if dtype == torch.bfloat16 else _dense_linear(w, dtype)

        qkv = torch.cat([get("self_attn.q_proj"), get("self_attn.k_proj"),
                         get("self_attn.v_proj")], 0)
        gate_up = torch.cat([get("mlp.gate_proj"), get("mlp.up_proj")], 0)
        return LayerWeights(
            input_norm=get("input_layernorm").to(dtype).contiguous(),
            qkv=lin(qkv),
            q_norm=get("self_attn.q_norm").to(dtype).contiguous(),
            k_norm=get("self_attn.k_norm").to(dtype).contiguous(),
            o=lin(get("self_attn.o_proj")),
            post_norm=get("post_attention_layernorm").to(dtype).contiguous(),
            gate_up=lin(gate_up),
            down=lin(get("mlp.down_proj")),
        )

    @classmethod
    def random_init(cls, cfg: Qwen3Config, *, weight_format: str = "bf16", seed: int = 0,
                    std: float = 0.02, device="cuda") -> "Qwen3DecodeModel":
        """Seeded N(0, std) weights drawn on the GPU one layer at a time (an
        8B model never needs a second full-precision copy)."""
        fmt = FORMATS[weight_format]
        dev = torch.device(device)
        glob = random_state_dict(cfg.with_layers(0), seed=seed, std=std, device=dev)
        layers = []
        for i in range(cfg.num_hidden_layers):
            sd = random_state_dict(cfg, seed=seed * 1000003 + i + 1, std=std, device=dev,
                                   layer_range=range(i, i + 1), with_globals=False)
            layers.append(cls._layer(cfg, lambda k, i=i, sd=sd: sd[f"layers.{i}.{k}.weight"],
                                     fmt, torch.bfloat16))
            del sd
        return cls(cfg, embed=glob["embed_tokens.weight"].contiguous(), layers=layers,
                   norm=glob["norm.weight"].contiguous(),
                   lm_head=QLinear.from_dense(glob["lm_head.weight"], fmt), dtype=torch.bfloat16)

    def weight_bytes(self) -> int:
        n = 0
        for L in self.layers:
            n += sum(x.nbytes() for x in (L.qkv, L.o, L.gate_up, L.down))
            n += sum(t.numel() * t.element_size()
                     for t in (L.input_norm, L.q_norm, L.k_norm, L.post_norm))
        n += self.lm_head.nbytes() + self.norm.numel() * self.norm.element_size()
        return n

    # ------------------------------------------------------------------ decode --
    def buffers(self, batch: int, max_pages: int, num_splits: int | None = None
                ) -> "StepBuffers":
        return StepBuffers(self, batch, max_pages, num_splits)

    def step(self, buf: "StepBuffers", k_pool: torch.Tensor, v_pool: torch.Tensor,
             num_blocks: int, page_size: int) -> None:
        """Launch one decode step on the current stream.

        Reads buf.ids/positions/pages/slots/lens/tables; writes buf.logits
        (bf16 [B, vocab]) and buf.next_ids (int64 [B], greedy). k_pool/v_pool
        are [layers, NB, P, KV, D]; layer l's new k/v go to
        (pages[b], slots[b]) before attention reads lens[b] tokens.
        """
        cfg = self.cfg
        L = lib()
        st = stream_ptr(self.device)
        B = buf.batch
        H, D = cfg.hidden_size, cfg.head_dim
        nq, nkv, inter = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.intermediate_size
        dt = dtype_code(buf.x)
        wdt = dtype_code(self.norm)
        eps = float(cfg.rms_norm_eps)
        layer_elems = num_blocks * page_size * nkv * D
        esz = k_pool.element_size()
        kbase, vbase = k_pool.data_ptr(), v_pool.data_ptr()

        check(L.acorn_embedding(ptr(self.embed), ptr(buf.ids), ptr(buf.x), B, cfg.vocab_size, H,
                                dt, st), "embedding")
        res_in = None           # residual stream; None before layer 0's K1
        prev_part, prev_ks = None, 0
        for li, lw in enumerate(self.layers):
            # K1: input norm (layer 0 from the embedding, later layers fuse
            # the previous down projection's split-K reduce + residual add).
            if prev_part is None:
                check(L.acorn_fused_add_rmsnorm(ptr(buf.x), None, ptr(buf.res), ptr(lw.input_norm),
                                                ptr(buf.normed), B, H, eps, dt, wdt, st), "K1")
            else:
                check(L.acorn_fused_add_rmsnorm_partials(
                    ptr(prev_part), prev_ks, ptr(res_in), ptr(buf.res), ptr(lw.input_norm),
                    ptr(buf.normed), None, B, H, eps, dt, wdt, st), "K1")
            res_in = buf.res
            # qkv projection -> partials -> K2 epilogue (+ KV scatter)
            cq = buf.cfgs["qkv"]
            lw.qkv.launch(buf.normed, B, cq, part=buf.part_qkv, stream=st)
            kp = kbase + li * layer_elems * esz
            vp = vbase + li * layer_elems * esz
            check(L.acorn_qkv_epilogue(
                ptr(buf.part_qkv), cq[2], ptr(buf.q), kp, vp, ptr(buf.pages), ptr(buf.slots),
                B, nq, nkv, D, page_size, num_blocks, ptr(lw.q_norm), ptr(lw.k_norm), eps,
                ptr(buf.positions), ptr(self.inv_freq), dt, wdt, st), "qkv_epilogue")
            # K3
            check(L.acorn_paged_attention(
                ptr(buf.q), kp, vp, ptr(buf.tables), ptr(buf.lens), ptr(buf.attn),
                ptr(buf.ws_acc), ptr(buf.ws_ml), B, nq, nkv, D, page_size, num_blocks,
                buf.max_pages, buf.num_splits, float(self.scale), dt, st), "K3")
            # o projection -> K1 (reduce + residual + post-attention norm)
            co = buf.cfgs["o"]
            lw.o.launch(buf.attn, B, co, part=buf.part_o, stream=st)
            check(L.acorn_fused_add_rmsnorm_partials(
                ptr(buf.part_o), co[2], ptr(buf.res), ptr(buf.res), ptr(lw.post_norm),
                ptr(buf.normed), None, B, H, eps, dt, wdt, st), "K1")
            # MLP
            cg = buf.cfgs["gate_up"]
            lw.gate_up.launch(buf.normed, B, cg, part=buf.part_gu, stream=st)
            check(L.acorn_silu_mul(ptr(buf.part_gu), cg[2], None, ptr(buf.act), B, inter, dt, st),
                  "silu_mul")
            cd = buf.cfgs["down"]
            lw.down.launch(buf.act, B, cd, part=buf.part_down, stream=st)
            prev_part, prev_ks = buf.part_down, cd[2]
        # final norm (reduce + residual) -> lm_head -> greedy
        check(L.acorn_fused_add_rmsnorm_partials(
            ptr(prev_part), prev_ks, ptr(res_in), ptr(buf.res), ptr(self.norm), ptr(buf.normed),
            None, B, H, eps, dt, wdt, st), "K1")
        self.lm_head.launch(buf.normed, B, buf.cfgs["lm_head"], out=buf.logits, stream=st)
        check(L.acorn_argmax(ptr(buf.logits), B, cfg.vocab_size, ptr(buf.next_ids),
                             dtype_code(buf.logits), st), "argmax")

    # Reference-shaped entry point (qwen3.py:520-595).
    def forward_decode(self, input_ids: torch.Tensor, views, *, prepared=None) -> torch.Tensor:
        """input_ids [B, 1] + one PagedCacheView per row -> fp32 logits [B, vocab].

        As in the reference: positions are each view's pre-write seq_len, the
        step first makes room for one token per view (allocating a block when
        the append starts a page), lens include the new token, and every
        layer's length advances by one. `prepared` = (positions, tables, lens,
        (pages, slots)) skips the host-side preparation.
        """
        if input_ids.shape[1] != 1:
            raise ValueError("forward_decode expects [B, 1] input_ids (decode step)")
        from acorninfer_amd.ops.paged_attention import build_tables
        cache = views[0].cache
        B = len(views)
        if prepared is None:
            positions = torch.tensor([v.seq_len for v in views], device=self.device)
            targets = [v.ensure_append_capacity(0) for v in views]
            pages = torch.tensor([p for p, _ in targets], device=self.device, dtype=torch.long)
            slots = torch.tensor([s for _, s in targets], device=self.device, dtype=torch.long)
            tables, lens = build_tables(views, cache.page_size, self.device,
                                        lens_override=[int(v.seq_len) + 1 for v in views])
        else:
            positions, tables, lens, (pages, slots) = prepared
        buf = self.buffers(B, tables.shape[1])
        buf.ids.copy_(input_ids.view(-1))
        buf.positions.copy_(positions)
        buf.pages.copy_(pages)
        buf.slots.copy_(slots)
        buf.lens.copy_(lens)
        buf.tables.copy_(tables)
        self.step(buf, cache.k_pool, cache.v_pool, cache.num_blocks, cache.page_size)
        for v in views:
            for li in range(self.cfg.num_hidden_layers):
                v._lens[li] = v._lens.get(li, 0) + 1
        return buf.logits.float()


def _dense_linear(w: torch.Tensor, dtype: torch.dtype) -> QLinear:
    """fp32 weights (parity path): kept dense in the activation dtype."""
    if dtype == torch.float32:
        return QLinear(_lib.WFMT_F32, w.float().contiguous(), w.shape[0], w.shape[1])
    raise ValueError(f"no dense weight format for activations of dtype {dtype}")


def attention_splits(batch: int, kv_heads: int, *, cu_count: int = MI355X_CUS,
                     waves_per_cu: int = 4, max_splits: int = 64) -> int:
    """K3 split count for a captured bucket: enough (split, kv head, sequence)
    wavefronts to give every CU `waves_per_cu` of them. Fixed per bucket (the
    kernel skips splits beyond a sequence's pages)."""
    return max(1, min(max_splits, -(-cu_count * waves_per_cu // max(1, batch * kv_heads))))


@dataclass
class StepBuffers:
    """Address-stable inputs, outputs and scratch of one decode step."""
    model: Qwen3DecodeModel
    batch: int
    max_pages: int
    num_splits: int | None = None
    cfgs: dict = field(default_factory=dict)

    def __post_init__(self):
        m = self.model
        cfg, dev, dt = m.cfg, m.device, m.dtype
        B = self.batch
        H, D = cfg.hidden_size, cfg.head_dim
        nq, nkv, inter = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.intermediate_size
        if self.num_splits is None:
            self.num_splits = attention_splits(B, nkv)
        lw = m.layers[0]
        for name, lin in (("qkv", lw.qkv), ("o", lw.o), ("gate_up", lw.gate_up),
                          ("down", lw.down)):
            self.cfgs[name] = lin.plan(B, partials=True)
        self.cfgs["lm_head"] = m.lm_head.plan(B, partials=False)
        # int64 block: ids | positions | pages | slots | next_ids ; int32 block: lens | tables
        self.flat_i64 = torch.zeros(5 * B, dtype=torch.int64, device=dev)
        self.flat_i32 = torch.zeros(B * (1 + self.max_pages), dtype=torch.int32, device=dev)
        self.ids = self.flat_i64[0:B]
        self.positions = self.flat_i64[B:2 * B]
        self.pages = self.flat_i64[2 * B:3 * B]
        self.slots = self.flat_i64[3 * B:4 * B]
        self.next_ids = self.flat_i64[4 * B:5 * B]
        self.meta_i64 = self.flat_i64[B:4 * B]        # host-written: positions|pages|slots
        self.lens = self.flat_i32[0:B]
        self.tables = self.flat_i32[B:].view(B, self.max_pages)
        self.lens.fill_(1)

        def z(*shape, dtype=dt):
            return torch.zeros(*shape, dtype=dtype, device=dev)

        f32 = torch.float32
        self.x = z(B, H)
        self.res = z(B, H)
        self.normed = z(B, H)
        self.q = z(B, nq, D)
        self.attn = z(B, nq * D)
        self.act = z(B, inter)
        self.part_qkv = z(self.cfgs["qkv"][2], B, (nq + 2 * nkv) * D, dtype=f32)
        self.part_o = z(self.cfgs["o"][2], B, H, dtype=f32)
        self.part_gu = z(self.cfgs["gate_up"][2], B, 2 * inter, dtype=f32)
        self.part_down = z(self.cfgs["down"][2], B, H, dtype=f32)
        S = self.num_splits
        self.ws_acc = z(B * nq * S * D, dtype=f32)
        self.ws_ml = z(2 * B * nq * S, dtype=f32)
        self.logits = z(B, cfg.vocab_size, dtype=dt)
