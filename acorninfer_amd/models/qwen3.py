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
    final K1 (reduce + residual + norm) ─► lm_head GEMM (bf16 logits) ─► sampler
    (argmax for temperature-0 rows)

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
from acorninfer_amd._lib import (BF16, WFMT_BF16, WFMT_BF16B, WFMT_W4, WFMT_W4B, WFMT_W8, WFMT_W8B,
                                 check,
                                 dtype_code, lib, ptr, stream_ptr)
from acorninfer_amd.config import Qwen3Config
from acorninfer_amd.ops.paged_attention import prefill_supported
from acorninfer_amd.quant import quantize as Q

MI355X_CUS = 256
FORMATS = {"bf16": WFMT_BF16, "w8a16": WFMT_W8, "w4a16": WFMT_W4}
# bf16 projections at prefill sizes run on the library's large-M kernel
# (its planner's default from DENSE_M_MIN rows, tiling rt == DENSE_RT: the
# 256 x 256 direct-to-LDS form; kDenseMinM in csrc/quant_gemm.hip).
DENSE_M_MIN = 256
DENSE_RT = -2
# int4 (W4B) projections from DEQUANT_M_MIN rows: the weights are
# dequantised to bf16 into a step workspace (acorn_dequant_w4b) and
# multiplied by the large-M bf16 kernel (tiling rt == DEQUANT_RT, the other
# fields the bf16 kernel's). At prefill sizes the MFMA work dominates and that
# kernel's rate outweighs the extra pass over the weights: on MI355X a W4A16
# 8B prefill of 512 / 768 tokens takes 15.0 / 19.7 ms this way against
# 15.9 / 25.4 ms on the int4 kernels; below 512 rows the int4 kernels win
# (8.5-9.2 vs 12.8 ms at 256 tokens).
DEQUANT_M_MIN = 512
DEQUANT_RT = -4
# prefill blocks from this many rows run gate|up with the large-M kernel's
# SwiGLU epilogue (act written directly: no fp32 gate|up output, no silu_mul);
# int4 weights once they take the dequantise route
PREFILL_SWIGLU_M = 512
# and from this many rows (the qkv epilogue's row form) qkv / o / down write
# the activation dtype directly when they run in one split on that kernel
PREFILL_DIRECT_M = 256


def dispatch_linear(mod, x: torch.Tensor) -> torch.Tensor:
    """The reference model's single entry for every projection and lm_head
    (acorninfer/models/qwen3.py:21-47), for callers that keep the reference's
    nn.Module model and quantise it with quant.apply_quant:

    - no `_m7_quant` marker: `mod(x)` (the module's own forward, unchanged);
    - "w8a16": quant_gemm(x, int8 weight, `_q_scale`, cls), cls looked up by
      the weight's (N, K) in `_CLS_BY_SHAPE` (an unknown shape is a
      ValueError, as in the reference);
    - "w4a16": quant_gemm_w4 on the packed weight (the reference rejects this
      mode; this build supports it, apply_quant sets it);
    - any other marker: ValueError.
    The result takes x's leading shape."""
    mode = getattr(mod, "_m7_quant", None)
    if mode is None:
        return mod(x)
    from acorninfer_amd.ops.quant_gemm import _CLS_BY_SHAPE, quant_gemm, quant_gemm_w4
    w = mod.weight.data
    if mode == "w8a16":
        N, K = w.shape
    elif mode == "w4a16":
        N, K = w.shape[0], 2 * w.shape[1]
    else:
        raise ValueError(f"dispatch_linear: unsupported _m7_quant={mode!r}")
    cls = _CLS_BY_SHAPE.get((N, K))
    if cls is None:
        raise ValueError(f"dispatch_linear: quantized linear shape {(N, K)} is not one of "
                         f"the CLASSES (apply_quant targets the production 8B shapes)")
    if mode == "w8a16":
        out = quant_gemm(x, w, mod._q_scale, cls)
    else:
        out = quant_gemm_w4(x, w, mod._q_scale, None, cls)
    return out.view(*x.shape[:-1], N)


# --------------------------------------------------------------------------- weights --

@dataclass
class QLinear:
    """One projection y = x @ W^T in a decode weight format.

    bf16: w [N,K] bf16; with N % 16 == 0 and K % 64 == 0 held in the bf16
    decode kernel's 1 KB block layout (fmt WFMT_BF16B, quantize.to_bf16b:
    the same shape). w8a16: w int8 [N,K], scale fp16 [N]; with N % 16
    == 0 and K % 64 == 0 held in the int8 decode kernel's 1 KB block layout
    (fmt WFMT_W8B, quantize.to_w8b: uint8 q + 128 of the same shape).
    w4a16: w uint8 [N,K/2] (low nibble = even k), scale fp16 [N,K/128], zero
    None (symmetric) or fp16 [N,K/128]; symmetric weights with N % 16 == 0
    and K % 512 == 0 are held in the int4 decode kernels' 1 KB block layout
    (fmt WFMT_W4B, quantize.to_w4b: the same tensor shapes).
    """
    fmt: int
    w: torch.Tensor
    N: int
    K: int
    scale: torch.Tensor | None = None
    zero: torch.Tensor | None = None
    il16: bool = False          # gate|up rows interleaved in 16-row blocks (fused SwiGLU)

    @classmethod
    def from_dense(cls, w: torch.Tensor, fmt: int) -> "QLinear":
        N, K = w.shape
        if fmt == WFMT_BF16:
            return cls(fmt, w.to(torch.bfloat16).contiguous(), N, K).blocked()
        if fmt == WFMT_W8:
            q, s = Q.quantize_w8(w)
            return cls(fmt, q.contiguous(), N, K, s.contiguous()).blocked()
        if fmt == WFMT_W4:
            u, s = Q.quantize_w4_sym(w)
            return cls(fmt, Q.pack_w4(u).contiguous(), N, K, s.contiguous()).blocked()
        raise ValueError(f"unknown weight format {fmt}")

    def blocked(self) -> "QLinear":
        """bf16 in the BF16B block layout and int8 in the W8B one (N % 16 ==
        0, K % 64 == 0), symmetric int4 in the W4B block layout (N % 16 == 0,
        K % 512 == 0) where the shape allows it; any other weight unchanged."""
        if self.fmt == WFMT_BF16 and not (self.N % 16 or self.K % 64):
            return QLinear(WFMT_BF16B, Q.to_bf16b(self.w), self.N, self.K, il16=self.il16)
        if self.fmt == WFMT_W8 and not (self.N % 16 or self.K % 64):
            return QLinear(WFMT_W8B, Q.to_w8b(self.w), self.N, self.K, self.scale, None,
                           il16=self.il16)
        if self.fmt != WFMT_W4 or self.zero is not None or self.N % 16 or self.K % 512:
            return self
        wb, sb = Q.to_w4b(self.w, self.scale)
        return QLinear(WFMT_W4B, wb, self.N, self.K, sb, None, il16=self.il16)

    def natural(self) -> "QLinear":
        """The same weight in the reference's layouts (bf16 and int8 [N, K],
        int4 [N, K/2])."""
        if self.fmt == WFMT_BF16B:
            return QLinear(WFMT_BF16, Q.from_bf16b(self.w), self.N, self.K, il16=self.il16)
        if self.fmt == WFMT_W8B:
            return QLinear(WFMT_W8, Q.from_w8b(self.w), self.N, self.K, self.scale, None,
                           il16=self.il16)
        if self.fmt != WFMT_W4B:
            return self
        w, s = Q.from_w4b(self.w, self.scale)
        return QLinear(WFMT_W4, w, self.N, self.K, s, None, il16=self.il16)

    def interleaved(self) -> "QLinear":
        """The same [gate; up] weight with rows (and scales, zeros) in the
        16-row gate/up blocks of the fused SwiGLU launch."""
        from acorninfer_amd.ops.quant_gemm import interleave16
        il = lambda t: None if t is None else interleave16(t)  # noqa: E731
        return QLinear(self.fmt, il(self.w), self.N, self.K, il(self.scale), il(self.zero),
                       il16=True)

    def dense(self) -> torch.Tensor:
        """fp32 dequantised weight [N, K] in [gate; up] row order (test helper)."""
        if self.fmt in (WFMT_BF16, _lib.WFMT_F32):
            d = self.w.float()
        elif self.fmt == WFMT_BF16B:
            d = self.natural().w.float()
        elif self.fmt in (WFMT_W8, WFMT_W8B):
            nat = self.natural()
            d = Q.dequant_w8(nat.w, nat.scale)
        else:
            nat = self.natural()
            u = Q.unpack_w4(nat.w)
            zero = nat.zero if nat.zero is not None else Q.sym_zero(nat.scale)
            d = Q.dequant_w4(u, nat.scale, zero)
        if self.il16:
            from acorninfer_amd.ops.quant_gemm import deinterleave16
            d = deinterleave16(d)
        return d

    def nbytes(self) -> int:
        n = self.w.numel() * self.w.element_size()
        for t in (self.scale, self.zero):
            if t is not None:
                n += t.numel() * t.element_size()
        return n

    def plan(self, M: int, tiling=None, workspace: bool = False):
        """(Tiling, output tiles) from the library planner. workspace: the
        caller holds a bf16 weight workspace, so int4 weights take the
        dequantise + bf16 GEMM route by default from DEQUANT_M_MIN rows (a
        DEQUANT_RT request takes it at any size)."""
        from acorninfer_amd.ops.quant_gemm import Tiling, plan
        if self.fmt == WFMT_W4B and (
                (tiling is not None and tiling[0] == DEQUANT_RT) or
                (workspace and (tiling is None or not any(tiling)) and M >= DEQUANT_M_MIN)):
            rest = tuple(tiling[1:]) if tiling is not None else (0, 0, 0, 0)
            t, tiles = plan(M, self.N, self.K, WFMT_BF16, Tiling(DENSE_RT, *rest))
            return Tiling(DEQUANT_RT, *t[1:]), tiles
        return plan(M, self.N, self.K, self.fmt, tiling)

    def _dequant(self, wtmp: torch.Tensor | None, M: int, stream: int) -> None:
        """W4B -> bf16 [N, K] into wtmp (the first half of a DEQUANT_RT launch)."""
        if self.fmt != WFMT_W4B:
            raise ValueError("a DEQUANT_RT tiling needs W4B weights")
        if wtmp is None or wtmp.dtype != torch.bfloat16 or wtmp.numel() < self.N * self.K:
            raise ValueError(f"int4 GEMM at {M} rows (DEQUANT_RT) needs a bf16 weight "
                             f"workspace of {self.N * self.K} elements")
        check(lib().acorn_dequant_w4b(ptr(self.w), ptr(self.scale), ptr(wtmp), self.N, self.K,
                                      stream), "dequant_w4b")

    def launch(self, x: torch.Tensor, M: int, tiling, *, out: torch.Tensor | None = None,
               part: torch.Tensor | None = None, wtmp: torch.Tensor | None = None,
               stream: int) -> None:
        """out given: bf16 [M, N] (part is the split-K workspace when
        tiling.ksplit > 1); out None: fp32 partials [ksplit, M, N] into part.
        fp32 weights always write fp32 through part. A DEQUANT_RT tiling
        dequantises into wtmp (bf16, at least N * K elements) first."""
        if self.fmt == _lib.WFMT_F32:
            part, out = (out if part is None else part), None
        if tiling[0] == DEQUANT_RT:
            self._dequant(wtmp, M, stream)
            arr = (ctypes.c_int * 6)(DENSE_RT, *tiling[1:], 0)
            rc = lib().acorn_quant_gemm(ptr(x), ptr(wtmp), None, None, ptr(out), ptr(part), M,
                                        self.N, self.K, WFMT_BF16, arr, stream)
            check(rc, "quant_gemm(dequantised int4)")
            return
        arr = (ctypes.c_int * 6)(*tiling, 0)
        rc = lib().acorn_quant_gemm(ptr(x), ptr(self.w), ptr(self.scale), ptr(self.zero),
                                    ptr(out), ptr(part), M, self.N, self.K, self.fmt, arr,
                                    stream)
        check(rc, "quant_gemm")

    def can_fold(self, M: int) -> bool:
        """The RMSNorm can be folded into this projection's launch (the direct
        decode kernels on the block layouts, M <= 16)."""
        return self.fmt in (WFMT_BF16B, WFMT_W8B, WFMT_W4B) and M <= 16 and self.K % 16 == 0

    def launch_norm(self, x: torch.Tensor, M: int, tiling, *, ss: torch.Tensor, eps: float,
                    stream: int, out: torch.Tensor | None = None,
                    part: torch.Tensor | None = None, act: torch.Tensor | None = None) -> None:
        """The projection of the normalised residual: x is a launch_resid
        producer's weighted rows bf16(v * norm_w) [M, K], and every result of
        row m is multiplied by inv = 1 / rms(v) from the producer's
        per-16-column sums of squares ss [M, K/16] before it is stored (the
        RMSNorm of acorninfer/ops/rmsnorm.py:39-82 split around the GEMM).
        Output as launch (act given: the fused SwiGLU of launch_swiglu)."""
        assert x.dtype == torch.bfloat16 and x.is_contiguous() and tuple(x.shape) == (M, self.K)
        assert ss.dtype == torch.float32 and ss.is_contiguous() and \
            tuple(ss.shape) == (M, self.K // 16), "sums of squares are [M, K/16] fp32"
        arr = (ctypes.c_int * 6)(*tiling, 0)
        rc = lib().acorn_quant_gemm_norm(
            ptr(x), ptr(self.w), ptr(self.scale), ptr(act if act is not None else out), ptr(part),
            M, self.N, self.K, self.fmt, arr, int(act is not None), ptr(ss), float(eps),
            None, None, None, None, None, stream)
        check(rc, "quant_gemm_norm")

    def launch_resid(self, x: torch.Tensor, M: int, tiling, *, res: torch.Tensor,
                     res_out: torch.Tensor, ss: torch.Tensor, norm_w: torch.Tensor,
                     xw: torch.Tensor, stream: int) -> None:
        """The projection whose output goes into the residual stream: stores
        res_out = v = bf16(res + bf16(x @ W^T)) (res_out may be res), the rows
        xw = bf16(v * norm_w) weighted by the next RMSNorm's weight, and the
        per-16-column sums of squares ss [M, N/16] of v: what a launch_norm
        consumer reads, in place of K1's residual add and norm (one split
        only)."""
        for t in (res, res_out, xw):
            assert t.dtype == torch.bfloat16 and t.is_contiguous() and \
                tuple(t.shape) == (M, self.N), "res, res_out, xw are [M, N] bf16"
        assert ss.dtype == torch.float32 and ss.is_contiguous() and \
            tuple(ss.shape) == (M, self.N // 16), "sums of squares are [M, N/16] fp32"
        assert norm_w.dtype == torch.bfloat16 and tuple(norm_w.shape) == (self.N,)
        arr = (ctypes.c_int * 6)(*tiling, 0)
        rc = lib().acorn_quant_gemm_norm(
            ptr(x), ptr(self.w), ptr(self.scale), None, None, M, self.N, self.K, self.fmt, arr,
            0, None, 0.0, ptr(res), ptr(res_out), ptr(ss), ptr(norm_w), ptr(xw), stream)
        check(rc, "quant_gemm_resid")

    def swiglu_plan(self, M: int, tiling=None, workspace: bool = False):
        """As plan, for the fused gate|up + SwiGLU launch (int4 at prefill
        sizes: dequantised onto the bf16 kernel's SwiGLU form)."""
        from acorninfer_amd.ops.quant_gemm import Tiling, swiglu_plan
        if self.fmt == WFMT_W4B and (
                (tiling is not None and tiling[0] == DEQUANT_RT) or
                (workspace and (tiling is None or not any(tiling)) and M >= DEQUANT_M_MIN)):
            rest = tuple(tiling[1:]) if tiling is not None else (0, 0, 0, 0)
            t, tiles = swiglu_plan(M, self.N, self.K, WFMT_BF16, Tiling(DENSE_RT, *rest))
            return Tiling(DEQUANT_RT, *t[1:]), tiles
        return swiglu_plan(M, self.N, self.K, self.fmt, tiling)

    def launch_swiglu(self, x: torch.Tensor, M: int, tiling, act: torch.Tensor,
                      stream: int, wtmp: torch.Tensor | None = None) -> None:
        """Fused gate|up + SwiGLU (il16 weights): act [M, N/2] bf16. A
        DEQUANT_RT tiling dequantises into wtmp first, as launch does."""
        w, fmt, arr = self.w, self.fmt, (ctypes.c_int * 6)(*tiling, 0)
        if tiling[0] == DEQUANT_RT:
            self._dequant(wtmp, M, stream)
            w, fmt, arr = wtmp, WFMT_BF16, (ctypes.c_int * 6)(DENSE_RT, *tiling[1:], 0)
        scale = self.scale if fmt not in (WFMT_BF16, WFMT_BF16B) else None
        rc = lib().acorn_quant_gemm_swiglu(ptr(x), ptr(w), ptr(scale), ptr(self.zero), ptr(act),
                                           M, self.N, self.K, fmt, arr, stream)
        check(rc, "quant_gemm_swiglu")


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
        # prefill attention as the query-tiled kernel where it is built for
        # the shapes (False: K3 with one row per prompt token)
        self.tiled_prefill = True
        # projections of prefill rows: "own" (bf16 on the library's large-M
        # kernel; int4 dequantised onto it from DEQUANT_M_MIN rows) or "int4"
        # (int4 weights on the int4 kernels at every size)
        self.prefill_gemm = "own"
        # prefill blocks whose qkv / o / down run on the large-M kernel in one
        # split take their output in the activation dtype (half the bytes of
        # an fp32 plane, the same bits after the consumer's rounding)
        self.prefill_direct = True
        # decode steps fold the RMSNorms between projections into them (o and
        # down store the residual and its sums of squares, qkv and gate|up
        # normalise on load) where the kernels support it: no K1 launch
        # between layers
        self.fold_norm = True
        # batch -> {projection name -> Tiling}, filled by tune()
        self.tilings: dict[int, dict] = {}
        self.swiglu_choice: dict[int, bool] = {}
        self.fold_choice: dict[int, bool] = {}

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
        gu = lin(gate_up)
        if gu.fmt != _lib.WFMT_F32 and gu.N % 32 == 0:
            gu = gu.interleaved()
        return LayerWeights(
            input_norm=get("input_layernorm").to(dtype).contiguous(),
            qkv=lin(qkv),
            q_norm=get("self_attn.q_norm").to(dtype).contiguous(),
            k_norm=get("self_attn.k_norm").to(dtype).contiguous(),
            o=lin(get("self_attn.o_proj")),
            post_norm=get("post_attention_layernorm").to(dtype).contiguous(),
            gate_up=gu,
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
    def buffers(self, batch: int, max_pages: int, num_splits: int | None = None,
                tilings: dict | None = None, *, prefill: bool = False) -> "StepBuffers":
        return StepBuffers(self, batch, max_pages, num_splits,
                           tilings if tilings is not None else self.tilings.get(batch),
                           prefill=prefill)

    def step(self, buf: "StepBuffers", k_pool: torch.Tensor, v_pool: torch.Tensor,
             num_blocks: int, page_size: int, *, fused_attn: bool = True,
             head_rows: torch.Tensor | None = None,
             segments: "PrefillSegments | None" = None) -> torch.Tensor | None:
        """Launch one decode step on the current stream.

        fused_attn=False keeps the qkv epilogue (which writes every row's new
        k/v) and K3 as two launches; rows that attend to each other's new
        tokens (prefill rows of one sequence) need that order. head_rows:
        int64 row indices; only their logits are computed, [len, vocab] in
        the activation dtype, returned instead of sampling. segments: the
        rows are runs of consecutive positions of a few sequences (a prefill
        chunk); attention then runs as the query-tiled prefill kernel over
        those runs (buf.tables / buf.lens unused) instead of one K3 row each.

        Reads buf.ids/positions/pages/slots/lens/tables and the sampling
        block (temperature 0 = greedy); writes buf.logits (bf16 [B, vocab]),
        buf.next_ids (int64 [B], the same memory as buf.ids: the next step's
        input), buf.logprob and buf.status. k_pool/v_pool
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
        # K3 runs the qkv epilogue itself where it supports the shape (one
        # launch fewer per layer, the same bits)
        fused_attn = fused_attn and not buf.direct and bool(
            L.acorn_paged_attention_qkv_supported(nq, nkv, D, page_size, buf.max_pages,
                                                  buf.num_splits, dt, wdt))

        def k1(first: bool, y, part, ks: int, w) -> None:
            """K1 after a projection: the residual add + RMSNorm from its
            output in the activation dtype (y), or from its fp32 partials; the
            first norm of the step takes the embedding as the residual."""
            if first:
                check(L.acorn_fused_add_rmsnorm(ptr(buf.x), None, ptr(buf.res), ptr(w),
                                                ptr(buf.normed), B, H, eps, dt, wdt, st), "K1")
            elif y is not None:
                check(L.acorn_fused_add_rmsnorm(ptr(y), ptr(buf.res), ptr(buf.res), ptr(w),
                                                ptr(buf.normed), B, H, eps, dt, wdt, st), "K1")
            else:
                check(L.acorn_fused_add_rmsnorm_partials(
                    ptr(part), ks, ptr(buf.res), ptr(buf.res), ptr(w), ptr(buf.normed), None, B,
                    H, eps, dt, wdt, st), "K1")

        y_qkv = buf.y_qkv if buf.direct else None
        y_o = buf.y_o if buf.direct else None
        y_down = buf.y_down if buf.direct else None
        prev_ks = 0             # splits of the previous layer's down-projection partials
        last = len(self.layers) - 1
        for li, lw in enumerate(self.layers):
            cq = buf.cfgs["qkv"]
            if buf.fold and li > 0:
                # the input norm folded into qkv: the previous down stored the
                # residual, its rows times this norm's weight and its sums of
                # squares
                lw.qkv.launch_norm(buf.normed, B, cq, ss=buf.ss_dn, eps=eps, stream=st,
                                   out=y_qkv, part=buf.part_qkv)
            else:
                # K1: input norm (layer 0 from the embedding; later layers reduce
                # the previous down projection's output and add the residual)
                k1(li == 0, y_down, buf.part_down, prev_ks, lw.input_norm)
                # qkv projection -> fp32 partials (or its T output) -> K2 epilogue (+ KV scatter)
                lw.qkv.launch(buf.normed, B, cq, out=y_qkv, part=buf.part_qkv, wtmp=buf.wtmp,
                              stream=st)
            kp = kbase + li * layer_elems * esz
            vp = vbase + li * layer_elems * esz
            if fused_attn:
                check(L.acorn_paged_attention_qkv(
                    ptr(buf.part_qkv), cq.ksplit, kp, vp, ptr(buf.pages), ptr(buf.slots),
                    ptr(buf.tables), ptr(buf.lens), ptr(buf.attn), ptr(buf.ws_acc),
                    ptr(buf.ws_ml), B, nq, nkv, D, page_size, num_blocks, buf.max_pages,
                    buf.num_splits, float(self.scale), ptr(lw.q_norm), ptr(lw.k_norm), eps,
                    ptr(buf.positions), ptr(self.inv_freq), dt, wdt, st), "K3+epilogue")
            else:
                check(L.acorn_qkv_epilogue(
                    ptr(y_qkv) if buf.direct else ptr(buf.part_qkv),
                    0 if buf.direct else cq.ksplit, ptr(buf.q), kp, vp, ptr(buf.pages),
                    ptr(buf.slots), B, nq, nkv, D, page_size, num_blocks, ptr(lw.q_norm),
                    ptr(lw.k_norm), eps, ptr(buf.positions), ptr(self.inv_freq), dt, wdt, st),
                    "qkv_epilogue")
                if segments is not None:
                    sg = segments
                    check(L.acorn_paged_prefill_attention(
                        ptr(buf.q), kp, vp, ptr(sg.tables), ptr(sg.row0), ptr(sg.pos0),
                        ptr(sg.nq), ptr(buf.attn), sg.count, B, sg.max_nq, nq, nkv, D,
                        page_size, num_blocks, sg.tables.shape[1], float(self.scale), dt, st),
                        "prefill attention")
                else:
                    # K3
                    check(L.acorn_paged_attention(
                        ptr(buf.q), kp, vp, ptr(buf.tables), ptr(buf.lens), ptr(buf.attn),
                        ptr(buf.ws_acc), ptr(buf.ws_ml), B, nq, nkv, D, page_size, num_blocks,
                        buf.max_pages, buf.num_splits, float(self.scale), dt, st), "K3")
            # o projection -> K1 (reduce + residual add + post-attention norm);
            # folded: o adds itself to the residual, gate|up normalises on load
            co = buf.cfgs["o"]
            cg = buf.cfgs["gate_up"]
            if buf.fold:
                lw.o.launch_resid(buf.attn, B, co, res=buf.res, res_out=buf.res, ss=buf.ss_o,
                                  norm_w=lw.post_norm, xw=buf.normed, stream=st)
                if buf.swiglu:
                    lw.gate_up.launch_norm(buf.normed, B, cg, ss=buf.ss_o, eps=eps, stream=st,
                                           act=buf.act)
                else:
                    lw.gate_up.launch_norm(buf.normed, B, cg, ss=buf.ss_o, eps=eps, stream=st,
                                           part=buf.part_gu)
            else:
                lw.o.launch(buf.attn, B, co, out=y_o, part=buf.part_o, wtmp=buf.wtmp, stream=st)
                k1(False, y_o, buf.part_o, co.ksplit, lw.post_norm)
                # MLP: gate|up (+ fused SwiGLU) -> act -> down partials
                if buf.swiglu:
                    lw.gate_up.launch_swiglu(buf.normed, B, cg, buf.act, st, wtmp=buf.wtmp)
                else:
                    lw.gate_up.launch(buf.normed, B, cg, part=buf.part_gu, wtmp=buf.wtmp,
                                      stream=st)
            if not buf.swiglu:
                check(L.acorn_silu_mul(ptr(buf.part_gu), cg.ksplit, None, ptr(buf.act), B, inter,
                                       int(lw.gate_up.il16), dt, st), "silu_mul")
            cd = buf.cfgs["down"]
            if buf.fold and li < last:
                # the next layer's input norm folded into its qkv
                lw.down.launch_resid(buf.act, B, cd, res=buf.res, res_out=buf.res,
                                     ss=buf.ss_dn, norm_w=self.layers[li + 1].input_norm,
                                     xw=buf.normed, stream=st)
            else:
                lw.down.launch(buf.act, B, cd, out=y_down, part=buf.part_down, wtmp=buf.wtmp,
                               stream=st)
            prev_ks = cd.ksplit
        # final norm (reduce + residual add) -> lm_head -> greedy
        k1(False, y_down, buf.part_down, prev_ks, self.norm)
        if head_rows is not None:
            n = int(head_rows.numel())
            if n == 0:
                return torch.empty(0, cfg.vocab_size, dtype=buf.x.dtype, device=self.device)
            hx = buf.normed.index_select(0, head_rows)
            ch, _ = self.lm_head.plan(n)
            out = torch.empty(n, cfg.vocab_size, dtype=buf.x.dtype, device=self.device)
            ws = (torch.empty(ch.ksplit, n, cfg.vocab_size, dtype=torch.float32,
                              device=self.device)
                  if ch.ksplit > 1 and self.lm_head.fmt != _lib.WFMT_F32 else None)
            self.lm_head.launch(hx, n, ch, out=out, part=ws, stream=st)
            return out
        self.lm_head.launch(buf.normed, B, buf.cfgs["lm_head"], out=buf.logits,
                            part=buf.ws_lm, stream=st)
        # next token: greedy rows (temperature 0) take the argmax, the others
        # temperature -> top-k -> top-p -> inverse-CDF draw of their uniform
        check(L.acorn_sample(ptr(buf.logits), B, cfg.vocab_size, dtype_code(buf.logits),
                             ptr(buf.temperature), ptr(buf.top_k), ptr(buf.top_p),
                             ptr(buf.uniform), ptr(buf.next_ids), ptr(buf.logprob), None,
                             ptr(buf.status), st), "sample")
        return None

    def prefill_swiglu(self, rows: int) -> bool:
        """A prefill block of `rows` runs gate|up with the SwiGLU epilogue of
        the large-M bf16 kernel (bf16 weights from PREFILL_SWIGLU_M rows, int4
        dequantised onto it from DEQUANT_M_MIN), gate|up in the 16-row
        interleave."""
        gu = self.layers[0].gate_up
        return gu.il16 and rows >= PREFILL_SWIGLU_M and (
            gu.fmt in (WFMT_BF16, WFMT_BF16B) or (gu.fmt == WFMT_W4B and rows >= DEQUANT_M_MIN))

    def fused_swiglu_possible(self, batch: int) -> bool:
        """The gate|up launch can carry the SwiGLU epilogue (decode sizes,
        interleaved gate|up rows)."""
        return batch <= 16 and self.layers[0].gate_up.il16

    def fused_swiglu(self, batch: int) -> bool:
        """The gate|up launch carries the SwiGLU epilogue (where possible, and
        unless tune() found the split-K launch + silu_mul faster)."""
        return self.fused_swiglu_possible(batch) and self.swiglu_choice.get(batch, True)

    def projections(self) -> dict[str, list[QLinear]]:
        """Each projection of the step with its per-layer weights."""
        return {"qkv": [L.qkv for L in self.layers], "o": [L.o for L in self.layers],
                "gate_up": [L.gate_up for L in self.layers],
                "down": [L.down for L in self.layers], "lm_head": [self.lm_head]}

    def fold_possible(self, batch: int, *, tuned: bool = True) -> bool:
        """Decode steps of `batch` rows fold the RMSNorms into the projections
        (given one-split o and down tilings): the kernels support it, and
        unless tune() found the plain launches with their K1s faster (tuned)."""
        lw = self.layers[0]
        ok = (self.fold_norm and self.dtype == torch.bfloat16 and
              self.cfg.hidden_size % 16 == 0 and
              all(lin.can_fold(batch) for lin in (lw.qkv, lw.o, lw.gate_up, lw.down)))
        return ok and (not tuned or self.fold_choice.get(batch, True))

    def time_projection(self, lins: list[QLinear], M: int, tiling, reps: int = 3,
                        swiglu: bool = False, with_act: bool = False,
                        with_reduce: bool = False, with_norm: bool = False,
                        norm_in: bool = False, resid: bool = False) -> float:
        """Average µs of one launch of `tiling`, measured as a hipGraph of one
        launch per weight in `lins` (distinct weights, so the 256 MB MALL does
        not hold them between launches) on a private stream with HIP events.
        The step's consumer of the partials is timed with it, because its cost
        grows with the split count: with_act adds the separate SwiGLU kernel
        the fused form saves; with_reduce a split-order reduction (the qkv
        epilogue's, spread over many workgroups); with_norm the step's own K1
        (one workgroup per row), which reads the o and down partials. norm_in /
        resid time the folded forms instead (launch_norm / launch_resid)."""
        from acorninfer_amd.ops.quant_gemm import _native_cfg
        lin0 = lins[0]
        planner = lin0.swiglu_plan if swiglu else lin0.plan
        t = planner(M, _native_cfg(tiling, M))[0]
        x = torch.randn(M, lin0.K, device=self.device).to(self.dtype)
        part = torch.empty(t.ksplit, M, lin0.N, dtype=torch.float32, device=self.device)
        wtmp = (torch.empty(lin0.N * lin0.K, dtype=torch.bfloat16, device=self.device)
                if t.rt == DEQUANT_RT else None)
        act = torch.empty(M, lin0.N // 2, dtype=self.dtype, device=self.device)
        red = torch.empty(M, lin0.N, dtype=self.dtype, device=self.device) if with_reduce else None
        if with_norm or resid:
            res = torch.zeros(M, lin0.N, dtype=self.dtype, device=self.device)
            nrm = torch.empty(M, lin0.N, dtype=self.dtype, device=self.device)
            nw = torch.ones(lin0.N, dtype=self.norm.dtype, device=self.device)
            ss_out = torch.empty(M, lin0.N // 16, dtype=torch.float32, device=self.device)
        if norm_in:
            ss_in = torch.full((M, lin0.K // 16), 16.0, dtype=torch.float32, device=self.device)
        if resid:
            xw = torch.empty(M, lin0.N, dtype=self.dtype, device=self.device)
        eps = float(self.cfg.rms_norm_eps)
        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            def body():
                for lin in lins:
                    if resid:
                        lin.launch_resid(x, M, t, res=res, res_out=res, ss=ss_out, norm_w=nw,
                                         xw=xw, stream=s.cuda_stream)
                    elif norm_in and swiglu:
                        lin.launch_norm(x, M, t, ss=ss_in, eps=eps, stream=s.cuda_stream,
                                        act=act)
                    elif swiglu:
                        lin.launch_swiglu(x, M, t, act, s.cuda_stream, wtmp=wtmp)
                    else:
                        if norm_in:
                            lin.launch_norm(x, M, t, ss=ss_in, eps=eps, stream=s.cuda_stream,
                                            part=part)
                        else:
                            lin.launch(x, M, t, part=part, wtmp=wtmp, stream=s.cuda_stream)
                        if with_act:   # the separate activation the fused form saves
                            check(lib().acorn_silu_mul(ptr(part), t.ksplit, None, ptr(act), M,
                                                       lin.N // 2, int(lin.il16),
                                                       dtype_code(act), s.cuda_stream),
                                  "silu_mul")
                        if with_reduce:
                            check(lib().acorn_splitk_reduce(ptr(part), t.ksplit, M * lin.N,
                                                            ptr(red), dtype_code(red),
                                                            s.cuda_stream), "splitk_reduce")
                        if with_norm:
                            check(lib().acorn_fused_add_rmsnorm_partials(
                                ptr(part), t.ksplit, ptr(res), ptr(res), ptr(nw), ptr(nrm), None,
                                M, lin.N, float(self.cfg.rms_norm_eps), dtype_code(nrm),
                                dtype_code(nw), s.cuda_stream), "K1")
            body()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                body()
            g.replay()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(reps):
                g.replay()
            e1.record(s)
        e1.synchronize()
        torch.cuda.current_stream(self.device).wait_stream(s)
        return e0.elapsed_time(e1) * 1e3 / (reps * len(lins))

    def tune(self, batch: int, *, names=None, verbose: bool = False,
             fold: bool | None = None) -> dict:
        """Load-time tiling choice for a decode bucket (the reference's
        quant_gemm.configure, acorninfer/ops/quant_gemm.py:449-492): every
        candidate tiling of each projection is timed in place, together with
        the work its split count puts on the consumer, the RETIME_TOP fastest
        are timed again with RETIME_REPS replays, and the fastest of those is
        kept in self.tilings[batch]; run before any graph capture."""
        if self.lm_head.fmt == _lib.WFMT_F32:
            return {}
        report = {}
        chosen = self.tilings.setdefault(batch, {})
        # the folded norms (o and down in one split with the residual
        # epilogue, qkv and gate|up normalising on load) are timed beside the
        # plain launches with their K1s, and kept where the four together are
        # faster (fold=True / False: only that form is timed, and kept)
        fold_ok = self.fold_possible(batch, tuned=False)
        if fold is not None:
            self.fold_choice[batch] = fold
        results = {}
        for name, lins in self.projections().items():
            if names is not None and name not in names:
                continue
            if name == "gate_up":
                self.swiglu_choice.pop(batch, None)
            modes = ((False, True) if fold is None else (fold,)) if fold_ok and name in FOLDED \
                else (False,)
            results[name] = {f: self._tune_one(name, lins, batch, f, verbose) for f in modes}
        if fold is None and fold_ok and all(n in results for n in FOLDED):
            plain = sum(results[n][False][0] for n in FOLDED)
            folded = sum(results[n][True][0] for n in FOLDED)
            self.fold_choice[batch] = folded < plain
            report["fold"] = {"chosen": folded < plain, "plain_us": round(plain, 3),
                              "folded_us": round(folded, 3)}
        fold = self.fold_possible(batch)
        for name, res in results.items():
            us, c, sw = res[fold] if fold in res else res[False]
            if name == "gate_up" and self.fused_swiglu_possible(batch):
                self.swiglu_choice[batch] = sw
            chosen[name] = c
            report[name] = {"tiling": tuple(c), "us": round(us, 3),
                            "bytes": self.projections()[name][0].nbytes()}
            if name == "gate_up":
                report[name]["fused_swiglu"] = sw
        return report

    def _tune_one(self, name: str, lins: list, batch: int, fold: bool,
                  verbose: bool) -> tuple:
        """(µs, tiling, swiglu) of the fastest candidate of one projection,
        each timed with the work its form puts on the step (see
        time_projection); fold times the folded forms."""
        from acorninfer_amd.ops.quant_gemm import candidates
        timed = []                             # (us, tiling, swiglu, consumer flags)
        modes = [False]
        if name == "gate_up" and self.fused_swiglu_possible(batch):
            modes = [True, False]
        for sw in modes:
            act = name == "gate_up" and not sw
            red = name == "qkv"                   # the qkv epilogue reads its partials
            nrm = name in ("o", "down") and not fold   # ... K1 those of o and down
            nin = fold and name in ("qkv", "gate_up")
            rsd = fold and name in ("o", "down")
            cands = candidates(batch, lins[0].N, lins[0].K, lins[0].fmt, swiglu=sw)
            if nin or rsd:
                # the folded forms are the direct kernels' (rt > 0); the
                # residual epilogue runs in one split
                cands = [c for c in cands if c.rt > 0 and (nin or c.ksplit == 1)]
            if red:
                # the fused K3 requests QKV_SPLITS_UP_FRONT split partials
                # with its first loads; each further split costs it a
                # round trip, which the timed reduction does not show
                cands = [c for c in cands if c.ksplit <= QKV_SPLITS_UP_FRONT] or cands
            for c in cands:
                us = self.time_projection(lins, batch, c, swiglu=sw, with_act=act,
                                          with_reduce=red, with_norm=nrm, norm_in=nin,
                                          resid=rsd)
                if verbose:
                    print(f"TUNE {name} M={batch} swiglu={sw} fold={fold} {tuple(c)} "
                          f"{us:.2f} us", flush=True)
                timed.append((us, c, sw, (act, red, nrm, nin, rsd)))
        # the closest few are timed again with more replays: single
        # timings of a few microseconds differ by more than the candidates do
        timed.sort(key=lambda t: t[0])
        best = None
        for _us, c, sw, (act, red, nrm, nin, rsd) in timed[:RETIME_TOP]:
            us = self.time_projection(lins, batch, c, reps=RETIME_REPS, swiglu=sw,
                                      with_act=act, with_reduce=red, with_norm=nrm,
                                      norm_in=nin, resid=rsd)
            if best is None or us < best[0]:
                best = (us, c, sw)
        return best

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

    def forward_prefill_batch(self, input_ids: torch.Tensor, views, *,
                              real_lens) -> torch.Tensor:
        """Batched prefill (qwen3.py:597-639): input_ids [N, Lmax] (right
        padded; pad values unused) + real_lens[i] -> fp32 logits [N, vocab]
        of each row's last real token. Every view starts empty; its KV gets
        the row's real_lens[i] tokens."""
        N, Lmax = input_ids.shape
        if len(views) != N or len(real_lens) != N:
            raise ValueError(f"views/real_lens must match the batch: N={N}, "
                             f"len(views)={len(views)}, len(real_lens)={len(real_lens)}")
        if min(real_lens) < 1 or max(real_lens) > Lmax:
            raise ValueError(f"real_lens must lie in [1, Lmax]: min={min(real_lens)}, "
                             f"max={max(real_lens)}, Lmax={Lmax}")
        if any(v.seq_len != 0 for v in views):
            raise ValueError("forward_prefill_batch: every view must start empty "
                             "(forward_extend continues a sequence)")
        return self.forward_extend(input_ids, views, starts=[0] * N, chunk_lens=list(real_lens))

    def forward_extend(self, input_ids: torch.Tensor, views, *, starts: list[int],
                       chunk_lens: list[int]) -> torch.Tensor:
        """Chunked prefill (qwen3.py:641-686): input_ids [N, Lc_max] (right
        padded) + starts[i] (= views[i]'s KV length) + chunk_lens[i] -> fp32
        logits [N, vocab] at each row's position start + len - 1.

        The rows of all chunks are packed into one launch sequence of the
        decode step, one row per token: token p of a sequence is a row with
        position p and KV target (table[p // P], p % P). The qkv epilogue
        writes every row's k/v before attention runs (fused_attn=False),
        which is what lets a row read the tokens of the same chunk before it.
        Attention is the query-tiled prefill kernel over each sequence's run
        of rows (causal over the cache, 16 query tokens per MFMA tile); for
        shapes it is not built for (fp32, head_dim 16/32), K3 with one row
        per token and length p + 1. GEMMs run at M = total rows; lm_head
        only for each chunk's last row."""
        N, Lc = input_ids.shape
        if len(views) != N or len(starts) != N or len(chunk_lens) != N:
            raise ValueError(f"views/starts/chunk_lens must match the batch: N={N}, "
                             f"len(views)={len(views)}, len(starts)={len(starts)}, "
                             f"len(chunk_lens)={len(chunk_lens)}")
        if min(chunk_lens) < 1 or max(chunk_lens) > Lc or min(starts) < 0:
            raise ValueError(f"chunk_lens must lie in [1, Lc_max] and starts be >= 0: "
                             f"min(len)={min(chunk_lens)}, max(len)={max(chunk_lens)}, "
                             f"Lc_max={Lc}, min(start)={min(starts)}")
        for v, s in zip(views, starts):
            if v.seq_len != s:
                raise ValueError(f"forward_extend: view KV length {v.seq_len} != start {s}")
        cache = views[0].cache
        P = cache.page_size
        cfg = self.cfg
        tiled = self.tiled_prefill and prefill_supported(
            self.dtype, cfg.head_dim, P, cfg.num_attention_heads, cfg.num_key_value_heads)
        targets = [v.reserve(n) for v, n in zip(views, chunk_lens)]
        W = max(len(v.table) for v in views)
        ids, pos, pages, slots, lens, tabs = [], [], [], [], [], []
        for i, (v, s, n) in enumerate(zip(views, starts, chunk_lens)):
            ids.append(input_ids[i, :n].to(torch.int64).cpu())
            pos += list(range(s, s + n))
            pages += [p for p, _ in targets[i]]
            slots += [q for _, q in targets[i]]
            lens += list(range(s + 1, s + n + 1))
            row = torch.zeros(W, dtype=torch.int32)
            row[:len(v.table)] = torch.tensor(v.table, dtype=torch.int32)
            tabs.append(row)
        R = len(pos)
        ids_all = torch.cat(ids)
        pos_all = torch.tensor(pos, dtype=torch.int64)
        pages_all = torch.tensor(pages, dtype=torch.int64)
        slots_all = torch.tensor(slots, dtype=torch.int64)
        lens_all = torch.tensor(lens, dtype=torch.int32)
        seq_tabs = torch.stack(tabs)                                  # [N, W]
        first = torch.tensor([0] + list(chunk_lens), dtype=torch.int64).cumsum(0)
        last = first[1:] - 1
        dev = self.device
        # Rows run in blocks of at most EXTEND_MAX_ROWS, in order: a block's
        # layer-l attention reads the k/v that earlier blocks wrote at layer l,
        # so this is chunked prefill over the packed rows.
        outs = []
        for r0 in range(0, R, EXTEND_MAX_ROWS):
            r1 = min(R, r0 + EXTEND_MAX_ROWS)
            Rb = r1 - r0
            # the step buffers of the last shape are kept (a prompt batch often repeats it)
            # (the prefill kernel reads per-sequence tables: no per-row table)
            key = (Rb, 1 if tiled else W, self.prefill_gemm, self.prefill_direct)
            cached = getattr(self, "_extend_buf", None)
            if cached is None or cached[0] != key:
                self._extend_buf = None
                lib_t = None
                lw = self.layers[0]
                if self.prefill_gemm not in ("own", "int4"):
                    raise ValueError(f"prefill_gemm must be 'own' or 'int4', not "
                                     f"{self.prefill_gemm!r}")
                if self.prefill_gemm == "int4" and lw.qkv.fmt == WFMT_W4B:
                    # the int4 planner's full choices (explicit: no dequantisation)
                    lib_t = {n: lin.plan(Rb)[0] for n, lin in (
                        ("qkv", lw.qkv), ("o", lw.o), ("gate_up", lw.gate_up),
                        ("down", lw.down))}
                self._extend_buf = (key, self.buffers(Rb, key[1], tilings=lib_t, prefill=True))
            buf = self._extend_buf[1]
            buf.ids.copy_(ids_all[r0:r1])
            buf.positions.copy_(pos_all[r0:r1])
            buf.pages.copy_(pages_all[r0:r1])
            buf.slots.copy_(slots_all[r0:r1])
            segs = None
            if tiled:
                segs = PrefillSegments.for_rows(first, starts, seq_tabs, r0, r1, dev)
            else:
                buf.lens.copy_(lens_all[r0:r1])
                for i in range(N):                 # each sequence's table on its rows
                    a, b = max(int(first[i]), r0), min(int(first[i + 1]), r1)
                    if a < b:
                        buf.tables[a - r0:b - r0].copy_(seq_tabs[i].expand(b - a, W))
            heads = last[(last >= r0) & (last < r1)] - r0
            outs.append(self.step(buf, cache.k_pool, cache.v_pool, cache.num_blocks, P,
                                  fused_attn=False, head_rows=heads.to(dev), segments=segs))
        for v, n in zip(views, chunk_lens):
            for li in range(self.cfg.num_hidden_layers):
                v._lens[li] = v._lens.get(li, 0) + n
        return torch.cat(outs).float()


@dataclass
class PrefillSegments:
    """The sequences of one block of prefill rows, as the prefill attention
    kernel reads them: sequence n's rows are block rows row0[n] ..
    row0[n] + nq[n] - 1 at positions pos0[n] + j, with block table tables[n]
    (all int32 on the device)."""
    tables: torch.Tensor    # [count, W]
    row0: torch.Tensor      # [count]
    pos0: torch.Tensor      # [count]
    nq: torch.Tensor        # [count]
    count: int
    max_nq: int

    @classmethod
    def for_rows(cls, first: torch.Tensor, starts: list[int], seq_tabs: torch.Tensor,
                 r0: int, r1: int, device) -> "PrefillSegments":
        """Rows [r0, r1) of a packing where sequence i holds rows
        first[i] .. first[i + 1] - 1 from KV position starts[i]."""
        sel, row0, pos0, nq = [], [], [], []
        for i in range(len(starts)):
            a, b = max(int(first[i]), r0), min(int(first[i + 1]), r1)
            if a < b:
                sel.append(i)
                row0.append(a - r0)
                pos0.append(starts[i] + a - int(first[i]))
                nq.append(b - a)
        meta = torch.tensor([row0, pos0, nq], dtype=torch.int32)
        blob = torch.cat([meta.reshape(-1), seq_tabs[sel].reshape(-1)]).to(device)
        n = len(sel)
        return cls(blob[3 * n:].view(n, seq_tabs.shape[1]), blob[0:n], blob[n:2 * n],
                   blob[2 * n:3 * n], n, max(nq))


def _dense_linear(w: torch.Tensor, dtype: torch.dtype) -> QLinear:
    """fp32 weights (parity path): kept dense in the activation dtype."""
    if dtype == torch.float32:
        return QLinear(_lib.WFMT_F32, w.float().contiguous(), w.shape[0], w.shape[1])
    raise ValueError(f"no dense weight format for activations of dtype {dtype}")


UNIT_PAGES = 4      # K3 split size the heuristic aims for (pages)
EXTEND_MAX_ROWS = 8192    # prefill rows per launch sequence (K3's grid holds <= 65535)
PREFILL_WS_BYTES = 256 << 20   # cap on a prefill launch's K3 split workspace
SMALL_GRID_PAGES = 1024   # below this many (sequence, kv head, page) units: 1-page splits
MAX_SPLITS = 64     # bound on K3 splits per (sequence, kv head)
WIDE_GRID = 256     # (sequence, kv head) pairs that fill the CUs on their own ...
ONE_SPLIT_MAX_PAGES = 64   # ... take one split over tables this wide,
WIDE_UNIT_PAGES = 16       # ... and splits of this many pages over wider ones
QKV_SPLITS_UP_FRONT = 4   # qkv split partials the fused K3 loads up front (kQB)
RETIME_TOP = 4      # tune(): candidates timed a second time ...
RETIME_REPS = 12    # ... with this many graph replays
FOLDED = ("qkv", "o", "gate_up", "down")   # the projections the RMSNorms fold into


def attention_splits(batch: int, kv_heads: int, max_pages: int, *,
                     unit_pages: int | None = None, max_splits: int = MAX_SPLITS,
                     q_per_kv: int = 1) -> int:
    """K3 split count S for block tables `max_pages` wide.

    K3 gives every split the same pps = ceil(max_pages / S) pages, so a
    sequence of n pages uses ceil(n / pps) splits and the rest exit at once.
    Small splits (here `unit_pages`, 64 tokens at P = 16) run as one-wave
    workgroups: many equal work units that the dispatcher spreads evenly over
    the CUs, whatever the mix of context lengths. S is capped at `max_splits`
    (workspace B*H*S*(D+2) floats; K3 writes and the combine reads one
    partial per used split), so very wide tables get proportionally larger
    splits. A small grid (batch * kv_heads * max_pages below
    SMALL_GRID_PAGES, e.g. one sequence) uses 1-page splits instead, so that
    its few waves each wait for one chunk rather than walk four. A grid that
    fills the CUs with (sequence, kv head) pairs alone (WIDE_GRID) over
    tables of at most ONE_SPLIT_MAX_PAGES pages takes one split: each pair
    is one workgroup of four waves merged in LDS, with no combine launch
    (C = 32 at 512 tokens: 4.43 against 4.56 ms per step). Over wider tables
    such a grid takes WIDE_UNIT_PAGES-page splits, the longest that still run
    as one-wave workgroups: half the partials of 8-page splits for the
    combine (C = 64 over prompts U[1024, 8192], 512-page tables: K3 + combine
    220 against 234 us per layer). With `q_per_kv` (q heads per kv head) the
    one-split rule counts the q heads: K3 gives a single split's q heads
    workgroups of their own while the pairs are fewer than the CUs (its head
    groups), so C = 8 at 512 tokens runs as 256 workgroups with no combine
    (bf16 step 3.11-3.13 against 3.14 ms)."""
    if unit_pages is None and batch * kv_heads * q_per_kv >= WIDE_GRID \
            and max_pages <= ONE_SPLIT_MAX_PAGES:
        return 1
    if unit_pages is None and batch * kv_heads >= WIDE_GRID:
        unit_pages = WIDE_UNIT_PAGES
    if unit_pages is None:
        unit_pages = 1 if batch * kv_heads * max_pages < SMALL_GRID_PAGES else UNIT_PAGES
    return max(1, min(-(-max_pages // unit_pages), max_splits))


@dataclass
class StepBuffers:
    """Address-stable inputs, outputs and scratch of one decode step."""
    model: Qwen3DecodeModel
    batch: int
    max_pages: int
    num_splits: int | None = None
    tilings: dict | None = None       # name -> requested Tiling (0 fields = planner)
    cfgs: dict = field(default_factory=dict)
    prefill: bool = False             # prompt rows: no decode logits / lm_head workspace

    def __post_init__(self):
        m = self.model
        cfg, dev, dt = m.cfg, m.device, m.dtype
        B = self.batch
        H, D = cfg.hidden_size, cfg.head_dim
        nq, nkv, inter = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.intermediate_size
        if self.num_splits is None:
            self.num_splits = attention_splits(B, nkv, self.max_pages,
                                               q_per_kv=1 if self.prefill else nq // nkv)
            if self.prefill:
                # one row per prompt token: bound the split workspace
                cap = PREFILL_WS_BYTES // max(1, B * nq * (D + 2) * 4)
                self.num_splits = max(1, min(self.num_splits, cap))
        lw = m.layers[0]
        tilings = self.tilings or {}
        # prefill blocks: the large-M kernel's SwiGLU epilogue unless a
        # tiling is requested for gate|up (the int4 kernels)
        self.swiglu = (m.prefill_swiglu(B) and "gate_up" not in tilings if self.prefill
                       else m.fused_swiglu(B))
        for name, lin in (("qkv", lw.qkv), ("o", lw.o), ("gate_up", lw.gate_up),
                          ("down", lw.down), ("lm_head", m.lm_head)):
            if name == "gate_up" and self.swiglu:
                self.cfgs[name] = lin.swiglu_plan(B, tilings.get(name), workspace=True)[0]
            else:
                self.cfgs[name] = lin.plan(B, tilings.get(name), workspace=name != "lm_head")[0]
        # bf16 copy of one int4 projection at a time (DEQUANT_RT tilings)
        nk = [lin.N * lin.K for name, lin in (("qkv", lw.qkv), ("o", lw.o),
                                             ("gate_up", lw.gate_up), ("down", lw.down))
              if self.cfgs[name][0] == DEQUANT_RT]
        self.wtmp = (torch.empty(max(nk), dtype=torch.bfloat16, device=dev) if nk else None)
        # The host-written inputs are one byte block, so a step needs one copy:
        # int64 ids | positions | pages | slots, then int32 lens | tables, then
        # the sampling block f32 temperature | top_p | uniform | top_k (int32
        # bits; temperature 0 = greedy). `meta_ends` are the ends of the three
        # parts in bytes. The sampler writes the next step's ids over `ids`.
        e64 = 8 * 4 * B
        e32 = e64 + 4 * B * (1 + self.max_pages)
        self.meta_ends = (e64, e32, e32 + 4 * 4 * B)
        self.meta = torch.zeros(self.meta_ends[2], dtype=torch.uint8, device=dev)
        self.flat_i64 = self.meta[:e64].view(torch.int64)
        self.flat_i32 = self.meta[e64:e32].view(torch.int32)
        self.flat_f32 = self.meta[e32:].view(torch.float32)
        self.ids = self.flat_i64[0:B]
        self.positions = self.flat_i64[B:2 * B]
        self.pages = self.flat_i64[2 * B:3 * B]
        self.slots = self.flat_i64[3 * B:4 * B]
        self.next_ids = self.ids
        self.lens = self.flat_i32[0:B]
        self.tables = self.flat_i32[B:].view(B, self.max_pages)
        self.lens.fill_(1)
        self.temperature = self.flat_f32[0:B]
        self.top_p = self.flat_f32[B:2 * B]
        self.uniform = self.flat_f32[2 * B:3 * B]
        self.top_k = self.flat_f32[3 * B:4 * B].view(torch.int32)
        self.top_p.fill_(1.0)
        self.logprob = torch.zeros(B, dtype=torch.float32, device=dev)
        self.status = torch.zeros(B, dtype=torch.int32, device=dev)

        def z(*shape, dtype=dt):
            return torch.zeros(*shape, dtype=dtype, device=dev)

        f32 = torch.float32
        self.x = z(B, H)
        self.res = z(B, H)
        self.normed = z(B, H)
        self.q = z(B, nq, D)
        self.attn = z(B, nq * D)
        self.act = z(B, inter)
        # prefill: qkv / o / down straight to the activation dtype when each is
        # one split on the large-M kernel (the epilogue and K1 read it as is)
        large = (DENSE_RT, DEQUANT_RT)
        self.direct = (self.prefill and m.prefill_direct and D == 128 and B >= PREFILL_DIRECT_M
                       and dt == torch.bfloat16 and
                       all(self.cfgs[n].rt in large and self.cfgs[n].ksplit == 1
                           for n in ("qkv", "o", "down")))
        if self.direct:
            self.y_qkv = z(B, (nq + 2 * nkv) * D)
            self.y_o = z(B, H)
            self.y_down = z(B, H)
            self.part_qkv = self.part_o = None
        else:
            self.part_qkv = z(self.cfgs["qkv"].ksplit, B, (nq + 2 * nkv) * D, dtype=f32)
            self.part_o = z(self.cfgs["o"].ksplit, B, H, dtype=f32)
        # (the fused SwiGLU writes act directly: no gate|up partials at prefill sizes)
        self.part_gu = (None if self.swiglu and self.prefill else
                        z(self.cfgs["gate_up"].ksplit, B, 2 * inter, dtype=f32))
        self.part_down = None if self.direct else z(self.cfgs["down"].ksplit, B, H, dtype=f32)
        # the RMSNorms folded into the projections (decode, block layouts, o
        # and down in one split): the sums of squares of the residual after o
        # (read by gate|up) and after down (read by the next layer's qkv)
        self.fold = (not self.prefill and m.fold_possible(B)
                     and self.cfgs["o"].ksplit == 1 and self.cfgs["down"].ksplit == 1)
        self.ss_o = z(B, H // 16, dtype=f32) if self.fold else None
        self.ss_dn = z(B, H // 16, dtype=f32) if self.fold else None
        ks_lm = self.cfgs["lm_head"].ksplit
        S = self.num_splits
        self.ws_acc = z(B * nq * S * D, dtype=f32) if S > 1 else None
        self.ws_ml = z(2 * B * nq * S, dtype=f32) if S > 1 else None
        if self.prefill:
            # step(head_rows=...) computes the few logits it needs on its own
            self.ws_lm = self.logits = None
        else:
            self.ws_lm = z(ks_lm, B, cfg.vocab_size, dtype=f32) if ks_lm > 1 else None
            self.logits = z(B, cfg.vocab_size, dtype=dt)
