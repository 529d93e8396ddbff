"""Weight-only quantised GEMM on the GPU (W8A16, W4A16 g128, and bf16).

Drop-in for acorninfer/ops/quant_gemm.py: `quant_gemm` (:257-294), `CLASSES`
(:67-73), `_CLS_BY_SHAPE` (:99), `M_BUCKETS_LARGE` (:82), `bucket_for`
(:86-94), `_state` (:101-107), `configure` (:449-492) and `reset` (:495-499).
New next to them (no reference counterpart in production): `quant_gemm_w4`
for packed int4 group-128 weights, and `gemm_partials`, the decode-step form
that leaves fp32 split-K partials for the consumer kernel to reduce.

All formats run on one MFMA kernel (csrc/quant_gemm.hip); a tiling is a
`Tiling` (rt, upw, nw, ksplit, tpw). The reference's 5-tuple configs are
accepted for compatibility; only their SPLIT_K field carries over. With
ksplit > 1 and a bf16 output the partials go through an address-stable
workspace (`_workspace`) and are summed in split order by a second launch.
"""
from __future__ import annotations

import ctypes
import time
from typing import NamedTuple

import torch

from acorninfer_amd._lib import (BF16, WFMT_BF16, WFMT_BF16B, WFMT_W4, WFMT_W4B, WFMT_W8, WFMT_W8B,
                                 check, lib,
                                 ptr, require_gpu, stream_ptr)

CLASSES = {
    "qo": (4096, 4096),
    "kv": (1024, 4096),
    "gate_up": (12288, 4096),
    "down": (4096, 12288),
    "lm_head": (151936, 4096),
}
# Fused projection shapes used by this build's decode step (qkv and gate|up
# concatenated along N).
FUSED_CLASSES = {
    "qkv": (6144, 4096),
    "gate_up2": (24576, 4096),
}
_CLS_BY_SHAPE = {v: k for k, v in CLASSES.items()}

DECODE_M_MAX = 16
W4B_M_MAX = 64      # the int4 decode kernel takes up to this many rows on request
MID_RT = -3         # Tiling.rt of the mid-M kernels (W4B and W8B, M > 16)
M_BUCKETS_LARGE = ("s", "m", "l")
_M_REP_M = {"s": 64, "m": 256, "l": 1024}

_state: dict = {
    "configs": {},     # cls -> Tiling   decode bucket (M <= 16)
    "m_configs": {},   # cls -> {bucket: Tiling}
    "shapes": {},      # cls -> (N, K)
    "workspaces": {},  # (rows, N, ksplit) -> fp32 [ksplit, rows, N]
    "device": None,
    "report": None,
}


def bucket_for(M: int) -> str:
    """M -> bucket name: d (M <= 16, decode) / s (<= 64) / m (<= 256) / l."""
    if M <= DECODE_M_MAX:
        return "d"
    if M <= 64:
        return "s"
    if M <= 256:
        return "m"
    return "l"


class Tiling(NamedTuple):
    """Native tiling of acorn_quant_gemm; 0 = planner's choice.

    Streaming kernel (the weight-stream form; M <= 16, or any M with rt >= 1):
    rt: 16-row weight tiles per wavefront row block; upw: 16-byte weight
    loads per lane per pipeline step; nw: wavefronts per workgroup (they
    split K); ksplit: workgroups along K; tpw: row tiles per workgroup.
    Tiled kernel (M > 16 with rt == 0, the default there): upw is the M tile
    BM (32 / 64 / 128), nw the N tile BN (64 / 128), ksplit the K split; the
    planner reports (0, BM, BN, ksplit, 1).
    int4 decode kernels (WFMT_W4B; M <= 16 the direct kernel, 16 < M <= 64
    with rt >= 1 the one that stages x in LDS): rt row tiles per wave, upw
    128-k groups per pipeline stage, nw the wave layout (M <= 16: 1 or 4
    waves each on its own rows; above: 2 or 4; 10*nw + kw: kw waves share
    rows and split K, 22 / 44 / 84 / 88 at M <= 16, 42 / 44 / 82 / 84
    above), ksplit, and tpw = stages in flight per wave.
    int8 decode kernel (WFMT_W8B, M <= 16): rt row tiles per wave, upw 64-k
    blocks per stage, nw the wave layout (1, 4, 22, 44), ksplit,
    tpw = stages in flight; above 16 rows W8B runs on the tiled kernel or the
    int8 mid-M kernel.
    bf16 decode kernel (WFMT_BF16B, M <= 16): rt row tiles per wave, upw
    32-k blocks per stage, nw the wave layout (1, 4, 22, 44), ksplit, tpw =
    stages in flight; above 16 rows BF16B runs on the tiled kernel and from
    256 rows on the large-M kernel (its direct-to-LDS and 64 / 128 forms).
    int4 / int8 mid-M kernels (WFMT_W4B / WFMT_W8B, M > 16, rt == -3): upw
    row tiles per wave (1 / 2), nw waves (4 / 8), ksplit, tpw 128-k steps in
    flight (2 / 4; 8 for the int4 one at one tile and 8 waves); 64 x rows per
    workgroup, streamed through LDS 128 k at a time.
    Large-M bf16 kernel (the default for bf16 from 256 rows, or rt == -2):
    upw is the M tile. 64 / 128: nw the weight rows per wave (64 / 128; a
    workgroup's weight tile is 4 nw), tpw the weight prefetch depth in 64-k
    steps (2 / 4). 256 (256 x 256 tiles): nw 64 with tpw 2 stages both
    operands through registers; nw 128 with tpw 4 loads them straight into
    LDS through a 4-stage ring (the default). Reported as (-2, BM, nw,
    ksplit, tpw).
    """
    rt: int = 0
    upw: int = 0
    nw: int = 0
    ksplit: int = 0
    tpw: int = 0


def plan(M: int, N: int, K: int, wfmt: int, cfg: Tiling | None = None
         ) -> tuple[Tiling, int]:
    """The library planner's full choice for (M, N, K, format), honouring the
    non-zero fields of `cfg`. Returns (tiling, output tiles of the launch)."""
    arr = (ctypes.c_int * 6)(*(tuple(cfg) if cfg is not None else (0,) * 5), 0)
    check(lib().acorn_gemm_plan(M, N, K, wfmt, arr), "gemm_plan")
    return Tiling(*arr[:5]), arr[5]


def swiglu_plan(M: int, N: int, K: int, wfmt: int, cfg: Tiling | None = None
                ) -> tuple[Tiling, int]:
    """Tiling of the fused gate|up + SwiGLU launch (rt = 2, ksplit = 1)."""
    arr = (ctypes.c_int * 6)(*(tuple(cfg) if cfg is not None else (0,) * 5), 0)
    check(lib().acorn_gemm_swiglu_plan(M, N, K, wfmt, arr), "gemm_swiglu_plan")
    return Tiling(*arr[:5]), arr[5]


def interleave16(t: torch.Tensor) -> torch.Tensor:
    """[gate (I rows); up (I rows)] -> 16-row blocks alternating gate and up
    (the weight layout of acorn_quant_gemm_swiglu). Works on weights, packed
    weights and per-row scales alike."""
    n2 = t.shape[0]
    assert n2 % 32 == 0, "gate|up rows must be a multiple of 32"
    rest = t.shape[1:]
    return t.reshape(2, n2 // 32, 16, *rest).transpose(0, 1).reshape(n2, *rest).contiguous()


def deinterleave16(t: torch.Tensor) -> torch.Tensor:
    """Inverse of interleave16."""
    n2 = t.shape[0]
    rest = t.shape[1:]
    return t.reshape(n2 // 32, 2, 16, *rest).transpose(0, 1).reshape(n2, *rest).contiguous()


def _native_cfg(cfg, M: int) -> Tiling | None:
    """A native Tiling from an explicit cfg.

    Accepted: a Tiling; a 3-tuple (rt, nw, ksplit); or the reference's
    5-tuple, read by M regime as the reference does: for M <= 16 it is
    (BN, BK, warps, stages, SPLIT_K) and SPLIT_K carries over; for M > 16 it
    is (BM, BN, BK, warps, stages) and nothing carries over (this kernel picks
    its own M tiling).
    """
    if cfg is None:
        return None
    if isinstance(cfg, Tiling):
        return cfg
    cfg = tuple(int(c) for c in cfg)
    if len(cfg) == 3:
        return Tiling(rt=cfg[0], nw=cfg[1], ksplit=cfg[2])
    if len(cfg) == 5:
        return Tiling(ksplit=cfg[4]) if M <= DECODE_M_MAX else Tiling()
    raise ValueError(f"quant_gemm cfg must be a Tiling, (rt, nw, ksplit) or a reference "
                     f"5-tuple: {cfg}")


def _workspace(rows: int, N: int, ksplit: int, device) -> torch.Tensor:
    """Address-stable fp32 split-K workspace [ksplit, rows, N]."""
    key = (rows, N, ksplit, str(device))
    ws = _state["workspaces"].get(key)
    if ws is None:
        ws = torch.empty(ksplit, rows, N, dtype=torch.float32, device=device)
        _state["workspaces"][key] = ws
    return ws


def _launch(x2: torch.Tensor, w: torch.Tensor, scale, zero, wfmt: int, N: int,
            cfg: Tiling | None, out: torch.Tensor | None) -> torch.Tensor:
    M, K = x2.shape
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=x2.device)
    assert out.shape == (M, N) and out.dtype == torch.bfloat16 and out.is_contiguous()
    tiling, _ = plan(M, N, K, wfmt, _native_cfg(cfg, M))
    part = _workspace(M, N, tiling.ksplit, x2.device) if tiling.ksplit > 1 else None
    arr = (ctypes.c_int * 6)(*tiling, 0)
    rc = lib().acorn_quant_gemm(ptr(x2), ptr(w), ptr(scale), ptr(zero), ptr(out), ptr(part),
                                M, N, K, wfmt, arr, stream_ptr(x2.device))
    check(rc, "quant_gemm")
    return out


def _prep_x(x: torch.Tensor) -> torch.Tensor:
    K = x.shape[-1]
    x2 = x.reshape(x.numel() // K, K)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    assert x2.dtype == torch.bfloat16, "activations must be bf16"
    return x2


def _pick_cfg(cls, M: int, cfg) -> tuple[int, int, int] | None:
    native = _native_cfg(cfg, M)
    if native is not None:
        return native
    if M <= DECODE_M_MAX:
        return _state["configs"].get(cls)
    table = _state["m_configs"].get(cls)
    if not table:
        raise RuntimeError(
            f"quant_gemm large-M bucket not configured: cls={cls} (M={M}); call "
            f"configure() at load time (tests may pass an explicit cfg)")
    bucket = bucket_for(M)
    if bucket not in table:
        raise RuntimeError(f"quant_gemm large-M bucket missing: cls={cls} bucket={bucket} (M={M})")
    return table[bucket]


def quant_gemm(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor, cls, cfg=None,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """W8A16: x [..., K] bf16, q int8 [N, K], scale fp16 [N] -> [M, N] bf16.

    y = x @ (q * scale)^T accumulated in fp32 (the products x*q are exact;
    the per-channel scale is applied once per output). M > 16 needs a
    configure()d large-M table or an explicit cfg, as in the reference.
    """
    require_gpu(x, q, scale)
    x2 = _prep_x(x)
    N, K = q.shape
    assert q.dtype == torch.int8 and q.is_contiguous(), "q must be contiguous int8 [N,K]"
    assert scale.dtype == torch.float16 and scale.numel() == N
    assert x2.shape[1] == K
    c = _pick_cfg(cls, x2.shape[0], cfg)
    return _launch(x2, q, scale.contiguous(), None, WFMT_W8, N, c, out)


def quant_gemm_w4(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor,
                  zero: torch.Tensor | None = None, cls=None, cfg=None,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """W4A16 group-128: x [..., K] bf16, packed uint8 [N, K/2] (low nibble =
    even k, quantize.pack_w4), scale fp16 [N, K/128], zero fp16 [N, K/128] or
    None -> [M, N] bf16.

    zero None means the symmetric format: stored u = v + 8, w = v * scale.
    With a zero (the reference's asymmetric quantize_w4), w = u*scale + zero.
    """
    require_gpu(x, packed, scale, zero)
    x2 = _prep_x(x)
    N, Kh = packed.shape
    K = 2 * Kh
    assert packed.dtype == torch.uint8 and packed.is_contiguous()
    assert K % 128 == 0, "K must be a multiple of the 128 group"
    assert scale.dtype == torch.float16 and scale.shape == (N, K // 128)
    if zero is not None:
        assert zero.dtype == torch.float16 and zero.shape == (N, K // 128)
        zero = zero.contiguous()
    assert x2.shape[1] == K
    M = x2.shape[0]
    c = _native_cfg(cfg, M) if cfg is not None else (
        _state["configs"].get(cls) if M <= DECODE_M_MAX else
        _state["m_configs"].get(cls, {}).get(bucket_for(M)))
    return _launch(x2, packed, scale.contiguous(), zero, WFMT_W4, N, c, out)


def bf16_gemm(x: torch.Tensor, w: torch.Tensor, cls=None, cfg=None,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """Dense bf16 x [..., K] @ w[N, K]^T -> [M, N] bf16 (fp32 accumulate)."""
    require_gpu(x, w)
    x2 = _prep_x(x)
    N, K = w.shape
    assert w.dtype == torch.bfloat16 and w.is_contiguous() and x2.shape[1] == K
    c = _native_cfg(cfg, x2.shape[0]) if cfg is not None else _state["configs"].get(cls)
    return _launch(x2, w, None, None, WFMT_BF16, N, c, out)


def gemm_partials(x2: torch.Tensor, w: torch.Tensor, scale, zero, wfmt: int,
                  part: torch.Tensor, cfg) -> None:
    """Decode-step form: write fp32 split-K partials part[ksplit, M, N]; the
    consumer kernel sums them (in split order) and applies the output cast."""
    M, K = x2.shape
    ks, Mp, N = part.shape
    assert Mp == M and part.dtype == torch.float32 and part.is_contiguous()
    tiling, _ = plan(M, N, K, wfmt, _native_cfg(cfg, M))
    assert tiling.ksplit == ks, f"partials buffer has {ks} splits, tiling wants {tiling.ksplit}"
    arr = (ctypes.c_int * 6)(*tiling, 0)
    rc = lib().acorn_quant_gemm(ptr(x2), ptr(w), ptr(scale), ptr(zero), None, ptr(part),
                                M, N, K, wfmt, arr, stream_ptr(x2.device))
    check(rc, "quant_gemm(partials)")


# ---------------------------------------------------------------- load time --

def _time_cfg(fn, reps: int = 20) -> float:
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / reps


def candidates(M: int, N: int, K: int, wfmt: int, swiglu: bool = False) -> list[Tiling]:
    """The planner's default plus a neighbourhood of valid tilings (distinct
    full choices only) for a load-time sweep."""
    planner = swiglu_plan if swiglu else plan
    base, _ = planner(M, N, K, wfmt)
    reqs = [Tiling()]
    if wfmt in (WFMT_W4B, WFMT_W8B, WFMT_BF16B) and M <= DECODE_M_MAX:
        reqs += {WFMT_W4B: _w4b_requests, WFMT_W8B: _w8b_requests,
                 WFMT_BF16B: _bf16b_requests}[wfmt](swiglu)
        if not swiglu:
            for bn in (64, 128):
                for ks in (1, 2, 4, 8, 16):
                    reqs.append(Tiling(0, 32, bn, ks, 0))
        return _resolve(reqs, planner, M, N, K, wfmt, base)
    for rt in (1, 2, 4):
        for upw in (2, 4, 8, 16):
            for nw in (2, 4, 8):
                for ks in (0, 1, 2, 3, 4):
                    reqs.append(Tiling(rt, upw, nw, ks, 0))
    for tpw in (1, 2, 4, 8):
        for upw in (2, 4, 8):
            for nw in (2, 4, 8):
                reqs.append(Tiling(0, upw, nw, 0, tpw))
    # more rows per workgroup over a shorter K range: the staged x (shared by
    # all workgroups) then costs less per weight byte, at the price of more
    # split partials
    for ks in (4, 6, 8, 12, 16):
        for tpw in (2, 4, 8, 12, 16, 24):
            for nw in (1, 2, 4):
                for upw in (2, 4):
                    reqs.append(Tiling(0, upw, nw, ks, tpw))
    if M > DECODE_M_MAX and not swiglu:
        reqs = [r for r in reqs if r.rt > 0]      # rt 0 means the tiled kernel here
        if wfmt == WFMT_W4B and M <= W4B_M_MAX:
            reqs = _w4b_wide_requests()           # the int4 kernel with 2 or 4 x blocks
        if wfmt in (WFMT_W4B, WFMT_W8B):
            reqs += [Tiling(MID_RT, rt, nw, ks, depth)   # the mid-M int4 / int8 kernels
                     for rt in (1, 2) for nw in (4, 8) for depth in (2, 4, 8)
                     for ks in (0, 1, 2, 4, 8, 16)]
        for bm in (32, 64, 128):
            for bn in (64, 128):
                for ks in (0, 1, 2, 4, 8):
                    reqs.append(Tiling(0, bm, bn, ks, 0))
    elif not swiglu:
        # the tiled kernel at its smallest M tile competes for decode sizes too
        for bn in (64, 128):
            for ks in (1, 2, 4, 8, 16):
                reqs.append(Tiling(0, 32, bn, ks, 0))
    return _resolve(reqs, planner, M, N, K, wfmt, base)


def _w4b_requests(swiglu: bool) -> list[Tiling]:
    """Requests covering the int4 direct kernel's knobs (M <= 16): 1, 2 or 4
    row tiles per wave, one group per stage with 2 or 4 stages in flight or
    two groups with 2 or 4 (4 where the paired-x form of M <= 8 fits it), one
    or four waves per workgroup on their own rows or 2,
    4 or 8 K slices over shared rows (22, 44, 84 = two row groups of four
    slices, 88), and split counts from one to sixteen (the fused SwiGLU runs
    in one split)."""
    reqs = []
    for rt in ((2, 4) if swiglu else (1, 2, 4)):
        for upw, depth in ((1, 2), (1, 4), (2, 2), (2, 4)):
            for nw in (1, 4, 22, 44, 84, 88):
                for ks in ((1,) if swiglu else (0, 1, 2, 3, 4, 6, 8, 12, 16)):
                    reqs.append(Tiling(rt, upw, nw, ks, depth))
    return reqs


def _w8b_requests(swiglu: bool) -> list[Tiling]:
    """Requests covering the int8 direct kernel's knobs (M <= 16): 1, 2 or 4
    row tiles per wave, one or two 64-k blocks per stage with 2 to 8 stages in
    flight, the same wave layouts as the int4 kernel (1, 4, 22, 44), and split
    counts from one to sixteen (the fused SwiGLU runs in one split)."""
    reqs = []
    for rt in ((2, 4) if swiglu else (1, 2, 4)):
        for upw, depth in ((1, 4), (1, 8), (2, 2), (2, 4), (2, 8)):
            for nw in (1, 4, 22, 44):
                for ks in ((1,) if swiglu else (0, 1, 2, 3, 4, 6, 8, 12, 16)):
                    reqs.append(Tiling(rt, upw, nw, ks, depth))
    return reqs


def _bf16b_requests(swiglu: bool) -> list[Tiling]:
    """Requests covering the bf16 direct kernel's knobs (M <= 16): 1, 2 or 4
    row tiles per wave, 1 / 2 / 4 blocks of 32 k per stage with 2 to 8 stages
    in flight, the wave layouts 1, 4, 22, 44, and split counts from one to
    eight (the fused SwiGLU runs in one split)."""
    reqs = []
    for rt in ((2, 4) if swiglu else (1, 2, 4)):
        for upw, depth in ((1, 8), (2, 4), (2, 8), (4, 2), (4, 4)):
            for nw in (1, 4, 22, 44):
                for ks in ((1,) if swiglu else (0, 1, 2, 3, 4, 6, 8)):
                    reqs.append(Tiling(rt, upw, nw, ks, depth))
    return reqs


def _w4b_wide_requests() -> list[Tiling]:
    """The int4 decode kernel's knobs for 16 < M <= 64 (32 or 64 staged x
    rows): rt * column blocks <= 8, one or two groups per stage, one or two
    stages in flight."""
    return [Tiling(rt, upw, nw, ks, depth)
            for rt in (1, 2, 4) for upw in (1, 2) for depth in (1, 2)
            for nw in (2, 4, 42, 44, 82, 84) for ks in (0, 1, 2, 3, 4, 6, 8, 12, 16)]


def _resolve(reqs, planner, M, N, K, wfmt, base) -> list[Tiling]:
    """The distinct full tilings the planner makes of `reqs`, the default first."""
    seen, out = set(), []
    for r in reqs:
        try:
            t, _ = planner(M, N, K, wfmt, r)
        except (AssertionError, ValueError, NotImplementedError):
            continue
        if t not in seen:
            seen.add(t)
            out.append(t)
    out.sort(key=lambda t: t != base)
    return out


def configure(classes=None, *, device="cuda:0", verbose=True, wfmt: int = WFMT_W8) -> dict:
    """Load-time tiling choice per class (before any graph capture).

    For each class: the planner's default and its neighbourhood
    (`candidates`), timed at M=8 on random weights rotated over 4 sets (to
    defeat the 256 MB MALL); the fastest becomes the decode (M <= 16) entry.
    Large-M buckets take the planner default for their representative M.
    """
    reset()
    classes = CLASSES if classes is None else dict(classes)
    _state["device"] = device
    _state["shapes"] = classes
    report = {"classes": {}}
    t0 = time.perf_counter()
    for cls, (n, k) in classes.items():
        t1 = time.perf_counter()
        if wfmt == WFMT_W8:
            sets = [(torch.randint(-127, 128, (n, k), dtype=torch.int8, device=device),
                     torch.rand(n, device=device).half() * 0.02, None) for _ in range(4)]
        elif wfmt == WFMT_W4:
            sets = [(torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=device),
                     torch.rand(n, k // 128, device=device).half() * 0.02, None)
                    for _ in range(4)]
        else:
            sets = [(torch.randn(n, k, device=device).bfloat16(), None, None) for _ in range(4)]
        x = torch.randn(8, k, device=device).bfloat16()
        best = None
        for c in candidates(8, n, k, wfmt):
            def run(c=c):
                for w, sc, z in sets:
                    _launch(x, w, sc, z, wfmt, n, c, None)
            try:
                us = _time_cfg(run) / len(sets)
            except (AssertionError, ValueError, NotImplementedError):
                continue
            if verbose:
                print(f"GEMM AUTOTUNE {cls} cfg={tuple(c)} us={us:.2f}", flush=True)
            if best is None or us < best[0]:
                best = (us, c)
        _state["configs"][cls] = best[1]
        _state["m_configs"][cls] = {
            b: plan(_M_REP_M[b], n, k, wfmt)[0] for b in M_BUCKETS_LARGE}
        report["classes"][cls] = {"config": best[1], "us": best[0],
                                  "autotune_s": time.perf_counter() - t1}
        del sets
    report["total_s"] = time.perf_counter() - t0
    _state["report"] = report
    if verbose:
        print(f"GEMM CONFIGURE total_s={report['total_s']:.2f} "
              f"cfgs={ {c: r['config'] for c, r in report['classes'].items()} }", flush=True)
    return report


def reset() -> None:
    """Clear all load-time state (test isolation)."""
    _state.clear()
    _state.update({"configs": {}, "m_configs": {}, "shapes": {}, "workspaces": {},
                   "device": None, "report": None})
