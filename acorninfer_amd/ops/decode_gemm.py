"""bf16 decode GEMM boundary (y = x @ w^T, bf16 in/out, fp32 accumulate).

Drop-in for acorninfer/ops/decode_gemm.py: `triton_gemm` (:236-257) forces the
kernel path, `linear_dispatch` (:260-277) consults the load-time dispatch
table, `configure` (:428-475) builds that table, `set_active_classes`
(:478-483) and `reset` (:486-493) manage it, `M_BUCKETS` (:64) are the decode
row buckets. The names are the reference's; the kernel behind them is this
build's MFMA GEMM (csrc/quant_gemm.hip, bf16 weight format), not Triton.

Table semantics follow the reference:

- layout "none" (the default) passes every call to `F.linear` unchanged, so a
  caller that never configures sees the framework's own linear;
- `configure("triton" | "hip", classes)` tunes the kernel's tiling per class
  at M = 8, times it against `F.linear` (torch's library GEMM) for each bucket
  on rotated weight sets (4 sets, beyond the 256 MB MALL), records per bucket
  which is faster ("triton" = this kernel, "cublas" = the library, the
  reference's labels), and adopts a class when the kernel beats the library
  by `valve` in some bucket;
- `linear_dispatch` runs the kernel for adopted classes whose bucket chose it,
  `F.linear` otherwise (and for M above the largest bucket).

The kernel path makes no host synchronisation and keeps its split-K
workspace address-stable (quant_gemm._workspace), so it can be captured.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from acorninfer_amd.ops import quant_gemm as _qg

M_BUCKETS = (1, 2, 4, 8)
_ROT_SETS = 4

_state: dict = {}


def reset() -> None:
    """Clear the dispatch table, tuned tilings and report (test isolation)."""
    _state.clear()
    _state.update({"layout": "none", "active": set(), "table": {}, "configs": {},
                   "shapes": {}, "adopted": set(), "device": None, "report": None})


reset()


def _bucket_for(m: int):
    for b in M_BUCKETS:
        if m <= b:
            return b
    return None


def _kernel(x2: torch.Tensor, w: torch.Tensor, cfg, out: torch.Tensor | None) -> torch.Tensor:
    return _qg._launch(x2, w, None, None, _qg.WFMT_BF16, w.shape[0], cfg, out)


def triton_gemm(x: torch.Tensor, w: torch.Tensor, cls, cfg=None,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Force the kernel path (the reference's name; unit tests and load-time
    timing use it). x [..., K] bf16, w [N, K] bf16 -> [M, N] bf16 (x
    flattened to M rows). cfg: a quant_gemm.Tiling, (rt, nw, ksplit), or the
    reference's (BLOCK_N, BLOCK_K, warps, stages, SPLIT_K), of which SPLIT_K
    carries over; None = the tiling configure() chose for `cls` (or the
    planner's default). out: None or a [M, N] bf16 buffer (graph capture)."""
    _qg.require_gpu(x, w)
    x2 = _qg._prep_x(x)
    assert w.dtype == torch.bfloat16 and w.is_contiguous() and w.shape[1] == x2.shape[1], \
        "w must be contiguous bf16 [N, K] matching x"
    c = cfg if cfg is not None else _state["configs"].get(cls)
    return _kernel(x2, w, _qg._native_cfg(c, x2.shape[0]), out)


def linear_dispatch(x: torch.Tensor, w: torch.Tensor, cls) -> torch.Tensor:
    """Call-site form: the table decides between the kernel and F.linear."""
    if _state["layout"] not in ("triton", "hip") or cls not in _state["active"]:
        return F.linear(x, w)
    K = w.shape[1]
    M = x.numel() // K
    b = _bucket_for(M)
    if b is None or _state["table"].get((cls, b)) != "triton":
        return F.linear(x, w)
    out = _kernel(_qg._prep_x(x), w, _state["configs"].get(cls), None)
    return out if x.dim() == 2 else out.view(*x.shape[:-1], w.shape[0])


def _time_us(fn, reps: int = 10) -> float:
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


def configure(layout, classes, *, device="cuda:0", dtype=torch.bfloat16,
              buckets=M_BUCKETS, valve=0.05, verbose=True) -> dict:
    """Load-time entry (before any graph capture). classes: {name: (N, K)}.
    Returns the report {"layout", "valve", "classes": {name: {"config",
    "adopted", "rows": {m: {...}}}}} with the reference's row fields:
    triton_us (this kernel), tn_us / best_cublas_us (F.linear), win_vs_best_pct,
    adopted_m, table."""
    reset()
    _state["layout"] = layout
    if layout not in ("triton", "hip"):
        return {"layout": "none"}
    assert dtype == torch.bfloat16, "the kernel computes bf16 x bf16 -> bf16"
    _state["device"] = device
    _state["shapes"] = dict(classes)
    report = {"layout": layout, "valve": valve, "classes": {}}
    for cls, (N, K) in classes.items():
        ws = [torch.randn(N, K, device=device).bfloat16() for _ in range(_ROT_SETS)]
        x8 = torch.randn(8, K, device=device).bfloat16()
        best = None
        for c in _qg.candidates(8, N, K, _qg.WFMT_BF16):
            us = _time_us(lambda c=c: [_kernel(x8, w, c, None) for w in ws]) / _ROT_SETS
            if best is None or us < best[0]:
                best = (us, c)
        cfg = best[1]
        _state["configs"][cls] = cfg
        rows, adopted = {}, False
        for m in buckets:
            x = torch.randn(m, K, device=device).bfloat16()
            k_us = _time_us(lambda: [_kernel(x, w, cfg, None) for w in ws]) / _ROT_SETS
            t_us = _time_us(lambda: [F.linear(x, w) for w in ws]) / _ROT_SETS
            adopted_m = k_us <= t_us * (1 - valve)
            adopted = adopted or adopted_m
            pick = "triton" if k_us < t_us else "cublas"
            _state["table"][(cls, m)] = pick
            rows[m] = {"triton_us": k_us, "tn_us": t_us, "best_cublas_us": t_us,
                       "win_vs_best_pct": (t_us / k_us - 1) * 100, "adopted_m": adopted_m,
                       "table": pick}
        if adopted:
            _state["active"].add(cls)
            _state["adopted"].add(cls)
        report["classes"][cls] = {"config": tuple(cfg), "adopted": adopted, "rows": rows}
        if verbose:
            print(f"DECODE GEMM {cls} cfg={tuple(cfg)} adopted={adopted} "
                  f"rows={ {m: (round(r['triton_us'], 1), round(r['tn_us'], 1)) for m, r in rows.items()} }",
                  flush=True)
        del ws
    _state["report"] = report
    return report


def set_active_classes(classes) -> None:
    """Narrow the active set to `classes` among the adopted ones (A/B)."""
    _state["active"] = set(classes) & _state["adopted"] if classes else set()
