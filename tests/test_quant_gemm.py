"""Weight-only GEMM (HIP MFMA) vs the dequantised-matmul oracle.

Anchor as in the reference (tests/test_quant_gemm.py:93-96): y_ref = x.float()
@ dequant(W).T, dequant from oracle/quant_ref.py. Bar: norm-wise relative
error <= 1e-2 (north star) and, for W8, the reference's per-class elementwise
tolerances TOL_W8 (test_quant_gemm.py:56-62).

Shapes: BASELINE config 3 — qkv 4096->6144, o 4096->4096, gate_up
4096->24576, down 12288->4096, M in {1, 8, 64, 256}; int4 symmetric g128
(v ~U{-8..7}, fp16 scale ~U(0.005, 0.02)), the same shapes in int8
per-channel (randn -> quantize_w8, the reference's distribution) and dense
bf16; plus the reference's asymmetric int4 (quantize_w4) format.
"""
import numpy as np
import pytest
import torch

from oracle.quant_ref import (dequant_w4_ref, dequant_w4_sym_ref, dequant_w8_ref,
                              pack_w4_ref, quantize_w4_ref, quantize_w8_ref)
from tolerances import GEMM_REL, rel_err
from gpu_utils import graph_replays_match

SHAPES = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (24576, 4096), "down": (4096, 12288)}
MS = [1, 8, 64, 256]
TOL_W8 = {"qkv": dict(rtol=2e-2, atol=1.5), "o": dict(rtol=2e-2, atol=1.5),
          "gate_up": dict(rtol=2e-2, atol=1.5), "down": dict(rtol=2e-2, atol=2.0)}

_W: dict = {}


def _w4(cls):
    key = ("w4", cls)
    if key not in _W:
        n, k = SHAPES[cls]
        g = torch.Generator().manual_seed(101)
        v = torch.randint(-8, 8, (n, k), generator=g, dtype=torch.int16).numpy()
        s = (0.005 + 0.015 * torch.rand(n, k // 128, generator=g)).half().numpy()
        u = (v + 8).astype(np.uint8)
        wref = torch.from_numpy(dequant_w4_sym_ref(u, s))
        _W[key] = (torch.from_numpy(pack_w4_ref(u)).cuda(), torch.from_numpy(s).cuda(), wref.cuda())
    return _W[key]


def _w8(cls):
    key = ("w8", cls)
    if key not in _W:
        n, k = SHAPES[cls]
        g = torch.Generator().manual_seed(11)
        w = torch.randn(n, k, generator=g).bfloat16().float().numpy()
        q, s = quantize_w8_ref(w)
        wref = torch.from_numpy(dequant_w8_ref(q, s))
        _W[key] = (torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(), wref.cuda())
    return _W[key]


def _bf(cls):
    key = ("bf16", cls)
    if key not in _W:
        n, k = SHAPES[cls]
        g = torch.Generator().manual_seed(7)
        w = (0.02 * torch.randn(n, k, generator=g)).bfloat16()
        _W[key] = (w.cuda(), w.float().cuda())
    return _W[key]


def _x(m, k, seed):
    g = torch.Generator().manual_seed(23 + m + seed)
    return torch.randn(m, k, generator=g).bfloat16().cuda()


def _ref(x, wref):
    return x.float() @ wref.T  # fp32 anchor on the GPU (torch matmul)


@pytest.mark.gpu
@pytest.mark.parametrize("cls", list(SHAPES))
@pytest.mark.parametrize("m", MS)
def test_w4_sym_matches_dequant_matmul(cls, m):
    from acorninfer_amd.ops.quant_gemm import quant_gemm_w4
    p, s, wref = _w4(cls)
    x = _x(m, SHAPES[cls][1], 0)
    out = quant_gemm_w4(x, p, s, cfg=(0, 0, 1))
    assert out.dtype == torch.bfloat16 and out.shape == (m, SHAPES[cls][0])
    r = rel_err(out, _ref(x, wref))
    assert r <= GEMM_REL, f"rel err {r:.3g}"


@pytest.mark.gpu
@pytest.mark.parametrize("cls", list(SHAPES))
@pytest.mark.parametrize("m", MS)
def test_w8_matches_dequant_matmul(cls, m):
    from acorninfer_amd.ops.quant_gemm import quant_gemm
    q, s, wref = _w8(cls)
    x = _x(m, SHAPES[cls][1], 1)
    out = quant_gemm(x, q, s, cls, cfg=(0, 0, 1))
    ref = _ref(x, wref)
    assert rel_err(out, ref) <= GEMM_REL
    torch.testing.assert_close(out.float(), ref, **TOL_W8[cls])


@pytest.mark.gpu
@pytest.mark.parametrize("cls", list(SHAPES))
@pytest.mark.parametrize("m", [1, 8, 64])
def test_bf16_matches_matmul(cls, m):
    from acorninfer_amd.ops.quant_gemm import bf16_gemm
    w, wref = _bf(cls)
    x = _x(m, SHAPES[cls][1], 2)
    out = bf16_gemm(x, w, cfg=(0, 0, 1))
    assert rel_err(out, _ref(x, wref)) <= GEMM_REL


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 8, 16, 33])
def test_w4_asymmetric_reference_format(m):
    """The reference's own int4 format (quantize_w4: u in [0,15], fp16 scale
    and zero per group) through the same kernel with a zero pointer."""
    from acorninfer_amd.ops.quant_gemm import quant_gemm_w4
    g = torch.Generator().manual_seed(5)
    w = torch.randn(1024, 4096, generator=g).bfloat16().float().numpy()
    u, s, z = quantize_w4_ref(w)
    wref = torch.from_numpy(dequant_w4_ref(u, s, z)).cuda()
    x = _x(m, 4096, 3)
    out = quant_gemm_w4(x, torch.from_numpy(pack_w4_ref(u)).cuda(), torch.from_numpy(s).cuda(),
                        torch.from_numpy(z).cuda(), cfg=(0, 0, 1))
    assert rel_err(out, _ref(x, wref)) <= GEMM_REL


@pytest.mark.gpu
@pytest.mark.parametrize("ks", [2, 3])
def test_split_k_partials_and_reduce(ks):
    """ksplit > 1 writes fp32 partials; summing them in order equals the
    reduce kernel's output; ksplit=1 and ksplit>1 agree to fp32 rounding."""
    from acorninfer_amd._lib import WFMT_W4
    from acorninfer_amd.ops.quant_gemm import gemm_partials, quant_gemm_w4
    p, s, wref = _w4("down")
    x = _x(8, 12288, 4)
    part = torch.empty(ks, 8, 4096, device="cuda")
    gemm_partials(x, p, s, None, WFMT_W4, part, (1, 0, ks))
    full = part.sum(0)
    one = quant_gemm_w4(x, p, s, cfg=(0, 0, 1))
    via = quant_gemm_w4(x, p, s, cfg=(0, 0, ks))
    torch.testing.assert_close(full, _ref(x, wref), rtol=1e-2, atol=5e-2)
    acc = part[0].clone()
    for i in range(1, ks):
        acc += part[i]
    assert torch.equal(via, acc.bfloat16())
    assert rel_err(one, via) < 5e-3


@pytest.mark.gpu
def test_deterministic_and_graph_replay():
    from acorninfer_amd.ops.quant_gemm import quant_gemm_w4
    p, s, _ = _w4("down")
    x = _x(8, 12288, 5)
    a = quant_gemm_w4(x, p, s, cfg=(0, 0, 3))
    b = quant_gemm_w4(x, p, s, cfg=(0, 0, 3))
    assert torch.equal(a, b)
    out = torch.empty(8, 4096, dtype=torch.bfloat16, device="cuda")
    assert graph_replays_match(lambda: quant_gemm_w4(x, p, s, cfg=(0, 0, 3), out=out),
                               lambda: out)


@pytest.mark.gpu
def test_no_host_sync_on_launch():
    from acorninfer_amd.ops import quant_gemm as qg
    q, s, _ = _w8("o")
    x = _x(8, 4096, 6)
    qg.reset()
    qg._state["configs"]["qo"] = (0, 0, 2)
    qg.quant_gemm(x, q, s, "qo")  # allocates the split workspace before the check
    torch.cuda.synchronize()
    prev = torch.cuda.get_sync_debug_mode()
    try:
        torch.cuda.set_sync_debug_mode(2)
        out = qg.quant_gemm(x, q, s, "qo")
    finally:
        torch.cuda.set_sync_debug_mode(prev)
    assert torch.equal(out, qg.quant_gemm(x, q, s, "qo", cfg=(0, 0, 2)))
    qg.reset()


@pytest.mark.gpu
def test_large_m_routing_contract():
    """As the reference (test_quant_gemm.py:208-221): M > 16 without
    configure() raises RuntimeError naming configure; an explicit cfg works."""
    from acorninfer_amd.ops import quant_gemm as qg
    q, s, _ = _w8("o")
    x = _x(17, 4096, 7)
    qg.reset()
    with pytest.raises(RuntimeError, match="configure"):
        qg.quant_gemm(x, q, s, "qo")
    assert qg.quant_gemm(x, q, s, "qo", cfg=(32, 64, 128, 4, 3)).shape == (17, 4096)


def test_bucket_boundaries_and_classes():
    from acorninfer_amd.ops import quant_gemm as qg
    assert qg.bucket_for(16) == "d" and qg.bucket_for(17) == "s"
    assert qg.bucket_for(66) == "m" and qg.bucket_for(256) == "m"
    assert qg.bucket_for(257) == "l" and qg.bucket_for(1024) == "l"
    assert qg.CLASSES == {"qo": (4096, 4096), "kv": (1024, 4096), "gate_up": (12288, 4096),
                          "down": (4096, 12288), "lm_head": (151936, 4096)}
    assert qg._CLS_BY_SHAPE[(4096, 12288)] == "down"


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["bf16", "bf16b", "w8", "w8b", "w4", "w4b"])
@pytest.mark.parametrize("m", [1, 8, 16, 40, 256])
def test_every_candidate_tiling_matches(fmt, m):
    """Every tiling the load-time sweep may pick (streaming kernel: row tiles
    per wave, loads per lane, waves, K splits, tiles per workgroup; for
    M > 16 also the tiled kernel at every M tile and K split, including a
    partial last M tile at M = 40) gives the oracle's result on the o shape
    (K=4096) and the down shape (K=12288); tilings differ only in fp32
    summation order."""
    from acorninfer_amd._lib import WFMT_BF16, WFMT_BF16B, WFMT_W4, WFMT_W4B, WFMT_W8, WFMT_W8B
    from acorninfer_amd.ops.quant_gemm import _launch, candidates
    from acorninfer_amd.quant.quantize import to_bf16b, to_w4b, to_w8b
    for cls in ("o", "down"):
        n, k = SHAPES[cls]
        if fmt == "bf16":
            w, wref = _bf(cls)
            args, wf = (w, None, None), WFMT_BF16
        elif fmt == "bf16b":
            w, wref = _bf(cls)
            args, wf = (to_bf16b(w), None, None), WFMT_BF16B
        elif fmt == "w8":
            q, s, wref = _w8(cls)
            args, wf = (q, s, None), WFMT_W8
        elif fmt == "w8b":
            q, s, wref = _w8(cls)
            args, wf = (to_w8b(q), s, None), WFMT_W8B
        elif fmt == "w4":
            p, s, wref = _w4(cls)
            args, wf = (p, s, None), WFMT_W4
        else:
            p, s, wref = _w4(cls)
            args, wf = (*to_w4b(p, s), None), WFMT_W4B
        x = _x(m, k, 9)
        ref = _ref(x, wref)
        cands = candidates(m, n, k, wf)
        assert len(cands) >= 8
        outs = []
        for c in cands:
            out = _launch(x, *args, wf, n, c, None)
            r = rel_err(out, ref)
            assert r <= GEMM_REL, f"{cls} {tuple(c)}: rel err {r:.3g}"
            outs.append(out)
        print(f"\n[{fmt} M={m} {cls}: {len(cands)} tilings ok]")


@pytest.mark.gpu
@pytest.mark.parametrize("cls", list(SHAPES))
@pytest.mark.parametrize("m", MS)
def test_w8b_config3_matches_dequant_matmul(cls, m):
    """The decode model's int8 layout (W8B blocks, q + 128) at every
    configuration-3 shape and M with the planner's tiling (the int8 decode
    kernel for M <= 16, the tiled kernel above) against the dequantised
    matmul (norm-wise GEMM_REL and the reference's per-class elementwise
    TOL_W8), and equal to the natural-layout int8 GEMM up to fp32 summation
    order."""
    from acorninfer_amd._lib import WFMT_W8, WFMT_W8B
    from acorninfer_amd.ops.quant_gemm import _launch
    from acorninfer_amd.quant.quantize import from_w8b, to_w8b
    q, s, wref = _w8(cls)
    wb = to_w8b(q)
    assert torch.equal(from_w8b(wb), q)
    n, k = SHAPES[cls]
    x = _x(m, k, 10)
    out = _launch(x, wb, s, None, WFMT_W8B, n, None, None)
    ref = _ref(x, wref)
    r = rel_err(out, ref)
    rn = rel_err(out, _launch(x, q, s, None, WFMT_W8, n, None, None))
    print(f"\n[w8b {cls} M={m}: rel err {r:.3g}, vs natural layout {rn:.3g}]")
    assert r <= GEMM_REL and rn <= 1e-2
    torch.testing.assert_close(out.float(), ref, **TOL_W8[cls])


@pytest.mark.gpu
@pytest.mark.parametrize("cls", list(SHAPES))
@pytest.mark.parametrize("m", MS + [16])
def test_bf16b_config3_matches_matmul(cls, m):
    """The decode model's bf16 layout (BF16B blocks) at every configuration-3
    shape and M with the planner's tiling (the bf16 decode kernel for
    M <= 16, the tiled kernel above, the large-M kernel from 256 rows)
    against the fp32 matmul, and equal to the natural-layout bf16 GEMM up to
    fp32 summation order (bit for bit where both run the same kernel: the
    tiled and large-M kernels)."""
    from acorninfer_amd._lib import WFMT_BF16, WFMT_BF16B
    from acorninfer_amd.ops.quant_gemm import _launch, plan
    from acorninfer_amd.quant.quantize import from_bf16b, to_bf16b
    w, wref = _bf(cls)
    wb = to_bf16b(w)
    assert torch.equal(from_bf16b(wb), w)
    n, k = SHAPES[cls]
    x = _x(m, k, 12)
    out = _launch(x, wb, None, None, WFMT_BF16B, n, None, None)
    r = rel_err(out, _ref(x, wref))
    tb = plan(m, n, k, WFMT_BF16B)[0]
    nat = _launch(x, w, None, None, WFMT_BF16, n, tb if m > 16 else None, None)
    rn = rel_err(out, nat)
    print(f"\n[bf16b {cls} M={m} {tuple(tb)}: rel err {r:.3g}, vs natural layout {rn:.3g}]")
    assert r <= GEMM_REL and rn <= 1e-2
    if m > 16:
        assert torch.equal(out, nat)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [40, 200])
def test_bf16b_tiled_equals_natural_bitwise(m):
    """The tiled kernel does the same arithmetic on both bf16 layouts, only
    its addressing differs: BF16B and natural bf16 give the same bits at
    every tiled candidate."""
    from acorninfer_amd._lib import WFMT_BF16, WFMT_BF16B
    from acorninfer_amd.ops.quant_gemm import _launch, candidates
    from acorninfer_amd.quant.quantize import to_bf16b
    w, _ = _bf("qkv")
    wb = to_bf16b(w)
    n, k = SHAPES["qkv"]
    x = _x(m, k, 13)
    cands = [c for c in candidates(m, n, k, WFMT_BF16B) if c.rt == 0]
    assert len(cands) >= 4
    for c in cands:
        a = _launch(x, wb, None, None, WFMT_BF16B, n, c, None)
        b = _launch(x, w, None, None, WFMT_BF16, n, c, None)
        assert torch.equal(a, b), tuple(c)


@pytest.mark.gpu
@pytest.mark.parametrize("cls", list(SHAPES))
@pytest.mark.parametrize("m", MS)
def test_w4b_config3_matches_dequant_matmul(cls, m):
    """The decode model's int4 layout (W4B blocks) at every configuration-3
    shape and M, with the planner's tiling: the int4 decode kernel for
    M <= 16, the tiled kernel above."""
    from acorninfer_amd._lib import WFMT_W4B
    from acorninfer_amd.ops.quant_gemm import _launch
    from acorninfer_amd.quant.quantize import to_w4b
    p, s, wref = _w4(cls)
    wb, sb = to_w4b(p, s)
    n, k = SHAPES[cls]
    x = _x(m, k, 10)
    out = _launch(x, wb, sb, None, WFMT_W4B, n, None, None)
    r = rel_err(out, _ref(x, wref))
    assert r <= GEMM_REL, f"rel err {r:.3g}"


@pytest.mark.gpu
@pytest.mark.parametrize("m", [40, 256])
def test_w4b_tiled_equals_natural_bitwise(m):
    """The tiled kernel does the same arithmetic on both int4 layouts, only
    its addressing differs: W4B and natural W4 give the same bits at every
    tiled candidate."""
    from acorninfer_amd._lib import WFMT_W4, WFMT_W4B
    from acorninfer_amd.ops.quant_gemm import _launch, candidates
    from acorninfer_amd.quant.quantize import to_w4b
    p, s, _ = _w4("down")
    wb, sb = to_w4b(p, s)
    n, k = SHAPES["down"]
    x = _x(m, k, 11)
    cands = [c for c in candidates(m, n, k, WFMT_W4B) if c.rt == 0]
    assert len(cands) >= 4
    for c in cands:
        a = _launch(x, wb, sb, None, WFMT_W4B, n, c, None)
        b = _launch(x, p, s, None, WFMT_W4, n, c, None)
        assert torch.equal(a, b), tuple(c)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [17, 32, 40, 64])
def test_w4b_wide_decode_kernel_matches(m):
    """The int4 decode kernel above 16 rows (two or four 16-column blocks of
    x per wave; the rows past M of the last block clamped to row M-1 and
    never stored) at every tiling the load-time sweep offers it, on the o
    shape (K=4096) and the down shape (K=12288), against the dequantised
    matmul; each output row also equals the same kernel's result for that
    row alone up to fp32 summation order (the blocks do not mix rows)."""
    from acorninfer_amd._lib import WFMT_W4B
    from acorninfer_amd.ops.quant_gemm import _launch, candidates
    from acorninfer_amd.quant.quantize import to_w4b
    for cls in ("o", "down"):
        p, s, wref = _w4(cls)
        wb, sb = to_w4b(p, s)
        n, k = SHAPES[cls]
        x = _x(m, k, 12)
        ref = _ref(x, wref)
        cands = [c for c in candidates(m, n, k, WFMT_W4B) if c.rt > 0]
        assert len(cands) >= 8, len(cands)
        for c in cands:
            out = _launch(x, wb, sb, None, WFMT_W4B, n, c, None)
            r = rel_err(out, ref)
            assert r <= GEMM_REL, f"{cls} M={m} {tuple(c)}: rel err {r:.3g}"
        # the column blocks do not mix rows: the last row equals that row of a
        # 17-row launch ending with it (the same kernel and tiling, two blocks)
        tail = _launch(x[m - 17:], wb, sb, None, WFMT_W4B, n, c, None)
        assert rel_err(out[m - 1:], tail[16:]) <= 1e-5
        # and the direct kernel's one-row result (its -136 X is formed by an
        # MFMA) agrees to bf16 rounding of a few outputs
        last = _launch(x[m - 1:], wb, sb, None, WFMT_W4B, n, None, None)
        assert rel_err(out[m - 1:], last) <= 1e-3
        print(f"\n[w4b wide M={m} {cls}: {len(cands)} tilings ok]")


@pytest.mark.gpu
@pytest.mark.parametrize("m", [17, 64, 100, 256])
def test_w4b_mid_kernel_matches(m):
    """The int4 mid-M kernel (x through LDS a group at a time, 64 x rows per
    workgroup; M = 17 and 100 leave a partial last block, 256 spreads four M
    blocks over an XCD) at every tiling the sweep offers it, on the qkv shape
    (N = 6144, 24 row blocks of 256) and the down shape (K = 12288), against
    the dequantised matmul; one split and four give the same result up to fp32
    summation order (bf16 outputs within one ulp)."""
    from acorninfer_amd._lib import WFMT_W4B
    from acorninfer_amd.ops.quant_gemm import MID_RT, Tiling, _launch, candidates
    from acorninfer_amd.quant.quantize import to_w4b
    for cls in ("qkv", "down"):
        p, s, wref = _w4(cls)
        wb, sb = to_w4b(p, s)
        n, k = SHAPES[cls]
        x = _x(m, k, 13)
        ref = _ref(x, wref)
        cands = [c for c in candidates(m, n, k, WFMT_W4B) if c.rt == MID_RT]
        assert len(cands) >= 8, len(cands)
        for c in cands:
            out = _launch(x, wb, sb, None, WFMT_W4B, n, c, None)
            r = rel_err(out, ref)
            assert r <= GEMM_REL, f"{cls} M={m} {tuple(c)}: rel err {r:.3g}"
        one = _launch(x, wb, sb, None, WFMT_W4B, n, Tiling(MID_RT, 2, 4, 1, 2), None)
        four = _launch(x, wb, sb, None, WFMT_W4B, n, Tiling(MID_RT, 2, 4, 4, 2), None)
        assert rel_err(one, four) <= 1e-3      # bf16 outputs: a few one-ulp flips
        print(f"\n[w4b mid M={m} {cls}: {len(cands)} tilings ok]")


@pytest.mark.gpu
@pytest.mark.parametrize("m", [17, 64, 100, 256])
def test_w8b_mid_kernel_matches(m):
    """The int8 mid-M kernel (x through LDS 128 k at a time, 64 x rows per
    workgroup, the -128 X correction from per-step column sums) at every
    tiling the sweep offers it, on the qkv shape (N = 6144) and the down
    shape (K = 12288), against the dequantised matmul (norm-wise GEMM_REL and
    the reference's per-class elementwise TOL_W8); one split and four agree
    up to fp32 summation order."""
    from acorninfer_amd._lib import WFMT_W8B
    from acorninfer_amd.ops.quant_gemm import MID_RT, Tiling, _launch, candidates
    from acorninfer_amd.quant.quantize import to_w8b
    for cls in ("qkv", "down"):
        q, s, wref = _w8(cls)
        wb = to_w8b(q)
        n, k = SHAPES[cls]
        x = _x(m, k, 14)
        ref = _ref(x, wref)
        cands = [c for c in candidates(m, n, k, WFMT_W8B) if c.rt == MID_RT]
        assert len(cands) >= 8, len(cands)
        for c in cands:
            out = _launch(x, wb, s, None, WFMT_W8B, n, c, None)
            r = rel_err(out, ref)
            assert r <= GEMM_REL, f"{cls} M={m} {tuple(c)}: rel err {r:.3g}"
            torch.testing.assert_close(out.float(), ref, **TOL_W8[cls])
        one = _launch(x, wb, s, None, WFMT_W8B, n, Tiling(MID_RT, 2, 4, 1, 2), None)
        four = _launch(x, wb, s, None, WFMT_W8B, n, Tiling(MID_RT, 2, 4, 4, 2), None)
        assert rel_err(one, four) <= 1e-3      # bf16 outputs: a few one-ulp flips
        print(f"\n[w8b mid M={m} {cls}: {len(cands)} tilings ok]")


@pytest.mark.gpu
@pytest.mark.parametrize("cls", ["qkv", "down"])
def test_dequant_w4b_bitwise(cls):
    """acorn_dequant_w4b writes the oracle's fp32 dequantised weight ((u - 8)
    * s) rounded once to bf16, bit for bit, in row order, also for rows in
    the gate|up 16-row interleave (the blocks move with their rows)."""
    from acorninfer_amd._lib import check, lib, ptr, stream_ptr
    from acorninfer_amd.ops.quant_gemm import interleave16
    from acorninfer_amd.quant.quantize import to_w4b
    p, s, wref = _w4(cls)
    n, k = SHAPES[cls]
    want = wref.to(torch.bfloat16)
    for perm in (False, True):
        pp, ss, ww = (interleave16(p), interleave16(s), interleave16(want)) if perm else (p, s, want)
        wb, sb = to_w4b(pp, ss)
        out = torch.full((n, k), float("nan"), dtype=torch.bfloat16, device="cuda")
        check(lib().acorn_dequant_w4b(ptr(wb), ptr(sb), ptr(out), n, k, stream_ptr(out.device)),
              "dequant_w4b")
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ww.view(torch.int16)), f"{cls} il16={perm}"
    # shape contract: rows in 16s, K in 512s (checked on the host, nothing launched)
    for bad in ((n - 8, k), (n, k - 128)):
        assert lib().acorn_dequant_w4b(ptr(wb), ptr(sb), ptr(out), *bad, None) == -1


@pytest.mark.gpu
@pytest.mark.parametrize("m", [2048, 2100])
def test_w4b_dequant_route_equals_bf16_gemm(m):
    """The int4 GEMM at prefill sizes (DEQUANT_RT: dequantise into a workspace,
    then the large-M bf16 kernel) gives bit for bit what that kernel gives on
    the bf16-rounded weights, within GEMM_REL of the float64 anchor on the
    unrounded ones; 2100 rows leave a ragged last M tile."""
    from acorninfer_amd._lib import WFMT_W4B
    from acorninfer_amd.models.qwen3 import DEQUANT_RT, QLinear
    from acorninfer_amd.ops.quant_gemm import Tiling, bf16_gemm
    from acorninfer_amd.quant.quantize import to_w4b
    from oracle.quant_ref import gemm_ref
    for cls in ("qkv", "down"):
        p, s, wref = _w4(cls)
        n, k = SHAPES[cls]
        wb, sb = to_w4b(p, s)
        lin = QLinear(WFMT_W4B, wb, n, k, sb)
        t, _ = lin.plan(m, workspace=True)
        assert t.rt == DEQUANT_RT, t
        assert lin.plan(m)[0].rt != DEQUANT_RT          # no workspace: the int4 kernels
        assert lin.plan(m, Tiling(DEQUANT_RT))[0] == t
        x = _x(m, k, 31)
        wtmp = torch.empty(n * k, dtype=torch.bfloat16, device="cuda")
        out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        part = torch.empty(t.ksplit, m, n, dtype=torch.float32, device="cuda")
        st = torch.cuda.current_stream().cuda_stream
        with pytest.raises(ValueError):
            lin.launch(x, m, t, out=out, part=part, stream=st)
        lin.launch(x, m, t, out=out, part=part, wtmp=wtmp, stream=st)
        want = bf16_gemm(x, wref.to(torch.bfloat16).contiguous())
        torch.cuda.synchronize()
        assert torch.equal(out, want), cls
        ref = torch.from_numpy(gemm_ref(x.float().cpu().numpy(), wref.cpu().numpy()))
        r = rel_err(out.cpu(), ref)
        print(f"\n[w4b dequant route M={m} {cls}: rel err {r:.3g} vs float64]")
        assert r <= GEMM_REL


@pytest.mark.gpu
def test_w4b_split_partials_deterministic_and_graph_replay():
    """W4B partials at several split counts sum (in split order) to the same
    result within fp32 rounding, repeat bitwise, and replay bitwise in a
    hipGraph."""
    from acorninfer_amd._lib import WFMT_W4B
    from acorninfer_amd.ops.quant_gemm import Tiling, _launch, gemm_partials
    from acorninfer_amd.quant.quantize import to_w4b
    for cls, splits in (("o", (1, 2)), ("down", (2, 3, 4, 6, 12))):
        p, s, wref = _w4(cls)
        wb, sb = to_w4b(p, s)
        n, k = SHAPES[cls]
        x = _x(8, k, 12)
        ref = _ref(x, wref)
        for ks in splits:               # ks = 1: fp32 output through the partials buffer
            t = Tiling(2, 2, 4, ks, 2)
            part = torch.empty(ks, 8, n, device="cuda")
            gemm_partials(x, wb, sb, None, WFMT_W4B, part, t)
            acc = part[0].clone()
            for i in range(1, ks):
                acc += part[i]
            assert rel_err(acc, ref) <= GEMM_REL, (cls, ks)
            part2 = torch.empty_like(part)
            gemm_partials(x, wb, sb, None, WFMT_W4B, part2, t)
            assert torch.equal(part, part2)
    p, s, _ = _w4("down")
    wb, sb = to_w4b(p, s)
    x = _x(8, 12288, 12)
    out = torch.empty(8, 4096, dtype=torch.bfloat16, device="cuda")
    t = Tiling(2, 2, 4, 3, 2)
    assert graph_replays_match(lambda: _launch(x, wb, sb, None, WFMT_W4B, 4096, t, out),
                               lambda: out)


def _swiglu_ref(x, wg, wu):
    """models/qwen3.py:392-396 in bf16 torch semantics on fp32-dequantised
    weights: each projection rounded to bf16, silu rounded, product rounded."""
    g = (x.float() @ wg.T).bfloat16()
    u = (x.float() @ wu.T).bfloat16()
    return (torch.nn.functional.silu(g.float()).bfloat16().float() * u.float()).bfloat16()


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["bf16", "bf16n", "w8", "w8b", "w4"])
@pytest.mark.parametrize("m", [1, 8, 16])
def test_fused_swiglu_every_tiling(fmt, m):
    """gate|up with the SwiGLU epilogue (interleaved 16-row gate/up blocks) vs
    the oracle's separate projections + activation; every candidate tiling;
    and the unfused path (partials + silu_mul on the interleaved layout).
    bf16n and w8 are bf16 and int8 in the natural layouts (the streaming
    kernel), bf16, w8b and w4 the decode model's block layouts (the bf16 /
    int8 / int4 direct kernels)."""
    import ctypes
    from acorninfer_amd import _lib
    from acorninfer_amd._lib import WFMT_BF16, WFMT_W4, WFMT_W8, lib, ptr, stream_ptr
    from acorninfer_amd.models.qwen3 import QLinear
    from acorninfer_amd.ops.quant_gemm import candidates
    inter, k = 1024, 4096
    g = torch.Generator().manual_seed(31)
    w = (0.02 * torch.randn(2 * inter, k, generator=g)).bfloat16().cuda()
    wf = {"bf16": WFMT_BF16, "bf16n": WFMT_BF16, "w8": WFMT_W8, "w8b": WFMT_W8, "w4": WFMT_W4}[fmt]
    lin = QLinear.from_dense(w, wf).interleaved()
    if fmt in ("w8", "bf16n"):
        lin = lin.natural()
    deq = lin.dense()
    x = (torch.randn(m, k, generator=g)).bfloat16().cuda()
    ref = _swiglu_ref(x, deq[:inter], deq[inter:])
    st = stream_ptr()
    cands = candidates(m, 2 * inter, k, lin.fmt, swiglu=True)
    assert len(cands) >= 4
    for c in cands:
        act = torch.full((m, inter), float("nan"), dtype=torch.bfloat16, device="cuda")
        lin.launch_swiglu(x, m, c, act, st)
        r = rel_err(act, ref)
        assert r <= 1e-2, f"{tuple(c)}: rel err {r:.3g}"
    # unfused: partials in interleaved column order -> silu_mul(il16)
    t, _ = lin.plan(m)
    part = torch.empty(t.ksplit, m, 2 * inter, device="cuda")
    lin.launch(x, m, t, part=part, stream=st)
    act2 = torch.empty(m, inter, dtype=torch.bfloat16, device="cuda")
    _lib.check(lib().acorn_silu_mul(ptr(part), t.ksplit, None, ptr(act2), m, inter, 1,
                                    _lib.BF16, st), "silu_mul")
    assert rel_err(act2, ref) <= 1e-2
    print(f"\n[swiglu {fmt} M={m}: {len(cands)} tilings ok]")


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["bf16", "bf16n", "w4"])
@pytest.mark.parametrize("m", [1100, 2048])
def test_fused_swiglu_at_prefill_sizes(fmt, m):
    """gate|up + SwiGLU at prefill sizes (the large-M kernel's epilogue; int4
    dequantised onto it): bit for bit the one-split fp32 output of the same
    kernel through silu_mul, and within 1e-2 of the oracle's separate
    projections + activation; bf16 (blocks) bit for bit bf16n (natural rows).
    inter = 1088: the last 256-row weight tile is half full; 1100 rows leave a
    ragged last M tile."""
    from acorninfer_amd import _lib
    from acorninfer_amd._lib import WFMT_BF16, WFMT_W4, lib, ptr, stream_ptr
    from acorninfer_amd.models.qwen3 import DENSE_RT, DEQUANT_RT, QLinear
    from acorninfer_amd.ops.quant_gemm import Tiling
    inter, k = 1088, 1024
    g = torch.Generator().manual_seed(37)
    w = (0.02 * torch.randn(2 * inter, k, generator=g)).bfloat16().cuda()
    lin = QLinear.from_dense(w, {"bf16": WFMT_BF16, "bf16n": WFMT_BF16,
                                 "w4": WFMT_W4}[fmt]).interleaved()
    if fmt == "bf16n":
        lin = lin.natural()
    deq = lin.dense()
    x = torch.randn(m, k, generator=g).bfloat16().cuda()
    ref = _swiglu_ref(x, deq[:inter], deq[inter:])
    st = stream_ptr()
    t, _ = lin.swiglu_plan(m, workspace=True)
    assert t.rt == (DEQUANT_RT if fmt == "w4" else DENSE_RT) and t.ksplit == 1, t
    wtmp = torch.empty(2 * inter * k, dtype=torch.bfloat16, device="cuda")
    act = torch.full((m, inter), float("nan"), dtype=torch.bfloat16, device="cuda")
    lin.launch_swiglu(x, m, t, act, st, wtmp=wtmp)
    # the unfused route on the same kernel: one fp32 plane -> silu_mul(il16)
    tp = Tiling(t.rt, t.upw, t.nw, 1, t.tpw)
    part = torch.empty(1, m, 2 * inter, device="cuda")
    lin.launch(x, m, tp, part=part, wtmp=wtmp, stream=st)
    act2 = torch.empty(m, inter, dtype=torch.bfloat16, device="cuda")
    _lib.check(lib().acorn_silu_mul(ptr(part), 1, None, ptr(act2), m, inter, 1, _lib.BF16, st),
               "silu_mul")
    torch.cuda.synchronize()
    assert torch.equal(act, act2)
    if fmt == "bf16":
        nat = lin.natural()
        act3 = torch.full_like(act, float("nan"))
        nat.launch_swiglu(x, m, nat.swiglu_plan(m, workspace=True)[0], act3, st)
        torch.cuda.synchronize()
        assert torch.equal(act, act3)
    r = rel_err(act, ref)
    print(f"\n[swiglu {fmt} M={m} at prefill size: rel err {r:.3g}]")
    assert r <= 1e-2
