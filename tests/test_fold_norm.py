"""The RMSNorm folded into the decode GEMMs (acorn_quant_gemm_norm), from
RMSNorm(v) @ W^T = inv * (bf16(v * w) @ W^T) per row: the producer form
against the plain launch followed by K1's residual add, the consumer form
against the plain launch on the weighted rows, and the decode step with the
fold against the step with K1 launches (rmsnorm.py:39-82, and
oracle/ops_ref.fused_add_rmsnorm_ref for the formula).

- producer (o, down; one split): res_out must be v = bf16(res + bf16(y)) bit
  for bit, y the plain launch's own output on the same tiling (the same
  accumulation order), xw = bf16(v * w_next) bit for bit, and ss_out the fp32
  sums of squares of v per 16 columns;
- consumer (qkv, gate|up): given xw and the producer's sums, every result of
  row m is the plain launch's on xw times inv, inv restated here in the
  kernel's order of additions (each quarter of a row's sums in order, then
  pairwise): bitwise for the fp32 partials, within one bf16 ulp per rounding
  for the fused SwiGLU (its silu goes through the device expf); inv itself is
  within 1e-6 of K1's float64 value, and the result is within bf16 rounding
  of the plain launch on K1's normalised rows bf16((v * inv) * w);
- the step: the bf16 and W4A16 models tuned with the fold against the same
  models with it switched off (K1 launches), greedy tokens equal where the
  top-2 margin clears the gate, logits within the bf16 tolerance.
"""
import ctypes

import numpy as np
import pytest
import torch

from acorninfer_amd import _lib
from tolerances import rel_err, ulp_distance

SHAPES = {"o": (4096, 4096), "down": (4096, 12288), "qkv": (6144, 4096),
          "gate_up": (24576, 4096)}
FMTS = {"bf16": _lib.WFMT_BF16, "w8": _lib.WFMT_W8, "w4": _lib.WFMT_W4}


def _lin(fmt, n, k, seed):
    from acorninfer_amd.models.qwen3 import QLinear
    g = torch.Generator().manual_seed(seed)
    w = (0.02 * torch.randn(n, k, generator=g)).bfloat16().cuda()
    return QLinear.from_dense(w, FMTS[fmt])


def _direct_tilings(lin, m, swiglu=False, one_split=False):
    from acorninfer_amd.ops.quant_gemm import candidates
    cs = [c for c in candidates(m, lin.N, lin.K, lin.fmt, swiglu=swiglu) if c.rt > 0]
    if one_split:
        cs = [c for c in cs if c.ksplit == 1]
    return cs


def _inv_kernel_order(ss: np.ndarray, cols: int, eps: float) -> np.ndarray:
    """1/rms per row from [M, nss] fp32 sums, added as the kernels do: mp =
    the power of two >= M, 64 / mp parts of ceil(nss mp / 64) sums each added
    in order, then the parts by an xor butterfly (neighbours first)."""
    m, nss = ss.shape
    mp = 1 << max(m - 1, 0).bit_length()
    parts = 64 // mp
    per = -(-nss // parts)
    out = np.empty(m, dtype=np.float32)
    for r in range(m):
        q = []
        for j in range(parts):
            s = np.float32(0)
            for t in range(j * per, min((j + 1) * per, nss)):
                s = np.float32(s + ss[r, t])
            q.append(s)
        while len(q) > 1:
            q = [np.float32(q[i] + q[i + 1]) for i in range(0, len(q), 2)]
        out[r] = np.float32(1.0) / np.sqrt(np.float32(q[0] / np.float32(cols) + np.float32(eps)))
    return out


def test_inv_order_restatement():
    """The restated order on a known case: M = 16 is four parts per row added
    as (q0 + q1) + (q2 + q3); M = 1 is 64 parts of one vector each; sums that
    need every bit of the order (a large value cancelled later) pin it."""
    nss = 256
    ss = np.full((1, nss), 1.0, dtype=np.float32)
    got = _inv_kernel_order(ss, 16 * nss, 0.0)
    assert np.isclose(got[0], 1.0 / np.sqrt(nss / (16 * nss)))
    # 2^24 + 1 is not an fp32: a part that adds 1.0 to 2^24 loses it, a part
    # that adds the ones first keeps them
    ss = np.zeros((16, nss), dtype=np.float32)
    ss[:, 0] = 2.0 ** 24
    ss[:, 1:64] = 1.0
    tot16 = _inv_kernel_order(ss, 1, 0.0)        # part 0 holds 2^24 and the 63 ones
    assert np.isclose(1.0 / tot16[0] ** 2, 2.0 ** 24, rtol=0, atol=0)
    ss1 = ss[:1].copy()
    tot1 = _inv_kernel_order(ss1, 1, 0.0)        # parts of 4: 2^24 + 3 ones, the rest exact
    assert 1.0 / tot1[0] ** 2 > 2.0 ** 24


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("m", [1, 5, 8, 16])
@pytest.mark.parametrize("cls", ["o", "down"])
def test_producer_residual_and_sums(fmt, m, cls):
    n, k = SHAPES[cls]
    lin = _lin(fmt, n, k, 3 + m)
    g = torch.Generator().manual_seed(11 + m)
    x = torch.randn(m, k, generator=g).bfloat16().cuda()
    res = torch.randn(m, n, generator=g).bfloat16().cuda()
    nw = (1.0 + 0.1 * torch.randn(n, generator=g)).bfloat16().cuda()
    st = _lib.stream_ptr()
    tilings = _direct_tilings(lin, m, one_split=True)
    assert len(tilings) >= 4
    for t in tilings:
        y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        lin.launch(x, m, t, out=y, part=torch.empty(1, m, n, device="cuda"), stream=st)
        res_out = torch.full_like(res, float("nan"))
        xw = torch.full_like(res, float("nan"))
        ss = torch.full((m, n // 16), float("nan"), device="cuda")
        lin.launch_resid(x, m, t, res=res, res_out=res_out, ss=ss, norm_w=nw, xw=xw, stream=st)
        torch.cuda.synchronize()
        want = (res.float() + y.float()).bfloat16()
        assert torch.equal(res_out.view(torch.int16), want.view(torch.int16)), tuple(t)
        want_xw = (want.float() * nw.float()).bfloat16()
        assert torch.equal(xw.view(torch.int16), want_xw.view(torch.int16)), tuple(t)
        sq = want.float().view(m, n // 16, 16).pow(2).sum(-1)
        torch.testing.assert_close(ss, sq, rtol=1e-6, atol=0)
    # in place (res_out = res), as the step runs it
    t = tilings[0]
    r2 = res.clone()
    lin.launch_resid(x, m, t, res=r2, res_out=r2, ss=ss, norm_w=nw, xw=xw, stream=st)
    y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    lin.launch(x, m, t, out=y, part=torch.empty(1, m, n, device="cuda"), stream=st)
    torch.cuda.synchronize()
    assert torch.equal(r2.view(torch.int16), (res.float() + y.float()).bfloat16().view(torch.int16))
    print(f"\n[fold producer {fmt} {cls} M={m}: {len(tilings)} tilings bitwise]")


def _swiglu_ref(part: torch.Tensor, inv: torch.Tensor) -> torch.Tensor:
    """The fused SwiGLU epilogue on one-split results [M, N] of interleaved
    gate|up rows (16-row blocks: gate, up, gate, ...), each row scaled by inv
    first: bf16(bf16(silu(bf16 g)) * bf16 u), the kernels' roundings."""
    m, n = part.shape
    v = (part * inv[:, None]).view(m, n // 32, 2, 16)
    gb = v[:, :, 0].bfloat16().float()
    ub = v[:, :, 1].bfloat16().float()
    sg = (gb / (1.0 + torch.exp(-gb))).bfloat16().float()
    return (sg * ub).bfloat16().reshape(m, n // 2)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("m", [1, 5, 8, 16])
@pytest.mark.parametrize("cls", ["qkv", "gate_up"])
def test_consumer_scales_rows_by_inv(fmt, m, cls):
    n, k = SHAPES[cls]
    lin = _lin(fmt, n, k, 5 + m)
    if cls == "gate_up":
        lin = lin.interleaved()
    g = torch.Generator().manual_seed(21 + m)
    v = torch.randn(m, k, generator=g).bfloat16()              # the residual rows
    nw = (1.0 + 0.1 * torch.randn(k, generator=g)).bfloat16()
    eps = 1e-6
    ss = v.float().view(m, k // 16, 16).pow(2).sum(-1)         # a producer's sums
    xw = (v.float() * nw.float()).bfloat16()                   # ... and weighted rows
    inv = _inv_kernel_order(ss.numpy(), k, eps)
    # K1's value of inv (float64) is within 1e-6
    ref = 1.0 / np.sqrt(v.double().pow(2).mean(-1).numpy() + eps)
    assert np.allclose(inv, ref, rtol=1e-6)
    invd = torch.from_numpy(inv).cuda()
    xn = ((v.float() * torch.from_numpy(inv)[:, None]) * nw.float()).bfloat16().cuda()
    xwd, ssd = xw.cuda(), ss.cuda()
    st = _lib.stream_ptr()
    for swiglu in ((False, True) if cls == "gate_up" else (False,)):
        tilings = _direct_tilings(lin, m, swiglu=swiglu)
        assert len(tilings) >= 4
        for t in tilings:
            if swiglu:
                p1 = torch.empty(1, m, n, device="cuda")
                lin.launch(xwd, m, t, part=p1, stream=st)
                b = torch.empty(m, n // 2, dtype=torch.bfloat16, device="cuda")
                lin.launch_norm(xwd, m, t, ss=ssd, eps=eps, stream=st, act=b)
                torch.cuda.synchronize()
                want = _swiglu_ref(p1[0], invd)
                d = ulp_distance(b, want)
                assert int(d.max()) <= 2 and float((d > 0).float().mean()) < 0.01, tuple(t)
                k1 = torch.empty_like(b)
                lin.launch_swiglu(xn, m, t, k1, st)
            else:
                a = torch.empty(t.ksplit, m, n, device="cuda")
                b = torch.full_like(a, float("nan"))
                lin.launch(xwd, m, t, part=a, stream=st)
                lin.launch_norm(xwd, m, t, ss=ssd, eps=eps, stream=st, part=b)
                torch.cuda.synchronize()
                assert torch.equal(b, a * invd[None, :, None]), (tuple(t), swiglu)
                k1 = torch.empty_like(a)
                lin.launch(xn, m, t, part=k1, stream=st)
            torch.cuda.synchronize()
            # the K1 pair (norm, then the plain launch) within bf16 rounding
            r = rel_err(b.float().sum(0) if b.dim() == 3 else b.float(),
                        k1.float().sum(0) if k1.dim() == 3 else k1.float())
            assert r < 1e-2, (tuple(t), swiglu, r)
        print(f"\n[fold consumer {fmt} {cls} M={m} swiglu={swiglu}: {len(tilings)} tilings]")


def test_fold_entry_rejects_bad_requests():
    """Exactly one of the two forms; the residual form needs its four outputs,
    one split and no SwiGLU; natural layouts are refused (the direct kernels
    read blocks)."""
    L = _lib.lib()
    arr = (ctypes.c_int * 6)()
    args = dict(x=None, w=None, scale=None, out=None, part=None, M=8, N=4096, K=4096,
                wfmt=_lib.WFMT_BF16B, cfg=arr, swiglu=0, ss_in=None, eps=1e-6, res=None,
                res_out=None, ss_out=None, norm_w=None, xw=None, stream=None)

    def call(**kw):
        return L.acorn_quant_gemm_norm(*{**args, **kw}.values())
    assert call() == _lib.ERR_VALUE                                    # neither form
    assert call(ss_in=1, res=1, res_out=1, ss_out=1, norm_w=1, xw=1) == _lib.ERR_VALUE  # both
    assert call(wfmt=_lib.WFMT_BF16, ss_in=1) == _lib.ERR_DTYPE        # natural rows
    assert call(wfmt=_lib.WFMT_W8B, swiglu=1, res=1, res_out=1, ss_out=1, norm_w=1,
                xw=1) == _lib.ERR_UNSUPPORTED                          # residual with SwiGLU
    assert call(res=1, res_out=1, ss_out=1, norm_w=1) == _lib.ERR_VALUE   # no xw
    assert call(res=1, res_out=1, ss_out=1, xw=1) == _lib.ERR_VALUE       # no norm weight
    assert call(M=8, N=4008, ss_in=1) == _lib.ERR_SHAPE


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["bf16", "w4a16"])
def test_step_with_folded_norms_matches_k1_step(fmt):
    """The 2-layer Qwen3-8B shape tuned at bucket 8 for the fold (one-split
    o and down, the folded forms timed): the same prompts prefilled, then the same forced
    tokens decoded through the step with the fold and with K1 launches. The
    residual stream's bits can differ only through inv (the sum of squares in
    another order), so the logits agree to bf16 rounding and the greedy
    tokens wherever the margin is clear."""
    from acorninfer_amd.cache.pager import PagedCacheView
    from acorninfer_amd.config import Qwen3Config
    from acorninfer_amd.models.qwen3 import Qwen3DecodeModel, random_state_dict
    from model_utils import new_cache
    cfg = Qwen3Config.qwen3_8b().with_layers(2)
    sd = random_state_dict(cfg, seed=77, std=0.02, dtype=torch.bfloat16)
    model = Qwen3DecodeModel.from_state_dict(cfg, sd, weight_format=fmt, device="cuda")
    model.tune(8, fold=True)
    assert model.fold_possible(8)
    B, L, steps = 8, 40, 4
    g = torch.Generator().manual_seed(5)
    prompts = torch.randint(0, cfg.vocab_size, (B, L), generator=g)
    forced = torch.randint(0, cfg.vocab_size, (steps, B), generator=g)
    runs = {}
    for fold in (True, False):
        model.fold_norm = fold
        assert model.buffers(B, 8).fold == fold
        _, cache = new_cache(model, B * 8)
        views = [PagedCacheView(cache) for _ in range(B)]
        model.forward_prefill_batch(prompts.cuda(), views, real_lens=[L] * B)
        out = [model.forward_decode(forced[t].view(B, 1).cuda(), views) for t in range(steps)]
        runs[fold] = torch.stack(out)
    model.fold_norm = True
    a, b = runs[True], runs[False]
    r = rel_err(a, b)
    assert r < 2e-2, r
    top2 = b.double().topk(2, -1).values
    clear = (top2[..., 0] - top2[..., 1]) > 0.1
    assert bool(((a.argmax(-1) == b.argmax(-1)) | ~clear).all())
    print(f"\n[{fmt} step: fold vs K1 rel err {r:.2e}, "
          f"{int(clear.sum())}/{clear.numel()} clear-margin tokens equal]")
