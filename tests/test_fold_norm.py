"""The RMSNorm folded into the decode GEMMs (acorn_quant_gemm_norm): the
producer form against the plain launch followed by K1's residual add, the
consumer form against the plain launch on rows normalised with K1's formula
(rmsnorm.py:39-82, oracle/ops_ref.fused_add_rmsnorm_ref for the formula), and
the decode step with the fold against the step with K1 launches.

- producer (o, down; one split): res_out must be bf16(res + bf16(y)) bit for bit,
  y the plain launch's own output on the same tiling (the same accumulation
  order), and ss_out the fp32 sums of squares of res_out per 16 columns;
- consumer (qkv, gate|up): given the producer's sums, every row is used as
  bf16((x * inv) * w); inv is restated here in the kernel's order of
  additions (each quarter of a row's sums in order, then pairwise), so the
  output must equal the plain launch on those normalised rows bit for bit;
  inv itself is within 1e-6 of K1's float64 value;
- the step: the bf16 and W4A16 models tuned with the fold against the same
  models with it switched off (K1 launches), greedy tokens equal where the
  top-2 margin clears the gate, logits within the bf16 tolerance.
"""
import ctypes

import numpy as np
import pytest
import torch

from acorninfer_amd import _lib
from tolerances import rel_err

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
    """1/rms per row from [M, nss] fp32 sums, added as the kernels do."""
    m, nss = ss.shape
    per = nss // 4
    out = np.empty(m, dtype=np.float32)
    for r in range(m):
        q = []
        for j in range(4):
            s = np.float32(0)
            for t in range(per):
                s = np.float32(s + ss[r, j * per + t])
            q.append(s)
        tot = np.float32(np.float32(q[0] + q[1]) + np.float32(q[2] + q[3]))
        out[r] = np.float32(1.0) / np.sqrt(np.float32(tot / np.float32(cols) + np.float32(eps)))
    return out


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
    st = _lib.stream_ptr()
    tilings = _direct_tilings(lin, m, one_split=True)
    assert len(tilings) >= 4
    for t in tilings:
        y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        lin.launch(x, m, t, out=y, part=torch.empty(1, m, n, device="cuda"), stream=st)
        res_out = torch.full_like(res, float("nan"))
        ss = torch.full((m, n // 16), float("nan"), device="cuda")
        lin.launch_resid(x, m, t, res=res, res_out=res_out, ss=ss, stream=st)
        torch.cuda.synchronize()
        want = (res.float() + y.float()).bfloat16()
        assert torch.equal(res_out.view(torch.int16), want.view(torch.int16)), tuple(t)
        sq = want.float().view(m, n // 16, 16).pow(2).sum(-1)
        torch.testing.assert_close(ss, sq, rtol=1e-6, atol=0)
    # in place (res_out = res), as the step runs it
    t = tilings[0]
    r2 = res.clone()
    lin.launch_resid(x, m, t, res=r2, res_out=r2, ss=ss, stream=st)
    y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    lin.launch(x, m, t, out=y, part=torch.empty(1, m, n, device="cuda"), stream=st)
    torch.cuda.synchronize()
    assert torch.equal(r2.view(torch.int16), (res.float() + y.float()).bfloat16().view(torch.int16))
    print(f"\n[fold producer {fmt} {cls} M={m}: {len(tilings)} tilings bitwise]")


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("m", [1, 5, 8, 16])
@pytest.mark.parametrize("cls", ["qkv", "gate_up"])
def test_consumer_normalises_on_load(fmt, m, cls):
    n, k = SHAPES[cls]
    lin = _lin(fmt, n, k, 5 + m)
    if cls == "gate_up":
        lin = lin.interleaved()
    g = torch.Generator().manual_seed(21 + m)
    x = torch.randn(m, k, generator=g).bfloat16()              # the residual rows
    nw = (1.0 + 0.1 * torch.randn(k, generator=g)).bfloat16()
    eps = 1e-6
    ss = x.float().view(m, k // 16, 16).pow(2).sum(-1)         # a producer's sums
    inv = _inv_kernel_order(ss.numpy(), k, eps)
    # K1's value of inv (float64) is within 1e-6
    ref = 1.0 / np.sqrt(x.double().pow(2).mean(-1).numpy() + eps)
    assert np.allclose(inv, ref, rtol=1e-6)
    xn = ((x.float() * torch.from_numpy(inv)[:, None]) * nw.float()).bfloat16().cuda()
    xd, nwd, ssd = x.cuda(), nw.cuda(), ss.cuda()
    st = _lib.stream_ptr()
    for swiglu in ((False, True) if cls == "gate_up" else (False,)):
        tilings = _direct_tilings(lin, m, swiglu=swiglu)
        assert len(tilings) >= 4
        for t in tilings:
            if swiglu:
                a = torch.empty(m, n // 2, dtype=torch.bfloat16, device="cuda")
                b = torch.empty_like(a)
                lin.launch_swiglu(xn, m, t, a, st)
                lin.launch_norm(xd, m, t, norm_w=nwd, ss=ssd, eps=eps, stream=st, act=b)
            else:
                a = torch.empty(t.ksplit, m, n, device="cuda")
                b = torch.full_like(a, float("nan"))
                lin.launch(xn, m, t, part=a, stream=st)
                lin.launch_norm(xd, m, t, norm_w=nwd, ss=ssd, eps=eps, stream=st, part=b)
            torch.cuda.synchronize()
            assert torch.equal(a, b), (tuple(t), swiglu)
        print(f"\n[fold consumer {fmt} {cls} M={m} swiglu={swiglu}: {len(tilings)} tilings bitwise]")


def test_fold_entry_rejects_bad_requests():
    """Exactly one of the two forms; the residual form needs one split and no
    SwiGLU; natural layouts are refused (the direct kernels read blocks)."""
    L = _lib.lib()
    arr = (ctypes.c_int * 6)()
    rc = L.acorn_quant_gemm_norm(None, None, None, None, None, 8, 4096, 4096, _lib.WFMT_BF16B,
                                 arr, 0, None, None, 1e-6, None, None, None, None)
    assert rc == _lib.ERR_VALUE                       # neither form
    rc = L.acorn_quant_gemm_norm(None, None, None, None, None, 8, 4096, 4096, _lib.WFMT_BF16,
                                 arr, 0, 1, 1, 1e-6, None, None, None, None)
    assert rc == _lib.ERR_DTYPE                       # natural rows
    rc = L.acorn_quant_gemm_norm(None, None, None, None, None, 8, 4096, 4096, _lib.WFMT_W8B,
                                 arr, 1, None, None, 1e-6, 1, 1, 1, None)
    assert rc == _lib.ERR_UNSUPPORTED                 # residual form with SwiGLU


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
