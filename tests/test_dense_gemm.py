"""Large-M bf16 GEMM (csrc/dense_gemm.hip, the bf16 projections at prefill
sizes: acorninfer/models/qwen3.py:21-47's F.linear; the planner's default
from 256 rows, DENSE_M_MIN).

Oracle: the float64 product of the same bf16 operands. fp32 output must
match it to fp32 accumulation drift (a dropped k step, a wrong row or column,
a transposed tile all fail by orders of magnitude); the bf16 output must be
exactly the fp32 output rounded once (the same sums, rounded in the
epilogue).
Shapes: ragged M and N (tile edges inside the launch), every (BM, depth)
variant, configuration 3's projections at M = 2048 against an fp32 matmul;
plus the planner's routing (CPU), determinism, graph replay and no writes
outside [M, N].
"""
import pytest
import torch

from gpu_utils import graph_replays_match

DENSE_RT = -2
SMALL = [(512, 256, 128), (513, 260, 256), (1000, 1028, 512), (1100, 4096, 1024),
         (777, 1536, 384)]
CONFIG3 = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (24576, 4096),
           "down": (4096, 12288)}


def _operands(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (0.02 * torch.randn(N, K, generator=g)).bfloat16()
    return x, w


def _planes(x, w, tiling):
    """fp32 split-K planes [ksplit, M, N] of the planned launch."""
    from acorninfer_amd._lib import WFMT_BF16
    from acorninfer_amd.ops.quant_gemm import gemm_partials, plan
    t, _ = plan(x.shape[0], w.shape[0], x.shape[1], WFMT_BF16, tiling)
    part = torch.full((t.ksplit, x.shape[0], w.shape[0]), float("nan"), device="cuda")
    gemm_partials(x, w, None, None, WFMT_BF16, part, t)
    return part


def _run(x, w, tiling, fp32):
    from acorninfer_amd.ops.quant_gemm import bf16_gemm
    if fp32:
        planes = _planes(x, w, tiling)
        total = planes[0].clone()
        for p in planes[1:]:              # in split order, as the consumers sum them
            total += p
        return total
    return bf16_gemm(x, w, cfg=tiling)


def test_planner_routes_prefill_sizes_to_the_dense_kernel():
    from acorninfer_amd._lib import WFMT_BF16, WFMT_W8
    from acorninfer_amd.ops.quant_gemm import Tiling, plan
    # from 256 rows: 256 x 256 tiles, both operands by direct-to-LDS loads,
    # split K while the tiles (16 x 2 here) leave CUs idle
    t, tiles = plan(512, 4096, 4096, WFMT_BF16)
    assert t == Tiling(DENSE_RT, 256, 128, 8, 4) and tiles == 16 * 2
    # ... but not into a second round of workgroups: 24 x 2 tiles take 4 splits,
    # 24 x 8 and 96 x 2 none
    assert plan(512, 6144, 4096, WFMT_BF16)[0] == Tiling(DENSE_RT, 256, 128, 4, 4)
    assert plan(2048, 6144, 4096, WFMT_BF16)[0] == Tiling(DENSE_RT, 256, 128, 1, 4)
    assert plan(512, 24576, 4096, WFMT_BF16)[0] == Tiling(DENSE_RT, 256, 128, 1, 4)
    assert plan(2048, 4096, 4096, WFMT_BF16)[0] == Tiling(DENSE_RT, 256, 128, 2, 4)
    assert plan(8192, 4096, 4096, WFMT_BF16)[0] == Tiling(DENSE_RT, 256, 128, 1, 4)
    assert plan(512, 4096, 4096, WFMT_BF16, Tiling(DENSE_RT, 128))[0] == \
        Tiling(DENSE_RT, 128, 64, 4, 4)                              # the 128-row form
    assert plan(8192, 4096, 4096, WFMT_BF16, Tiling(DENSE_RT, 256, 64))[0] == \
        Tiling(DENSE_RT, 256, 64, 1, 2)                              # register-staged form
    assert plan(255, 4096, 4096, WFMT_BF16)[0].rt != DENSE_RT       # tiled kernel below 256
    assert plan(256, 6144, 4096, WFMT_BF16)[0] == Tiling(DENSE_RT, 256, 128, 8, 4)
    assert plan(256, 4096, 12288, WFMT_BF16)[0] == Tiling(DENSE_RT, 256, 128, 16, 4)
    assert plan(4096, 4096, 192, WFMT_BF16)[0] == Tiling(DENSE_RT, 256, 128, 1, 4)  # 6 stages of 32
    assert plan(4096, 4096, 4096, WFMT_W8)[0].rt != DENSE_RT        # bf16 weights only
    assert plan(64, 4096, 4096, WFMT_BF16, Tiling(DENSE_RT, 64, 0, 1, 4))[0] == \
        Tiling(DENSE_RT, 64, 64, 1, 4)                               # on request at any M
    with pytest.raises(NotImplementedError):
        plan(4096, 4096, 4096, WFMT_BF16, Tiling(DENSE_RT, 32, 0, 0, 2))


@pytest.mark.gpu
@pytest.mark.parametrize("wn,bm,depth", [(64, 128, 2), (64, 128, 4), (64, 64, 2), (64, 64, 4),
                                         (128, 64, 2), (64, 256, 2), (128, 256, 4)])
def test_dense_gemm_matches_float64(wn, bm, depth):
    from acorninfer_amd.ops.quant_gemm import Tiling
    for i, (M, N, K) in enumerate(SMALL):
        # the direct-to-LDS form (256, 128) runs 32-k stages in pairs
        if ((K // 32) % 2 if (bm, wn) == (256, 128) else (K // 64) % depth):
            continue
        print(f"\n[dense GEMM M={M} N={N} K={K} wn={wn} bm={bm} depth={depth}]", flush=True)
        x, w = _operands(M, N, K, 100 + i)
        ref = x.double() @ w.double().T
        t = Tiling(DENSE_RT, bm, wn, 0, depth)
        got32 = _run(x.cuda(), w.cuda(), t, True).cpu()
        torch.testing.assert_close(got32.double(), ref, rtol=1e-5, atol=1e-5)
        # the bf16 output is the same fp32 sums rounded once (same tiles, same order)
        got16 = _run(x.cuda(), w.cuda(), t, False).cpu()
        assert torch.equal(got16, got32.to(torch.bfloat16))


@pytest.mark.gpu
@pytest.mark.parametrize("M", [2048, 256, 300])
@pytest.mark.parametrize("cls", list(CONFIG3))
def test_dense_gemm_config3_at_prefill_m(cls, M):
    """The default plan at M = 2048 (a 2048-token prompt) and at 256 / 300
    rows (the smallest that take the 256 x 256 form, up to 16 K splits, a
    ragged last tile) on configuration 3's shapes, fp32 partials against the
    fp32 matmul of the same operands."""
    from acorninfer_amd._lib import WFMT_BF16
    from acorninfer_amd.ops.quant_gemm import plan
    N, K = CONFIG3[cls]
    assert plan(M, N, K, WFMT_BF16)[0][:3] == (DENSE_RT, 256, 128)
    x, w = _operands(M, N, K, 7)
    xd, wd = x.cuda(), w.cuda()
    got = _run(xd, wd, None, True)
    ref = xd.float() @ wd.float().T
    rel = ((got - ref).norm() / ref.norm()).item()
    print(f"\n[dense GEMM {cls} M={M}: rel err vs fp32 matmul {rel:.3g}]", flush=True)
    assert rel < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("bm,wn,depth", [(128, 0, 2), (256, 0, 2), (256, 128, 4)])
def test_dense_gemm_deterministic_graph_and_bounds(bm, wn, depth):
    from acorninfer_amd._lib import WFMT_BF16
    from acorninfer_amd.ops.quant_gemm import Tiling, gemm_partials
    M, N, K = 600, 516, 256
    x, w = _operands(M, N, K, 3)
    xd, wd = x.cuda(), w.cuda()
    t = Tiling(DENSE_RT, bm, wn, 1, depth)
    big = torch.full((M + 7, N), 9.0, device="cuda")       # 7 guard rows after the output
    part = big[:M].view(1, M, N)
    gemm_partials(xd, wd, None, None, WFMT_BF16, part, t)
    first = big.clone()
    gemm_partials(xd, wd, None, None, WFMT_BF16, part, t)
    assert torch.equal(big, first)
    assert bool((big[M:] == 9.0).all())

    def fn():
        gemm_partials(xd, wd, None, None, WFMT_BF16, part, t)

    assert graph_replays_match(fn, lambda: part)


@pytest.mark.gpu
@pytest.mark.parametrize("ks", [2, 4])
def test_dense_gemm_split_planes_are_k_range_products(ks):
    """Split s writes the product over its own K range: each plane against the
    float64 product of the matching column slices of x and w."""
    from acorninfer_amd.ops.quant_gemm import Tiling
    M, N, K = 300, 520, 1024
    x, w = _operands(M, N, K, 17)
    planes = _planes(x.cuda(), w.cuda(), Tiling(DENSE_RT, 64, 64, ks, 2)).cpu()
    assert planes.shape[0] == ks
    kr = K // ks
    for s in range(ks):
        ref = x[:, s * kr:(s + 1) * kr].double() @ w[:, s * kr:(s + 1) * kr].double().T
        torch.testing.assert_close(planes[s].double(), ref, rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(513, 272, 256), (1000, 1040, 512), (777, 1536, 384),
                                   (300, 4096, 1024)])
@pytest.mark.parametrize("tiling", [(DENSE_RT, 256, 128, 1, 4), (DENSE_RT, 256, 128, 2, 4),
                                    (DENSE_RT, 128, 64, 1, 2), (DENSE_RT, 128, 64, 2, 4),
                                    (DENSE_RT, 64, 64, 1, 4), (DENSE_RT, 64, 128, 1, 2)])
def test_dense_gemm_blocked_weights_bitwise(M, N, K, tiling):
    """The decode model's bf16 weights in 1 KB blocks (BF16B) on every form of
    the large-M kernel that reads them (direct-to-LDS 256 x 256; the
    register-direct 64 / 128 forms): the same operands in the same order as
    the natural rows, so the fp32 planes are bit for bit those of the natural
    layout. Ragged N (272, 1040: a last 256-row tile cut inside) and M, K
    splits, 6 and 12 k-pairs."""
    from acorninfer_amd._lib import WFMT_BF16, WFMT_BF16B
    from acorninfer_amd.ops.quant_gemm import Tiling, gemm_partials, plan
    from acorninfer_amd.quant.quantize import to_bf16b
    x, w = _operands(M, N, K, 29)
    xd, wd = x.cuda(), w.cuda()
    wb = to_bf16b(wd)
    t = Tiling(*tiling)
    try:
        tb, _ = plan(M, N, K, WFMT_BF16B, t)
    except NotImplementedError:
        pytest.skip(f"{tiling} not built for K={K}")
    assert tb == plan(M, N, K, WFMT_BF16, t)[0]
    outs = []
    for wf, ww in ((WFMT_BF16B, wb), (WFMT_BF16, wd)):
        part = torch.full((tb.ksplit, M, N), float("nan"), device="cuda")
        gemm_partials(xd, ww, None, None, wf, part, tb)
        outs.append(part)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]), tiling
    ref = xd.float() @ wd.float().T
    rel = ((outs[0].sum(0) - ref).norm() / ref.norm()).item()
    assert rel < 1e-5


def test_planner_refuses_blocked_weights_on_the_staged_form():
    """BF16B is read by the direct-to-LDS and register-direct forms only."""
    from acorninfer_amd._lib import WFMT_BF16B
    from acorninfer_amd.ops.quant_gemm import Tiling, plan
    with pytest.raises(NotImplementedError):
        plan(4096, 4096, 4096, WFMT_BF16B, Tiling(DENSE_RT, 256, 64, 1, 2))
    assert plan(4096, 4096, 4096, WFMT_BF16B)[0] == Tiling(DENSE_RT, 256, 128, 1, 4)
