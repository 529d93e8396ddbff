"""The bf16 decode layout (ACORN_WFMT_BF16B) on the CPU: the conversion from
the reference's bf16 [N, K] rows moves each 8-value piece (row n, k in
[8c, 8c+8)) to the place the C-ABI's index map says (include/acorn_hip.h),
it round-trips, it commutes with the 16-row gate|up interleave, and the
planner's BF16B tilings satisfy the kernels' constraints: the direct decode
kernel at M <= 16, the tiled kernel above, and the large-M kernel's forms
that read blocks (never the register-staged 256 x 256 one). No GPU: the
planner is host code."""
import ctypes

import pytest
import torch

from acorninfer_amd import _lib
from acorninfer_amd.ops.quant_gemm import interleave16
from acorninfer_amd.quant.quantize import from_bf16b, to_bf16b


def _piece_offset(n, c, K):
    """Element offset of row n's values k = 8c .. 8c + 7 (the header's map)."""
    return ((n // 16) * (K // 32) + c // 4) * 512 + ((c % 4) * 16 + n % 16) * 8


def _random(n, k, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, k, generator=g).bfloat16()


@pytest.mark.parametrize("n,k", [(16, 64), (48, 256), (64, 3072)])
def test_round_trip_and_index_map(n, k):
    w = _random(n, k, n + k)
    wb = to_bf16b(w)
    assert wb.shape == w.shape and wb.dtype == torch.bfloat16
    assert torch.equal(from_bf16b(wb), w)
    fb = wb.flatten()
    for row in range(n):
        for c in range(k // 8):
            o = _piece_offset(row, c, k)
            assert torch.equal(fb[o:o + 8], w[row, 8 * c:8 * c + 8]), (row, c)


def test_known_positions():
    """Hand-computed: row 17, k 40..47 (piece 5) lies in the second tile's
    second block (K = 256: 8 blocks of 32 k per tile row), lane
    (5 % 4) * 16 + 1 = 17, i.e. element (1 * 8 + 1) * 512 + 17 * 8 = 4744.
    That is also the MFMA A operand: lane 17 = lg 1, r 1 holds row 1 of the
    tile at k 8 .. 15 of the block."""
    K = 256
    assert _piece_offset(17, 5, K) == 4744
    w = torch.zeros(32, K, dtype=torch.bfloat16)
    w[17, 41] = 3.0
    w[0, 0] = -1.0
    wb = to_bf16b(w).flatten()
    assert wb[4745] == 3.0 and wb[0] == -1.0
    assert int((wb != 0).sum()) == 2


def test_interleave_commutes_with_blocking():
    w = _random(64, 256, 3)
    assert torch.equal(interleave16(to_bf16b(w)), to_bf16b(interleave16(w)))


def test_shape_and_dtype_guard():
    with pytest.raises(ValueError):
        to_bf16b(_random(16, 96, 4))               # K % 64 != 0
    with pytest.raises(ValueError):
        to_bf16b(_random(24, 64, 4))               # N % 16 != 0
    with pytest.raises(ValueError):
        to_bf16b(_random(16, 64, 4).float())


def _plan(M, N, K, req, swiglu=False):
    lib = _lib.lib()
    cfg = (ctypes.c_int * 6)(*req, 0)
    fn = lib.acorn_gemm_swiglu_plan if swiglu else lib.acorn_gemm_plan
    return fn(M, N, K, _lib.WFMT_BF16B, cfg), tuple(cfg[:5])


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
@pytest.mark.parametrize("M", [1, 8, 16])
@pytest.mark.parametrize("N,K", [(6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288),
                                 (151936, 4096), (2048, 1024), (1024, 3072)])
def test_planner_bf16b_decode(M, N, K):
    """The default tiling, and every requested one the planner accepts, obey
    the bf16 decode kernel's contract: rt in {1,2,4} dividing N/16, upw in
    {1,2,4}, a wave layout of 1 or 4 waves on their own rows or 10 nw + kw
    (22, 44), depth in {2,4,8} within the register ring's budget (stage = 4 rt
    upw + 4 upw dwords), and each wave's K range holding a whole number of
    depth-stage rounds of 32-k blocks."""
    reqs = [(0, 0, 0, 0, 0), (4, 1, 1, 0, 8), (1, 2, 4, 3, 2), (2, 2, 4, 5, 4), (2, 1, 1, 1, 4),
            (4, 4, 1, 2, 4), (1, 1, 4, 16, 1), (2, 1, 2, 0, 4), (1, 4, 1, 0, 2), (2, 1, 44, 1, 8),
            (2, 2, 84, 2, 2), (4, 1, 22, 0, 4), (1, 8, 1, 0, 2)]
    for r in reqs:
        rc, (rt, upw, nwf, ks, depth) = _plan(M, N, K, r)
        if r != reqs[0] and rc == _lib.ERR_UNSUPPORTED:
            continue                  # a request the shape cannot honour is refused
        assert rc == 0, (r, rc)
        assert r[2] in (0, 1, 4, 22, 44) and r[1] in (0, 1, 2, 4), r  # refused knobs never plan
        assert r[4] != 1, r                                            # no depth-1 form
        kw = 1 if nwf < 10 else nwf % 10
        assert nwf in (1, 4, 22, 44)
        assert rt in (1, 2, 4) and (N // 16) % rt == 0
        assert upw in (1, 2, 4) and depth in (2, 4, 8)
        # x registers per stage: 4 per block, half in the paired-x form (M <= 8, even upw)
        xd = 4 * (upw // 2 if M <= 8 and upw % 2 == 0 else upw)
        assert depth * (4 * rt * upw + xd) <= 192
        blocks = K // 32
        assert blocks % (ks * kw) == 0 and (blocks // ks // kw) % (upw * depth) == 0
        if r[3] == 0:
            waves = N // 16 // rt * kw
            assert waves * ks >= 768 or ks == blocks // (kw * upw * depth)


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
@pytest.mark.parametrize("M", [1, 8, 16])
def test_planner_bf16b_swiglu_decode(M):
    """The fused SwiGLU at decode sizes: two or four row tiles per wave (gate
    and up tiles in pairs), one split."""
    for r in [(0, 0, 0, 0, 0), (4, 2, 22, 0, 4), (1, 1, 44, 0, 8)]:
        rc, (rt, upw, nwf, ks, depth) = _plan(M, 24576, 4096, r, swiglu=True)
        assert rc == 0, (r, rc)
        assert rt in (2, 4) and ks == 1


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
@pytest.mark.parametrize("M", [17, 64, 200, 256, 1024, 4096])
@pytest.mark.parametrize("N,K", [(6144, 4096), (4096, 12288), (24576, 4096)])
def test_planner_bf16b_prefill_routes(M, N, K):
    """Above 16 rows BF16B plans onto the tiled kernel (rt 0) and from 256
    rows onto the large-M kernel's direct-to-LDS form (-2, 256, 128, ks, 4);
    the register-staged 256 x 256 form and the streaming kernel are refused."""
    rc, t = _plan(M, N, K, (0, 0, 0, 0, 0))
    assert rc == 0
    if M >= 256:
        assert t[0] == -2 and t[1:3] == (256, 128) and t[4] == 4, t
    else:
        assert t[0] == 0 and t[1] in (32, 64, 128) and t[2] in (64, 128), t
    assert _plan(M, N, K, (-2, 256, 64, 1, 2))[0] == _lib.ERR_UNSUPPORTED
    assert _plan(M, N, K, (1, 2, 4, 0, 0))[0] == _lib.ERR_UNSUPPORTED
    rc, t = _plan(M, N, K, (-2, 128, 64, 0, 4))
    assert rc == 0 and t[:3] == (-2, 128, 64)
    if M >= 512:
        rc, t = _plan(M, N, K, (0, 0, 0, 0, 0), swiglu=True)
        assert rc == 0 and t[0] == -2 and t[3] == 1


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_planner_bf16b_rejects_unblockable_shapes():
    lib = _lib.lib()
    for N, K in ((4096, 4128), (4104, 4096)):
        for M in (8, 64, 512):
            rc = lib.acorn_gemm_plan(M, N, K, _lib.WFMT_BF16B, (ctypes.c_int * 6)())
            with pytest.raises(AssertionError):
                _lib.check(rc, "plan")


def test_qlinear_blocks_bf16_weights():
    """from_dense keeps bf16 weights of blockable shapes in BF16B, the rest
    natural; natural() and dense() give the reference's rows back."""
    from acorninfer_amd.models.qwen3 import QLinear
    w = _random(64, 256, 9)
    lin = QLinear.from_dense(w, _lib.WFMT_BF16)
    assert lin.fmt == _lib.WFMT_BF16B
    assert torch.equal(lin.natural().w, w) and torch.equal(lin.dense(), w.float())
    odd = QLinear.from_dense(_random(24, 96, 9), _lib.WFMT_BF16)
    assert odd.fmt == _lib.WFMT_BF16
    il = QLinear.from_dense(w, _lib.WFMT_BF16).interleaved()
    assert il.fmt == _lib.WFMT_BF16B and torch.equal(il.dense(), w.float())
