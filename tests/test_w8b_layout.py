"""The int8 decode layout (ACORN_WFMT_W8B) on the CPU: the conversion from
the reference's int8 [N, K] rows (quant/quantize.py:89-107) stores every byte
as q + 128 and moves each 16-byte piece (row n, k in [16c, 16c+16)) to the
place the C-ABI's index map says (include/acorn_hip.h), it round-trips, it
commutes with the 16-row gate|up interleave, and the planner's W8B tilings
satisfy the int8 decode kernel's constraints. No GPU: the planner is host
code."""
import ctypes

import pytest
import torch

from acorninfer_amd import _lib
from acorninfer_amd.ops.quant_gemm import interleave16
from acorninfer_amd.quant.quantize import from_w8b, to_w8b


def _chunk_offset(n, c, K):
    return ((n // 16) * (K // 64) + c // 4) * 1024 + ((c % 4) * 16 + n % 16) * 16


def _random(n, k, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)


@pytest.mark.parametrize("n,k", [(16, 64), (48, 256), (64, 3072)])
def test_round_trip_and_index_map(n, k):
    q = _random(n, k, n + k)
    wb = to_w8b(q)
    assert wb.shape == q.shape and wb.dtype == torch.uint8
    assert torch.equal(from_w8b(wb), q)
    fb = wb.flatten()
    qb = (q.to(torch.int16) + 128).to(torch.uint8)
    for row in range(n):
        for c in range(k // 16):
            o = _chunk_offset(row, c, k)
            assert torch.equal(fb[o:o + 16], qb[row, 16 * c:16 * c + 16]), (row, c)


def test_known_positions():
    """Hand-computed: row 17, k 48..63 (chunk 3) is the second tile's first
    block (K = 256: 4 blocks per tile row), lane 3 * 16 + 1 = 49; the byte
    holds q + 128."""
    K = 256
    assert _chunk_offset(17, 3, K) == (1 * 4 + 0) * 1024 + 49 * 16
    q = torch.zeros(32, K, dtype=torch.int8)
    q[17, 48] = -5
    q[0, 0] = 127
    wb = to_w8b(q).flatten()
    assert wb[4 * 1024 + 49 * 16] == 123 and wb[0] == 255
    assert int((wb != 128).sum()) == 2


def test_interleave_commutes_with_blocking():
    q = _random(64, 256, 3)
    assert torch.equal(interleave16(to_w8b(q)), to_w8b(interleave16(q)))


def test_shape_and_dtype_guard():
    with pytest.raises(ValueError):
        to_w8b(_random(16, 96, 4))               # K % 64 != 0
    with pytest.raises(ValueError):
        to_w8b(_random(24, 64, 4))               # N % 16 != 0
    with pytest.raises(ValueError):
        to_w8b(_random(16, 64, 4).to(torch.uint8))


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
@pytest.mark.parametrize("M", [1, 8, 16])
@pytest.mark.parametrize("N,K", [(6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288),
                                 (151936, 4096), (2048, 1024), (1024, 3072)])
def test_planner_w8b_decode(M, N, K):
    """The default tiling, and every requested one the planner accepts, obey
    the int8 decode kernel's contract: rt in {1,2,4} dividing N/16, upw in
    {1,2}, a wave layout of 1 or 4 waves on their own rows or 10 nw + kw (22,
    44), depth in {1,2,4,8} within the register ring's budget (stage = 4 rt
    upw + 8 upw dwords), and each wave's K range holding a whole number of
    depth-stage rounds of 64-k blocks."""
    lib = _lib.lib()
    reqs = [(0, 0, 0, 0, 0), (4, 1, 1, 0, 4), (1, 2, 4, 3, 2), (2, 2, 4, 5, 4), (2, 1, 1, 1, 4),
            (4, 2, 1, 2, 4), (1, 1, 4, 16, 1), (2, 1, 2, 0, 4), (1, 4, 1, 0, 2), (2, 1, 44, 1, 4),
            (2, 2, 84, 2, 2), (4, 1, 22, 0, 4), (1, 2, 44, 1, 8), (2, 1, 1, 0, 8)]
    for r in reqs:
        cfg = (ctypes.c_int * 6)(*r, 0)
        rc = lib.acorn_gemm_plan(M, N, K, _lib.WFMT_W8B, cfg)
        if r != reqs[0] and rc == _lib.ERR_UNSUPPORTED:
            continue                  # a request the shape cannot honour is refused
        assert rc == 0, (r, rc)
        rt, upw, nwf, ks, depth = cfg[:5]
        assert r[2] in (0, 1, 4, 22, 44) and r[1] in (0, 1, 2), r   # refused knobs never plan
        kw = 1 if nwf < 10 else nwf % 10
        assert nwf in (1, 4, 22, 44)
        assert rt in (1, 2, 4) and (N // 16) % rt == 0
        assert upw in (1, 2) and depth in (1, 2, 4, 8)
        # x registers per stage: 8 per block, half in the paired-x form (M <= 8, upw 2)
        xd = 8 * (upw // 2 if M <= 8 and upw == 2 else upw)
        assert depth * (4 * rt * upw + xd) <= 192
        blocks = K // 64
        assert blocks % (ks * kw) == 0 and (blocks // ks // kw) % (upw * depth) == 0
        if r[3] == 0:
            waves = N // 16 // rt * kw
            assert waves * ks >= 768 or ks == blocks // (kw * upw * depth)


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_planner_w8b_rejects_unblockable_shapes():
    lib = _lib.lib()
    for N, K in ((4096, 4128), (4104, 4096)):
        rc = lib.acorn_gemm_plan(8, N, K, _lib.WFMT_W8B, (ctypes.c_int * 6)())
        with pytest.raises(AssertionError):
            _lib.check(rc, "plan")
