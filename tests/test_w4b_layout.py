"""The int4 decode layout (ACORN_WFMT_W4B) on the CPU: the conversion from
the reference's packing (quant/quantize.py:122-131, u_even | u_odd << 4 in
[N, K/2] rows) is a byte permutation that round-trips, it places bytes where
the C-ABI's index maps say (include/acorn_hip.h), it commutes with the
16-row gate|up interleave, and the planner's W4B tilings satisfy the
kernel's constraints. No GPU: the planner is host code."""
import ctypes

import pytest
import torch

from acorninfer_amd import _lib
from acorninfer_amd.ops.quant_gemm import interleave16
from acorninfer_amd.quant.quantize import from_w4b, to_w4b


def _chunk_offset(n, c, K):
    return ((n // 16) * (K // 128) + c // 4) * 1024 + ((c % 4) * 16 + n % 16) * 16


def _half_index(n, g, K):
    return ((n // 16) * (K // 512) + g // 4) * 64 + ((n % 16) // 4) * 16 + (g % 4) * 4 + n % 4


def _random(n, k, seed=0):
    g = torch.Generator().manual_seed(seed)
    p = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.uint8)
    s = torch.rand(n, k // 128, generator=g).half()
    return p, s


@pytest.mark.parametrize("n,k", [(16, 512), (48, 1024), (64, 3072)])
def test_round_trip_and_index_maps(n, k):
    p, s = _random(n, k, n + k)
    wb, sb = to_w4b(p, s)
    assert wb.shape == p.shape and sb.shape == s.shape
    back = from_w4b(wb, sb)
    assert torch.equal(back[0], p) and torch.equal(back[1], s)
    fw, fs = wb.flatten(), sb.flatten()
    for row in range(n):
        for c in range(k // 32):
            o = _chunk_offset(row, c, k)
            assert torch.equal(fw[o:o + 16], p[row, 16 * c:16 * c + 16]), (row, c)
        for g in range(k // 128):
            assert fs[_half_index(row, g, k)] == s[row, g], (row, g)


def test_known_positions():
    """Hand-computed positions: row 17, k 96..127 (chunk 3) is the second
    tile's first block, lane 3*16 + 1 = 49; row 5, group 6's scale is record
    (tile 0, groups 4..7, lane group 1) at position 2*4 + 1."""
    K = 1024
    assert _chunk_offset(17, 3, K) == (1 * 8 + 0) * 1024 + 49 * 16
    assert _half_index(5, 6, K) == (0 * 2 + 1) * 64 + 1 * 16 + 2 * 4 + 1
    p = torch.zeros(32, K // 2, dtype=torch.uint8)
    p[17, 48] = 0xAB                 # k = 96, 97: chunk 3, byte 0
    s = torch.zeros(32, K // 128, dtype=torch.float16)
    s[5, 6] = 2.0
    wb, sb = to_w4b(p, s)
    assert wb.flatten()[(8 * 1024) + 49 * 16] == 0xAB and int(wb.sum()) == 0xAB
    assert sb.flatten()[64 + 16 + 9] == 2.0 and float(sb.float().sum()) == 2.0


def test_interleave_commutes_with_blocking():
    p, s = _random(64, 1024, 3)
    wb, sb = to_w4b(p, s)
    wi, si = to_w4b(interleave16(p), interleave16(s))
    assert torch.equal(interleave16(wb), wi) and torch.equal(interleave16(sb), si)


def test_shape_guard():
    p, s = _random(16, 384, 4)        # K % 512 != 0
    with pytest.raises(ValueError):
        to_w4b(p, s)


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
@pytest.mark.parametrize("M", [1, 8, 16])
@pytest.mark.parametrize("N,K", [(6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288),
                                 (151936, 4096), (2048, 1024), (1024, 3072)])
def test_planner_w4b_decode(M, N, K):
    """The default W4B tiling, and every requested one the planner accepts,
    obey the kernel's contract:
    rt divides N/16, upw in {1,2,4}, rt*upw*depth <= 16, a supported wave
    layout, each wave's K range holds a whole number of depth-stage rounds,
    LDS fits."""
    lib = _lib.lib()
    reqs = [(0, 0, 0, 0, 0), (4, 1, 2, 0, 2), (1, 4, 4, 3, 2), (2, 2, 4, 5, 4), (1, 2, 84, 1, 4),
            (2, 1, 42, 2, 8)]
    for r in reqs:
        cfg = (ctypes.c_int * 6)(*r, 0)
        rc = lib.acorn_gemm_plan(M, N, K, _lib.WFMT_W4B, cfg)
        if r != reqs[0] and rc == _lib.ERR_UNSUPPORTED:
            continue                  # a request the shape cannot honour is refused
        assert rc == 0, (r, rc)
        rt, upw, nwf, ks, depth = cfg[:5]
        nw, kw = (nwf, 1) if nwf < 10 else (nwf // 10, nwf % 10)
        assert (nw, kw) in ((2, 1), (4, 1), (4, 2), (4, 4), (8, 2), (8, 4))
        assert rt in (1, 2, 4) and (N // 16) % rt == 0
        assert upw in (1, 2, 4) and depth in (1, 2, 4, 8)
        assert rt * upw <= 8 and rt * upw * depth <= 16
        groups = K // 128
        assert groups % (ks * kw * upw) == 0
        assert (groups // ks // kw // upw) % depth == 0
        R = 1 << (M - 1).bit_length()
        red = nw * rt * 4 * 64 * 4 if kw > 1 else 0
        assert (K // ks) * R * 2 + (K // ks // 128) * 64 + red <= 160 * 1024


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_planner_w4b_rejects_unblockable_shapes():
    lib = _lib.lib()
    for N, K in ((4096, 4224), (4104, 4096)):
        rc = lib.acorn_gemm_plan(8, N, K, _lib.WFMT_W4B, (ctypes.c_int * 6)())
        with pytest.raises(AssertionError):
            _lib.check(rc, "plan")
