"""The int4 decode layout (ACORN_WFMT_W4B) on the CPU: the conversion from
the reference's packing (quant/quantize.py:122-131, u_even | u_odd << 4 in
[N, K/2] rows) moves 16-byte chunks where the C-ABI's index maps say
(include/acorn_hip.h) with each word's nibbles in the pair order the kernels
unpack, it round-trips, it commutes with the 16-row gate|up interleave, and
the planner's W4B tilings satisfy the kernel's constraints. No GPU: the
planner is host code."""
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


# k offset held by nibble p of a W4B word (the decode kernels unpack nibbles
# (q, q + 4) as one bf16 pair, which must be k offsets (2q, 2q + 1))
NIBBLE_K = (0, 2, 4, 6, 1, 3, 5, 7)


def _w4b_word_bytes(natural: bytes) -> bytes:
    """4 bytes in the reference's packing (low nibble = even k) -> the W4B word."""
    w = int.from_bytes(natural, "little")
    out = sum(((w >> (4 * NIBBLE_K[p])) & 15) << (4 * p) for p in range(8))
    return out.to_bytes(4, "little")


def test_nibble_order_pairs_natural_k():
    """Unpacking pair q of a W4B word as (nibble q, nibble q + 4) yields the
    natural k pair (2q, 2q + 1) of the source bytes."""
    src = bytes([0xAB, 0xCD, 0xEF, 0x12])          # k0..k7 = B, A, D, C, F, E, 2, 1
    w = int.from_bytes(_w4b_word_bytes(src), "little")
    assert w == 0x1ECA2FDB
    ks = [(int.from_bytes(src, "little") >> (4 * k)) & 15 for k in range(8)]
    for q in range(4):
        assert ((w >> 4 * q) & 15, (w >> (4 * q + 16)) & 15) == (ks[2 * q], ks[2 * q + 1])


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
    pb = p.numpy().tobytes()
    fb = fw.numpy().tobytes()
    for row in range(n):
        for c in range(k // 32):
            o = _chunk_offset(row, c, k)
            src = pb[row * (k // 2) + 16 * c:row * (k // 2) + 16 * c + 16]
            want = b"".join(_w4b_word_bytes(src[4 * j:4 * j + 4]) for j in range(4))
            assert fb[o:o + 16] == want, (row, c)
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
    p[17, 48] = 0xAB                 # k = 96 (B), 97 (A): chunk 3, word 0
    s = torch.zeros(32, K // 128, dtype=torch.float16)
    s[5, 6] = 2.0
    wb, sb = to_w4b(p, s)
    # word 0 = 0x000A000B: k 96 in nibble 0, k 97 in nibble 4
    o = (8 * 1024) + 49 * 16
    assert wb.flatten()[o] == 0x0B and wb.flatten()[o + 2] == 0x0A
    assert int(wb.sum()) == 0x0B + 0x0A
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
    """M <= 16 (the direct kernel): the default tiling, and every requested
    one the planner accepts, obey the kernel's contract: rt in {1,2,4}
    dividing N/16, upw in {1,2}, a wave layout of 1 or 4 waves on their own
    rows or 10 nw + kw (22, 44, 84, 88), depth in {1,2,4} within the register
    ring's budget, and each wave's K range holding a whole number of
    depth-stage rounds."""
    lib = _lib.lib()
    reqs = [(0, 0, 0, 0, 0), (4, 1, 1, 0, 4), (1, 2, 4, 3, 2), (2, 2, 4, 5, 4), (2, 1, 1, 1, 4),
            (4, 2, 1, 2, 2), (1, 1, 4, 16, 1), (2, 1, 2, 0, 4), (1, 4, 1, 0, 2), (2, 1, 44, 1, 4),
            (2, 2, 84, 2, 2), (4, 1, 22, 0, 4), (2, 1, 42, 1, 2), (1, 1, 88, 1, 4),
            (1, 2, 88, 1, 2), (2, 1, 84, 0, 4), (1, 2, 44, 1, 4), (2, 2, 1, 1, 4)]
    for r in reqs:
        cfg = (ctypes.c_int * 6)(*r, 0)
        rc = lib.acorn_gemm_plan(M, N, K, _lib.WFMT_W4B, cfg)
        if r != reqs[0] and rc == _lib.ERR_UNSUPPORTED:
            continue                  # a request the shape cannot honour is refused
        assert rc == 0, (r, rc)
        rt, upw, nwf, ks, depth = cfg[:5]
        assert r[2] in (0, 1, 4, 22, 44, 84, 88) and r[1] in (0, 1, 2), r   # refused knobs never plan
        assert nwf in (1, 4, 22, 44, 84, 88)
        kw = 1 if nwf < 10 else nwf % 10
        assert rt in (1, 2, 4) and (N // 16) % rt == 0
        assert upw in (1, 2) and depth in (1, 2, 4)
        # x registers per stage: 16 per group, half in the paired-x form (M <= 8, upw 2)
        xd = 16 * (upw // 2 if M <= 8 and upw == 2 else upw)
        assert depth * (4 * rt * upw + xd + 2 * rt * upw) <= 160
        groups = K // 128
        assert groups % (ks * kw) == 0 and (groups // ks // kw) % (upw * depth) == 0
        if r[3] == 0:
            # the default split: the fewest that launch three waves per CU
            waves = N // 16 // rt * kw
            assert waves * ks >= 768 or ks == groups // (kw * upw * depth)


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_planner_w4b_rejects_unblockable_shapes():
    lib = _lib.lib()
    for N, K in ((4096, 4224), (4104, 4096)):
        rc = lib.acorn_gemm_plan(8, N, K, _lib.WFMT_W4B, (ctypes.c_int * 6)())
        with pytest.raises(AssertionError):
            _lib.check(rc, "plan")
