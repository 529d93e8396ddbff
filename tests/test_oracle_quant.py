"""Pins for oracle/quant_ref.py (CPU): the reference's known answers and
theoretical bounds (tests/test_quantize.py in the reference), the symmetric
bridge identity, and the product quantiser agreeing with the oracle."""
import numpy as np
import torch

from oracle.quant_ref import (dequant_w4_ref, dequant_w4_sym_ref, dequant_w8_ref, gemm_ref,
                              pack_w4_ref, quantize_w4_ref, quantize_w4_sym_ref,
                              quantize_w8_ref, unpack_w4_ref)


def _w(seed, n=256, k=4096):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, k, generator=g).bfloat16().float().numpy()


def test_pack_known_answer_and_roundtrip():
    q2 = np.array([[1, 2, 3, 4, 15, 0]], dtype=np.uint8)
    assert pack_w4_ref(q2).tolist() == [[0x21, 0x43, 0x0F]]
    assert np.array_equal(unpack_w4_ref(pack_w4_ref(q2)), q2)
    u = np.random.default_rng(0).integers(0, 16, (64, 256)).astype(np.uint8)
    assert np.array_equal(unpack_w4_ref(pack_w4_ref(u)), u)


def test_w8_bound_and_zero_row():
    w = _w(0)
    w[0] = 0.0
    w[1] = 0.5
    q, s = quantize_w8_ref(w)
    assert q.dtype == np.int8 and s.dtype == np.float16 and np.abs(q).max() <= 127
    assert float(s[0]) == 0.0                          # 1e-8/127 underflows fp16
    assert np.all(q[1] == 127)
    sf = s.astype(np.float32)
    bound = sf / 2 + sf * 127 * 2.0 ** -11 + 1e-6
    assert np.all(np.abs(dequant_w8_ref(q, s) - w) <= bound[:, None])


def test_w4_asym_bound():
    w = _w(1)
    w[0] = 0.0
    w[1, :128] = -2.0
    u, s, z = quantize_w4_ref(w)
    assert u.max() <= 15 and s.shape == (256, 32) and z.shape == (256, 32)
    sf, zf = s.astype(np.float32), z.astype(np.float32)
    bound = sf / 2 + sf * 15 * 2.0 ** -11 + np.abs(zf) * 2.0 ** -11 + 1e-6
    err = np.abs(dequant_w4_ref(u, s, z) - w).reshape(256, 32, 128)
    assert np.all(err <= bound[..., None])


def test_symmetric_bridge_is_bitwise():
    """dequant_w4(v+8, s, -8s) == v*s exactly in fp32.

    -8s is exact in fp16 (a power-of-two multiple), (v+8)*s needs at most
    4 + 11 mantissa bits and fits fp32, and so does its difference with 8s."""
    rng = np.random.default_rng(3)
    v = rng.integers(-8, 8, (128, 512))
    s = (0.005 + 0.015 * rng.random((128, 4))).astype(np.float16)
    u = (v + 8).astype(np.uint8)
    zero = (-8.0 * s.astype(np.float32)).astype(np.float16)
    a = dequant_w4_ref(u, s, zero)
    b = v.astype(np.float32) * np.repeat(s.astype(np.float32), 128, axis=1)
    assert np.array_equal(a, b)
    assert np.array_equal(dequant_w4_sym_ref(u, s), b)


def test_w4_sym_bound():
    w = _w(4)
    u, s = quantize_w4_sym_ref(w)
    assert u.min() >= 0 and u.max() <= 15
    sf = np.repeat(s.astype(np.float32), 128, axis=1)
    err = np.abs(dequant_w4_sym_ref(u, s) - w)
    assert np.all(err <= sf / 2 + 1e-6 + sf * 2.0 ** -10 * 8)


def test_gemm_ref_matches_hand_expanded_group_sum():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    u = rng.integers(0, 16, (8, 256)).astype(np.uint8)
    s = (0.01 + 0.01 * rng.random((8, 2))).astype(np.float16)
    y = gemm_ref(x, dequant_w4_sym_ref(u, s))
    for m in range(3):
        for n in range(8):
            tot = 0.0
            for g in range(2):
                tot += float(s[n, g]) * sum(float(x[m, k]) * (int(u[n, k]) - 8)
                                            for k in range(128 * g, 128 * g + 128))
            assert abs(y[m, n] - tot) < 1e-9 * max(1.0, abs(tot))


def test_product_quantize_agrees_with_oracle():
    from acorninfer_amd.quant import quantize as qz
    w = _w(6)
    wt = torch.from_numpy(w).bfloat16()
    q, s = qz.quantize_w8(wt)
    q_r, s_r = quantize_w8_ref(w)
    assert np.array_equal(q.numpy(), q_r) and np.array_equal(s.numpy(), s_r)
    u, s4, z4 = qz.quantize_w4(wt)
    u_r, s4_r, z4_r = quantize_w4_ref(w)
    assert np.array_equal(u.numpy(), u_r) and np.array_equal(s4.numpy(), s4_r)
    assert np.array_equal(z4.numpy(), z4_r)
    us, ss = qz.quantize_w4_sym(wt)
    us_r, ss_r = quantize_w4_sym_ref(w)
    assert np.array_equal(us.numpy(), us_r) and np.array_equal(ss.numpy(), ss_r)
    assert np.array_equal(qz.pack_w4(us).numpy(), pack_w4_ref(us_r))
    assert np.array_equal(qz.unpack_w4(qz.pack_w4(us)).numpy(), us_r)
    assert np.array_equal(qz.dequant_w4(us, ss, qz.sym_zero(ss)).numpy(), dequant_w4_sym_ref(us_r, ss_r))
