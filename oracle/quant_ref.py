"""Restatement of acorninfer/quant/quantize.py (numpy) and the GEMM reference.

Pins (tests/test_oracle_quant.py):
- pack_w4_ref: the reference's known answer test_quantize.py:87-90
  ([[1,2,3,4,15,0]] -> [[0x21,0x43,0x0F]]) and unpack(pack(u)) == u.
- quantize_w8_ref / quantize_w4_ref: the reference's theoretical error bounds
  test_quantize.py:38-79 and its all-zero-row case (fp16 scale stores 0.0).
- symmetric int4 bridge: dequant_w4(v+8, s, -8s) == v*s bitwise in fp32.
- gemm_ref: float64 matmul of the fp32 dequantised weights (a library
  routine); checked against a per-group hand-expanded sum on small shapes.
"""
from __future__ import annotations

import numpy as np

EPS = np.float32(1e-8)


def _bf16_to_f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32)


def quantize_w8_ref(w) -> tuple[np.ndarray, np.ndarray]:
    """quantize.py:89-99: scale = max|w|/127 (clamp EPS), q = rint(w/scale) in [-127,127]."""
    w32 = _bf16_to_f32(w)
    scale = np.maximum(np.abs(w32).max(axis=1), EPS) / np.float32(127.0)
    q = np.clip(np.rint(w32 / scale[:, None]), -127, 127).astype(np.int8)
    return q, scale.astype(np.float16)


def quantize_w4_ref(w, group: int = 128) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """quantize.py:102-119 (asymmetric): scale = (max-min)/15, zero = min."""
    w32 = _bf16_to_f32(w)
    n, k = w32.shape
    wg = w32.reshape(n, k // group, group)
    wmax, wmin = wg.max(axis=2), wg.min(axis=2)
    scale = np.maximum((wmax - wmin) / np.float32(15.0), EPS).astype(np.float32)
    q = np.clip(np.rint((wg - wmin[..., None]) / scale[..., None]), 0, 15)
    return q.astype(np.uint8).reshape(n, k), scale.astype(np.float16), wmin.astype(np.float16)


def quantize_w4_sym_ref(w, group: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric int4 (BASELINE config 3 format): s = max|w_g|/7 stored fp16,
    v = clip(rint(w / s), -8, 7), stored u = v + 8."""
    w32 = _bf16_to_f32(w)
    n, k = w32.shape
    wg = w32.reshape(n, k // group, group)
    s16 = (np.maximum(np.abs(wg).max(axis=2), EPS) / np.float32(7.0)).astype(np.float16)
    s = np.maximum(s16.astype(np.float32), EPS)
    v = np.clip(np.rint(wg / s[..., None]), -8, 7)
    return (v + 8).astype(np.uint8).reshape(n, k), s16


def pack_w4_ref(u: np.ndarray) -> np.ndarray:
    """quantize.py:122-131: byte = u[:, 2j] | u[:, 2j+1] << 4."""
    u = np.asarray(u, dtype=np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def unpack_w4_ref(p: np.ndarray) -> np.ndarray:
    """quantize.py:134-142."""
    p = np.asarray(p, dtype=np.uint8)
    out = np.empty((p.shape[0], p.shape[1] * 2), dtype=np.uint8)
    out[:, 0::2] = p & 0xF
    out[:, 1::2] = p >> 4
    return out


def dequant_w8_ref(q, scale) -> np.ndarray:
    """quantize.py:145-147 (fp32)."""
    return np.asarray(q, np.float32) * np.asarray(scale, np.float32)[:, None]


def dequant_w4_ref(u, scale, zero) -> np.ndarray:
    """quantize.py:150-164 (fp32): u * s_g + z_g."""
    u = np.asarray(u, np.float32)
    rep = u.shape[1] // np.asarray(scale).shape[1]
    s = np.repeat(np.asarray(scale, np.float32), rep, axis=1)
    z = np.repeat(np.asarray(zero, np.float32), rep, axis=1)
    return u * s + z


def dequant_w4_sym_ref(u, scale) -> np.ndarray:
    """v * s with v = u - 8 (fp32)."""
    rep = np.asarray(u).shape[1] // np.asarray(scale).shape[1]
    s = np.repeat(np.asarray(scale, np.float32), rep, axis=1)
    return (np.asarray(u, np.float32) - 8.0) * s


def gemm_ref(x, w_deq) -> np.ndarray:
    """float64 x[M,K] @ w_deq[N,K]^T — the reference's fp32 dequantised
    matmul anchor (test_quant_gemm.py:93-96) evaluated without fp32 drift."""
    return np.asarray(x, np.float64) @ np.asarray(w_deq, np.float64).T
