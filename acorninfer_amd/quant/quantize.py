"""Load-time RTN weight quantisation (torch, any device).

Drop-in for acorninfer/quant/quantize.py. Formats:
- W8 per-channel symmetric (quantize.py:89-99): scale fp16 [N] =
  max|w[n,:]| / 127 (clamped at EPS before the fp16 cast), q int8 in
  [-127, 127].
- W4 group-128 asymmetric, the reference's spike format (quantize.py:102-119):
  per (row, group) scale = (max-min)/15, zero = min, u uint8 in [0, 15].
- W4 group-128 symmetric (this build's production W4A16): v int in [-8, 7],
  scale fp16 = max|w_g| / 7; stored as u = v + 8 with the same packing, so
  `dequant_w4(u, s, -8*s)` equals v*s exactly in fp32.
- Packing (quantize.py:122-131): byte = u_even | u_odd << 4.
Shape guard (quantize.py:78-86): N and K multiples of 128, else ValueError.

`apply_quant(model, mode)` is the load-time module walk (quantize.py:33-76):
"w8a16" as in the reference; "w4a16" is implemented here (the reference
raises NotImplementedError), storing the packed weight, `_q_scale` and the
marker `_m7_quant`.
"""
from __future__ import annotations

import torch

EPS = 1e-8
_SHAPE_MULT = 128
GROUP = 128

QUANT_ATTRS = frozenset({
    "q_proj", "k_proj", "v_proj", "o_proj",
    "gate_proj", "up_proj", "down_proj", "lm_head",
})


def _guard_shape(w: torch.Tensor) -> tuple[int, int]:
    if w.dim() != 2:
        raise ValueError(f"w must be 2D [N,K], got shape={tuple(w.shape)}")
    n, k = w.shape
    if k % _SHAPE_MULT != 0:
        raise ValueError(f"K={k} is not a multiple of {_SHAPE_MULT}")
    if n % _SHAPE_MULT != 0:
        raise ValueError(f"N={n} is not a multiple of {_SHAPE_MULT}")
    return n, k


def quantize_w8(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """w [N,K] -> (q int8 [N,K] in [-127,127], scale fp16 [N])."""
    _guard_shape(w)
    w32 = w.float()
    scale = w32.abs().amax(dim=1).clamp_min(EPS) / 127.0
    q = torch.round(w32 / scale[:, None]).clamp_(-127, 127).to(torch.int8)
    return q, scale.half()


def quantize_w4(w: torch.Tensor, group: int = GROUP
                ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Asymmetric: w [N,K] -> (u uint8 [N,K] in [0,15], scale fp16 [N,K/g], zero fp16 [N,K/g])."""
    n, k = _guard_shape(w)
    if k % group != 0:
        raise ValueError(f"K={k} is not divisible by group={group}")
    wg = w.float().view(n, k // group, group)
    wmax, wmin = wg.amax(dim=2), wg.amin(dim=2)
    scale = ((wmax - wmin) / 15.0).clamp_min(EPS)
    zp = wmin
    q = torch.round((wg - zp[..., None]) / scale[..., None]).clamp_(0, 15)
    return q.to(torch.uint8).view(n, k), scale.half(), zp.half()


def quantize_w4_sym(w: torch.Tensor, group: int = GROUP
                    ) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric: w [N,K] -> (u uint8 [N,K] = v + 8 with v in [-8,7], scale fp16 [N,K/g]).

    scale = max|w_g| / 7 (clamped at EPS), v = clamp(round(w / scale_fp16), -8, 7)
    computed against the stored fp16 scale so that v*scale is the nearest grid point.
    """
    n, k = _guard_shape(w)
    if k % group != 0:
        raise ValueError(f"K={k} is not divisible by group={group}")
    wg = w.float().view(n, k // group, group)
    s16 = (wg.abs().amax(dim=2).clamp_min(EPS) / 7.0).half()
    s = s16.float().clamp_min(EPS)  # a scale that underflowed fp16 divides by EPS
    v = torch.round(wg / s[..., None]).clamp_(-8, 7)
    return (v + 8).to(torch.uint8).view(n, k), s16


def pack_w4(q: torch.Tensor) -> torch.Tensor:
    """u uint8 [N,K] in [0,15] -> uint8 [N,K/2], byte = u_even | u_odd << 4."""
    if q.dim() != 2 or q.shape[1] % 2 != 0:
        raise ValueError(f"pack_w4 needs 2D with even K, got shape={tuple(q.shape)}")
    qq = q.reshape(q.shape[0], q.shape[1] // 2, 2)
    return (qq[..., 0] | (qq[..., 1] << 4)).contiguous()


def unpack_w4(p: torch.Tensor) -> torch.Tensor:
    """Inverse of pack_w4: even column = p & 0xF, odd column = p >> 4."""
    if p.dim() != 2:
        raise ValueError(f"unpack_w4 needs 2D, got shape={tuple(p.shape)}")
    n, kh = p.shape
    out = torch.empty(n, kh * 2, dtype=torch.uint8, device=p.device)
    out[:, 0::2] = p & 0xF
    out[:, 1::2] = p >> 4
    return out


# Nibble order inside each 32-bit word of the W4B layout: position p (bits
# 4p .. 4p+3) holds the word's k offset W4B_NIBBLE_K[p]. The kernels turn a
# word into four bf16 pairs as (nibble q, nibble q + 4), q = 0..3, so with k
# offsets (2q, 2q + 1) in that pair the unpacked operand is in natural k order
# and x needs no reordering.
W4B_NIBBLE_K = (0, 2, 4, 6, 1, 3, 5, 7)


def _w4b_nibbles(packed: torch.Tensor, order) -> torch.Tensor:
    """Each group of 4 bytes (8 nibbles, low nibble first) with nibble p
    replaced by nibble order[p]."""
    b = packed.reshape(-1, 4).to(torch.int32)
    nib = torch.stack([(b >> 4 * (p % 2)) & 15 for p in range(2)], 2).reshape(-1, 8)
    nib = nib[:, list(order)]
    out = (nib[:, 0::2] | (nib[:, 1::2] << 4)).to(torch.uint8)
    return out.reshape(packed.shape)


def to_w4b(packed: torch.Tensor, scale: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Natural packed int4 [N, K/2] + scale [N, K/128] -> the decode kernels'
    1 KB block layout (ACORN_WFMT_W4B), kept in tensors of the same shapes:
    16-byte chunk (row n, k in [32c, 32c+32)) moves to block (n // 16, c // 4),
    lane (c % 4) * 16 + n % 16, with the nibbles of each 32-bit word in the
    W4B_NIBBLE_K order; the scale of (n, g) to record (n // 16, g // 4,
    (n % 16) // 4) at position (g % 4) * 4 + n % 4. Rows 16t..16t+15 of both
    tensors hold row tile t, so 16-row block permutations (interleave16)
    commute with the conversion. N % 16 == 0 and K % 512 == 0."""
    n, kh = packed.shape
    k = 2 * kh
    if n % 16 or k % 512 or scale.shape != (n, k // 128):
        raise ValueError(f"to_w4b needs N % 16 == 0, K % 512 == 0 and scale [N, K/128]: "
                         f"packed {tuple(packed.shape)}, scale {tuple(scale.shape)}")
    wb = (_w4b_nibbles(packed, W4B_NIBBLE_K)
          .reshape(n // 16, 16, k // 128, 4, 16)           # tile, row, group, chunk, byte
          .permute(0, 2, 3, 1, 4).reshape(n, kh).contiguous())
    sb = (scale.reshape(n // 16, 4, 4, k // 512, 4)        # tile, lg, i, g4, gg
          .permute(0, 3, 1, 4, 2).reshape(n, k // 128).contiguous())
    return wb, sb


def from_w4b(wb: torch.Tensor, sb: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Inverse of to_w4b."""
    n, kh = wb.shape
    k = 2 * kh
    if n % 16 or k % 512 or sb.shape != (n, k // 128):
        raise ValueError(f"from_w4b needs N % 16 == 0, K % 512 == 0 and scale [N, K/128]: "
                         f"packed {tuple(wb.shape)}, scale {tuple(sb.shape)}")
    inv = [W4B_NIBBLE_K.index(j) for j in range(8)]
    packed = _w4b_nibbles(wb.reshape(n // 16, k // 128, 4, 16, 16)   # tile, group, chunk, row, byte
                          .permute(0, 3, 1, 2, 4).reshape(n, kh), inv).contiguous()
    scale = (sb.reshape(n // 16, k // 512, 4, 4, 4)        # tile, g4, lg, gg, i
             .permute(0, 2, 4, 1, 3).reshape(n, k // 128).contiguous())
    return packed, scale


def to_w8b(q: torch.Tensor) -> torch.Tensor:
    """int8 [N, K] -> the int8 decode kernel's 1 KB block layout
    (ACORN_WFMT_W8B) in a uint8 tensor of the same shape: every byte stored
    as q + 128, and the 16 bytes of row n, k in [16c, 16c+16) moved to block
    (n // 16, c // 4), lane (c % 4) * 16 + n % 16. The per-channel scale keeps
    its [N] layout. Rows 16t..16t+15 hold row tile t, so 16-row block
    permutations (interleave16) commute with the conversion. N % 16 == 0 and
    K % 64 == 0."""
    n, k = q.shape
    if q.dtype != torch.int8 or n % 16 or k % 64:
        raise ValueError(f"to_w8b needs int8 [N, K] with N % 16 == 0 and K % 64 == 0: "
                         f"{q.dtype} {tuple(q.shape)}")
    u = (q.to(torch.int16) + 128).to(torch.uint8)
    return (u.reshape(n // 16, 16, k // 64, 4, 16)        # tile, row, block, chunk, byte
            .permute(0, 2, 3, 1, 4).reshape(n, k).contiguous())


def from_w8b(wb: torch.Tensor) -> torch.Tensor:
    """Inverse of to_w8b."""
    n, k = wb.shape
    if wb.dtype != torch.uint8 or n % 16 or k % 64:
        raise ValueError(f"from_w8b needs uint8 [N, K] with N % 16 == 0 and K % 64 == 0: "
                         f"{wb.dtype} {tuple(wb.shape)}")
    u = (wb.reshape(n // 16, k // 64, 4, 16, 16)           # tile, block, chunk, row, byte
         .permute(0, 3, 1, 2, 4).reshape(n, k))
    return (u.to(torch.int16) - 128).to(torch.int8).contiguous()


def to_bf16b(w: torch.Tensor) -> torch.Tensor:
    """bf16 [N, K] -> the bf16 decode kernel's 1 KB block layout
    (ACORN_WFMT_BF16B) in a bf16 tensor of the same shape: the 8 values of row
    n, k in [8c, 8c+8) moved to block (n // 16, c // 4), lane (c % 4) * 16 +
    n % 16, so a block is the MFMA A operand of 16 rows x 32 k. Rows
    16t..16t+15 hold row tile t, so 16-row block permutations (interleave16)
    commute with the conversion. N % 16 == 0 and K % 64 == 0."""
    n, k = w.shape
    if w.dtype != torch.bfloat16 or n % 16 or k % 64:
        raise ValueError(f"to_bf16b needs bf16 [N, K] with N % 16 == 0 and K % 64 == 0: "
                         f"{w.dtype} {tuple(w.shape)}")
    return (w.reshape(n // 16, 16, k // 32, 4, 8)          # tile, row, block, chunk, value
            .permute(0, 2, 3, 1, 4).reshape(n, k).contiguous())


def from_bf16b(wb: torch.Tensor) -> torch.Tensor:
    """Inverse of to_bf16b."""
    n, k = wb.shape
    if wb.dtype != torch.bfloat16 or n % 16 or k % 64:
        raise ValueError(f"from_bf16b needs bf16 [N, K] with N % 16 == 0 and K % 64 == 0: "
                         f"{wb.dtype} {tuple(wb.shape)}")
    return (wb.reshape(n // 16, k // 32, 4, 16, 8)          # tile, block, chunk, row, value
            .permute(0, 3, 1, 2, 4).reshape(n, k).contiguous())


def dequant_w8(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32 [N,K] = q * scale[:, None]."""
    return q.float() * scale.float()[:, None]


def dequant_w4(q: torch.Tensor, scale: torch.Tensor, zp: torch.Tensor) -> torch.Tensor:
    """fp32 [N,K] = u * scale_g + zero_g for unpacked u [N,K]."""
    n, k = q.shape
    g = scale.shape[1]
    if k % g != 0:
        raise ValueError(f"K={k} is incompatible with {g} scale groups")
    rep = k // g
    s = scale.float().repeat_interleave(rep, dim=1)
    z = zp.float().repeat_interleave(rep, dim=1)
    return q.float() * s + z


def sym_zero(scale: torch.Tensor) -> torch.Tensor:
    """The zero point that makes the symmetric format an instance of dequant_w4."""
    return (-8.0 * scale.float()).half()


def apply_quant(model, mode: str) -> None:
    """Load-time walk: quantise every nn.Linear whose last name is in QUANT_ATTRS.

    "none": no change. "w8a16": weight.data <- int8, `_q_scale` fp16 [N].
    "w4a16": weight.data <- packed uint8 [N,K/2] (symmetric g128),
    `_q_scale` fp16 [N,K/128]. Both set `_m7_quant` to the mode.
    """
    if mode == "none":
        return
    if mode not in ("w8a16", "w4a16"):
        raise NotImplementedError(f"apply_quant: mode {mode!r} is not supported")
    hit = 0
    for name, mod in model.named_modules():
        if name.split(".")[-1] in QUANT_ATTRS and isinstance(mod, torch.nn.Linear):
            w = mod.weight.data
            if mode == "w8a16":
                q, s = quantize_w8(w)
            else:
                u, s = quantize_w4_sym(w)
                q = pack_w4(u)
            mod.weight.requires_grad_(False)
            mod.weight.data = q
            mod._q_scale = s
            mod._m7_quant = mode
            hit += 1
    if hit == 0:
        raise ValueError("apply_quant matched no quantisation target (projections + lm_head)")
