"""On-disk format of a quantised Qwen3 decode model (safetensors).

The reference quantises at load time only (`apply_quant`, acorninfer/quant/
quantize.py:33-76) and has no file format for int4. This one stores exactly
what the decode kernels read, so a checkpoint quantised once loads with no
re-quantisation and no full-precision copy:

- every projection under the reference's module names
  (`layers.{i}.self_attn.q_proj`, `k_proj`, `v_proj`, `o_proj`,
  `layers.{i}.mlp.gate_proj`, `up_proj`, `down_proj`, `lm_head`):
  - w4a16: `{name}.qweight` uint8 [N, K/2] (low nibble = even k, the
    reference's pack_w4 order), `{name}.scales` fp16 [N, K/128] and, for the
    asymmetric form only, `{name}.zeros` fp16 [N, K/128] (symmetric weights
    dequantise as (u - 8) * s);
  - w8a16: `{name}.qweight` int8 [N, K], `{name}.scales` fp16 [N];
  - bf16: `{name}.weight` bf16 [N, K];
- `embed_tokens.weight` and the RMSNorm weights (`norm.weight`,
  `layers.{i}.input_layernorm.weight`, `post_attention_layernorm.weight`,
  `self_attn.q_norm.weight`, `self_attn.k_norm.weight`) in bf16;
- metadata: `format`, `group_size`, `packing` and the model config as JSON.

Rows are stored in the reference's order (separate q/k/v and gate/up, gate
and up not interleaved); `load_quantized` fuses them into this build's qkv
and 16-row-interleaved gate|up launches. Loading goes through
safetensors.torch.load_file, which executes nothing from the file.
"""
from __future__ import annotations

import dataclasses
import json

import torch

from acorninfer_amd.config import Qwen3Config
from acorninfer_amd.models.qwen3 import (FORMATS, WFMT_BF16, WFMT_BF16B, WFMT_W4, WFMT_W4B, WFMT_W8,
                                         WFMT_W8B, LayerWeights, QLinear, Qwen3DecodeModel)
from acorninfer_amd.ops.quant_gemm import deinterleave16

FORMAT_NAMES = {v: k for k, v in FORMATS.items()}
FORMAT_NAMES[WFMT_W4B] = "w4a16"      # the in-memory block layouts of int4, int8 and bf16
FORMAT_NAMES[WFMT_W8B] = "w8a16"
FORMAT_NAMES[WFMT_BF16B] = "bf16"
_NORMS = ("input_layernorm", "post_attention_layernorm", "self_attn.q_norm", "self_attn.k_norm")


def _linear_tensors(name: str, lin: QLinear, out: dict) -> None:
    lin = lin.natural()                   # files hold the reference's layouts
    if lin.fmt == WFMT_BF16:
        out[f"{name}.weight"] = lin.w
    elif lin.fmt in (WFMT_W8, WFMT_W4):
        out[f"{name}.qweight"] = lin.w
        out[f"{name}.scales"] = lin.scale
        if lin.zero is not None:
            out[f"{name}.zeros"] = lin.zero
    else:
        raise ValueError(f"no on-disk form for weight format {lin.fmt}")


def _rows(lin: QLinear, bounds: list[int], names: list[str], out: dict) -> None:
    """Split a fused projection back into the reference's modules by rows."""
    lin = lin.natural()
    t = {"w": lin.w, "scale": lin.scale, "zero": lin.zero}
    if lin.il16:
        t = {k: (None if v is None else deinterleave16(v)) for k, v in t.items()}
    for name, lo, hi in zip(names, bounds[:-1], bounds[1:]):
        part = QLinear(lin.fmt, t["w"][lo:hi].contiguous(), hi - lo, lin.K,
                       None if t["scale"] is None else t["scale"][lo:hi].contiguous(),
                       None if t["zero"] is None else t["zero"][lo:hi].contiguous())
        _linear_tensors(name, part, out)


def save_quantized(model: Qwen3DecodeModel, path: str) -> None:
    """Write `model` (bf16 / w8a16 / w4a16 weights) to a safetensors file."""
    from safetensors.torch import save_file
    cfg = model.cfg
    if model.lm_head.fmt not in FORMAT_NAMES:
        raise ValueError("only bf16 / w8a16 / w4a16 models have an on-disk form")
    out: dict[str, torch.Tensor] = {"embed_tokens.weight": model.embed, "norm.weight": model.norm}
    qn, kvn = cfg.num_attention_heads * cfg.head_dim, cfg.num_key_value_heads * cfg.head_dim
    for i, L in enumerate(model.layers):
        p = f"layers.{i}"
        for n, w in zip(_NORMS, (L.input_norm, L.post_norm, L.q_norm, L.k_norm)):
            out[f"{p}.{n}.weight"] = w
        _rows(L.qkv, [0, qn, qn + kvn, qn + 2 * kvn],
              [f"{p}.self_attn.q_proj", f"{p}.self_attn.k_proj", f"{p}.self_attn.v_proj"], out)
        _linear_tensors(f"{p}.self_attn.o_proj", L.o, out)
        half = L.gate_up.N // 2
        _rows(L.gate_up, [0, half, 2 * half], [f"{p}.mlp.gate_proj", f"{p}.mlp.up_proj"], out)
        _linear_tensors(f"{p}.mlp.down_proj", L.down, out)
    _linear_tensors("lm_head", model.lm_head, out)
    meta = {"format": FORMAT_NAMES[model.lm_head.fmt], "group_size": "128",
            "packing": "uint8 [N, K/2], low nibble = even k",
            "config": json.dumps(dataclasses.asdict(cfg))}
    save_file({k: v.detach().contiguous().cpu() for k, v in out.items()}, path, metadata=meta)


def load_quantized(path: str, *, device="cuda") -> Qwen3DecodeModel:
    """Build a decode model from a file written by save_quantized."""
    from safetensors import safe_open
    from safetensors.torch import load_file
    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
    for key in ("format", "config"):
        if key not in meta:
            raise ValueError(f"{path}: metadata has no {key!r} entry (not a save_quantized file)")
    if meta["format"] not in FORMATS:
        raise ValueError(f"{path}: unknown weight format {meta['format']!r}")
    fmt = FORMATS[meta["format"]]
    if fmt != WFMT_BF16:
        if meta.get("group_size") != "128":
            raise ValueError(f"{path}: group size {meta.get('group_size')!r}; the kernels use 128")
        if fmt == WFMT_W4 and not meta.get("packing", "").startswith("uint8 [N, K/2], low nibble"):
            raise ValueError(f"{path}: int4 packing {meta.get('packing')!r} is not low-nibble-even")
    # JSON has no tuples: sequence fields of the config come back as lists
    cfg = Qwen3Config(**{k: tuple(v) if isinstance(v, list) else v
                         for k, v in json.loads(meta["config"]).items()})
    sd = load_file(path, device=str(torch.device(device)))

    def tensor(name: str, shape: tuple, dtype: torch.dtype) -> torch.Tensor:
        t = sd.get(name)
        if t is None:
            raise ValueError(f"{path}: tensor {name} is missing")
        if tuple(t.shape) != shape or t.dtype != dtype:
            raise ValueError(f"{path}: {name} is {tuple(t.shape)} {t.dtype}, "
                             f"the config needs {shape} {dtype}")
        return t

    H, D, I = cfg.hidden_size, cfg.head_dim, cfg.intermediate_size
    qn, kvn = cfg.num_attention_heads * D, cfg.num_key_value_heads * D
    shapes = {"q_proj": (qn, H), "k_proj": (kvn, H), "v_proj": (kvn, H), "o_proj": (H, qn),
              "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I),
              "lm_head": (cfg.vocab_size, H)}

    def lin(*names: str) -> QLinear:
        parts = []
        for n in names:
            N, K = shapes[n.rsplit(".", 1)[-1]]
            if fmt == WFMT_BF16:
                parts.append((tensor(f"{n}.weight", (N, K), torch.bfloat16), None, None))
                continue
            if K % 128:
                raise ValueError(f"{path}: {n} has K={K}, not a multiple of the group size 128")
            if fmt == WFMT_W8:
                parts.append((tensor(f"{n}.qweight", (N, K), torch.int8),
                              tensor(f"{n}.scales", (N,), torch.float16), None))
            else:
                zs = (tensor(f"{n}.zeros", (N, K // 128), torch.float16)
                      if f"{names[0]}.zeros" in sd else None)
                parts.append((tensor(f"{n}.qweight", (N, K // 2), torch.uint8),
                              tensor(f"{n}.scales", (N, K // 128), torch.float16), zs))
        w = torch.cat([p[0] for p in parts], 0).contiguous()
        K = shapes[names[0].rsplit(".", 1)[-1]][1]
        if fmt == WFMT_BF16:
            return QLinear(fmt, w, w.shape[0], K).blocked()
        s = torch.cat([p[1] for p in parts], 0).contiguous()
        z = None if parts[0][2] is None else torch.cat([p[2] for p in parts], 0).contiguous()
        return QLinear(fmt, w, w.shape[0], K, s, z).blocked()

    layers = []
    for i in range(cfg.num_hidden_layers):
        p = f"layers.{i}"
        gu = lin(f"{p}.mlp.gate_proj", f"{p}.mlp.up_proj")
        if gu.N % 32 == 0:
            gu = gu.interleaved()
        norms = [tensor(f"{p}.{n}.weight", (D if "self_attn" in n else H,), torch.bfloat16)
                 for n in _NORMS]
        layers.append(LayerWeights(
            input_norm=norms[0], post_norm=norms[1], q_norm=norms[2], k_norm=norms[3],
            qkv=lin(f"{p}.self_attn.q_proj", f"{p}.self_attn.k_proj", f"{p}.self_attn.v_proj"),
            o=lin(f"{p}.self_attn.o_proj"), gate_up=gu, down=lin(f"{p}.mlp.down_proj")))
    return Qwen3DecodeModel(cfg, embed=tensor("embed_tokens.weight", (cfg.vocab_size, H),
                                              torch.bfloat16),
                            layers=layers, norm=tensor("norm.weight", (H,), torch.bfloat16),
                            lm_head=lin("lm_head"), dtype=torch.bfloat16)


__all__ = ["save_quantized", "load_quantized"]
