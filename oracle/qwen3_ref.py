"""CPU restatement of the reference's Qwen3 SDPA path — TEST INFRASTRUCTURE ONLY.

Follows acorninfer/models/qwen3.py (RMSNorm :50-60, RotaryEmbedding :68-84,
_rotate_half/_apply_rope :63-95, _repeat_kv :98-103, Qwen3Attention.forward
:119-152, Qwen3MLP :392-396, Qwen3Block.forward :407-410,
Qwen3ForCausalLM.forward :491-518) and the greedy loop
acorninfer/generate.py:55-110 (prefill of the whole prompt with a causal
mask, then one token per step attending to the whole cache; the chosen id
is appended before the EOS check).

Weights come as a reference-named state dict (`embed_tokens.weight`,
`layers.{i}.self_attn.q_proj.weight`, ...), the same dict the GPU model is
built from.

Pins (tests/test_oracle_model.py):
- HF transformers' Qwen3ForCausalLM (the reference's own golden oracle,
  tests/test_golden_m0.py) on the same weights: logits agree in fp32;
- prefill logits of the last position equal the step-by-step decode logits
  (the reference's bitwise invariant, tests/test_forward_decode.py:32-48);
- each op it calls is pinned in tests/test_oracle_ops.py.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle.ops_ref import inv_freq_ref, rmsnorm_ref


class Qwen3Ref:
    """Functional Qwen3 over a state dict; KV cache = per-layer contiguous tensors."""

    def __init__(self, cfg, sd: dict[str, torch.Tensor], dtype: torch.dtype = torch.float32,
                 weight_dtype: torch.dtype | None = None):
        """dtype: activations (every op's output rounded to it, as the
        reference's torch path rounds in that dtype). weight_dtype: the
        projection and lm_head weights (default dtype); fp32 with bf16
        activations keeps dequantised int4 / int8 weights exact while every
        activation is rounded as in the bf16 path: F.linear then runs on the
        activation widened to fp32 and its output is rounded to dtype."""
        self.cfg = cfg
        self.dtype = dtype
        wdt = dtype if weight_dtype is None else weight_dtype
        self.w = {k: v.to(device="cpu", dtype=wdt if self._is_projection(k) else dtype)
                  for k, v in sd.items()}
        self.inv_freq = inv_freq_ref(cfg.head_dim, cfg.rope_theta)

    @staticmethod
    def _is_projection(name: str) -> bool:
        return name == "lm_head.weight" or name.endswith("_proj.weight")

    def new_cache(self) -> list[list[torch.Tensor | None]]:
        return [[None, None] for _ in range(self.cfg.num_hidden_layers)]

    def _rope(self, positions: torch.Tensor):
        """RotaryEmbedding.forward (qwen3.py:76-84): fp32 angles, cos/sin cast to dtype."""
        freqs = torch.outer(positions.float(), self.inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(self.dtype), emb.sin().to(self.dtype)

    @staticmethod
    def _rotate_half(x):
        x1, x2 = x.chunk(2, dim=-1)
        return torch.cat((-x2, x1), dim=-1)

    def _linear(self, x, name):
        w = self.w[name + ".weight"]
        if w.dtype == x.dtype:
            return F.linear(x, w)
        return F.linear(x.to(w.dtype), w).to(self.dtype)

    def _attention(self, i, h, cos, sin, cache):
        cfg = self.cfg
        b, s, _ = h.shape
        nq, nkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        p = f"layers.{i}.self_attn."
        q = self._linear(h, p + "q_proj").view(b, s, nq, D).transpose(1, 2)
        k = self._linear(h, p + "k_proj").view(b, s, nkv, D).transpose(1, 2)
        v = self._linear(h, p + "v_proj").view(b, s, nkv, D).transpose(1, 2)
        q = rmsnorm_ref(q, self.w[p + "q_norm.weight"], cfg.rms_norm_eps)
        k = rmsnorm_ref(k, self.w[p + "k_norm.weight"], cfg.rms_norm_eps)
        c, sn = cos[None, None], sin[None, None]
        q = q * c + self._rotate_half(q) * sn
        k = k * c + self._rotate_half(k) * sn
        if cache is not None:
            kc, vc = cache[i]
            k = k if kc is None else torch.cat([kc, k], dim=2)
            v = v if vc is None else torch.cat([vc, v], dim=2)
            cache[i] = [k, v]
        past = k.shape[2] - s
        rep = nq // nkv
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
        if past == 0:
            out = F.scaled_dot_product_attention(q, k, v, is_causal=(s > 1))
        elif s == 1:
            out = F.scaled_dot_product_attention(q, k, v)
        else:
            qp = torch.arange(past, past + s)
            kp = torch.arange(past + s)
            out = F.scaled_dot_product_attention(q, k, v, attn_mask=qp[:, None] >= kp[None, :])
        out = out.transpose(1, 2).reshape(b, s, -1)
        return self._linear(out, p + "o_proj")

    def _mlp(self, i, x):
        p = f"layers.{i}.mlp."
        return self._linear(F.silu(self._linear(x, p + "gate_proj")) * self._linear(x, p + "up_proj"),
                            p + "down_proj")

    @torch.no_grad()
    def forward(self, ids: torch.Tensor, cache=None, num_logits_to_keep: int | None = None
                ) -> torch.Tensor:
        """ids [b, s] -> fp32 logits [b, s', vocab] (qwen3.py:491-518)."""
        cfg = self.cfg
        s = ids.shape[1]
        past = 0 if cache is None or cache[0][0] is None else cache[0][0].shape[2]
        cos, sin = self._rope(torch.arange(past, past + s))
        h = self.w["embed_tokens.weight"][ids]
        eps = cfg.rms_norm_eps
        for i in range(cfg.num_hidden_layers):
            p = f"layers.{i}."
            h = h + self._attention(i, rmsnorm_ref(h, self.w[p + "input_layernorm.weight"], eps),
                                    cos, sin, cache)
            h = h + self._mlp(i, rmsnorm_ref(h, self.w[p + "post_attention_layernorm.weight"], eps))
        h = rmsnorm_ref(h, self.w["norm.weight"], eps)
        if num_logits_to_keep is not None:
            h = h[:, -num_logits_to_keep:, :]
        return self._linear(h, "lm_head").float()

    @torch.no_grad()
    def decode_ragged(self, ids: list[int], caches: list) -> torch.Tensor:
        """One decode step of B sequences whose caches hold different
        lengths (Qwen3ForCausalLM.forward_decode, qwen3.py:520-595, batched
        over per-sequence caches): the projections run on all B rows at once,
        RoPE uses each row's own position (its cache length) and attention
        reads each row's own cache, as `forward([[id]], cache_b)` does for one
        sequence. Returns fp32 logits [B, vocab]; each cache grows by one.
        Pinned against B separate `forward` calls (tests/test_oracle_model.py)."""
        cfg = self.cfg
        B = len(ids)
        nq, nkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        eps = cfg.rms_norm_eps
        pos = [0 if c[0][0] is None else c[0][0].shape[2] for c in caches]
        rope = [self._rope(torch.tensor([p])) for p in pos]
        h = self.w["embed_tokens.weight"][torch.tensor(ids)][:, None]          # [B, 1, H]
        for i in range(cfg.num_hidden_layers):
            p = f"layers.{i}."
            a = f"layers.{i}.self_attn."
            x = rmsnorm_ref(h, self.w[p + "input_layernorm.weight"], eps)
            q = self._linear(x, a + "q_proj").view(B, 1, nq, D).transpose(1, 2)
            k = self._linear(x, a + "k_proj").view(B, 1, nkv, D).transpose(1, 2)
            v = self._linear(x, a + "v_proj").view(B, 1, nkv, D).transpose(1, 2)
            q = rmsnorm_ref(q, self.w[a + "q_norm.weight"], eps)
            k = rmsnorm_ref(k, self.w[a + "k_norm.weight"], eps)
            outs = []
            for b in range(B):
                c, sn = rope[b][0][None, None], rope[b][1][None, None]
                qb = q[b:b + 1] * c + self._rotate_half(q[b:b + 1]) * sn
                kb = k[b:b + 1] * c + self._rotate_half(k[b:b + 1]) * sn
                kc, vc = caches[b][i]
                kb = kb if kc is None else torch.cat([kc, kb], dim=2)
                vb = v[b:b + 1] if vc is None else torch.cat([vc, v[b:b + 1]], dim=2)
                caches[b][i] = [kb, vb]
                rep = nq // nkv
                outs.append(F.scaled_dot_product_attention(
                    qb, kb.repeat_interleave(rep, dim=1), vb.repeat_interleave(rep, dim=1)))
            attn = torch.cat(outs).transpose(1, 2).reshape(B, 1, -1)
            h = h + self._linear(attn, a + "o_proj")
            h = h + self._mlp(i, rmsnorm_ref(h, self.w[p + "post_attention_layernorm.weight"], eps))
        h = rmsnorm_ref(h, self.w["norm.weight"], eps)
        return self._linear(h, "lm_head").float()[:, 0]


@torch.no_grad()
def generate_greedy(model: Qwen3Ref, prompt: list[int], max_new_tokens: int, *,
                    eos_ids=frozenset(), forced: list[int] | None = None
                    ) -> tuple[list[int], list[torch.Tensor]]:
    """generate.py:55-110 with greedy choice. Returns (generated ids, the fp32
    logits each choice was made from). With `forced`, the fed-back ids are
    `forced[t]` instead of the argmax (forced-token stream)."""
    cache = model.new_cache()
    last = model.forward(torch.tensor([prompt]), cache, num_logits_to_keep=1)[0, -1]
    out, logits = [], []
    for t in range(max_new_tokens):
        logits.append(last.clone())
        nxt = int(last.argmax()) if forced is None else int(forced[t])
        out.append(nxt)
        if nxt in eos_ids:
            break
        last = model.forward(torch.tensor([[nxt]]), cache)[0, -1]
    return out, logits
