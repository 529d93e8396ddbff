"""Model shapes the decode path reads (acorninfer/config.py:17-66).

Only the fields the Qwen3 decode step needs. `tiny()` is the reference's unit
test shape (config.py:51-66); `qwen3_0_6b()` and `qwen3_8b()` are the shapes
the benchmark configurations name.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

QWEN3_EOS_IDS: frozenset[int] = frozenset({151643, 151645})


@dataclass(frozen=True)
class Qwen3Config:
    num_hidden_layers: int
    hidden_size: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    rms_norm_eps: float
    rope_theta: float
    vocab_size: int
    tie_word_embeddings: bool = False
    bos_token_id: int = 151643
    eos_token_id: tuple[int, ...] = (151645,)

    @classmethod
    def from_json(cls, path: Path | str) -> "Qwen3Config":
        raw = json.loads(Path(path).read_text())
        eos = raw["eos_token_id"]
        return cls(
            num_hidden_layers=raw["num_hidden_layers"],
            hidden_size=raw["hidden_size"],
            num_attention_heads=raw["num_attention_heads"],
            num_key_value_heads=raw["num_key_value_heads"],
            head_dim=raw["head_dim"],
            intermediate_size=raw["intermediate_size"],
            rms_norm_eps=raw["rms_norm_eps"],
            rope_theta=raw["rope_theta"],
            vocab_size=raw["vocab_size"],
            tie_word_embeddings=raw.get("tie_word_embeddings", False),
            bos_token_id=raw.get("bos_token_id", 151643),
            eos_token_id=tuple(eos if isinstance(eos, list) else [eos]),
        )

    @classmethod
    def tiny(cls) -> "Qwen3Config":
        """2 layers, hidden 64, 4/2 heads, head_dim 16, vocab 256."""
        return cls(num_hidden_layers=2, hidden_size=64, num_attention_heads=4,
                   num_key_value_heads=2, head_dim=16, intermediate_size=128,
                   rms_norm_eps=1e-6, rope_theta=10_000.0, vocab_size=256,
                   bos_token_id=0, eos_token_id=(1,))

    @classmethod
    def qwen3_0_6b(cls) -> "Qwen3Config":
        """Qwen3-0.6B shape: 28 layers, hidden 1024, 16/8 heads, intermediate 3072."""
        return cls(num_hidden_layers=28, hidden_size=1024, num_attention_heads=16,
                   num_key_value_heads=8, head_dim=128, intermediate_size=3072,
                   rms_norm_eps=1e-6, rope_theta=1_000_000.0, vocab_size=151936)

    @classmethod
    def qwen3_8b(cls) -> "Qwen3Config":
        """Qwen3-8B shape: 36 layers, hidden 4096, 32/8 heads, intermediate 12288."""
        return cls(num_hidden_layers=36, hidden_size=4096, num_attention_heads=32,
                   num_key_value_heads=8, head_dim=128, intermediate_size=12288,
                   rms_norm_eps=1e-6, rope_theta=1_000_000.0, vocab_size=151936)

    def with_layers(self, n: int) -> "Qwen3Config":
        d = dict(self.__dict__)
        d["num_hidden_layers"] = n
        return Qwen3Config(**d)
