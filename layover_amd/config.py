"""Model shapes the KV data path depends on (mirrors layover/config.py:12-102 of the reference,
restricted to what sizes the pool and the records)."""

from __future__ import annotations

from dataclasses import dataclass, replace

DTYPE_BYTES = {"fp8": 1, "bf16": 2, "fp16": 2, "fp32": 4}


@dataclass(frozen=True)
class ModelConfig:
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int

    @classmethod
    def qwen3_4b(cls) -> "ModelConfig":
        """Qwen3-4B: 36 layers, 32 query heads over 8 KV heads, head_dim 128."""
        return cls(num_hidden_layers=36, num_attention_heads=32, num_key_value_heads=8, head_dim=128)

    @classmethod
    def micro(cls, **overrides) -> "ModelConfig":
        """The reference's test shape (config.py:70-89): head_dim 24, 2 layers, GQA 2."""
        return replace(cls(num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=24), **overrides)

    @property
    def kv_groups(self) -> int:
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("num_attention_heads must be divisible by num_key_value_heads")
        return self.num_attention_heads // self.num_key_value_heads

    def kv_bytes_per_token(self, dtype: str = "bf16") -> int:
        return self.num_hidden_layers * 2 * self.num_key_value_heads * self.head_dim * DTYPE_BYTES[dtype]
