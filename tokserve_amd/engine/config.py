"""Llama architecture configuration (tokserve/reference/llama/config.py)."""

from __future__ import annotations

from dataclasses import dataclass

__all__ = ["LlamaConfig", "tinyllama_1_1b"]


@dataclass(frozen=True)
class LlamaConfig:
    """Architectural sizes of a Llama-style decoder, validated on construction."""

    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    max_position_embeddings: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10_000.0

    def __post_init__(self) -> None:
        for name in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
                     "num_attention_heads", "num_key_value_heads", "max_position_embeddings"):
            if getattr(self, name) < 1:
                raise ValueError(f"{name} must be positive")
        if self.hidden_size % self.num_attention_heads != 0:
            raise ValueError("hidden_size must be divisible by num_attention_heads")
        if self.num_attention_heads % self.num_key_value_heads != 0:
            raise ValueError("num_attention_heads must be divisible by num_key_value_heads")
        if self.rms_norm_eps <= 0.0:
            raise ValueError("rms_norm_eps must be positive")
        if self.rope_theta <= 0.0:
            raise ValueError("rope_theta must be positive")

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def num_key_value_groups(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads


def tinyllama_1_1b(max_position_embeddings: int = 2048) -> LlamaConfig:
    """TinyLlama-1.1B: 22 layers, hidden 2048, 32 query / 4 KV heads of 64, MLP 5632,
    vocabulary 32000, eps 1e-5, theta 1e4."""

    return LlamaConfig(vocab_size=32_000, hidden_size=2048, intermediate_size=5632,
                       num_hidden_layers=22, num_attention_heads=32, num_key_value_heads=4,
                       max_position_embeddings=max_position_embeddings, rms_norm_eps=1e-5,
                       rope_theta=10_000.0)
