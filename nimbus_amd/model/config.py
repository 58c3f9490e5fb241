"""Model shape and RoPE settings of a Llama-family decoder.

Field for field nimbus/config.py:10-81 (RopeScaling, ModelConfig with
from_hf / from_dir / kv_bytes_per_token), so a config built for Nimbus
builds the same model here. The engine configuration (EngineConfig) is the
reference's scheduler and server settings and has no counterpart here.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass


@dataclass(frozen=True)
class RopeScaling:
    """Llama 3.1 frequency scaling ("rope_type": "llama3")."""

    factor: float
    low_freq_factor: float
    high_freq_factor: float
    original_max_position: int


@dataclass(frozen=True)
class ModelConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    max_position: int
    tie_word_embeddings: bool = False
    rope_scaling: RopeScaling | None = None
    bos_token_id: int | None = None
    eos_token_ids: tuple[int, ...] = ()

    @classmethod
    def from_hf(cls, d: dict) -> "ModelConfig":
        """From a HuggingFace Llama config.json dict (nimbus/config.py:37-72):
        RoPE settings either at the top level or under "rope_parameters"."""
        rope = d.get("rope_parameters") or {}
        theta = d.get("rope_theta", rope.get("rope_theta", 10000.0))
        scaling_d = d.get("rope_scaling") or (rope if rope.get("rope_type") == "llama3" else None)
        scaling = None
        if scaling_d and scaling_d.get("rope_type", scaling_d.get("type")) == "llama3":
            scaling = RopeScaling(
                factor=scaling_d["factor"], low_freq_factor=scaling_d["low_freq_factor"],
                high_freq_factor=scaling_d["high_freq_factor"],
                original_max_position=scaling_d["original_max_position_embeddings"])
        heads = d["num_attention_heads"]
        eos = d.get("eos_token_id")
        eos_ids = tuple(eos) if isinstance(eos, list) else ((eos,) if eos is not None else ())
        return cls(
            vocab_size=d["vocab_size"], hidden_size=d["hidden_size"], intermediate_size=d["intermediate_size"],
            num_layers=d["num_hidden_layers"], num_heads=heads, num_kv_heads=d.get("num_key_value_heads", heads),
            head_dim=d.get("head_dim") or d["hidden_size"] // heads, rms_norm_eps=d.get("rms_norm_eps", 1e-6),
            rope_theta=float(theta), max_position=d.get("max_position_embeddings", 2048),
            tie_word_embeddings=d.get("tie_word_embeddings", False), rope_scaling=scaling,
            bos_token_id=d.get("bos_token_id"), eos_token_ids=eos_ids)

    @classmethod
    def from_dir(cls, path: str) -> "ModelConfig":
        with open(os.path.join(path, "config.json")) as f:
            return cls.from_hf(json.load(f))

    def kv_bytes_per_token(self, dtype_bytes: int = 2) -> int:
        return self.num_layers * 2 * self.num_kv_heads * self.head_dim * dtype_bytes


# Shapes used by the tests and the benchmark (random weights: no checkpoint
# is loaded anywhere in this build).
LLAMA3_8B = ModelConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_layers=32, num_heads=32,
                        num_kv_heads=8, head_dim=128, rms_norm_eps=1e-5, rope_theta=500000.0, max_position=8192,
                        rope_scaling=RopeScaling(8.0, 1.0, 4.0, 8192))
TINYLLAMA = ModelConfig(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_layers=22, num_heads=32,
                        num_kv_heads=4, head_dim=64, rms_norm_eps=1e-5, rope_theta=10000.0, max_position=2048)
