"""Model shape and RoPE settings of a Llama-family decoder.

The fields of nimbus/config.py:10-35 (RopeScaling, ModelConfig), so a config
built for Nimbus builds the same model here. Nothing here reads checkpoints
or config files: the model is the caller the decode-step graphs replay, built
with random weights. The engine configuration (EngineConfig) is the
reference's scheduler and server settings and has no counterpart here.
"""

from __future__ import annotations

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


# Shapes used by the tests and the benchmark (random weights: no checkpoint
# is loaded anywhere in this build).
LLAMA3_8B = ModelConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_layers=32, num_heads=32,
                        num_kv_heads=8, head_dim=128, rms_norm_eps=1e-5, rope_theta=500000.0, max_position=8192,
                        rope_scaling=RopeScaling(8.0, 1.0, 4.0, 8192))
TINYLLAMA = ModelConfig(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_layers=22, num_heads=32,
                        num_kv_heads=4, head_dim=64, rms_norm_eps=1e-5, rope_theta=10000.0, max_position=2048)
