"""Model hyper-parameters (ModelConfig, src/config.rs:10-30) and the synthetic
configurations this backend is measured on."""
from __future__ import annotations

from dataclasses import dataclass, replace


@dataclass(frozen=True)
class ModelConfig:
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    vocab_size: int
    rms_norm_eps: float
    rope_theta: float = 10000.0          # default_rope_theta, src/config.rs:50-52
    max_position_embeddings: int = 4096  # default_max_pos, src/config.rs:54-56
    head_dim: int = 0                    # 0 = hidden / heads (config.rs:92-95)

    def head_dim_(self) -> int:
        return self.head_dim or self.hidden_size // self.num_attention_heads

    def kv_dim(self) -> int:
        return self.num_key_value_heads * self.head_dim_()

    def q_dim(self) -> int:
        return self.num_attention_heads * self.head_dim_()

    def with_(self, **kw) -> "ModelConfig":
        return replace(self, **kw)


# Shapes of the three model families the benchmarks name.
SMOLLM2_135M = ModelConfig(hidden_size=576, intermediate_size=1536, num_hidden_layers=30, num_attention_heads=9,
                           num_key_value_heads=3, vocab_size=49152, rms_norm_eps=1e-5, rope_theta=10000.0,
                           max_position_embeddings=8192)
QWEN25_05B = ModelConfig(hidden_size=896, intermediate_size=4864, num_hidden_layers=24, num_attention_heads=14,
                         num_key_value_heads=2, vocab_size=151936, rms_norm_eps=1e-6, rope_theta=1000000.0,
                         max_position_embeddings=32768)
TINYLLAMA_11B = ModelConfig(hidden_size=2048, intermediate_size=5632, num_hidden_layers=22, num_attention_heads=32,
                            num_key_value_heads=4, vocab_size=32000, rms_norm_eps=1e-5, rope_theta=10000.0,
                            max_position_embeddings=2048)

CONFIGS = {
    "smollm2-135m": SMOLLM2_135M,
    "qwen2.5-0.5b": QWEN25_05B,
    "tinyllama-1.1b": TINYLLAMA_11B,
}
