"""Seeded synthetic checkpoints in GGUF tensor layouts.

Every tensor gets its own 64-bit seed derived from (model seed, tensor name),
so any tensor can be regenerated alone and both the HIP engine and the CPU
oracle read the very same bytes.  Layouts are GGUF's: Q8_0 rows of 34-byte
blocks (f16 d, 32 x i8), Q4_K rows of 144-byte super-blocks (f16 d, f16 dmin,
12 packed 6-bit scale/min bytes, 128 nibble bytes), Q4_0 (18 B), Q5_0 (22 B),
Q5_K (176 B), Q6_K (210 B) blocks, F16 / F32 little-endian
(src/gguf/dequant.rs:98-119, :203-230, :484-533).

Value distributions:
  F16 linear weights   N(0, 0.02)
  Q8_0 blocks          q ~ U[-127, 127] int8, d = f16(|N(0, 0.002)|)
  Q4_K super-blocks    random bytes, d and dmin = f16(U[2^-10, 2^-6])
  Q4_0 / Q5_0 blocks   random bytes, d = f16(+-U[2^-9, 2^-6])
  Q5_K super-blocks    random bytes, d and dmin = f16(U[2^-13, 2^-9])
  Q6_K super-blocks    random bytes (int8 scales), d = f16(U[2^-15, 2^-12])
  RMSNorm gains        N(1, 0.1)   (f32)
  q/k/v biases         N(0, 0.02)  (f32, Qwen2-style models only)
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np

from .config import ModelConfig

F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 6, 8, 12, 13, 14
BLK = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144),
       Q5_K: (256, 176), Q6_K: (256, 210)}


@dataclass
class Tensor:
    """One named tensor as a TensorStore hands it over (src/weights.rs:77-97)."""
    name: str
    ggml_type: int
    dims: tuple          # row-major: (rows, cols) or (n,)
    data: np.ndarray     # raw little-endian bytes, uint8

    @property
    def nbytes(self) -> int:
        return int(self.data.size)


def row_bytes(ggml_type: int, n: int) -> int:
    e, b = BLK[ggml_type]
    if n % e:
        raise ValueError(f"{n} values is not a whole number of blocks of {e}")
    return n // e * b


def tensor_seed(seed: int, name: str) -> int:
    h = hashlib.sha256(f"{seed}:{name}".encode()).digest()
    return int.from_bytes(h[:8], "little")


def rng_for(seed: int, name: str) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(tensor_seed(seed, name)))


def gen_f16(rng, n: int, std: float = 0.02) -> np.ndarray:
    return (rng.standard_normal(n, dtype=np.float32) * np.float32(std)).astype(np.float16).view(np.uint8)


def gen_f32(rng, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    v = rng.standard_normal(n, dtype=np.float32) * np.float32(std) + np.float32(mean)
    return v.astype(np.float32).view(np.uint8)


def gen_q8_0(rng, n: int, d_std: float = 0.002) -> np.ndarray:
    nb = n // 32
    d = np.abs(rng.standard_normal(nb, dtype=np.float32) * np.float32(d_std)).astype(np.float16)
    q = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8)
    out = np.empty((nb, 34), dtype=np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def gen_q4_k(rng, n: int) -> np.ndarray:
    nb = n // 256
    out = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    lo, hi = 2.0 ** -10, 2.0 ** -6
    d = rng.uniform(lo, hi, nb).astype(np.float16)
    dmin = rng.uniform(lo, hi, nb).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return out.reshape(-1)


def _f16_field(out, at, v):
    out[:, at:at + 2] = v.astype(np.float16).view(np.uint8).reshape(-1, 2)


def gen_blocks(rng, n: int, ggml_type: int) -> np.ndarray:
    """Q4_0 / Q5_0 / Q5_K / Q6_K: random bytes with the f16 fields set."""
    e, b = BLK[ggml_type]
    nb = n // e
    out = rng.integers(0, 256, size=(nb, b), dtype=np.uint8)
    if ggml_type in (Q4_0, Q5_0):
        d = rng.uniform(2.0 ** -9, 2.0 ** -6, nb) * rng.choice([-1.0, 1.0], nb)
        _f16_field(out, 0, d)
    elif ggml_type == Q5_K:
        _f16_field(out, 0, rng.uniform(2.0 ** -13, 2.0 ** -9, nb))
        _f16_field(out, 2, rng.uniform(2.0 ** -13, 2.0 ** -9, nb))
    else:  # Q6_K: d is the last field
        _f16_field(out, 208, rng.uniform(2.0 ** -15, 2.0 ** -12, nb))
    return out.reshape(-1)


def gen_weight(ggml_type: int, seed: int, name: str, rows: int, cols: int) -> Tensor:
    rng = rng_for(seed, name)
    n = rows * cols
    if ggml_type == F16:
        data = gen_f16(rng, n)
    elif ggml_type == Q8_0:
        data = gen_q8_0(rng, n)
    elif ggml_type == Q4_K:
        data = gen_q4_k(rng, n)
    elif ggml_type in (Q4_0, Q5_0, Q5_K, Q6_K):
        data = gen_blocks(rng, n, ggml_type)
    elif ggml_type == F32:
        data = gen_f32(rng, n, 0.0, 0.02)
    else:
        raise ValueError(f"unsupported synthetic type {ggml_type}")
    assert data.size == rows * row_bytes(ggml_type, cols)
    return Tensor(name, ggml_type, (rows, cols), data)


def gen_vec(seed: int, name: str, n: int, mean: float, std: float) -> Tensor:
    return Tensor(name, F32, (n,), gen_f32(rng_for(seed, name), n, mean, std))


def use_more_bits(i: int, n: int) -> bool:
    """llama.cpp's k-quant mix rule: the layers whose attn_v / ffn_down a
    *_K_M file stores in Q6_K (the first and last eighth, every third between)."""
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


def k_mix(base: int, cfg: ModelConfig):
    """Type chooser of a Q4_K_M / Q5_K_M-style file: `base` everywhere, Q6_K
    for v_proj / down_proj of the use_more_bits layers and for lm_head."""
    n = cfg.num_hidden_layers

    def choose(layer, proj):
        if proj == "lm_head":
            return Q6_K
        if proj in ("v_proj", "down_proj") and use_more_bits(layer, n):
            return Q6_K
        return base
    return choose


def synth_model(cfg: ModelConfig, weight_type: int, seed: int = 0, *, tied: bool = True,
                qkv_bias: bool = False, embed_type: int | None = None, type_of=None) -> list[Tensor]:
    """All tensors of a Llama/Qwen2-shaped checkpoint under HF names
    (the names src/model.rs:160-186 reads).  type_of(layer, proj) -> GGUF
    type overrides weight_type per matrix (proj "q_proj" .. "down_proj",
    "lm_head"; layer None for lm_head)."""
    h, I, hd = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim_()
    qd, kvd = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd
    et = weight_type if embed_type is None else embed_type

    def ty(layer, proj):
        return type_of(layer, proj) if type_of else weight_type
    out: list[Tensor] = []
    for L in range(cfg.num_hidden_layers):
        p = f"model.layers.{L}."
        out.append(gen_vec(seed, p + "input_layernorm.weight", h, 1.0, 0.1))
        out.append(gen_vec(seed, p + "post_attention_layernorm.weight", h, 1.0, 0.1))
        out.append(gen_weight(ty(L, "q_proj"), seed, p + "self_attn.q_proj.weight", qd, h))
        out.append(gen_weight(ty(L, "k_proj"), seed, p + "self_attn.k_proj.weight", kvd, h))
        out.append(gen_weight(ty(L, "v_proj"), seed, p + "self_attn.v_proj.weight", kvd, h))
        out.append(gen_weight(ty(L, "o_proj"), seed, p + "self_attn.o_proj.weight", h, qd))
        if qkv_bias:
            out.append(gen_vec(seed, p + "self_attn.q_proj.bias", qd, 0.0, 0.02))
            out.append(gen_vec(seed, p + "self_attn.k_proj.bias", kvd, 0.0, 0.02))
            out.append(gen_vec(seed, p + "self_attn.v_proj.bias", kvd, 0.0, 0.02))
        out.append(gen_weight(ty(L, "gate_proj"), seed, p + "mlp.gate_proj.weight", I, h))
        out.append(gen_weight(ty(L, "up_proj"), seed, p + "mlp.up_proj.weight", I, h))
        out.append(gen_weight(ty(L, "down_proj"), seed, p + "mlp.down_proj.weight", h, I))
    out.append(gen_weight(et, seed, "model.embed_tokens.weight", cfg.vocab_size, h))
    out.append(gen_vec(seed, "model.norm.weight", h, 1.0, 0.1))
    if not tied:
        out.append(gen_weight(ty(None, "lm_head"), seed, "lm_head.weight", cfg.vocab_size, h))
    return out


def synth_named(name: str, seed: int = 0, cfg: ModelConfig | None = None) -> tuple[ModelConfig, list[Tensor]]:
    """The benchmark workloads: 'smollm2-135m' (F16, tied), 'qwen2.5-0.5b-q8_0'
    (Q8_0 everywhere, tied, q/k/v biases), 'tinyllama-1.1b-q4_k' (Q4_K, untied).
    `cfg` overrides the shape (tests use shrunken copies)."""
    from .config import CONFIGS
    if name == "smollm2-135m":
        c = cfg or CONFIGS["smollm2-135m"]
        return c, synth_model(c, F16, seed, tied=True)
    if name == "qwen2.5-0.5b-q8_0":
        c = cfg or CONFIGS["qwen2.5-0.5b"]
        return c, synth_model(c, Q8_0, seed, tied=True, qkv_bias=True)
    if name == "tinyllama-1.1b-q4_k":
        c = cfg or CONFIGS["tinyllama-1.1b"]
        return c, synth_model(c, Q4_K, seed, tied=False)
    raise KeyError(name)
