"""Writes GGUF v3 files from HF-named synthetic tensors, for the reader tests.

The layout follows the GGUF container as lokal reads it
(src/gguf/container.rs:162-261): magic, version, tensor and KV counts, the
metadata KVs, the tensor infos (name, n_dims, ne fastest-first, type,
offset), then the data section at the next alignment boundary with each
tensor at an aligned offset.  Names go HF -> GGUF by the inverse of
hf_name (src/gguf/arch.rs:229-270); for the llama architecture the q/k
rows are permuted the way the converter does, which load_f32 undoes
(src/gguf/dequant.rs:538-557, unpermute_llama_qk in src/gguf/arch.rs:274-286).
"""
from __future__ import annotations

import struct

import numpy as np

from lokal_amd import synth

_HF_TO_GGUF = {
    "input_layernorm": "attn_norm", "post_attention_layernorm": "ffn_norm",
    "self_attn.q_proj": "attn_q", "self_attn.k_proj": "attn_k", "self_attn.v_proj": "attn_v",
    "self_attn.o_proj": "attn_output", "mlp.gate_proj": "ffn_gate", "mlp.up_proj": "ffn_up",
    "mlp.down_proj": "ffn_down",
}


def gguf_name(hf: str) -> str:
    if hf == "model.embed_tokens.weight":
        return "token_embd.weight"
    if hf == "model.norm.weight":
        return "output_norm.weight"
    if hf == "lm_head.weight":
        return "output.weight"
    assert hf.startswith("model.layers.")
    rest = hf[len("model.layers."):]
    idx, tail = rest.split(".", 1)
    part, kind = tail.rsplit(".", 1)
    return f"blk.{idx}.{_HF_TO_GGUF[part]}.{kind}"


def permute_rows(t: synth.Tensor, n_heads: int, head_dim: int) -> np.ndarray:
    """The llama converter's row order for a q/k weight: within each head,
    GGUF row 2*i + s holds HF row s*(head_dim/2) + i."""
    rows, cols = t.dims
    rb = synth.row_bytes(t.ggml_type, cols)
    src = t.data.reshape(rows, rb)
    half = head_dim // 2
    out = np.empty_like(src)
    for h in range(n_heads):
        for i in range(half):
            for s in range(2):
                out[h * head_dim + 2 * i + s] = src[h * head_dim + s * half + i]
    return out.reshape(-1)


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, kind: str, value) -> bytes:
    out = _str(key)
    if kind == "u32":
        out += struct.pack("<II", 4, value)
    elif kind == "f32":
        out += struct.pack("<If", 6, value)
    elif kind == "str":
        out += struct.pack("<I", 8) + _str(value)
    elif kind == "strs":
        out += struct.pack("<IIQ", 9, 8, len(value)) + b"".join(_str(v) for v in value)
    else:
        raise ValueError(kind)
    return out


def write_gguf(path, cfg, tensors, arch: str = "qwen2", align: int = 32, with_tokens: bool = True,
               version: int = 3, extra_kv: list | None = None) -> None:
    hd = cfg.head_dim_()
    kvs = [_kv("general.architecture", "str", arch)]
    if align != 32:
        kvs.append(_kv("general.alignment", "u32", align))
    for key, kind, val in [
        ("embedding_length", "u32", cfg.hidden_size), ("feed_forward_length", "u32", cfg.intermediate_size),
        ("block_count", "u32", cfg.num_hidden_layers), ("attention.head_count", "u32", cfg.num_attention_heads),
        ("attention.head_count_kv", "u32", cfg.num_key_value_heads),
        ("attention.layer_norm_rms_epsilon", "f32", cfg.rms_norm_eps), ("rope.freq_base", "f32", cfg.rope_theta),
        ("context_length", "u32", cfg.max_position_embeddings),
    ]:
        kvs.append(_kv(f"{arch}.{key}", kind, val))
    if with_tokens:
        kvs.append(_kv("tokenizer.ggml.tokens", "strs", [f"t{i}" for i in range(cfg.vocab_size)]))
    for item in extra_kv or []:
        kvs.append(_kv(*item))
    infos, blobs, off = [], [], 0
    for t in tensors:
        data = t.data
        if arch == "llama" and t.name.endswith(("q_proj.weight", "k_proj.weight")):
            nh = cfg.num_attention_heads if "q_proj" in t.name else cfg.num_key_value_heads
            data = permute_rows(t, nh, hd)
        ne = list(reversed(t.dims))  # fastest first
        info = _str(gguf_name(t.name)) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        info += struct.pack("<IQ", t.ggml_type, off)
        infos.append(info)
        blobs.append((off, data.tobytes()))
        off = (off + data.nbytes + align - 1) // align * align
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)) + b"".join(kvs) + b"".join(infos)
    pad = (-len(head)) % align
    body = bytearray(off)
    for o, b in blobs:
        body[o:o + len(b)] = b
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad + bytes(body))
