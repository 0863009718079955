"""A CPU reading of a GGUF file the way lokal's CPU path loads one.

TEST INFRASTRUCTURE ONLY (the parity checker; the product reads GGUF in
lokal_amd/csrc/gguf.hip).  Restates, in Python over the file's bytes:
  - GgufFile::open (src/gguf/container.rs:162-261): magic, version 2/3,
    little-endian, the KV section (container.rs:79-125: every integer kind
    read as an integer, f32/f64 as float, arrays of strings / numbers), the
    tensor infos (name, n_dims, ne fastest-first, type, offset), the data
    section at the next general.alignment boundary (default 32), and dims
    reversed to row-major;
  - model_config (src/gguf/arch.rs:164-223): the per-architecture keys, the
    token list as the vocabulary, head_dim from attention.key_length;
  - hf_name (src/gguf/arch.rs:229-270): GGUF tensor names to HF names;
  - load_f32's permutation rule (src/gguf/dequant.rs:538-557): llama-arch
    files carry q/k rows in the converter's RoPE order, undone at load.
The tensors come back as raw bytes under HF names with the llama flag; the
oracle Model dequantizes them and undoes the permutation itself
(oracle_unpermute_llama_qk, src/gguf/arch.rs:274-286).  The container walk
(read_container) is pinned on the reference's own tiny_gguf fixture and its
asserted facts (src/gguf/testutil.rs:9-42, container.rs:474-513); of the
reader's refusals it restates the ones those tests assert (bad magic,
big-endian, version, truncation); the rest are tested against the product
directly (tests/test_gguf.py).
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

from lokal_amd.config import ModelConfig
from lokal_amd.synth import Tensor, row_bytes

# GGUF value kinds (container.rs:79-92); 9 = array
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}


class _Rd:
    def __init__(self, b: bytes):
        self.b, self.p = b, 0

    def take(self, n: int) -> bytes:
        if self.p + n > len(self.b):
            raise ValueError("GGUF header truncated")
        out = self.b[self.p:self.p + n]
        self.p += n
        return out

    def unpack(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def str(self) -> str:
        return self.take(self.unpack("<Q")).decode("utf-8")

    def value(self, ty: int):
        if ty == 8:
            return self.str()
        if ty == 9:
            et, n = self.unpack("<I"), self.unpack("<Q")
            return [self.value(et) for _ in range(n)]
        v = self.unpack(_SCALAR[ty])
        return bool(v) if ty == 7 else v


def hf_name(g: str) -> str | None:
    """src/gguf/arch.rs:229-270."""
    top = {"token_embd.weight": "model.embed_tokens.weight", "output_norm.weight": "model.norm.weight",
           "output.weight": "lm_head.weight"}
    if g in top:
        return top[g]
    if g == "rope_freqs.weight" or not g.startswith("blk."):
        return None
    idx, rest = g[len("blk."):].split(".", 1)
    mid, kind = rest.rsplit(".", 1)
    if kind not in ("weight", "bias"):
        return None
    m = {"attn_norm": "input_layernorm", "ffn_norm": "post_attention_layernorm", "attn_q": "self_attn.q_proj",
         "attn_k": "self_attn.k_proj", "attn_v": "self_attn.v_proj", "attn_output": "self_attn.o_proj",
         "attn_q_norm": "self_attn.q_norm", "attn_k_norm": "self_attn.k_norm", "ffn_gate": "mlp.gate_proj",
         "ffn_up": "mlp.up_proj", "ffn_down": "mlp.down_proj"}.get(mid, f"gguf.{mid}")
    return f"model.layers.{int(idx)}.{m}.{kind}"


def read_container(src) -> tuple[int, dict, list[tuple[str, tuple[int, ...], int, np.ndarray]]]:
    """GgufFile::open (src/gguf/container.rs:161-288) over a path or the
    file's bytes: (version, kv, [(name, dims row-major, ggml type, data
    bytes)]).  Raises ValueError with the reference's reasons for a bad magic,
    a big-endian file, a version other than 2/3, a header that ends early and
    a tensor whose data runs past the file."""
    b = bytes(src) if isinstance(src, (bytes, bytearray, memoryview)) else Path(src).read_bytes()
    rd = _Rd(b)
    if rd.take(4) != b"GGUF":
        raise ValueError("not a GGUF file (bad magic)")
    version = rd.unpack("<I")
    swapped = int.from_bytes(version.to_bytes(4, "little"), "big")
    if swapped in (2, 3):
        raise ValueError("big-endian GGUF files are not supported")
    if version not in (2, 3):
        raise ValueError(f"GGUF version {version} unsupported")
    n_tensors, n_kv = rd.unpack("<Q"), rd.unpack("<Q")
    kv = {}
    for _ in range(n_kv):
        key = rd.str()
        kv[key] = rd.value(rd.unpack("<I"))
    infos = []
    for _ in range(n_tensors):
        name = rd.str()
        nd = rd.unpack("<I")
        ne = [rd.unpack("<Q") for _ in range(nd)]
        ty, off = rd.unpack("<I"), rd.unpack("<Q")
        infos.append((name, ne, ty, off))
    align = int(kv.get("general.alignment", 32))
    data_start = (rd.p + align - 1) // align * align
    out = []
    for name, ne, ty, off in infos:
        nb = row_bytes(ty, int(np.prod(ne)))
        start = data_start + off
        if start + nb > len(b):
            raise ValueError(f"tensor {name}: {nb} bytes at data offset {off} run past the file")
        data = np.frombuffer(b, dtype=np.uint8, count=nb, offset=start).copy()
        out.append((name, tuple(reversed(ne)), ty, data))  # fastest-first -> row-major
    return version, kv, out


def read_gguf(path) -> tuple[ModelConfig, list[Tensor], bool]:
    """(config, tensors under HF names with the file's raw bytes, llama_permuted)."""
    _, kv, raw = read_container(path)
    arch = kv["general.architecture"]
    k = lambda s: kv[f"{arch}.{s}"]  # noqa: E731
    heads, hidden = int(k("attention.head_count")), int(k("embedding_length"))
    vocab = len(kv["tokenizer.ggml.tokens"]) if "tokenizer.ggml.tokens" in kv else int(k("vocab_size"))
    cfg = ModelConfig(hidden_size=hidden, intermediate_size=int(k("feed_forward_length")),
                      num_hidden_layers=int(k("block_count")), num_attention_heads=heads,
                      num_key_value_heads=int(k("attention.head_count_kv")), vocab_size=vocab,
                      rms_norm_eps=float(np.float32(k("attention.layer_norm_rms_epsilon"))),
                      rope_theta=float(np.float32(kv.get(f"{arch}.rope.freq_base", 10000.0))),
                      max_position_embeddings=int(kv.get(f"{arch}.context_length", 4096)),
                      head_dim=int(kv.get(f"{arch}.attention.key_length", 0)))
    tensors = []
    for name, dims, ty, data in raw:
        hf = hf_name(name)
        if hf is None:
            continue
        tensors.append(Tensor(hf, ty, dims, data))
    return cfg, tensors, arch == "llama"
