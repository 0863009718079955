"""The "hip" backend behind lokal's Engine / Session / Batcher seam
(src/engine.rs:13-71), over the C ABI of include/lokal_hip.h.

    engine = Engine.from_tensors(cfg, tensors)     # engine::create / create_metal_quant
    sess = engine.session(max_seq)                 # Engine::session
    logits = sess.forward(token, pos)              # Session::forward
    logits = sess.prefill(ids)                     # Session::prefill (token loop)
    ids = sess.decode_greedy(token, pos, n)        # generate.rs greedy loop, on device
    b = engine.batcher(n_slots, max_seq)           # Engine::batcher
    b.decode_step([BatchRow(token, pos, slot)])    # Batcher::decode_step

Errors surface as LokalHipError carrying the backend's one-line reason.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import Config, LokalHipError, Profile, Row, TensorDesc, check, lib
from .config import ModelConfig


def create(backend: str, cfg: ModelConfig, tensors, llama_permuted: bool = False,
           win: tuple[int, int] | None = None) -> "Engine":
    """engine::create by backend name (src/engine.rs:76-111); this build has one: "hip".
    win = (context window, attention sink) as src/main.rs:159-162 builds it;
    the hip backend refuses a window (lkhip_context_window)."""
    if backend != "hip":
        raise LokalHipError(-1, f'unknown backend "{backend}" — available: hip')
    check_window(win)
    return Engine.from_tensors(cfg, tensors, llama_permuted)


def check_window(win: tuple[int, int] | None) -> None:
    """The hip arm's --context-window contract (src/engine.rs:84-87 for the CPU arm)."""
    if win is not None:
        check(lib().lkhip_context_window(max(int(win[0]), 1), int(win[1])))


def _cfg_struct(cfg: ModelConfig) -> Config:
    return Config(cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers, cfg.num_attention_heads,
                  cfg.num_key_value_heads, cfg.vocab_size, cfg.head_dim, cfg.max_position_embeddings,
                  cfg.rms_norm_eps, cfg.rope_theta)


def _cfg_from_struct(c: Config) -> ModelConfig:
    return ModelConfig(c.hidden_size, c.intermediate_size, c.num_hidden_layers, c.num_attention_heads,
                       c.num_key_value_heads, c.vocab_size, c.rms_norm_eps, c.rope_theta,
                       c.max_position_embeddings, c.head_dim)


def gguf_config(path: str) -> tuple[ModelConfig, int, bool]:
    """Config, tensor count and llama-permutation flag of a GGUF file (no device needed)."""
    c, n, perm = Config(), C.c_size_t(), C.c_int()
    check(lib().lkhip_gguf_config(str(path).encode(), C.byref(c), C.byref(n), C.byref(perm)))
    return _cfg_from_struct(c), int(n.value), bool(perm.value)


def _f32p(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _u32p(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


@dataclass
class BatchRow:
    """One active request in a batched decode step (src/engine.rs:30-34)."""
    token: int
    pos: int
    slot: int


class Engine:
    name = "hip"

    def __init__(self, handle, cfg: ModelConfig):
        self._h = handle
        self.cfg = cfg

    @classmethod
    def from_tensors(cls, cfg: ModelConfig, tensors, llama_permuted: bool = False) -> "Engine":
        L = lib()
        arr = (TensorDesc * len(tensors))()
        keep = []
        for i, t in enumerate(tensors):
            data = np.ascontiguousarray(t.data).view(np.uint8).reshape(-1)
            keep.append(data)
            name = t.name.encode()
            keep.append(name)
            dims = (C.c_uint64 * 2)(*(list(t.dims) + [0])[:2])
            arr[i] = TensorDesc(name, t.ggml_type, len(t.dims), dims, data.ctypes.data, data.size)
        h = C.c_void_p()
        check(L.lkhip_engine_create_tensors(C.byref(_cfg_struct(cfg)), arr, len(tensors), int(llama_permuted),
                                            C.byref(h)))
        return cls(h, cfg)

    @classmethod
    def from_gguf(cls, path: str, win: tuple[int, int] | None = None) -> "Engine":
        """engine::create_metal_quant's counterpart (src/engine.rs:150-162):
        weights stay quantized; a context window is refused as check_window does."""
        check_window(win)
        h = C.c_void_p()
        check(lib().lkhip_engine_create_gguf(str(path).encode(), C.byref(h)))
        c = Config()
        check(lib().lkhip_engine_config(h, C.byref(c)))
        return cls(h, _cfg_from_struct(c))

    def config(self) -> ModelConfig:
        return self.cfg

    @property
    def matvec_bytes(self) -> float:
        """Algorithmic weight bytes one decode token streams through the matvecs."""
        return float(lib().lkhip_engine_matvec_bytes(self._h))

    def session(self, max_seq: int, kv_dtype: str = "f16") -> "Session":
        """kv_dtype "f16" (the GPU path's cache format) or "f32" (the CPU path's)."""
        kv = {"f16": _lib.LKHIP_F16, "f32": _lib.LKHIP_F32}.get(kv_dtype)
        if kv is None:
            raise LokalHipError(-1, f"session: the KV cache is f16 or f32, not {kv_dtype}")
        h = C.c_void_p()
        check(lib().lkhip_session_create_ex(self._h, max_seq, kv, C.byref(h)))
        return Session(self, h, max_seq)

    def batcher(self, n_slots: int, max_seq: int) -> "Batcher":
        h = C.c_void_p()
        check(lib().lkhip_batch_create(self._h, n_slots, max_seq, C.byref(h)))
        return Batcher(self, h, n_slots)

    def close(self):
        if self._h:
            lib().lkhip_engine_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class Session:
    def __init__(self, engine: Engine, handle, max_seq: int):
        self.engine = engine
        self._h = handle
        self.max_seq = max_seq
        self.vocab = engine.cfg.vocab_size

    def forward(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.vocab, dtype=np.float32)
        check(lib().lkhip_session_forward(self._h, int(token), int(pos), _f32p(out)))
        return out

    def prefill(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(self.vocab, dtype=np.float32)
        check(lib().lkhip_session_prefill(self._h, _u32p(ids), ids.size, _f32p(out)))
        return out

    def forward_batch(self, ids, pos0: int) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty((ids.size, self.vocab), dtype=np.float32)
        check(lib().lkhip_session_forward_batch(self._h, _u32p(ids), ids.size, pos0, _f32p(out)))
        return out

    def decode_greedy(self, token: int, pos: int, n_steps: int, want_logits: bool = False):
        ids = np.empty(max(n_steps, 1), dtype=np.uint32)
        logits = np.empty(self.vocab, dtype=np.float32) if want_logits else None
        check(lib().lkhip_session_decode_greedy(self._h, int(token), int(pos), int(n_steps), _u32p(ids),
                                                _f32p(logits) if want_logits else None))
        ids = ids[:n_steps]
        return (ids, logits) if want_logits else ids

    def read_kv(self, layer: int, pos: int, which_v: bool) -> np.ndarray:
        out = np.empty(self.engine.cfg.kv_dim(), dtype=np.float32)
        check(lib().lkhip_session_read_kv(self._h, layer, pos, int(which_v), _f32p(out)))
        return out

    def read_kv_rows(self, layer: int, pos0: int, n: int, which_v: bool) -> np.ndarray:
        """Cache rows pos0..pos0+n-1 of one layer, [n][kv_dim] f32."""
        out = np.empty((n, self.engine.cfg.kv_dim()), dtype=np.float32)
        check(lib().lkhip_session_read_kv_rows(self._h, layer, pos0, n, int(which_v), _f32p(out)))
        return out

    def set_profiling(self, on: bool) -> None:
        check(lib().lkhip_session_set_profiling(self._h, int(on)))

    def profile(self, reset: bool = False) -> dict:
        p = Profile()
        check(lib().lkhip_session_profile(self._h, C.byref(p), int(reset)))
        return p.as_dict()

    def set_trace(self, block: int) -> None:
        """Record the stage timeline of workgroup `block` (< 0: stop)."""
        check(lib().lkhip_session_set_trace(self._h, int(block)))

    def trace_ticks(self) -> np.ndarray:
        """Timestamps (100 MHz) of the last one-kernel step, [workgroup][2 + 6L + 1 + 24]:
        start, after the embedding, after each of the 6 stages of every layer, end,
        then 24 sub-step marks of layer 1."""
        n = int(lib().lkhip_session_trace_len(self._h))
        t = np.zeros(max(n, 1), dtype=np.uint64)
        check(lib().lkhip_session_trace(self._h, t.ctypes.data_as(C.POINTER(C.c_uint64)), n))
        L = self.engine.cfg.num_hidden_layers
        return t.reshape(-1, 2 + 6 * L + 1 + 24)

    def stage_times_us(self, block: int = 0) -> dict:
        """Stage durations (us) of the last one-kernel step, for one workgroup
        (the final norm + lm_head + argmax is a separate launch, not traced)."""
        L = self.engine.cfg.num_hidden_layers
        t = self.trace_ticks()[block][:2 + 6 * L + 1]
        us = np.diff(t.astype(np.float64)) / 100.0  # 100 MHz counter
        names = ["qkv", "attn", "merge", "o_proj", "gate_up", "down"]
        per = us[1:1 + 6 * L].reshape(L, 6)
        return {"embed": float(us[0]), **{n_: per[:, i].tolist() for i, n_ in enumerate(names)},
                "end": float(us[1 + 6 * L]), "total": float((t[-1] - t[0]) / 100.0)}

    def close(self):
        if self._h:
            lib().lkhip_session_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class Batcher:
    def __init__(self, engine: Engine, handle, n_slots: int):
        self.engine = engine
        self._h = handle
        self.n_slots = n_slots
        self.vocab = engine.cfg.vocab_size

    def prefill(self, slot: int, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(self.vocab, dtype=np.float32)
        check(lib().lkhip_batch_prefill(self._h, slot, _u32p(ids), ids.size, _f32p(out)))
        return out

    def decode_step(self, rows) -> list:
        arr = (Row * len(rows))(*[Row(r.token, r.slot, r.pos) for r in rows])
        out = np.empty((len(rows), self.vocab), dtype=np.float32)
        check(lib().lkhip_batch_decode_step(self._h, arr, len(rows), _f32p(out)))
        return [out[i] for i in range(len(rows))]

    def decode_greedy(self, rows, n_steps: int) -> np.ndarray:
        """Greedy decode of every row for n_steps steps on the device; returns
        the [n_steps, n_rows] argmax ids."""
        arr = (Row * len(rows))(*[Row(r.token, r.slot, r.pos) for r in rows])
        out = np.empty((n_steps, len(rows)), dtype=np.uint32)
        check(lib().lkhip_batch_decode_greedy(self._h, arr, len(rows), n_steps, _u32p(out)))
        return out

    def trace_ticks(self) -> np.ndarray:
        """Phase timestamps (100 MHz) of the last persistent multi-row step:
        start, after the embedding, then 5 per layer (LKHIP_BSTEP_TRACE=1)."""
        n = int(lib().lkhip_batch_trace_len(self._h))
        t = np.zeros(max(n, 1), dtype=np.uint64)
        check(lib().lkhip_batch_trace(self._h, t.ctypes.data_as(C.POINTER(C.c_uint64)), n))
        return t

    def read_kv_rows(self, slot: int, layer: int, pos0: int, n: int, which_v: bool) -> np.ndarray:
        """One slot's cache rows pos0..pos0+n-1 of one layer, [n][kv_dim] f32."""
        out = np.empty((n, self.engine.cfg.kv_dim()), dtype=np.float32)
        check(lib().lkhip_batch_read_kv_rows(self._h, slot, layer, pos0, n, int(which_v), _f32p(out)))
        return out

    def close(self):
        if self._h:
            lib().lkhip_batch_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


__all__ = ["Engine", "Session", "Batcher", "BatchRow", "create", "gguf_config", "LokalHipError", "_lib"]
