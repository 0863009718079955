"""ctypes bindings of the CPU oracle (lokal_oracle.c).

TEST INFRASTRUCTURE ONLY: a restatement of lokal's Rust CPU path
(src/math.rs, src/model.rs, src/gguf/dequant.rs, src/sampler.rs) used by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker.  The product (lokal_amd) never imports it.

Pinned by tests/test_oracle.py against every hand vector the reference's own
tests hold (dequant.rs:568-780, math.rs:77-107, sampler.rs:82-86,
arch.rs:807-824), closed forms in float64 and invariants.  The libm boundary
(expf / powf / sinf / cosf as Apple's libm computes them) is parity unpinned:
no reference test fixes those bits; glibc's are used.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liblokal_oracle.so"
_lib = None

F32P = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
U8P = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")


class OracleConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32), ("intermediate", C.c_uint32), ("n_layers", C.c_uint32),
        ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("vocab", C.c_uint32),
        ("head_dim", C.c_uint32), ("rms_eps", C.c_float), ("rope_theta", C.c_float),
    ]


def select(variant: str) -> None:
    """Chooses the build this process loads, before its first use: "o2" (the
    parity build every test checks against, the default) or "o3" (the same
    source at -O3 -mavx2, bit-identical results, timed as the CPU baseline)."""
    global _LIB_PATH
    path = {"o2": _HERE / "liblokal_oracle.so", "o3": _HERE / "liblokal_oracle_o3.so"}[variant]
    if _lib is not None and path != _LIB_PATH:
        raise RuntimeError(f"oracle: {_LIB_PATH.name} is already loaded in this process")
    _LIB_PATH = path


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            from . import build as _b
            _b.build()
        L = C.CDLL(str(_LIB_PATH))
        L.oracle_f16_to_f32.argtypes = [C.c_uint16]
        L.oracle_f16_to_f32.restype = C.c_float
        L.oracle_blk_elems.argtypes = [C.c_uint32]
        L.oracle_blk_bytes.argtypes = [C.c_uint32]
        L.oracle_row_bytes.argtypes = [C.c_uint32, C.c_size_t]
        L.oracle_row_bytes.restype = C.c_size_t
        L.oracle_scale_min_k4.argtypes = [C.c_int, U8P, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]
        L.oracle_dequant_row.argtypes = [C.c_uint32, U8P, C.c_size_t, F32P, C.c_size_t]
        L.oracle_unpermute_llama_qk.argtypes = [F32P, C.c_size_t, C.c_size_t, C.c_size_t]
        L.oracle_dot.argtypes = [F32P, F32P, C.c_size_t]
        L.oracle_dot.restype = C.c_float
        L.oracle_matvec.argtypes = [F32P, F32P, C.c_size_t, C.c_size_t, F32P]
        L.oracle_rmsnorm.argtypes = [F32P, F32P, C.c_size_t, C.c_float, F32P]
        L.oracle_softmax.argtypes = [F32P, C.c_size_t]
        L.oracle_silu.argtypes = [C.c_float]
        L.oracle_silu.restype = C.c_float
        L.oracle_swiglu.argtypes = [F32P, F32P, C.c_size_t, F32P]
        L.oracle_rope.argtypes = [F32P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_float]
        L.oracle_attention.argtypes = [F32P, F32P, F32P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t,
                                       C.c_size_t, F32P]
        L.oracle_argmax.argtypes = [F32P, C.c_size_t]
        L.oracle_argmax.restype = C.c_uint32
        L.oracle_set_threads.argtypes = [C.c_int]
        L.oracle_get_threads.restype = C.c_int
        L.oracle_model_new.argtypes = [C.POINTER(OracleConfig)]
        L.oracle_model_new.restype = C.c_void_p
        L.oracle_model_set.argtypes = [C.c_void_p, C.c_char_p, C.c_uint32, U8P, C.c_size_t, C.c_size_t,
                                       C.c_size_t, C.c_int]
        L.oracle_model_set_f32.argtypes = [C.c_void_p, C.c_char_p, F32P, C.c_size_t, C.c_size_t]
        L.oracle_model_finalize.argtypes = [C.c_void_p]
        L.oracle_model_free.argtypes = [C.c_void_p]
        L.oracle_session_new.argtypes = [C.c_void_p, C.c_size_t]
        L.oracle_session_new.restype = C.c_void_p
        L.oracle_session_free.argtypes = [C.c_void_p]
        L.oracle_forward.argtypes = [C.c_void_p, C.c_uint32, C.c_size_t, F32P]
        L.oracle_session_hidden.argtypes = [C.c_void_p, F32P]
        L.oracle_session_kv.argtypes = [C.c_void_p, C.c_uint32, C.c_size_t, C.c_int, F32P]
        L.oracle_session_set_kv_f16.argtypes = [C.c_void_p, C.c_int]
        L.oracle_session_load_kv.argtypes = [C.c_void_p, C.c_uint32, C.c_size_t, C.c_size_t, C.c_int, F32P]
        L.oracle_f32_to_f16.argtypes = [C.c_float]
        L.oracle_f32_to_f16.restype = C.c_uint16
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def f16_to_f32(bits: int) -> float:
    return float(lib().oracle_f16_to_f32(bits))


def f32_to_f16(x: float) -> int:
    return int(lib().oracle_f32_to_f16(x))


def blk_elems(t: int) -> int:
    return lib().oracle_blk_elems(t)


def blk_bytes(t: int) -> int:
    return lib().oracle_blk_bytes(t)


def row_bytes(t: int, n: int) -> int:
    return lib().oracle_row_bytes(t, n)


def scale_min_k4(j: int, q) -> tuple[int, int]:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    sc, m = C.c_uint8(), C.c_uint8()
    lib().oracle_scale_min_k4(j, q, C.byref(sc), C.byref(m))
    return sc.value, m.value


def dequant_row(ggml_type: int, data, n: int) -> np.ndarray:
    """dequant_row_ref (src/gguf/dequant.rs:191-535)."""
    data = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8) if isinstance(data, (bytes, bytearray))
                                else data, dtype=np.uint8).reshape(-1)
    out = np.empty(n, dtype=np.float32)
    rc = lib().oracle_dequant_row(ggml_type, data, data.size, out, n)
    if rc != 0:
        raise ValueError(f"src/out size mismatch for type {ggml_type}")
    return out


def unpermute_llama_qk(w: np.ndarray, head_dim: int) -> np.ndarray:
    w = _f32(w).copy()
    rows, cols = w.shape
    lib().oracle_unpermute_llama_qk(w.reshape(-1), rows, cols, head_dim)
    return w


def dot(a, b) -> float:
    a, b = _f32(a), _f32(b)
    return float(lib().oracle_dot(a, b, a.size))


def matvec(w, x) -> np.ndarray:
    w, x = _f32(w), _f32(x)
    out_dim, in_dim = w.shape
    y = np.empty(out_dim, dtype=np.float32)
    lib().oracle_matvec(w.reshape(-1), x, out_dim, in_dim, y)
    return y


def rmsnorm(x, w, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    y = np.empty_like(x)
    lib().oracle_rmsnorm(x, w, x.size, eps, y)
    return y


def softmax(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().oracle_softmax(x, x.size)
    return x


def silu(x: float) -> float:
    return float(lib().oracle_silu(x))


def swiglu(g, u) -> np.ndarray:
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    lib().oracle_swiglu(g, u, g.size, out)
    return out


def rope(x, pos: int, head_dim: int, theta: float) -> np.ndarray:
    x = _f32(x).copy()
    lib().oracle_rope(x, x.size, pos, head_dim, theta)
    return x


def attention(q, k_cache, v_cache, pos: int, n_heads: int, n_kv_heads: int, head_dim: int) -> np.ndarray:
    """model::attention over cached rows 0..=pos; caches are [max_seq][kv_dim]."""
    q, k, v = _f32(q), _f32(k_cache), _f32(v_cache)
    kvd = n_kv_heads * head_dim
    out = np.empty(n_heads * head_dim, dtype=np.float32)
    lib().oracle_attention(q, k.reshape(-1), v.reshape(-1), pos, n_heads, n_kv_heads, head_dim, kvd, out)
    return out


def argmax(x) -> int:
    x = _f32(x)
    return int(lib().oracle_argmax(x, x.size))


def set_threads(n: int) -> None:
    lib().oracle_set_threads(n)


def get_threads() -> int:
    return int(lib().oracle_get_threads())


class Model:
    """Model::from_store + forward (src/model.rs:140-262) on dequantized f32."""

    def __init__(self, cfg, tensors, llama_permuted: bool = False):
        L = lib()
        oc = OracleConfig(cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers, cfg.num_attention_heads,
                          cfg.num_key_value_heads, cfg.vocab_size, cfg.head_dim or 0, cfg.rms_norm_eps,
                          cfg.rope_theta)
        self.cfg = cfg
        self._sessions = []
        self._m = L.oracle_model_new(C.byref(oc))
        for t in tensors:
            data = np.ascontiguousarray(np.frombuffer(t.data, dtype=np.uint8) if not isinstance(t.data, np.ndarray)
                                        else t.data.view(np.uint8).reshape(-1))
            rows, cols = (t.dims if len(t.dims) == 2 else (1, t.dims[0]))
            unperm = int(llama_permuted and (t.name.endswith("q_proj.weight") or t.name.endswith("k_proj.weight")))
            rc = L.oracle_model_set(self._m, t.name.encode(), t.ggml_type, data, data.size, rows, cols, unperm)
            if rc != 0:
                raise ValueError(f"oracle: cannot take tensor {t.name}")
        rc = L.oracle_model_finalize(self._m)
        if rc != 0:
            raise ValueError(f"oracle: model incomplete (code {rc})")

    def session(self, max_seq: int, kv_f16: bool = False) -> "Session":
        """kv_f16: test-only variant storing K/V through f16 (the GPU cache format)."""
        s = Session(self, max_seq)
        if kv_f16:
            lib().oracle_session_set_kv_f16(s._s, 1)
        self._sessions.append(s)
        return s

    def close(self):
        for s in self._sessions:
            s.close()
        self._sessions = []
        if self._m:
            lib().oracle_model_free(self._m)
            self._m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Session:
    def __init__(self, model: Model, max_seq: int):
        self.model = model
        self.max_seq = max_seq
        self._s = lib().oracle_session_new(model._m, max_seq)

    def forward(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.model.cfg.vocab_size, dtype=np.float32)
        if lib().oracle_forward(self._s, token, pos, out) != 0:
            raise ValueError("oracle forward: token or position out of range")
        return out

    def prefill(self, ids) -> np.ndarray:
        logits = None
        for pos, t in enumerate(ids):
            logits = self.forward(int(t), pos)
        return logits

    def kv(self, layer: int, pos: int, which_v: bool) -> np.ndarray:
        kvd = self.model.cfg.num_key_value_heads * (self.model.cfg.head_dim or
                                                    self.model.cfg.hidden_size // self.model.cfg.num_attention_heads)
        out = np.empty(kvd, dtype=np.float32)
        lib().oracle_session_kv(self._s, layer, pos, int(which_v), out)
        return out

    def load_kv(self, layer: int, pos0: int, which_v: bool, rows) -> None:
        """Overwrite cached rows [pos0, pos0 + len(rows)) of one layer (test
        helper: continue from a cache another implementation filled)."""
        rows = np.ascontiguousarray(rows, dtype=np.float32)
        if lib().oracle_session_load_kv(self._s, layer, pos0, rows.shape[0], int(which_v), rows) != 0:
            raise ValueError("oracle load_kv: layer or positions out of range")

    def close(self):
        if self._s:
            lib().oracle_session_free(self._s)
            self._s = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
