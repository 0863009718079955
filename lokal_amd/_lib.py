"""ctypes view of liblokal_hip.so (include/lokal_hip.h).

The library is loaded from this package directory (or from $LOKAL_HIP_LIB,
to compare builds); if it is missing the import fails loudly -- there is no
CPU fallback behind this API.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("LOKAL_HIP_LIB") or Path(__file__).resolve().parent / "liblokal_hip.so")

LKHIP_OK = 0
LKHIP_F32, LKHIP_F16, LKHIP_Q8_0, LKHIP_Q4_K = 0, 1, 8, 12
LKHIP_Q4_0, LKHIP_Q5_0, LKHIP_Q5_K, LKHIP_Q6_K = 2, 6, 13, 14


class LokalHipError(RuntimeError):
    """A refusal or failure reported by the HIP backend (its lkhip_last_error text)."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class Config(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_uint32), ("intermediate_size", C.c_uint32), ("num_hidden_layers", C.c_uint32),
        ("num_attention_heads", C.c_uint32), ("num_key_value_heads", C.c_uint32), ("vocab_size", C.c_uint32),
        ("head_dim", C.c_uint32), ("max_position_embeddings", C.c_uint32), ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float),
    ]


class TensorDesc(C.Structure):
    _fields_ = [
        ("name", C.c_char_p), ("ggml_type", C.c_uint32), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 2),
        ("data", C.c_void_p), ("nbytes", C.c_uint64),
    ]


class Row(C.Structure):
    _fields_ = [("token", C.c_uint32), ("slot", C.c_uint32), ("pos", C.c_uint64)]


class Profile(C.Structure):
    _fields_ = [
        ("tokens", C.c_uint64), ("matvec_launches", C.c_uint64), ("matvec_ms", C.c_double),
        ("matvec_bytes", C.c_double), ("lm_head_launches", C.c_uint64), ("lm_head_ms", C.c_double),
        ("lm_head_bytes", C.c_double), ("attn_ms", C.c_double), ("other_ms", C.c_double),
    ]

    def as_dict(self) -> dict:
        return {k: getattr(self, k) for k, _ in self._fields_}


_P = C.c_void_p
_F = C.POINTER(C.c_float)
_U32 = C.POINTER(C.c_uint32)
_U16 = C.POINTER(C.c_uint16)

# name -> (restype, argtypes); mirrors include/lokal_hip.h one to one.
SIGNATURES = {
    "lkhip_last_error": (C.c_char_p, []),
    "lkhip_device_count": (C.c_int, []),
    "lkhip_version": (C.c_char_p, []),
    "lkhip_engine_create_tensors": (C.c_int, [C.POINTER(Config), C.POINTER(TensorDesc), C.c_size_t, C.c_int,
                                              C.POINTER(_P)]),
    "lkhip_engine_create_gguf": (C.c_int, [C.c_char_p, C.POINTER(_P)]),
    "lkhip_context_window": (C.c_int, [C.c_size_t, C.c_size_t]),
    "lkhip_gguf_config": (C.c_int, [C.c_char_p, C.POINTER(Config), C.POINTER(C.c_size_t), C.POINTER(C.c_int)]),
    "lkhip_engine_destroy": (None, [_P]),
    "lkhip_engine_config": (C.c_int, [_P, C.POINTER(Config)]),
    "lkhip_engine_matvec_bytes": (C.c_double, [_P]),
    "lkhip_session_create": (C.c_int, [_P, C.c_size_t, C.POINTER(_P)]),
    "lkhip_session_create_ex": (C.c_int, [_P, C.c_size_t, C.c_uint32, C.POINTER(_P)]),
    "lkhip_session_destroy": (None, [_P]),
    "lkhip_session_forward": (C.c_int, [_P, C.c_uint32, C.c_size_t, _F]),
    "lkhip_session_prefill": (C.c_int, [_P, _U32, C.c_size_t, _F]),
    "lkhip_session_forward_batch": (C.c_int, [_P, _U32, C.c_size_t, C.c_size_t, _F]),
    "lkhip_session_decode_greedy": (C.c_int, [_P, C.c_uint32, C.c_size_t, C.c_size_t, _U32, _F]),
    "lkhip_session_read_kv": (C.c_int, [_P, C.c_uint32, C.c_size_t, C.c_int, _F]),
    "lkhip_session_read_kv_rows": (C.c_int, [_P, C.c_uint32, C.c_size_t, C.c_size_t, C.c_int, _F]),
    "lkhip_batch_read_kv_rows": (C.c_int, [_P, C.c_uint32, C.c_uint32, C.c_size_t, C.c_size_t, C.c_int, _F]),
    "lkhip_batch_trace_len": (C.c_size_t, [_P]),
    "lkhip_batch_trace": (C.c_int, [_P, C.POINTER(C.c_uint64), C.c_size_t]),
    "lkhip_session_set_profiling": (C.c_int, [_P, C.c_int]),
    "lkhip_session_profile": (C.c_int, [_P, C.POINTER(Profile), C.c_int]),
    "lkhip_session_set_trace": (C.c_int, [_P, C.c_int]),
    "lkhip_session_trace_len": (C.c_size_t, [_P]),
    "lkhip_session_trace": (C.c_int, [_P, C.POINTER(C.c_uint64), C.c_size_t]),
    "lkhip_batch_create": (C.c_int, [_P, C.c_size_t, C.c_size_t, C.POINTER(_P)]),
    "lkhip_batch_destroy": (None, [_P]),
    "lkhip_batch_prefill": (C.c_int, [_P, C.c_uint32, _U32, C.c_size_t, _F]),
    "lkhip_batch_decode_step": (C.c_int, [_P, C.POINTER(Row), C.c_size_t, _F]),
    "lkhip_batch_decode_greedy": (C.c_int, [_P, C.POINTER(Row), C.c_size_t, C.c_size_t, _U32]),
    "lkhip_malloc": (C.c_int, [C.POINTER(_P), C.c_size_t]),
    "lkhip_free": (C.c_int, [_P]),
    "lkhip_memcpy_htod": (C.c_int, [_P, _P, C.c_size_t]),
    "lkhip_memcpy_dtoh": (C.c_int, [_P, _P, C.c_size_t]),
    "lkhip_memcpy_dtod": (C.c_int, [_P, _P, C.c_size_t]),
    "lkhip_memset": (C.c_int, [_P, C.c_int, C.c_size_t]),
    "lkhip_synchronize": (C.c_int, []),
    "lkhip_stream_create": (C.c_int, [C.POINTER(_P)]),
    "lkhip_stream_destroy": (C.c_int, [_P]),
    "lkhip_stream_synchronize": (C.c_int, [_P]),
    "lkhip_event_create": (C.c_int, [C.POINTER(_P)]),
    "lkhip_event_destroy": (C.c_int, [_P]),
    "lkhip_event_record": (C.c_int, [_P, _P]),
    "lkhip_event_elapsed_ms": (C.c_int, [_P, _P, _F]),
    "lkhip_weight_create": (C.c_int, [C.c_uint32, C.c_size_t, C.c_size_t, _P, C.c_size_t, C.POINTER(_P)]),
    "lkhip_weight_destroy": (None, [_P]),
    "lkhip_weight_bytes": (C.c_double, [_P]),
    "lkhip_dequant_rows": (C.c_int, [_P, C.c_size_t, C.c_size_t, _P, _P]),
    "lkhip_matvec": (C.c_int, [_P, _P, _P, _P, C.c_int, _P]),
    "lkhip_q8_0_matvec": (C.c_int, [_P, _P, _P, _P, C.c_int, _P]),
    "lkhip_q4_k_matvec": (C.c_int, [_P, _P, _P, _P, C.c_int, _P]),
    "lkhip_matmul": (C.c_int, [_P, _P, C.c_size_t, C.c_size_t, _P, _P, C.c_size_t, C.c_int, _P]),
    "lkhip_rmsnorm": (C.c_int, [_P, _P, C.c_size_t, C.c_size_t, C.c_float, _P, _P]),
    "lkhip_rope_pairs": (C.c_int, [_P, C.c_size_t, C.c_size_t, C.c_size_t, _P, C.c_float, _P]),
    "lkhip_swiglu": (C.c_int, [_P, _P, C.c_size_t, _P, _P]),
    "lkhip_embed_gather": (C.c_int, [_P, _P, C.c_size_t, _P, _P]),
    "lkhip_attn_decode": (C.c_int, [_P, _P, _P, _P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t,
                                    _P, _P]),
    "lkhip_attn_decode_noalloc": (C.c_int, [_P, _P, _P, _P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t,
                                            C.c_size_t, _P, _P]),
    "lkhip_argmax": (C.c_int, [_P, C.c_size_t, C.c_size_t, _P, _P]),
}

_lib = None


def lib():
    """Load liblokal_hip.so once and bind every declared symbol."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m lokal_amd.build` "
                              "(the HIP backend has no CPU fallback)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != LKHIP_OK:
        msg = lib().lkhip_last_error()
        raise LokalHipError(rc, msg.decode("utf-8", "replace") if msg else f"lkhip error {rc}")
