"""Kernel-level entry points of the HIP backend on device buffers.

These wrap the "kernels" part of include/lokal_hip.h: device memory
(DeviceArray), weights uploaded in their GGUF type (Weight), and one call per
hot-path kernel.  Calls are asynchronous on the given stream (None = null
stream); DeviceArray.numpy() synchronises.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib


class DeviceArray:
    """A device allocation with a numpy dtype and shape."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        check(lib().lkhip_malloc(C.byref(p), max(self.nbytes, 4)))
        self.ptr = p

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if d.nbytes:
            check(lib().lkhip_memcpy_htod(d.ptr, a.ctypes.data, d.nbytes))
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        check(lib().lkhip_synchronize())
        if self.nbytes:
            check(lib().lkhip_memcpy_dtoh(out.ctypes.data, self.ptr, self.nbytes))
        return out

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        check(lib().lkhip_memcpy_htod(self.ptr, a.ctypes.data, self.nbytes))

    def zero(self) -> None:
        check(lib().lkhip_memset(self.ptr, 0, self.nbytes))

    def free(self) -> None:
        if self.ptr:
            check(lib().lkhip_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr:
                lib().lkhip_free(self.ptr)
        except Exception:
            pass


class Weight:
    """A weight matrix in its GGUF type (F16, Q8_0, Q4_0, Q5_0, Q4_K, Q5_K, Q6_K), resident on device."""

    def __init__(self, ggml_type: int, rows: int, cols: int, data: np.ndarray):
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        h = C.c_void_p()
        check(lib().lkhip_weight_create(ggml_type, rows, cols, data.ctypes.data, data.size, C.byref(h)))
        self._h = h
        self.ggml_type, self.rows, self.cols = ggml_type, rows, cols

    @property
    def nbytes(self) -> float:
        return float(lib().lkhip_weight_bytes(self._h))

    def close(self):
        if self._h:
            lib().lkhip_weight_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _p(d):
    return None if d is None else d.ptr


def dequant_rows(w: Weight, row0: int, n_rows: int, out: DeviceArray, stream=None) -> None:
    check(lib().lkhip_dequant_rows(w._h, row0, n_rows, out.ptr, stream))


def matvec(w: Weight, x: DeviceArray, y: DeviceArray, bias: DeviceArray | None = None, accumulate=False,
           stream=None) -> None:
    check(lib().lkhip_matvec(w._h, x.ptr, _p(bias), y.ptr, int(accumulate), stream))


def matmul(w: Weight, x: DeviceArray, n_rows: int, y: DeviceArray, bias: DeviceArray | None = None,
           accumulate=False, ldx: int | None = None, ldy: int | None = None, stream=None) -> None:
    """y[r, :rows] (+)= W x[r, :cols] (+ bias) for n_rows rows (multi-row GEMM)."""
    check(lib().lkhip_matmul(w._h, x.ptr, n_rows, ldx or w.cols, _p(bias), y.ptr, ldy or w.rows, int(accumulate),
                             stream))


def q8_0_matvec(w, x, y, bias=None, accumulate=False, stream=None) -> None:
    check(lib().lkhip_q8_0_matvec(w._h, x.ptr, _p(bias), y.ptr, int(accumulate), stream))


def q4_k_matvec(w, x, y, bias=None, accumulate=False, stream=None) -> None:
    check(lib().lkhip_q4_k_matvec(w._h, x.ptr, _p(bias), y.ptr, int(accumulate), stream))


def rmsnorm(x: DeviceArray, w: DeviceArray, n_rows: int, n: int, eps: float, y: DeviceArray, stream=None) -> None:
    check(lib().lkhip_rmsnorm(x.ptr, w.ptr, n_rows, n, eps, y.ptr, stream))


def rope_pairs(x: DeviceArray, n_rows: int, n: int, head_dim: int, pos: DeviceArray, theta: float,
               stream=None) -> None:
    check(lib().lkhip_rope_pairs(x.ptr, n_rows, n, head_dim, pos.ptr, theta, stream))


def swiglu(g: DeviceArray, u: DeviceArray, n: int, out: DeviceArray, stream=None) -> None:
    check(lib().lkhip_swiglu(g.ptr, u.ptr, n, out.ptr, stream))


def embed_gather(table: Weight, ids: DeviceArray, n_ids: int, out: DeviceArray, stream=None) -> None:
    check(lib().lkhip_embed_gather(table._h, ids.ptr, n_ids, out.ptr, stream))


def attn_decode(q: DeviceArray, k: DeviceArray, v: DeviceArray, ctx_len: DeviceArray, n_seq: int, n_heads: int,
                n_kv_heads: int, head_dim: int, max_seq: int, out: DeviceArray, stream=None) -> None:
    check(lib().lkhip_attn_decode(q.ptr, k.ptr, v.ptr, ctx_len.ptr, n_seq, n_heads, n_kv_heads, head_dim, max_seq,
                                  out.ptr, stream))


def attn_decode_noalloc(q: DeviceArray, k: DeviceArray, v: DeviceArray, ctx_len: DeviceArray, n_seq: int,
                        n_heads: int, n_kv_heads: int, head_dim: int, max_seq: int, out: DeviceArray,
                        stream=None) -> None:
    check(lib().lkhip_attn_decode_noalloc(q.ptr, k.ptr, v.ptr, ctx_len.ptr, n_seq, n_heads, n_kv_heads, head_dim,
                                          max_seq, out.ptr, stream))


def argmax(x: DeviceArray, n_rows: int, n: int, out: DeviceArray, stream=None) -> None:
    check(lib().lkhip_argmax(x.ptr, n_rows, n, out.ptr, stream))


def memset(d: DeviceArray, value: int) -> None:
    check(lib().lkhip_memset(d.ptr, value, d.nbytes))


def memcpy_dtod(dst: DeviceArray, src: DeviceArray) -> None:
    check(lib().lkhip_memcpy_dtod(dst.ptr, src.ptr, min(dst.nbytes, src.nbytes)))


def synchronize() -> None:
    check(lib().lkhip_synchronize())


def device_count() -> int:
    return int(lib().lkhip_device_count())


class Stream:
    def __init__(self):
        p = C.c_void_p()
        check(lib().lkhip_stream_create(C.byref(p)))
        self.ptr = p

    def synchronize(self):
        check(lib().lkhip_stream_synchronize(self.ptr))

    def close(self):
        if self.ptr:
            check(lib().lkhip_stream_destroy(self.ptr))
            self.ptr = None


class Event:
    def __init__(self):
        p = C.c_void_p()
        check(lib().lkhip_event_create(C.byref(p)))
        self.ptr = p

    def record(self, stream=None):
        check(lib().lkhip_event_record(self.ptr, None if stream is None else stream.ptr))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib().lkhip_event_elapsed_ms(self.ptr, end.ptr, C.byref(ms)))
        return float(ms.value)
