"""lkhip_attn_decode_noalloc: the attention entry point that allocates no
device memory (its partials live in a fixed per-device buffer).  Its output
must equal lkhip_attn_decode's bit for bit -- the same kernels on the same
inputs -- and the oracle's within the attention tolerance, on consecutive
calls that reuse the buffer (the second with a smaller input)."""
import ctypes as C

import numpy as np
import pytest

import oracle
from lokal_amd import _lib
from lokal_amd import kernels as K

TOL = 1e-3
SCRATCH_FLOATS = 2 << 20


def rel_err(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def _inputs(n_seq, nh, nkv, ctxs, max_seq, seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n_seq, nkv, max_seq, 64)).astype(np.float16)
    v = rng.standard_normal((n_seq, nkv, max_seq, 64)).astype(np.float16)
    q = rng.standard_normal((n_seq, nh * 64)).astype(np.float32)
    return q, k, v, np.array(ctxs, np.uint32)


def _both(n_seq, nh, nkv, ctxs, max_seq, seed):
    q, k, v, ctx = _inputs(n_seq, nh, nkv, ctxs, max_seq, seed)
    qd, kd, vd, cd = (K.DeviceArray.from_numpy(q), K.DeviceArray.from_numpy(k.view(np.uint16)),
                      K.DeviceArray.from_numpy(v.view(np.uint16)), K.DeviceArray.from_numpy(ctx))
    o1, o2 = K.DeviceArray((n_seq, nh * 64)), K.DeviceArray((n_seq, nh * 64))
    K.attn_decode(qd, kd, vd, cd, n_seq, nh, nkv, 64, max_seq, o1)
    K.attn_decode_noalloc(qd, kd, vd, cd, n_seq, nh, nkv, 64, max_seq, o2)
    a, b = o1.numpy(), o2.numpy()
    for s in range(n_seq):
        c = int(ctx[s])
        Kc = k[s, :, :c, :].astype(np.float32).transpose(1, 0, 2).reshape(c, nkv * 64)
        Vc = v[s, :, :c, :].astype(np.float32).transpose(1, 0, 2).reshape(c, nkv * 64)
        want = oracle.attention(q[s], Kc, Vc, c - 1, nh, nkv, 64)
        assert rel_err(b[s], want) < TOL, (s, c)
    return a, b


@pytest.mark.gpu
def test_noalloc_matches_allocating_entry_point_twice():
    """Config 5 shape (4 sequences, Qwen2.5-0.5B GQA 14/2) at 32768 positions,
    then a smaller ragged call on the same buffer: bit-identical to
    lkhip_attn_decode each time, and within 1e-3 of the oracle."""
    print("noalloc: 4 seq x 14/2 heads, max_seq 32768", flush=True)
    a, b = _both(4, 14, 2, [32768, 4096, 16384, 777], 32768, seed=41)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    print("noalloc: 3 seq x 9/3 heads, max_seq 1024", flush=True)
    a, b = _both(3, 9, 3, [1000, 1, 300], 1024, seed=42)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_noalloc_refuses_more_than_its_buffer():
    """The size check runs on the host before any device work (no GPU needed):
    8 sequences x 32 heads x 32768 positions need 8*32*128*66 floats > 2^21."""
    L = _lib.lib()
    dummy = C.c_void_p(256)
    rc = L.lkhip_attn_decode_noalloc(dummy, dummy, dummy, dummy, 8, 32, 4, 64, 32768, dummy, None)
    assert rc == -1
    msg = L.lkhip_last_error().decode()
    assert "lkhip_attn_decode" in msg and "8 MiB" in msg
    assert 8 * 32 * 128 * 66 > SCRATCH_FLOATS >= 4 * 14 * 128 * 66
    # a zero-size call is a no-op, like the allocating entry point
    assert L.lkhip_attn_decode_noalloc(dummy, dummy, dummy, dummy, 0, 14, 2, 64, 1024, dummy, None) == 0
