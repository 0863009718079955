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
CNT_WORDS = 1024 * 64  # 1024 counters, one per 256-byte line


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


def _scratch_floats(n_seq, nh, max_seq):
    """Floats the call needs: 1024 counters 64 words apart, then per
    (sequence, head) min(32, ceil(max_seq / 64)) chunk slots of 2 + 64 floats."""
    return CNT_WORDS + n_seq * nh * min(32, -(-max_seq // 64)) * 66


def test_noalloc_refuses_more_than_its_buffer():
    """The size checks run on the host before any device work (no GPU
    needed).  The pointers are dummies, so the sizes are first checked here
    to be refused: a call that passed the checks would launch on them."""
    L = _lib.lib()
    dummy = C.c_void_p(256)
    # 64 sequences x 32 heads x 32768 positions: 64*32*32*66 partial floats > 2^21
    assert _scratch_floats(64, 32, 32768) > SCRATCH_FLOATS >= _scratch_floats(4, 14, 32768)
    rc = L.lkhip_attn_decode_noalloc(dummy, dummy, dummy, dummy, 64, 32, 4, 64, 32768, dummy, None)
    assert rc == -1
    msg = L.lkhip_last_error().decode()
    assert "lkhip_attn_decode" in msg and "8 MiB" in msg
    # 512 sequences x 4 kv heads need more than the 1024 arrival counters
    assert _scratch_floats(512, 8, 64) <= SCRATCH_FLOATS
    rc = L.lkhip_attn_decode_noalloc(dummy, dummy, dummy, dummy, 512, 8, 4, 64, 64, dummy, None)
    assert rc == -1
    assert "arrival counters" in L.lkhip_last_error().decode()
    # a zero-size call is a no-op, like the allocating entry point
    assert L.lkhip_attn_decode_noalloc(dummy, dummy, dummy, dummy, 0, 14, 2, 64, 1024, dummy, None) == 0
