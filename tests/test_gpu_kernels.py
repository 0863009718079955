"""Kernel-level parity of the HIP backend against the CPU oracle, through the
C ABI.  Dequantization and embedding gather are bit-exact; the one-hot matvec
(the reference's metal.rs:4790-4976 gate) is bit-exact; everything with fp32
accumulation is within 1e-3 relative error, measured as
max|got - want| / max|want| over the output."""
import numpy as np
import pytest

import oracle
from lokal_amd import kernels as K
from lokal_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def weight_bytes(t, rows, cols, seed):
    return synth.gen_weight(t, seed, f"w{rows}x{cols}", rows, cols).data


def oracle_rows(t, data, rows, cols):
    return oracle.dequant_row(t, data, rows * cols).reshape(rows, cols)


TYPES = [synth.Q8_0, synth.Q4_K, synth.F16]


@pytest.mark.parametrize("t", TYPES)
def test_dequant_rows_bit_exact(t):
    rows, cols = 64, 2048
    data = weight_bytes(t, rows, cols, 1)
    w = K.Weight(t, rows, cols, data)
    out = K.DeviceArray((rows - 5, cols))
    K.dequant_rows(w, 5, rows - 5, out)
    assert np.array_equal(out.numpy(), oracle_rows(t, data, rows, cols)[5:])


def test_dequant_reference_hand_vectors():
    import json
    from pathlib import Path
    gold = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
    for v in gold["dequant"]:
        if v["type"] not in (8, 12):
            continue
        w = K.Weight(v["type"], 1, v["n"], np.array(v["bytes"], np.uint8))
        out = K.DeviceArray(v["n"])
        K.dequant_rows(w, 0, 1, out)
        y = out.numpy()
        for i, want in v["expect"].items():
            assert y[int(i)] == np.float32(want), v["ref"]


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("cols", [512, 2048])
def test_onehot_matvec_is_bit_exact(t, cols):
    """A one-hot x returns column c of the dequantized weight bit-for-bit."""
    rows = 96
    data = weight_bytes(t, rows, cols, 2)
    want = oracle_rows(t, data, rows, cols)
    w = K.Weight(t, rows, cols, data)
    x = K.DeviceArray(cols)
    y = K.DeviceArray(rows)
    for c in (0, 1, 31, 32, 255, 256, cols - 1, cols // 2 + 17):
        xh = np.zeros(cols, np.float32)
        xh[c] = 1.0
        x.upload(xh)
        K.matvec(w, x, y)
        assert np.array_equal(y.numpy(), want[:, c]), (t, cols, c)


QWEN_SHAPES = [(896, 896), (128, 896), (4864, 896), (896, 4864), (151936, 896)]


@pytest.mark.parametrize("rows,cols", QWEN_SHAPES)
def test_q8_0_matvec_qwen_shapes(rows, cols):
    data = weight_bytes(synth.Q8_0, rows, cols, 3)
    wf = oracle_rows(synth.Q8_0, data, rows, cols)
    x = np.random.default_rng(rows + cols).standard_normal(cols).astype(np.float32)
    want = oracle.matvec(wf, x)
    w = K.Weight(synth.Q8_0, rows, cols, data)
    xd, yd = K.DeviceArray.from_numpy(x), K.DeviceArray(rows)
    K.q8_0_matvec(w, xd, yd)
    assert rel_err(yd.numpy(), want) < TOL


@pytest.mark.parametrize("rows,cols", [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632), (32000, 2048)])
def test_q4_k_matvec_tinyllama_shapes(rows, cols):
    data = weight_bytes(synth.Q4_K, rows, cols, 4)
    wf = oracle_rows(synth.Q4_K, data, rows, cols)
    x = np.random.default_rng(rows * 3 + cols).standard_normal(cols).astype(np.float32)
    want = oracle.matvec(wf, x)
    w = K.Weight(synth.Q4_K, rows, cols, data)
    xd, yd = K.DeviceArray.from_numpy(x), K.DeviceArray(rows)
    K.q4_k_matvec(w, xd, yd)
    assert rel_err(yd.numpy(), want) < TOL


@pytest.mark.parametrize("rows,cols", [(576, 576), (192, 576), (1536, 576), (576, 1536), (49152, 576)])
def test_f16_matvec_smollm2_shapes(rows, cols):
    data = weight_bytes(synth.F16, rows, cols, 5)
    wf = oracle_rows(synth.F16, data, rows, cols)
    x = np.random.default_rng(rows * 5 + cols).standard_normal(cols).astype(np.float32)
    want = oracle.matvec(wf, x)
    w = K.Weight(synth.F16, rows, cols, data)
    xd, yd = K.DeviceArray.from_numpy(x), K.DeviceArray(rows)
    K.matvec(w, xd, yd)
    assert rel_err(yd.numpy(), want) < TOL


def test_matvec_bias_and_residual_modes():
    rows, cols = 300, 896
    data = weight_bytes(synth.Q8_0, rows, cols, 6)
    wf = oracle_rows(synth.Q8_0, data, rows, cols)
    rng = np.random.default_rng(6)
    x = rng.standard_normal(cols).astype(np.float32)
    b = rng.standard_normal(rows).astype(np.float32)
    r = rng.standard_normal(rows).astype(np.float32)
    w = K.Weight(synth.Q8_0, rows, cols, data)
    xd, bd = K.DeviceArray.from_numpy(x), K.DeviceArray.from_numpy(b)
    yd = K.DeviceArray(rows)
    K.matvec(w, xd, yd, bias=bd)
    assert rel_err(yd.numpy(), oracle.matvec(wf, x) + b) < TOL
    yd.upload(r)
    K.matvec(w, xd, yd, accumulate=True)
    assert rel_err(yd.numpy(), r + oracle.matvec(wf, x)) < TOL


def test_matvec_refuses_wrong_type():
    from lokal_amd import LokalHipError
    w = K.Weight(synth.F16, 8, 64, weight_bytes(synth.F16, 8, 64, 0))
    x, y = K.DeviceArray(64), K.DeviceArray(8)
    with pytest.raises(LokalHipError, match="q8_0_matvec"):
        K.q8_0_matvec(w, x, y)


@pytest.mark.parametrize("rows", [1, 8, 64])
def test_rmsnorm_rows(rows):
    rng = np.random.default_rng(rows)
    x = rng.standard_normal((rows, 896)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(896)).astype(np.float32)
    xd, gd, yd = K.DeviceArray.from_numpy(x), K.DeviceArray.from_numpy(g), K.DeviceArray((rows, 896))
    K.rmsnorm(xd, gd, rows, 896, 1e-6, yd)
    y = yd.numpy()
    for r in range(rows):
        assert rel_err(y[r], oracle.rmsnorm(x[r], g, 1e-6)) < TOL


@pytest.mark.parametrize("rows", [1, 8, 64])
def test_rope_rows(rows):
    rng = np.random.default_rng(100 + rows)
    n = 14 * 64
    x = rng.standard_normal((rows, n)).astype(np.float32)
    pos = rng.integers(0, 32768, rows).astype(np.uint32)
    xd, pd = K.DeviceArray.from_numpy(x), K.DeviceArray.from_numpy(pos)
    K.rope_pairs(xd, rows, n, 64, pd, 1e6)
    y = xd.numpy()
    for r in range(rows):
        assert rel_err(y[r], oracle.rope(x[r], int(pos[r]), 64, 1e6)) < TOL


@pytest.mark.parametrize("rows", [1, 8, 64])
def test_swiglu_rows(rows):
    rng = np.random.default_rng(200 + rows)
    g = rng.standard_normal(rows * 4864).astype(np.float32)
    u = rng.standard_normal(rows * 4864).astype(np.float32)
    gd, ud, od = K.DeviceArray.from_numpy(g), K.DeviceArray.from_numpy(u), K.DeviceArray(rows * 4864)
    K.swiglu(gd, ud, rows * 4864, od)
    assert rel_err(od.numpy(), oracle.swiglu(g, u)) < TOL


@pytest.mark.parametrize("t", [synth.F16, synth.Q8_0])
def test_embed_gather_bit_exact(t):
    vocab, h = 151936, 896
    data = synth.gen_weight(t, 9, "model.embed_tokens.weight", vocab, h).data
    table = K.Weight(t, vocab, h, data)
    ids = np.random.default_rng(9).integers(0, vocab, 64).astype(np.uint32)
    ids[:3] = [0, vocab - 1, 12345]
    idd, out = K.DeviceArray.from_numpy(ids), K.DeviceArray((64, h))
    K.embed_gather(table, idd, 64, out)
    y = out.numpy()
    rb = synth.row_bytes(t, h)
    for i, tok in enumerate(ids):
        row = data[int(tok) * rb:(int(tok) + 1) * rb]
        assert np.array_equal(y[i], oracle.dequant_row(t, row, h))


def _attn_case(n_seq, nh, nkv, ctxs, max_seq, seed):
    rng = np.random.default_rng(seed)
    hd = 64
    k = rng.standard_normal((n_seq, nkv, max_seq, hd)).astype(np.float16)
    v = rng.standard_normal((n_seq, nkv, max_seq, hd)).astype(np.float16)
    q = rng.standard_normal((n_seq, nh * hd)).astype(np.float32)
    ctx = np.array(ctxs, np.uint32)
    qd, kd, vd, cd = (K.DeviceArray.from_numpy(q), K.DeviceArray.from_numpy(k.view(np.uint16)),
                      K.DeviceArray.from_numpy(v.view(np.uint16)), K.DeviceArray.from_numpy(ctx))
    od = K.DeviceArray((n_seq, nh * hd))
    K.attn_decode(qd, kd, vd, cd, n_seq, nh, nkv, hd, max_seq, od)
    out = od.numpy()
    for s in range(n_seq):
        c = int(ctx[s])
        # oracle caches are [pos][kv_dim]: transpose [kv][pos][hd] -> [pos][kv*hd]
        Kc = k[s, :, :c, :].astype(np.float32).transpose(1, 0, 2).reshape(c, nkv * hd)
        Vc = v[s, :, :c, :].astype(np.float32).transpose(1, 0, 2).reshape(c, nkv * hd)
        want = oracle.attention(q[s], Kc, Vc, c - 1, nh, nkv, hd)
        assert rel_err(out[s], want) < TOL, (s, c)


@pytest.mark.parametrize("nh,nkv", [(14, 2), (9, 3), (32, 4)])
@pytest.mark.parametrize("ctx", [1, 17, 256, 300, 1000])
def test_attention_single_sequence(nh, nkv, ctx):
    _attn_case(1, nh, nkv, [ctx], 1024, seed=nh * 1000 + ctx)


def test_attention_four_sequences_ragged():
    _attn_case(4, 14, 2, [4096, 1, 2500, 777], 4096, seed=5)


def test_attention_long_context():
    _attn_case(2, 14, 2, [16384, 9999], 16384, seed=6)


def test_attention_config5_four_sequences_32k():
    """Long-context GQA flash-decoding at the Qwen2.5-0.5B shape: 4 sequences
    with independent contexts up to 32768, one query token each."""
    _attn_case(4, 14, 2, [32768, 32768, 16384, 4096], 32768, seed=7)


def test_attention_merge_boundary_and_repeat():
    """Contexts on both sides of 8192 positions in one call, repeated on the
    same cached scratch buffer with other shapes in between."""
    for rep in range(3):
        _attn_case(3, 14, 2, [8192, 8193, 8191], 8448, seed=21 + rep)
        _attn_case(2, 14, 2, [8192, 256], 8192, seed=31 + rep)


def test_attention_chunk_plans():
    """Each chunk plan of the launch (A active waves of 8 per block, T tiles
    per wave, at most 32 chunks per sequence and kv head): A = 8 with T = 1
    and 2, A = 4, A = 2 with T = 3, A = 1, on ragged contexts; then the
    first shape again on the same scratch buffer."""
    _attn_case(4, 14, 2, [16384, 16383, 1, 300], 16384, seed=51)      # A=8, T=1
    _attn_case(4, 14, 2, [32768, 20000, 16385, 64], 32768, seed=52)   # A=8, T=2
    _attn_case(4, 14, 2, [4096, 4000, 129, 65], 4096, seed=53)        # A=4, T=1
    _attn_case(3, 14, 2, [8448, 8192, 4097], 8448, seed=54)           # A=2, T=3
    _attn_case(1, 14, 2, [1000], 1024, seed=55)                       # A=1, T=1
    _attn_case(4, 14, 2, [16384, 16383, 1, 300], 16384, seed=51)


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
def test_attention_one_chunk_per_pair(kernel, monkeypatch):
    """64 or more (sequence, kv head) pairs over a cache of at most 1024
    positions take one chunk each, whose block writes the output without the
    partial / count / fold round trip: ragged contexts from 1 to 1024 (one
    and two tiles per wave), 4 kv heads, and 1025 positions (the chunked plan
    again), on both f16 kernels, repeated on the same scratch buffer."""
    monkeypatch.setenv("LKHIP_ATTN", kernel)
    rng = np.random.default_rng(61)
    ctx32 = [1, 2, 63, 64, 65, 511, 512, 513, 1023, 1024] + [int(c) for c in rng.integers(1, 1025, 22)]
    _attn_case(32, 14, 2, ctx32, 1024, seed=61)
    _attn_case(40, 32, 4, [int(c) for c in rng.integers(1, 513, 40)], 512, seed=62)
    _attn_case(32, 14, 2, [1025] + ctx32[1:], 1025, seed=63)
    _attn_case(32, 14, 2, ctx32, 1024, seed=61)


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
def test_attention_both_f16_kernels(kernel, monkeypatch):
    """The vector-ALU and matrix-core partial kernels (the matrix-core one by
    default, LKHIP_ATTN=valu selects the other) on the same cases, short and long."""
    monkeypatch.setenv("LKHIP_ATTN", kernel)
    _attn_case(1, 14, 2, [1], 64, seed=11)
    _attn_case(3, 9, 3, [300, 17, 1000], 1024, seed=12)
    _attn_case(4, 32, 4, [4096, 1, 2500, 777], 4096, seed=13)
    _attn_case(2, 14, 2, [16384, 9999], 16384, seed=14)
    _attn_case(3, 14, 2, [8192, 8193, 8191], 8448, seed=15)


def test_argmax_first_max_wins():
    x = np.random.default_rng(1).standard_normal((3, 151936)).astype(np.float32)
    x[1, 500] = x[1, 900] = 100.0
    xd, od = K.DeviceArray.from_numpy(x), K.DeviceArray(3, np.uint32)
    K.argmax(xd, 3, 151936, od)
    got = od.numpy()
    assert list(got) == [oracle.argmax(x[i]) for i in range(3)]
    assert got[1] == 500
