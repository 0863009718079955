"""Pins the CPU oracle (oracle/lokal_oracle.c) before anything is checked
against it: the reference's own known-answer vectors (tests/golden), closed
forms in float64, exhaustive bit-level checks, and invariants chosen so that a
dropped term, a wrong sign or index, or a swapped operand fails one of them."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from lokal_amd import synth
from lokal_amd.config import ModelConfig
from tests import ref64

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


# ------------------------------------------------------------ dequant

@pytest.mark.parametrize("vec", GOLD["dequant"], ids=lambda v: v["ref"])
def test_reference_hand_vectors(vec):
    y = oracle.dequant_row(vec["type"], bytes(vec["bytes"]), vec["n"])
    for idx, want in vec["expect"].items():
        assert y[int(idx)] == np.float32(want), (vec["ref"], idx, y[int(idx)], want)


def test_block_sizes_match_ggml_structs():
    s = GOLD["sizes"]
    for t, b in s["blk_bytes"].items():
        assert oracle.blk_bytes(int(t)) == b
    for t, n, rb in s["row_bytes"]:
        assert oracle.row_bytes(t, n) == rb


def test_q8_0_roundtrip_within_half_lsb():
    """dequant.rs:699-711: quantize an LCG vector at d=1/32, dequantize, |x-y| <= d/2."""
    r = GOLD["q8_0_roundtrip"]
    d = np.float32(r["d"])
    state = r["seed"]
    xs = np.empty(32, np.float32)
    for i in range(32):
        state = (state * r["mul"] + r["add"]) & 0xFFFFFFFF
        xs[i] = (np.float32(state >> 8) / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0)) \
            * np.float32(127.0) * d
    blk = np.zeros(34, np.uint8)
    blk[:2] = np.array([d], np.float16).view(np.uint8)
    blk[2:] = np.clip(np.round(xs / d), -127, 127).astype(np.int8).view(np.uint8)
    y = oracle.dequant_row(8, blk, 32)
    assert np.all(np.abs(xs - y) <= d * 0.5 + 1e-7)


def _f16_scales():
    # normal, subnormal, largest and a few ordinary f16 scales
    bits = np.array([0x0001, 0x03FF, 0x0400, 0x3C00, 0x3800, 0x7BFF, 0x1234, 0x2E66, 0x8001, 0xBC00], np.uint16)
    return bits


def test_q8_0_exhaustive_against_exact_product():
    """All 256 int8 codes x f16 scales incl. subnormal / max: (i8)q*d is exact in f32."""
    ds = _f16_scales()
    nb = ds.size * 8
    blocks = np.zeros((nb, 34), np.uint8)
    q = np.arange(-128, 128, dtype=np.int16).astype(np.int8)
    for b in range(nb):
        blocks[b, :2] = ds[b // 8 : b // 8 + 1].view(np.uint8)
        blocks[b, 2:] = q[(b % 8) * 32 : (b % 8 + 1) * 32].view(np.uint8)
    y = oracle.dequant_row(8, blocks.reshape(-1), nb * 32)
    d64 = ds.view(np.float16).astype(np.float64)
    want = np.concatenate([q[(b % 8) * 32:(b % 8 + 1) * 32].astype(np.float64) * d64[b // 8] for b in range(nb)])
    assert np.array_equal(y.astype(np.float64), want)


def _pack_scale_min_k4(sc, m):
    """ggml's quantize_row_q4_K packing of 8 (scale, min) 6-bit pairs into 12 bytes
    -- the encoder, an independent path to the decoder under test."""
    q = [0] * 12
    for j in range(8):
        ls, lm = sc[j], m[j]
        if j < 4:
            q[j] = ls
            q[j + 4] = lm
        else:
            q[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            q[j - 4] |= (ls >> 4) << 6
            q[j] |= (lm >> 4) << 6
    return np.array(q, np.uint8)


def test_scale_min_k4_inverts_the_ggml_packing():
    rng = np.random.default_rng(7)
    for _ in range(2000):
        sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        packed = _pack_scale_min_k4(sc, m)
        for j in range(8):
            assert oracle.scale_min_k4(j, packed) == (sc[j], m[j])


def test_scale_min_k4_is_six_bit_for_every_byte_pattern():
    rng = np.random.default_rng(1)
    for _ in range(512):
        q = rng.integers(0, 256, 12).astype(np.uint8)
        for j in range(8):
            sc, m = oracle.scale_min_k4(j, q)
            assert 0 <= sc < 64 and 0 <= m < 64


def test_q4_k_closed_form():
    """y = d*sc*q - dmin*m per sub-block (float64, within 2 ulp of the f32 value)."""
    rng = np.random.default_rng(3)
    nsb = 64
    raw = synth.gen_q4_k(rng, nsb * 256).reshape(nsb, 144)
    y = oracle.dequant_row(12, raw.reshape(-1), nsb * 256).reshape(nsb, 256).astype(np.float64)
    for b in range(nsb):
        d = raw[b, 0:2].view(np.float16)[0].astype(np.float64)
        dmin = raw[b, 2:4].view(np.float16)[0].astype(np.float64)
        qs = raw[b, 16:]
        for e in range(256):
            grp, within = divmod(e, 64)
            hi, l = divmod(within, 32)
            sc, m = oracle.scale_min_k4(2 * grp + hi, raw[b, 4:16])
            byte = int(qs[grp * 32 + l])
            qv = (byte >> 4) if hi else (byte & 0xF)
            want = d * sc * qv - dmin * m
            assert abs(y[b, e] - want) <= 2 * np.spacing(np.float32(max(abs(want), 1e-30))) + 1e-12


def test_f16_decode_exact():
    bits = np.arange(0, 1 << 16, 97, dtype=np.uint16)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    want = bits.view(np.float16).astype(np.float32)
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_dequant_refuses_size_mismatch():
    with pytest.raises(ValueError):
        oracle.dequant_row(8, bytes(33), 32)


# ---------------------------------------------------------------- math

def test_math_hand_vectors():
    m = GOLD["math"]
    w = np.array(m["matvec"]["w"], np.float32).reshape(m["matvec"]["out"], m["matvec"]["in"])
    assert list(oracle.matvec(w, np.array(m["matvec"]["x"], np.float32))) == m["matvec"]["y"]
    a = np.array(m["dot_len11"]["a"], np.float32)
    assert oracle.dot(a, a) == m["dot_len11"]["expect"]
    s = oracle.softmax(m["softmax"]["x"])
    assert abs(s.sum() - 1) < 1e-6 and s[1] > s[2] > s[0]
    r = m["rmsnorm"]
    y = oracle.rmsnorm(r["x"], r["w"], r["eps"])
    assert np.all(np.abs(y - r["expect"]) < r["tol"])


def test_argmax_first_max_wins():
    s = GOLD["sampler"]
    assert oracle.argmax(s["logits"]) == s["argmax"]
    assert oracle.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert oracle.argmax([-1.0, -1.0]) == 0


def test_dot_and_matvec_against_float64():
    rng = np.random.default_rng(11)
    for n in (1, 7, 8, 9, 64, 896, 4867):
        a, b = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
        want = float(a.astype(np.float64) @ b.astype(np.float64))
        assert abs(oracle.dot(a, b) - want) <= 1e-5 * (np.abs(a) @ np.abs(b) + 1e-30)
    w = rng.standard_normal((37, 91)).astype(np.float32)
    x = rng.standard_normal(91).astype(np.float32)
    want = w.astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(oracle.matvec(w, x), want, rtol=1e-5, atol=1e-5)


def test_rmsnorm_closed_form_and_scale_invariance():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(896).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(896)).astype(np.float32)
    y = oracle.rmsnorm(x, w, 1e-6)
    assert np.allclose(y, ref64.rmsnorm(x, w, 1e-6), rtol=1e-5, atol=1e-6)
    y2 = oracle.rmsnorm(x * np.float32(8.0), w, 1e-6)
    assert np.allclose(y, y2, rtol=1e-5, atol=1e-6)


def test_silu_and_swiglu_closed_form():
    rng = np.random.default_rng(2)
    g, u = rng.standard_normal(4864).astype(np.float32), rng.standard_normal(4864).astype(np.float32)
    assert np.allclose(oracle.swiglu(g, u), ref64.silu(g) * u, rtol=1e-6, atol=1e-7)
    assert oracle.silu(0.0) == 0.0


def test_rope_identity_norm_and_composition():
    rng = np.random.default_rng(9)
    hd, theta = 64, 1e6
    x = rng.standard_normal(14 * hd).astype(np.float32)
    assert np.array_equal(oracle.rope(x, 0, hd, theta), x)
    for pos in (1, 17, 1000, 32767):
        y = oracle.rope(x, pos, hd, theta)
        assert np.allclose(y, ref64.rope(x, pos, hd, theta, f32_angle=True), rtol=0, atol=2e-6)
        # each (i, i+hd/2) pair keeps its length
        xr, yr = x.reshape(-1, hd).astype(np.float64), y.reshape(-1, hd).astype(np.float64)
        n0 = xr[:, :32] ** 2 + xr[:, 32:] ** 2
        n1 = yr[:, :32] ** 2 + yr[:, 32:] ** 2
        assert np.allclose(n0, n1, rtol=1e-5)
    # rotating by p then q equals rotating by p+q (float64 closed form)
    p, q = 123, 456
    assert np.allclose(ref64.rope(ref64.rope(x, p, hd, 1e4), q, hd, 1e4), ref64.rope(x, p + q, hd, 1e4))
    assert np.allclose(oracle.rope(x, p + q, hd, 1e4), ref64.rope(x, p + q, hd, 1e4, f32_angle=True), atol=2e-6)


def test_attention_special_cases_and_float64():
    rng = np.random.default_rng(4)
    nh, nkv, hd = 14, 2, 64
    kvd = nkv * hd
    ctx = 50
    K = rng.standard_normal((ctx, kvd)).astype(np.float32)
    V = rng.standard_normal((ctx, kvd)).astype(np.float32)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    # ctx = 1: output is the V row of the head's kv head
    out = oracle.attention(q, K, V, 0, nh, nkv, hd)
    for h in range(nh):
        assert np.allclose(out[h * hd:(h + 1) * hd], V[0, (h // 7) * hd:(h // 7 + 1) * hd], rtol=1e-6)
    # uniform K: output is the mean of V
    Ku = np.tile(K[:1], (ctx, 1))
    out = oracle.attention(q, Ku, V, ctx - 1, nh, nkv, hd)
    for h in range(nh):
        assert np.allclose(out[h * hd:(h + 1) * hd], V[:, (h // 7) * hd:(h // 7 + 1) * hd].mean(0), atol=1e-5)
    # general case against float64; GQA equals MHA with repeated kv heads
    out = oracle.attention(q, K, V, ctx - 1, nh, nkv, hd)
    assert np.allclose(out, ref64.attention(q, K, V, nh, nkv, hd), atol=1e-5)
    Kr = np.repeat(K.reshape(ctx, nkv, hd), 7, axis=1).reshape(ctx, nh * hd)
    Vr = np.repeat(V.reshape(ctx, nkv, hd), 7, axis=1).reshape(ctx, nh * hd)
    out_mha = oracle.attention(q, Kr, Vr, ctx - 1, nh, nh, hd)
    assert np.allclose(out, out_mha, rtol=1e-6, atol=1e-7)


def test_unpermute_inverts_the_converter_permute():
    u = GOLD["unpermute"]
    rows, hd, cols = u["rows"], u["head_dim"], u["cols"]
    hf = np.arange(rows * cols, dtype=np.float32).reshape(rows, cols)
    # conversion/llama.py: reshape(h, 2, hd/2, cols).swapaxes(1, 2).reshape
    gguf = hf.reshape(rows // hd, 2, hd // 2, cols).swapaxes(1, 2).reshape(rows, cols)
    assert np.array_equal(oracle.unpermute_llama_qk(gguf, hd), hf)
    rng = np.random.default_rng(0)
    hf = rng.standard_normal((4 * 64, 5)).astype(np.float32)
    gguf = hf.reshape(4, 2, 32, 5).swapaxes(1, 2).reshape(256, 5)
    assert np.array_equal(oracle.unpermute_llama_qk(gguf, 64), hf)


# --------------------------------------------------------------- model

TINY = ModelConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                   num_key_value_heads=2, vocab_size=300, rms_norm_eps=1e-6, rope_theta=1e6)


@pytest.mark.parametrize("wtype,bias,tied", [(synth.Q8_0, True, True), (synth.F16, False, True),
                                             (synth.Q4_K, False, False)])
def test_model_forward_against_float64_statement(wtype, bias, tied):
    tensors = synth.synth_model(TINY, wtype, seed=42, tied=tied, qkv_bias=bias)
    m = oracle.Model(TINY, tensors)
    s = m.session(16)
    W = {}
    for t in tensors:
        n = int(np.prod(t.dims))
        W[t.name] = oracle.dequant_row(t.ggml_type, t.data, n).reshape(t.dims)
    m64 = ref64.Model64(TINY, W)
    for pos, tok in enumerate([5, 299, 0, 17, 123]):
        got = s.forward(tok, pos)
        want = m64.forward(tok, pos)
        err = np.max(np.abs(got - want)) / np.max(np.abs(want))
        assert err < 1e-4, (pos, err)


def test_llama_permuted_upload_matches_hf_layout():
    tensors = synth.synth_model(TINY, synth.F16, seed=3)
    m_hf = oracle.Model(TINY, tensors)
    perm = []
    for t in tensors:
        if t.name.endswith(("q_proj.weight", "k_proj.weight")):
            rows, cols = t.dims
            a = t.data.view(np.float16).reshape(rows, cols)
            a = a.reshape(rows // 64, 2, 32, cols).swapaxes(1, 2).reshape(rows, cols)
            perm.append(synth.Tensor(t.name, t.ggml_type, t.dims, np.ascontiguousarray(a).view(np.uint8).reshape(-1)))
        else:
            perm.append(t)
    m_p = oracle.Model(TINY, perm, llama_permuted=True)
    a, b = m_hf.session(4), m_p.session(4)
    assert np.array_equal(a.forward(7, 0), b.forward(7, 0))


def test_oracle_refuses_out_of_range():
    tensors = synth.synth_model(TINY, synth.F16, seed=1)
    s = oracle.Model(TINY, tensors).session(4)
    with pytest.raises(ValueError):
        s.forward(300, 0)
    with pytest.raises(ValueError):
        s.forward(1, 4)


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(12)
    xs = np.concatenate([rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
                         np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                                   3 * 2.0 ** -26, 2.0 ** -14, np.inf, -np.inf], np.float32)]).astype(np.float32)
    got = np.array([oracle.f32_to_f16(float(x)) for x in xs], np.uint16)
    want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert oracle.f32_to_f16(float("nan")) & 0x7c00 == 0x7c00


_O3_SCRIPT = r"""
import sys, numpy as np
sys.path.insert(0, sys.argv[1])
import oracle
from lokal_amd import synth
from lokal_amd.config import ModelConfig
oracle.select("o3")
oracle.set_threads(4)
cfg = ModelConfig(576, 1536, 2, 9, 3, 2048, 1e-5, 1e4)
m = oracle.Model(cfg, synth.synth_model(cfg, synth.Q8_0, seed=3, qkv_bias=True))
s = m.session(40)
out = [s.prefill(np.arange(1, 31, dtype=np.uint32) * 61)]
for i in range(5):
    out.append(s.forward(int(oracle.argmax(out[-1])), 30 + i))
np.save(sys.argv[2], np.stack(out))
"""


def test_o3_baseline_build_is_bit_identical(tmp_path):
    """The -O3 -mavx2 build timed as bench.py's CPU baseline computes the same
    bits as the -O2 parity build (vectorised lanes round as scalar ones; no
    contraction): prefill + 5 greedy steps of a 2-layer model, logits compared
    as raw bits."""
    import subprocess
    import sys
    root = Path(__file__).resolve().parent.parent
    out = tmp_path / "o3.npy"
    subprocess.run([sys.executable, "-c", _O3_SCRIPT, str(root), str(out)], check=True, timeout=300)
    cfg = ModelConfig(576, 1536, 2, 9, 3, 2048, 1e-5, 1e4)
    m = oracle.Model(cfg, synth.synth_model(cfg, synth.Q8_0, seed=3, qkv_bias=True))
    s = m.session(40)
    ref = [s.prefill(np.arange(1, 31, dtype=np.uint32) * 61)]
    for i in range(5):
        ref.append(s.forward(int(oracle.argmax(ref[-1])), 30 + i))
    got = np.load(out)
    assert np.array_equal(np.stack(ref).view(np.uint32), got.view(np.uint32))
