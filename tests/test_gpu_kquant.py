"""Q4_0, Q5_0, Q5_K and Q6_K weights on the HIP backend, against the CPU
oracle's dequant_row arms (src/gguf/dequant.rs:203-230, :484-533), through the
C ABI.

These types are repacked at upload (Q4_0 / Q5_0 as int8 + the block's f16
scale, Q5_K / Q6_K as int8 + an f32 (scale, min) pair per 16 values), so the
device must hand back the reference's values bit for bit: dequantization,
embedding gather and the one-hot matvec / GEMM are compared exactly; matvec,
GEMM and whole models with fp32 accumulation within 1e-3 relative error
(max|got - want| / max|want|), as for the other types.

Models: a Q4_K_M-style mix (Q4_K, with Q6_K for v_proj / down_proj of the
layers llama.cpp's mix rule picks and for lm_head), the same over Q5_K, and
all-Q5_0 / all-Q4_0 models of the Qwen2.5-0.5B layer widths, which run the
one-kernel step (their device form is Q8_0's)."""
import json
import os
from pathlib import Path

import numpy as np
import pytest

import oracle
from lokal_amd import BatchRow, Engine
from lokal_amd import kernels as K
from lokal_amd import synth
from lokal_amd.config import ModelConfig

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL_F16_KV = TOL + 2.0 ** -10
NEW = [synth.Q4_0, synth.Q5_0, synth.Q5_K, synth.Q6_K]


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def weight_bytes(t, rows, cols, seed):
    return synth.gen_weight(t, seed, f"w{rows}x{cols}", rows, cols).data


def oracle_rows(t, data, rows, cols):
    return oracle.dequant_row(t, data, rows * cols).reshape(rows, cols)


@pytest.mark.parametrize("t", NEW)
def test_dequant_rows_bit_exact(t):
    rows, cols = 64, 2048
    data = weight_bytes(t, rows, cols, 1)
    w = K.Weight(t, rows, cols, data)
    out = K.DeviceArray((rows - 5, cols))
    K.dequant_rows(w, 5, rows - 5, out)
    assert np.array_equal(out.numpy().view(np.uint32), oracle_rows(t, data, rows, cols)[5:].view(np.uint32))


def test_dequant_reference_hand_vectors():
    """The reference's own hand-built blocks (dequant.rs:580-594 Q4_0,
    :665-681 Q5_0, :733-748 Q5_K, :750-767 Q6_K) through the device."""
    gold = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
    seen = set()
    for v in gold["dequant"]:
        if v["type"] not in NEW:
            continue
        seen.add(v["type"])
        w = K.Weight(v["type"], 1, v["n"], np.array(v["bytes"], np.uint8))
        out = K.DeviceArray(v["n"])
        K.dequant_rows(w, 0, 1, out)
        y = out.numpy()
        for i, want in v["expect"].items():
            assert y[int(i)] == np.float32(want), v["ref"]
    assert seen == set(NEW)


@pytest.mark.parametrize("t", NEW)
@pytest.mark.parametrize("cols", [512, 2048])
def test_onehot_matvec_is_bit_exact(t, cols):
    rows = 96
    data = weight_bytes(t, rows, cols, 2)
    want = oracle_rows(t, data, rows, cols)
    w = K.Weight(t, rows, cols, data)
    x, y = K.DeviceArray(cols), K.DeviceArray(rows)
    for c in (0, 1, 15, 16, 31, 32, 255, 256, cols - 1, cols // 2 + 17):
        xh = np.zeros(cols, np.float32)
        xh[c] = 1.0
        x.upload(xh)
        K.matvec(w, x, y)
        assert np.array_equal(y.numpy(), want[:, c]), (t, cols, c)


@pytest.mark.parametrize("t", NEW)
@pytest.mark.parametrize("rows,cols", [(2048, 2048), (256, 2048), (2048, 5632), (32000, 2048)])
def test_matvec_matches_float64(t, rows, cols):
    data = weight_bytes(t, rows, cols, 3)
    wf = oracle_rows(t, data, rows, cols).astype(np.float64)
    x = np.random.default_rng(3).standard_normal(cols).astype(np.float32)
    w = K.Weight(t, rows, cols, data)
    xd, y = K.DeviceArray.from_numpy(x), K.DeviceArray(rows)
    K.matvec(w, xd, y)
    assert rel_err(y.numpy(), wf @ x) < TOL


@pytest.mark.parametrize("t", [synth.Q5_K, synth.Q6_K])
def test_matvec_bias_and_residual(t):
    rows, cols = 512, 1024
    data = weight_bytes(t, rows, cols, 6)
    wf = oracle_rows(t, data, rows, cols).astype(np.float64)
    rng = np.random.default_rng(6)
    x, b, r = (rng.standard_normal(n).astype(np.float32) for n in (cols, rows, rows))
    w = K.Weight(t, rows, cols, data)
    xd, bd, y = K.DeviceArray.from_numpy(x), K.DeviceArray.from_numpy(b), K.DeviceArray.from_numpy(r)
    K.matvec(w, xd, y, bias=bd, accumulate=True)
    assert rel_err(y.numpy(), r + (wf @ x + b)) < TOL


@pytest.mark.parametrize("t", NEW)
@pytest.mark.parametrize("rows,cols", [(2048, 2048), (256, 512), (1000, 5632)])
def test_matmul_one_hot_bit_exact_and_float64(t, rows, cols):
    data = weight_bytes(t, rows, cols, 7)
    ref = oracle_rows(t, data, rows, cols)
    w = K.Weight(t, rows, cols, data)
    hit = np.array([0, 1, 15, 16, 31, 32, 127, 128, cols // 2 + 3, cols - 1])
    n = len(hit)
    x = np.zeros((n, cols), np.float32)
    x[np.arange(n), hit] = 1.0
    xd, y = K.DeviceArray.from_numpy(x), K.DeviceArray((n, rows))
    K.matmul(w, xd, n, y)
    got = y.numpy()
    for i, c in enumerate(hit):
        assert np.array_equal(got[i], ref[:, c]), (i, c)
    for n_rows in (1, 17, 40):
        xr = np.random.default_rng(n_rows).standard_normal((n_rows, cols)).astype(np.float32)
        xd, y = K.DeviceArray.from_numpy(xr), K.DeviceArray((n_rows, rows))
        K.matmul(w, xd, n_rows, y)
        assert rel_err(y.numpy(), xr.astype(np.float64) @ ref.T.astype(np.float64)) < TOL, n_rows


@pytest.mark.parametrize("t", NEW)
def test_embed_gather_bit_exact(t):
    vocab, h = 32000, 2048
    data = synth.gen_weight(t, 9, "model.embed_tokens.weight", vocab, h).data
    table = K.Weight(t, vocab, h, data)
    ids = np.random.default_rng(9).integers(0, vocab, 32).astype(np.uint32)
    ids[:2] = [0, vocab - 1]
    idd, out = K.DeviceArray.from_numpy(ids), K.DeviceArray((32, h))
    K.embed_gather(table, idd, 32, out)
    y = out.numpy()
    rb = synth.row_bytes(t, h)
    for i, tok in enumerate(ids):
        row = data[int(tok) * rb:(int(tok) + 1) * rb]
        assert np.array_equal(y[i], oracle.dequant_row(t, row, h))


def test_typed_matvec_refuses_transcoded_types():
    """lkhip_q8_0_matvec takes GGUF Q8_0 only: a Q5_0 weight stored in the
    same device form is still refused."""
    from lokal_amd import LokalHipError
    w = K.Weight(synth.Q5_0, 8, 64, weight_bytes(synth.Q5_0, 8, 64, 0))
    with pytest.raises(LokalHipError, match="q8_0_matvec: weight is Q5_0"):
        K.q8_0_matvec(w, K.DeviceArray(64), K.DeviceArray(8))


# ----------------------------------------------------------------- models

MIX_CFG = ModelConfig(512, 1024, 8, 8, 2, 1000, 1e-5, 1e4)  # 8 layers: the mix rule picks 0, 3, 6, 7
QWEN_CFG = ModelConfig(896, 4864, 3, 14, 2, 1000, 1e-6, 1e6)


def mixed_model(base, seed):
    tensors = synth.synth_model(MIX_CFG, base, seed, tied=False, type_of=synth.k_mix(base, MIX_CFG))
    types = {t.name: t.ggml_type for t in tensors}
    assert types["model.layers.3.self_attn.v_proj.weight"] == synth.Q6_K
    assert types["model.layers.1.mlp.down_proj.weight"] == base
    assert types["lm_head.weight"] == synth.Q6_K
    return MIX_CFG, tensors


def _fused(on):
    class Ctx:
        def __enter__(self):
            self.old = os.environ.get("LKHIP_FUSED")
            os.environ["LKHIP_FUSED"] = "1" if on else "0"

        def __exit__(self, *a):
            if self.old is None:
                del os.environ["LKHIP_FUSED"]
            else:
                os.environ["LKHIP_FUSED"] = self.old
    return Ctx()


MODELS = {
    "q4_k_m": lambda s: mixed_model(synth.Q4_K, s),
    "q5_k_m": lambda s: mixed_model(synth.Q5_K, s),
    "q5_0": lambda s: (QWEN_CFG, synth.synth_model(QWEN_CFG, synth.Q5_0, s, tied=True, qkv_bias=True)),
    "q4_0": lambda s: (QWEN_CFG, synth.synth_model(QWEN_CFG, synth.Q4_0, s, tied=True, qkv_bias=True)),
}


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("kv", ["f32", "f16"])
@pytest.mark.parametrize("kind", list(MODELS))
def test_decode_logits_match_oracle(kind, kv, fused):
    cfg, tensors = MODELS[kind](0)
    with _fused(fused):
        eng = Engine.from_tensors(cfg, tensors)
    om = oracle.Model(cfg, tensors)
    s, o = eng.session(80, kv_dtype=kv), om.session(80, kv_f16=(kv == "f16"))
    toks = np.random.default_rng(1).integers(0, cfg.vocab_size, 66)
    worst = 0.0
    for pos, t in enumerate(toks):
        e = rel_err(s.forward(int(t), pos), o.forward(int(t), pos))
        worst = max(worst, e)
        assert e < TOL, (kind, kv, pos, e)
    print(f"{kind}/{kv}/fused={fused}: worst logits rel err {worst:.3g}")
    s.close()
    o.close()
    eng.close()
    om.close()


@pytest.mark.parametrize("kind", list(MODELS))
def test_prefill_batcher_and_greedy_match(kind):
    """Chunked prefill (rows path, per-projection QKV GEMMs where q/k/v types
    differ), a Batcher step over ragged sequences, and 32 greedy steps on the
    device against the oracle with an f32 cache."""
    cfg, tensors = MODELS[kind](2)
    eng = Engine.from_tensors(cfg, tensors)
    om = oracle.Model(cfg, tensors)
    rng = np.random.default_rng(2)
    prompt = rng.integers(0, cfg.vocab_size, 37).astype(np.uint32)
    s, o = eng.session(80, kv_dtype="f32"), om.session(80)
    lg, lo = s.prefill(prompt), o.prefill(prompt)
    assert rel_err(lg, lo) < TOL
    first = int(oracle.argmax(lo))
    ids = list(s.decode_greedy(first, len(prompt), 32))
    cur, want = first, []
    for k in range(32):
        cur = int(oracle.argmax(o.forward(cur, len(prompt) + k)))
        want.append(cur)
    assert ids == want
    s.close()
    o.close()

    lens = (5, 40, 1)
    prompts = [rng.integers(0, cfg.vocab_size, n).astype(np.uint32) for n in lens]
    bat = eng.batcher(len(lens), 64)
    orc = [om.session(64, kv_f16=True) for _ in lens]
    for slot, p in enumerate(prompts):
        assert rel_err(bat.prefill(slot, p), orc[slot].prefill(p)) < TOL_F16_KV
    rows = [BatchRow(int(rng.integers(0, cfg.vocab_size)), lens[sl], sl) for sl in (2, 0, 1)]
    for r, out in zip(rows, bat.decode_step(rows)):
        assert rel_err(out, orc[r.slot].forward(r.token, r.pos)) < TOL_F16_KV, r.slot
    bat.close()
    for x in orc:
        x.close()
    eng.close()
    om.close()


@pytest.mark.parametrize("attn", ["mfma", "valu"])
@pytest.mark.parametrize("kind", ["q4_k_m", "q5_0"])
def test_batcher_per_layer_step_rope_in_attention(kind, attn, monkeypatch):
    """Batcher steps of 12 rows (the per-layer launches), where the attention
    launch rotates q and appends each row's own k / v: on a mixed model whose
    q/k/v types differ in some layers (per-projection QKV sums, no split-K
    partials) and on a model with q/k/v biases; with the vector-ALU kernel the
    RoPE + KV append runs as its own launch first.  Ragged positions, rows
    out of slot order, three steps, each row against the oracle's sequence."""
    monkeypatch.setenv("LKHIP_ATTN", attn)
    cfg, tensors = MODELS[kind](4)
    eng = Engine.from_tensors(cfg, tensors)
    om = oracle.Model(cfg, tensors)
    rng = np.random.default_rng(4)
    lens = (3, 70, 1, 33, 12, 5, 64, 2, 17, 40, 9, 1)
    bat = eng.batcher(len(lens), 128)
    orc = [om.session(128, kv_f16=True) for _ in lens]
    for slot, n in enumerate(lens):
        p = rng.integers(0, cfg.vocab_size, n).astype(np.uint32)
        assert rel_err(bat.prefill(slot, p), orc[slot].prefill(p)) < TOL_F16_KV
    pos = list(lens)
    for step in range(3):
        order = list(rng.permutation(len(lens)))
        rows = [BatchRow(int(rng.integers(0, cfg.vocab_size)), pos[s], int(s)) for s in order]
        for r, out in zip(rows, bat.decode_step(rows)):
            assert rel_err(out, orc[r.slot].forward(r.token, r.pos)) < TOL_F16_KV, (step, r.slot)
            pos[r.slot] += 1
    bat.close()
    for x in orc:
        x.close()
    eng.close()
    om.close()
