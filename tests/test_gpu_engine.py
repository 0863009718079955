"""End-to-end parity of the HIP decode step against the CPU oracle (lokal's
CPU path restated), through the C ABI's Engine / Session / Batcher.

Logits are within 1e-3 relative error (max|d| / max|want|); KV rows within
f16 rounding; greedy token streams are identical for the first 64 steps at the
benchmark shapes.  The GPU keeps an f16 KV cache and the CPU an f32 one, as
the reference's GPU and CPU paths do."""
import numpy as np
import pytest

import oracle
from lokal_amd import BatchRow, Engine, LokalHipError, synth
from lokal_amd.config import CONFIGS, ModelConfig

pytestmark = pytest.mark.gpu

TOL = 1e-3


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


TINY = ModelConfig(hidden_size=512, intermediate_size=1024, num_hidden_layers=3, num_attention_heads=8,
                   num_key_value_heads=2, vocab_size=1000, rms_norm_eps=1e-6, rope_theta=1e6)

KINDS = {
    "q8_0": dict(weight_type=synth.Q8_0, tied=True, qkv_bias=True),
    "q4_k": dict(weight_type=synth.Q4_K, tied=False, qkv_bias=False),
    "f16": dict(weight_type=synth.F16, tied=True, qkv_bias=False),
}


def build(cfg, kind, seed=0):
    k = KINDS[kind]
    tensors = synth.synth_model(cfg, k["weight_type"], seed, tied=k["tied"], qkv_bias=k["qkv_bias"])
    return tensors, Engine.from_tensors(cfg, tensors), oracle.Model(cfg, tensors)


@pytest.mark.parametrize("kind", list(KINDS))
def test_forward_logits_and_kv_match_oracle(kind):
    tensors, eng, om = build(TINY, kind)
    s, o = eng.session(64), om.session(64)
    rng = np.random.default_rng(1)
    toks = rng.integers(0, TINY.vocab_size, 40)
    for pos, t in enumerate(toks):
        got = s.forward(int(t), pos)
        want = o.forward(int(t), pos)
        assert rel_err(got, want) < TOL, (kind, pos)
    for layer in (0, TINY.num_hidden_layers - 1):
        for pos in (0, 39):
            for which_v in (False, True):
                want = o.kv(layer, pos, which_v)
                got = s.read_kv(layer, pos, which_v)
                assert np.allclose(got, want, rtol=2 ** -10, atol=1e-6 * np.abs(want).max()), (layer, pos, which_v)
    s.close()
    eng.close()


@pytest.mark.parametrize("kind", list(KINDS))
def test_prefill_and_greedy_decode_match_token_loop(kind):
    tensors, eng, om = build(TINY, kind, seed=3)
    prompt = np.random.default_rng(2).integers(0, TINY.vocab_size, 20).astype(np.uint32)
    a = eng.session(128)
    la = a.prefill(prompt)
    b = eng.session(128)
    for pos, t in enumerate(prompt):
        lb = b.forward(int(t), pos)
    assert np.array_equal(la, lb)
    # greedy on device == host loop of forward + argmax
    first = int(np.argmax(la))
    ids = a.decode_greedy(first, len(prompt), 30)
    cur, pos, host_ids = first, len(prompt), []
    for _ in range(30):
        lg = b.forward(cur, pos)
        cur = int(oracle.argmax(lg))
        host_ids.append(cur)
        pos += 1
    assert list(ids) == host_ids
    a.close()
    b.close()
    eng.close()


def test_batcher_rows_match_independent_sessions():
    tensors, eng, om = build(TINY, "q8_0", seed=4)
    bat = eng.batcher(3, 64)
    sess = [eng.session(64) for _ in range(3)]
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, TINY.vocab_size, n).astype(np.uint32) for n in (5, 9, 1)]
    for slot, p in enumerate(prompts):
        assert np.array_equal(bat.prefill(slot, p), sess[slot].prefill(p))
    rows = [BatchRow(int(rng.integers(0, 1000)), len(prompts[s]), s) for s in (2, 0, 1)]
    outs = bat.decode_step(rows)
    for r, out in zip(rows, outs):
        assert np.array_equal(out, sess[r.slot].forward(r.token, r.pos))
    bat.close()
    eng.close()


def test_refusals_are_errors_not_crashes():
    tensors, eng, om = build(TINY, "q8_0")
    s = eng.session(8)
    with pytest.raises(LokalHipError, match="outside the vocabulary"):
        s.forward(TINY.vocab_size, 0)
    with pytest.raises(LokalHipError, match="exceeds"):
        s.forward(1, 8)
    with pytest.raises(LokalHipError, match="exceeds"):
        s.decode_greedy(1, 4, 5)
    with pytest.raises(LokalHipError, match="empty prompt"):
        s.prefill(np.zeros(0, np.uint32))
    bad = [t for t in tensors if t.name != "model.layers.1.mlp.up_proj.weight"]
    with pytest.raises(LokalHipError, match="missing tensor"):
        Engine.from_tensors(TINY, bad)
    with pytest.raises(LokalHipError, match="head_dim"):
        Engine.from_tensors(TINY.with_(head_dim=32), tensors)
    s.close()
    eng.close()


def _greedy_identity(name, prompt_len, steps, seed=0):
    cfg, tensors = synth.synth_named(name, seed)
    eng = Engine.from_tensors(cfg, tensors)
    om = oracle.Model(cfg, tensors)
    del tensors
    prompt = np.random.default_rng(seed + 1).integers(0, cfg.vocab_size, prompt_len).astype(np.uint32)
    max_seq = prompt_len + steps
    s, o = eng.session(max_seq), om.session(max_seq)
    lg = s.prefill(prompt)
    lo = o.prefill(prompt)
    assert rel_err(lg, lo) < TOL
    first = int(oracle.argmax(lo))
    assert int(np.argmax(lg)) == first
    gpu_ids = [first] + list(s.decode_greedy(first, prompt_len, steps - 1))
    cpu_ids, margins = [first], []
    cur = first
    for i in range(steps - 1):
        lo = o.forward(cur, prompt_len + i)
        top2 = np.sort(lo)[-2:]
        margins.append(float(top2[1] - top2[0]))
        cur = int(oracle.argmax(lo))
        cpu_ids.append(cur)
    print(f"{name}: min top-2 margin {min(margins):.4g}")
    assert gpu_ids == cpu_ids
    s.close()
    eng.close()
    om.close()


@pytest.mark.parametrize("name", ["qwen2.5-0.5b-q8_0", "smollm2-135m", "tinyllama-1.1b-q4_k"])
def test_greedy_64_steps_identical_at_full_shape(name):
    _greedy_identity(name, prompt_len=16, steps=64)
