"""The multi-row path through the C ABI: the matrix-core GEMM (lkhip_matmul),
chunked prefill and forward_batch of a Session, and the Batcher's decode step
and device greedy loop, against the CPU oracle (lokal's CPU path restated).

The GEMM is pinned three ways: a one-hot activation row returns a weight
column bit-for-bit (every other product is an exact zero, so this fixes the
lane/row/column index maps of the MFMA tiles), random rows agree with a
float64 product of the oracle's dequantized weights to fp32 rounding, and
split-K, bias, residual accumulation and row strides are exercised at the
model widths.  End to end, logits are within 1e-3 relative error of the
oracle (summation order is the only difference) and greedy ids agree."""
import numpy as np
import pytest

import oracle
from lokal_amd import BatchRow, Engine, LokalHipError, synth
from lokal_amd import kernels as K
from lokal_amd.config import ModelConfig

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL_F16_KV = TOL + 2.0 ** -10


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def dequant(t, data, rows, cols):
    return oracle.dequant_row(t, data, rows * cols).reshape(rows, cols)


SHAPES = [  # (type, rows, cols)
    (synth.Q8_0, 896, 896), (synth.Q8_0, 1152, 896), (synth.Q8_0, 896, 4864), (synth.Q8_0, 4864, 896),
    (synth.F16, 576, 576), (synth.F16, 1536, 576), (synth.F16, 576, 1536),
    (synth.Q4_K, 2048, 2048), (synth.Q4_K, 2048, 5632), (synth.Q4_K, 256, 512),
]


@pytest.mark.parametrize("t,rows,cols", SHAPES)
@pytest.mark.parametrize("n", [8, 150])
def test_matmul_one_hot_is_bit_exact(t, rows, cols, n):
    """One-hot activation rows return weight columns bit for bit (this pins
    the tile and lane maps); 150 rows take the prefill-sized tiles, with the
    one-hot rows spread over its column blocks and zero rows between."""
    data = synth.gen_weight(t, 7, f"w{rows}x{cols}", rows, cols).data
    w = K.Weight(t, rows, cols, data)
    ref = dequant(t, data, rows, cols)
    cols_hit = np.array([0, 1, 31, 32, 127, 128, cols // 2 + 3, cols - 1])
    at = np.arange(len(cols_hit)) if n == len(cols_hit) else np.array([0, 17, 40, 63, 64, 100, 128, 149])
    x = np.zeros((n, cols), np.float32)
    x[at, cols_hit] = 1.0
    xd, y = K.DeviceArray.from_numpy(x), K.DeviceArray((n, rows))
    K.matmul(w, xd, n, y)
    got = y.numpy()
    for i, c in zip(at, cols_hit):
        assert np.array_equal(got[i], ref[:, c]), (i, c)
    assert not np.delete(got, at, axis=0).any()


@pytest.mark.parametrize("t,rows,cols", SHAPES)
@pytest.mark.parametrize("n_rows", [1, 5, 16, 17, 40, 130, 256])
def test_matmul_matches_float64(t, rows, cols, n_rows):
    data = synth.gen_weight(t, 3, f"w{rows}x{cols}", rows, cols).data
    w = K.Weight(t, rows, cols, data)
    ref = dequant(t, data, rows, cols).astype(np.float64)
    rng = np.random.default_rng(n_rows)
    x = rng.standard_normal((n_rows, cols)).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32)
    y0 = rng.standard_normal((n_rows, rows)).astype(np.float32)
    xd, bd = K.DeviceArray.from_numpy(x), K.DeviceArray.from_numpy(bias)
    y = K.DeviceArray.from_numpy(y0)
    K.matmul(w, xd, n_rows, y, bias=bd)
    want = x.astype(np.float64) @ ref.T + bias
    got = y.numpy()
    # fp32 accumulation over cols products: relative to the row's |terms| sum
    scale = np.abs(x).astype(np.float64) @ np.abs(ref).T
    assert np.max(np.abs(got - want) / (scale + 1e-30)) < 1e-6
    assert rel_err(got, want) < 1e-5
    # residual accumulation (src/model.rs:235-237)
    y.upload(y0)
    K.matmul(w, xd, n_rows, y, accumulate=True)
    assert rel_err(y.numpy(), y0 + x.astype(np.float64) @ ref.T) < 1e-5


@pytest.mark.parametrize("t,rows,cols", [(synth.Q8_0, 20000, 896), (synth.F16, 16400, 576), (synth.Q8_0, 16400, 512)])
def test_matmul_wide_lm_head_shapes(t, rows, cols, monkeypatch):
    """Wide, shallow store GEMMs (the lm_head: >= 16384 rows, K <= 896, no
    bias) take gemm16_wide_kernel, which converts X once per block: one-hot
    columns bit-exact, random rows within the float64 bound, an output row
    stride, and every result bit-identical to gemm16_kernel's
    (LKHIP_GEMM_WIDE=0), at 1-64 activation rows."""
    data = synth.gen_weight(t, 9, f"w{rows}x{cols}", rows, cols).data
    w = K.Weight(t, rows, cols, data)
    ref = dequant(t, data, rows, cols).astype(np.float64)
    rng = np.random.default_rng(rows + cols)
    for n in (1, 5, 16, 17, 40, 64):
        x = rng.standard_normal((n, cols)).astype(np.float32)
        hit = rng.integers(0, cols, n)
        x[: n // 2] = 0.0
        x[np.arange(n // 2), hit[: n // 2]] = 1.0  # the first half one-hot
        xd = K.DeviceArray.from_numpy(x)
        outs = []
        for wide in ("1", "0"):
            monkeypatch.setenv("LKHIP_GEMM_WIDE", wide)
            y = K.DeviceArray((n, rows + 16))
            y.zero()
            K.matmul(w, xd, n, y, ldy=rows + 16)
            outs.append(y.numpy())
        got, base = outs
        assert np.array_equal(got, base), n
        assert not got[:, rows:].any()
        got = got[:, :rows]
        for i in range(n // 2):
            assert np.array_equal(got[i], ref[:, hit[i]].astype(np.float32)), (n, i)
        want = x.astype(np.float64) @ ref.T
        scale = np.abs(x).astype(np.float64) @ np.abs(ref).T
        assert np.max(np.abs(got - want) / (scale + 1e-30)) < 1e-6, n


def test_matmul_row_strides():
    t, rows, cols, n = synth.Q8_0, 896, 896, 7
    data = synth.gen_weight(t, 5, "w", rows, cols).data
    w = K.Weight(t, rows, cols, data)
    ref = dequant(t, data, rows, cols).astype(np.float64)
    x = np.random.default_rng(1).standard_normal((n, cols + 32)).astype(np.float32)
    y = K.DeviceArray((n, rows + 48))
    y.zero()
    K.matmul(w, K.DeviceArray.from_numpy(x), n, y, ldx=cols + 32, ldy=rows + 48)
    got = y.numpy()
    assert rel_err(got[:, :rows], x[:, :cols].astype(np.float64) @ ref.T) < 1e-5
    assert not got[:, rows:].any()


def test_matmul_ragged_rows_and_refusals():
    """A row count off the 16-row tile (a vocabulary like 1000) is computed and
    nothing past the last row is written; strides it cannot load are refused."""
    t, rows, cols, n = synth.Q8_0, 1000, 64, 3
    data = synth.gen_weight(t, 1, "w", rows, cols).data
    w = K.Weight(t, rows, cols, data)
    x = np.random.default_rng(2).standard_normal((n, cols)).astype(np.float32)
    y = K.DeviceArray((n, rows + 8))
    y.upload(np.full((n, rows + 8), 7.0, np.float32))
    K.matmul(w, K.DeviceArray.from_numpy(x), n, y, ldy=rows + 8)
    got = y.numpy()
    assert rel_err(got[:, :rows], x.astype(np.float64) @ dequant(t, data, rows, cols).T) < 1e-5
    assert np.all(got[:, rows:] == 7.0)
    n2 = 131  # the prefill-sized tiles, ragged in both directions
    x2 = np.random.default_rng(3).standard_normal((n2, cols)).astype(np.float32)
    y2 = K.DeviceArray((n2, rows + 8))
    y2.upload(np.full((n2, rows + 8), 7.0, np.float32))
    K.matmul(w, K.DeviceArray.from_numpy(x2), n2, y2, ldy=rows + 8)
    got2 = y2.numpy()
    assert rel_err(got2[:, :rows], x2.astype(np.float64) @ dequant(t, data, rows, cols).T) < 1e-5
    assert np.all(got2[:, rows:] == 7.0)
    with pytest.raises(LokalHipError, match="multiple of 4"):
        K.matmul(w, K.DeviceArray((n, 70)), n, y, ldx=66)


KINDS = {
    "q8_0": dict(cfg=ModelConfig(896, 4864, 3, 14, 2, 1000, 1e-6, 1e6), weight_type=synth.Q8_0, tied=True,
                 qkv_bias=True),
    "q4_k": dict(cfg=ModelConfig(2048, 5632, 2, 32, 4, 1008, 1e-5, 1e4), weight_type=synth.Q4_K, tied=False,
                 qkv_bias=False),
    "f16": dict(cfg=ModelConfig(576, 1536, 3, 9, 3, 1008, 1e-5, 1e4), weight_type=synth.F16, tied=True,
                qkv_bias=False),
}


def build(kind, seed=0):
    k = KINDS[kind]
    cfg = k["cfg"]
    tensors = synth.synth_model(cfg, k["weight_type"], seed, tied=k["tied"], qkv_bias=k["qkv_bias"])
    return cfg, Engine.from_tensors(cfg, tensors), oracle.Model(cfg, tensors)


@pytest.mark.parametrize("kind", list(KINDS))
@pytest.mark.parametrize("n_rows", [2, 3])
def test_batcher_head_rows_kernel_matches_the_gemm_head(kind, n_rows, monkeypatch):
    """The 2-row one-kernel step ends with lm_head_rows_kernel (final norm +
    lm_head of both rows in one launch; 3 rows keep the GEMM either way);
    LKHIP_HEAD_ROWS=0 keeps the norm launch + lm_head GEMM.  Same rows, same steps: logits within 1e-5 of each
    other (different summation orders), the oracle within the f16-KV bound."""
    set_batch_path(monkeypatch, "fused")
    cfg, eng, om = build(kind, seed=40 + n_rows)
    rng = np.random.default_rng(40 + n_rows)
    lens = [33, 70, 5, 64][:n_rows]
    prompts = [rng.integers(0, cfg.vocab_size, n).astype(np.uint32) for n in lens]
    toks = [[int(rng.integers(0, cfg.vocab_size)) for _ in lens] for _ in range(3)]
    outs = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("LKHIP_HEAD_ROWS", mode)
        bat = eng.batcher(4, 128)
        for i, p in enumerate(prompts):
            bat.prefill(i, p)
        outs[mode] = [bat.decode_step([BatchRow(t[i], lens[i] + k, i) for i in range(n_rows)])
                      for k, t in enumerate(toks)]
        bat.close()
    orc = [om.session(128, kv_f16=True) for _ in lens]
    for i, p in enumerate(prompts):
        orc[i].prefill(p)
    for k, t in enumerate(toks):
        for i in range(n_rows):
            assert rel_err(outs["1"][k][i], outs["0"][k][i]) < 1e-5, (k, i)
            assert rel_err(outs["1"][k][i], orc[i].forward(t[i], lens[i] + k)) < TOL_F16_KV, (k, i)
    eng.close()
    om.close()


@pytest.mark.parametrize("kind", list(KINDS))
@pytest.mark.parametrize("n", [1, 37, 600])
def test_chunked_prefill_matches_oracle(kind, n):
    """Prefill through the rows path (512-position chunks) against the CPU
    path's token loop: last logits within 1e-3, every KV row of layer 0 within
    one f16 ulp (f16 cache) or 1e-5 (f32 cache)."""
    cfg, eng, om = build(kind, seed=2)
    prompt = np.random.default_rng(n).integers(0, cfg.vocab_size, n).astype(np.uint32)
    for kv in ("f32", "f16"):
        s, o = eng.session(n + 4, kv_dtype=kv), om.session(n + 4, kv_f16=(kv == "f16"))
        lg, lo = s.prefill(prompt), o.prefill(prompt)
        assert rel_err(lg, lo) < (TOL if kv == "f32" else TOL_F16_KV), (kv, rel_err(lg, lo))
        for pos in sorted({0, n // 2, n - 1}):
            for which_v in (False, True):
                got, want = s.read_kv(0, pos, which_v), o.kv(0, pos, which_v)
                if kv == "f32":
                    assert rel_err(got, want) < 1e-5
                else:  # one f16 step, or fp32 noise on the row's scale
                    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
                    excess = float(np.max(np.abs(got - want) - ulp - 1e-5 * np.max(np.abs(want))))
                    assert excess <= 0.0, (pos, which_v, excess)
        # decode continues from the batched prefill's cache
        t = int(np.argmax(lo))
        assert rel_err(s.forward(t, n), o.forward(t, n)) < (TOL if kv == "f32" else TOL_F16_KV)
        s.close()
        o.close()
    eng.close()
    om.close()


@pytest.mark.parametrize("kind", list(KINDS))
def test_forward_batch_matches_oracle_per_position(kind):
    cfg, eng, om = build(kind, seed=4)
    ids = np.random.default_rng(4).integers(0, cfg.vocab_size, 70).astype(np.uint32)
    s, o = eng.session(80, kv_dtype="f32"), om.session(80)
    got = s.forward_batch(ids[:10], 0)  # one pass
    got = np.concatenate([got, s.forward_batch(ids[10:], 10)])  # 64 + 6 rows
    for pos, t in enumerate(ids):
        assert rel_err(got[pos], o.forward(int(t), pos)) < TOL, pos
    s.close()
    o.close()
    eng.close()
    om.close()


# The Batcher's three device paths: the persistent multi-row step
# (batch_step.hip, "bstep"), the multi-row one-kernel step (fused_rows.hip, up
# to 8 rows, "fused") and the per-layer launches ("layers").
BATCH_PATHS = ["bstep", "fused", "layers"]


def set_batch_path(monkeypatch, path):
    monkeypatch.setenv("LKHIP_BATCH_FUSED", "0" if path == "layers" else "1")
    monkeypatch.setenv("LKHIP_BATCH_STEP", "1" if path == "bstep" else "0")
    monkeypatch.setenv("LKHIP_BATCH_STEP_MIN", "2")


@pytest.fixture
def batch_path(request, monkeypatch):
    set_batch_path(monkeypatch, request.param)
    return request.param


@pytest.mark.parametrize("batch_path", BATCH_PATHS, indirect=True)
@pytest.mark.parametrize("kind", list(KINDS))
def test_batcher_decode_step_matches_independent_sequences(kind, batch_path):
    """Rows of different slots, lengths and positions in one step: each row's
    logits equal the oracle's for its own sequence (src/engine.rs:42-47)."""
    cfg, eng, om = build(kind, seed=5)
    rng = np.random.default_rng(5)
    lens = (5, 130, 1, 64)
    prompts = [rng.integers(0, cfg.vocab_size, n).astype(np.uint32) for n in lens]
    bat = eng.batcher(len(lens), 256)
    orc = [om.session(256, kv_f16=True) for _ in lens]
    for slot, p in enumerate(prompts):
        assert rel_err(bat.prefill(slot, p), orc[slot].prefill(p)) < TOL_F16_KV
    pos = list(lens)
    for step in range(3):
        order = [(step + i) % len(lens) for i in range(len(lens))][: len(lens) - (step == 1)]
        rows = [BatchRow(int(rng.integers(0, cfg.vocab_size)), pos[s], s) for s in order]
        outs = bat.decode_step(rows)
        for r, out in zip(rows, outs):
            assert rel_err(out, orc[r.slot].forward(r.token, r.pos)) < TOL_F16_KV, (step, r.slot)
            pos[r.slot] += 1
    bat.close()
    eng.close()
    om.close()


@pytest.mark.parametrize("batch_path", BATCH_PATHS, indirect=True)
def test_batcher_greedy_matches_per_sequence_greedy(batch_path):
    """lkhip_batch_decode_greedy: every row's ids equal that sequence's own
    greedy ids from a per-sequence decode_step loop with host argmax, and the
    oracle's ids up to a near-tie within tolerance."""
    cfg, eng, om = build("q8_0", seed=6)
    rng = np.random.default_rng(6)
    lens = (17, 3, 40)
    steps = 24
    prompts = [rng.integers(0, cfg.vocab_size, n).astype(np.uint32) for n in lens]
    bat = eng.batcher(len(lens), 128)
    ref = eng.batcher(len(lens), 128)
    first = []
    for slot, p in enumerate(prompts):
        lg = bat.prefill(slot, p)
        ref.prefill(slot, p)
        first.append(int(np.argmax(lg)))
    rows = [BatchRow(first[s], lens[s], s) for s in range(len(lens))]
    ids = bat.decode_greedy(rows, steps)
    assert ids.shape == (steps, len(lens))
    cur = list(first)
    for k in range(steps):
        outs = ref.decode_step([BatchRow(cur[s], lens[s] + k, s) for s in range(len(lens))])
        cur = [int(oracle.argmax(o)) for o in outs]
        assert list(ids[k]) == cur, k
    # against the CPU path, row by row
    for s, p in enumerate(prompts):
        o = om.session(128, kv_f16=True)
        lo = o.prefill(p)
        t, agree = int(oracle.argmax(lo)), 0
        for k in range(steps):
            t = int(oracle.argmax(o.forward(t, lens[s] + k)))
            if t != ids[k, s]:
                break
            agree += 1
        o.close()
        print(f"slot {s}: {agree}/{steps} greedy ids agree with the CPU path")
        assert agree >= steps // 2
    bat.close()
    ref.close()
    eng.close()
    om.close()


def test_batcher_refusals():
    cfg, eng, om = build("q8_0")
    bat = eng.batcher(2, 16)
    with pytest.raises(LokalHipError, match="out of range"):
        bat.decode_step([BatchRow(1, 0, 2)])
    with pytest.raises(LokalHipError, match="twice"):
        bat.decode_step([BatchRow(1, 0, 1), BatchRow(2, 0, 1)])
    with pytest.raises(LokalHipError, match="exceeds"):
        bat.decode_step([BatchRow(1, 16, 0)])
    with pytest.raises(LokalHipError, match="exceeds"):
        bat.decode_greedy([BatchRow(1, 10, 0)], 8)
    with pytest.raises(LokalHipError, match="outside the vocabulary"):
        bat.prefill(0, np.array([cfg.vocab_size], np.uint32))
    bat.close()
    eng.close()
    om.close()


@pytest.mark.parametrize("kind", ["q8_0", "f16", "q4_k"])
@pytest.mark.parametrize("n_rows", [1, 2, 3, 4, 5, 6, 7, 8])
def test_batcher_fused_step_every_row_count(kind, n_rows, monkeypatch):
    """The one-kernel Batcher step at 1-8 rows (1 row: the single-row kernel;
    2-8 rows: the 2-, 4- and 8-row kernels, fewer rows padded; at the Q4_K
    shape the 8-row kernel's LDS does not fit, so 5-8 rows run the per-layer
    launches there), on slots
    other than 0..n-1: every row against the oracle over steps that cross a
    64-position tile, then greedy ids against the oracle's."""
    set_batch_path(monkeypatch, "fused")
    cfg, eng, om = build(kind, seed=10 + n_rows)
    rng = np.random.default_rng(n_rows)
    lens = [60, 3, 127, 64, 1, 100, 20, 63][:n_rows]
    slots = [i + 8 - n_rows for i in range(n_rows)]
    prompts = [rng.integers(0, cfg.vocab_size, n).astype(np.uint32) for n in lens]
    bat = eng.batcher(8, 192)
    orc = [om.session(192, kv_f16=True) for _ in lens]
    for i, p in enumerate(prompts):
        bat.prefill(slots[i], p)
        orc[i].prefill(p)
    pos = list(lens)
    for step in range(6):
        toks = [int(rng.integers(0, cfg.vocab_size)) for _ in lens]
        outs = bat.decode_step([BatchRow(toks[i], pos[i], slots[i]) for i in range(n_rows)])
        for i in range(n_rows):
            assert rel_err(outs[i], orc[i].forward(toks[i], pos[i])) < TOL_F16_KV, (step, i)
            pos[i] += 1
    first = [int(rng.integers(0, cfg.vocab_size)) for _ in lens]
    ids = bat.decode_greedy([BatchRow(first[i], pos[i], slots[i]) for i in range(n_rows)], 12)
    for i in range(n_rows):
        t, want = first[i], []
        for k in range(12):
            t = int(oracle.argmax(orc[i].forward(t, pos[i] + k)))
            want.append(t)
        agree = next((k for k in range(12) if ids[k, i] != want[k]), 12)
        print(f"{kind} rows={n_rows} row {i}: {agree}/12 greedy ids agree with the CPU path")
        assert agree >= 6
    bat.close()
    eng.close()
    om.close()


@pytest.mark.parametrize("kind", list(KINDS))
def test_batcher_one_row_steps_mixed_with_multi_row_steps_and_a_session(kind, monkeypatch):
    """A 1-row decode_step runs the single-row one-kernel step on the
    Batcher's row table (token, position, KV slot); it interleaves with
    multi-row steps on the same slots and with a Session of the same engine
    stepping in between, and every row stays equal to the oracle's own
    sequence (src/engine.rs:42-47)."""
    set_batch_path(monkeypatch, "fused")
    cfg, eng, om = build(kind, seed=21)
    rng = np.random.default_rng(21)
    lens = [70, 2, 33]
    slots = [5, 0, 3]
    prompts = [rng.integers(0, cfg.vocab_size, n).astype(np.uint32) for n in lens]
    bat = eng.batcher(6, 160)
    orc = [om.session(160, kv_f16=True) for _ in lens]
    for i, p in enumerate(prompts):
        bat.prefill(slots[i], p)
        orc[i].prefill(p)
    sp = rng.integers(0, cfg.vocab_size, 9).astype(np.uint32)
    ses = eng.session(160)
    so = om.session(160, kv_f16=True)
    ses.prefill(sp)
    so.prefill(sp)
    spos = len(sp)
    pos = list(lens)
    # 1 row, all rows, 1 row of another slot, 2 rows, 1 row ...
    plan = [[0], [0, 1, 2], [2], [1, 0], [1], [2], [0, 2], [0]]
    for step, which in enumerate(plan):
        toks = {i: int(rng.integers(0, cfg.vocab_size)) for i in which}
        outs = bat.decode_step([BatchRow(toks[i], pos[i], slots[i]) for i in which])
        for i, out in zip(which, outs):
            assert rel_err(out, orc[i].forward(toks[i], pos[i])) < TOL_F16_KV, (step, i)
            pos[i] += 1
        t = int(rng.integers(0, cfg.vocab_size))
        assert rel_err(ses.forward(t, spos), so.forward(t, spos)) < TOL_F16_KV, step
        spos += 1
    ses.close()
    so.close()
    bat.close()
    eng.close()
    om.close()


@pytest.mark.parametrize("batch_path", BATCH_PATHS, indirect=True)
def test_batcher_graph_replay_matches_direct_launches(batch_path, monkeypatch):
    """LKHIP_GRAPH=1 replays the Batcher's steps as HIP graphs (by default
    they are launched directly): greedy ids and decode_step logits equal the
    direct launches' bit for bit, at 1 and 3 rows, over repeated calls."""
    cfg, eng, om = build("q8_0", seed=33)
    rng = np.random.default_rng(33)
    lens = (9, 30, 2)
    prompts = [rng.integers(0, cfg.vocab_size, n).astype(np.uint32) for n in lens]
    runs = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("LKHIP_GRAPH", mode)
        bat = eng.batcher(3, 128)
        for slot, p in enumerate(prompts):
            bat.prefill(slot, p)
        out = []
        pos = list(lens)
        for n in (1, 3, 1, 3):
            rows = [BatchRow(int(7 + s), pos[s], s) for s in range(n)]
            out.append([o.copy() for o in bat.decode_step(rows)])
            for s in range(n):
                pos[s] += 1
        ids = bat.decode_greedy([BatchRow(5 + s, pos[s], s) for s in range(3)], 12)
        runs[mode] = (out, ids.copy())
        bat.close()
    for a, b in zip(runs["1"][0], runs["0"][0]):
        for x, y in zip(a, b):
            assert np.array_equal(x, y)
    assert np.array_equal(runs["1"][1], runs["0"][1])
    eng.close()
    om.close()


def _batcher_against_oracle_on_its_cache(kind, max_seq, lens, plan, seed):
    """Prefill each slot through the Batcher, hand the oracle every slot's f16
    cache rows, then run the steps of `plan` (lists of slots stepped
    together): every row's logits must match the oracle continuing from the
    same cache, within the f16 bar (the current row's own K/V is rounded by
    each side), and after each step the oracle takes the row the GPU wrote."""
    cfg, eng, om = build(kind, seed=seed)
    rng = np.random.default_rng(seed)
    bat = eng.batcher(len(lens), max_seq)
    orc = []
    L = cfg.num_hidden_layers
    for slot, n in enumerate(lens):
        bat.prefill(slot, rng.integers(0, cfg.vocab_size, n).astype(np.uint32))
        o = om.session(max_seq, kv_f16=True)
        for layer in range(L):
            for which_v in (False, True):
                o.load_kv(layer, 0, which_v, bat.read_kv_rows(slot, layer, 0, n, which_v))
        orc.append(o)
    print(f"{kind} max_seq {max_seq}: {len(lens)} slots prefilled, caches loaded", flush=True)
    pos = list(lens)
    worst = 0.0
    for step, slots in enumerate(plan):
        rows = [BatchRow(int(rng.integers(0, cfg.vocab_size)), pos[s], s) for s in slots]
        outs = bat.decode_step(rows)
        for r, out in zip(rows, outs):
            e = rel_err(out, orc[r.slot].forward(r.token, r.pos))
            worst = max(worst, e)
            assert e < TOL_F16_KV, (step, r.slot, r.pos, e)
            for layer in range(L):
                for which_v in (False, True):
                    orc[r.slot].load_kv(layer, r.pos, which_v, bat.read_kv_rows(r.slot, layer, r.pos, 1, which_v))
            pos[r.slot] += 1
    print(f"{kind} max_seq {max_seq}: {len(plan)} steps, worst logits rel err {worst:.3g}, last positions {pos}")
    for o in orc:
        o.close()
    bat.close()
    eng.close()
    om.close()
    return pos


@pytest.mark.parametrize("kind", ["q8_0", "f16"])
def test_batcher_rows_near_4096_positions_across_the_path_switch(kind):
    """A Batcher whose cache holds 4096 positions runs 2-row steps on the
    multi-row one-kernel step up to position 4095 (its attention stage takes
    64 tiles per row there), 3-row steps on the per-layer launches (too many
    attention items for one grid) and 1-row steps on the single-row kernel,
    interleaved on the same slots up to the cache's last position."""
    plan = [[0, 1], [0, 1, 2], [2], [1, 2], [0, 1, 2, 3], [3], [0, 3]] * 3
    lens = [4060, 4070, 4050, 4000]
    pos = _batcher_against_oracle_on_its_cache(kind, 4096, lens, plan, seed=40)
    assert max(pos) <= 4096


@pytest.mark.parametrize("kind", ["q8_0", "f16"])
def test_batcher_rows_from_4000_to_4200_positions(kind):
    """A Batcher past the multi-row kernel's 4096-position cache runs its
    multi-row steps as per-layer launches and 1-row steps on the single-row
    kernel: rows cross position 4096 (the 65th 64-position tile) in both."""
    plan = [[0, 1, 2]] * 6 + [[0]] * 3 + [[1, 2]] * 4 + [[2]] * 2
    lens = [4090, 4093, 4095]
    pos = _batcher_against_oracle_on_its_cache(kind, 4200, lens, plan, seed=41)
    assert min(pos) > 4096


def test_batcher_four_rows_at_16k_positions():
    """BASELINE config 5's batched decode shape: 4 concurrent sequences with
    independent contexts near 16384 positions, one query token each per step
    (4-row steps), then single-row steps (the one-kernel step with 64 chunks
    of 4 tiles per head)."""
    plan = [[0, 1, 2, 3]] * 4 + [[1]] * 2 + [[0, 1, 2, 3]] * 2
    lens = [16300, 16000, 16200, 16100]
    _batcher_against_oracle_on_its_cache("q8_0", 16384, lens, plan, seed=42)


@pytest.mark.parametrize("kind", list(KINDS))
@pytest.mark.parametrize("n_rows", [2, 9, 16, 33, 64])
def test_batcher_persistent_step_every_row_band(kind, n_rows, monkeypatch):
    """The persistent multi-row step (one launch per step, grid barriers
    between its phases) at 2-64 rows on slots in scrambled order, rows at
    different positions: every row's logits against the oracle's own
    sequence over three steps (crossing a 64-position tile for some rows),
    then 8 greedy steps on the device against a per-step host loop."""
    set_batch_path(monkeypatch, "bstep")
    monkeypatch.setenv("LKHIP_BSTEP_TRACE", "1")  # its barrier times show the step ran
    cfg, eng, om = build(kind, seed=60 + n_rows)
    rng = np.random.default_rng(60 + n_rows)
    lens = [int(rng.integers(1, 140)) for _ in range(n_rows)]
    lens[0] = 63
    slots = list(rng.permutation(64)[:n_rows])
    prompts = [rng.integers(0, cfg.vocab_size, n).astype(np.uint32) for n in lens]
    bat = eng.batcher(64, 192)
    orc = [om.session(192, kv_f16=True) for _ in lens]
    for i, p in enumerate(prompts):
        bat.prefill(int(slots[i]), p)
        orc[i].prefill(p)
    pos = list(lens)
    worst = 0.0
    for step in range(3):
        toks = [int(rng.integers(0, cfg.vocab_size)) for _ in lens]
        outs = bat.decode_step([BatchRow(toks[i], pos[i], int(slots[i])) for i in range(n_rows)])
        for i in range(n_rows):
            e = rel_err(outs[i], orc[i].forward(toks[i], pos[i]))
            worst = max(worst, e)
            assert e < TOL_F16_KV, (step, i, e)
            pos[i] += 1
    print(f"{kind} rows={n_rows}: worst logits rel err {worst:.3g}")
    first = [int(rng.integers(0, cfg.vocab_size)) for _ in lens]
    ids = bat.decode_greedy([BatchRow(first[i], pos[i], int(slots[i])) for i in range(n_rows)], 8)
    assert ids.shape == (8, n_rows)
    ticks = bat.trace_ticks().astype(np.int64)
    assert ticks.size == 2 + 5 * cfg.num_hidden_layers and ticks[0] > 0 and np.all(np.diff(ticks) >= 0), ticks
    short = 0
    for i in range(n_rows):
        t, agree = first[i], 8
        for k in range(8):
            t = int(oracle.argmax(orc[i].forward(t, pos[i] + k)))
            if t != ids[k, i]:
                agree = k
                break
        short += agree < 8
        assert agree >= 4, (i, agree)
    print(f"{kind} rows={n_rows}: {n_rows - short}/{n_rows} rows with 8/8 greedy ids equal to the CPU path's")
    bat.close()
    for o in orc:
        o.close()
    eng.close()
    om.close()
