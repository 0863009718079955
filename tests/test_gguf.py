"""The GGUF container reader (lkhip_gguf_config / lkhip_engine_create_gguf):
header walk, metadata, alignment, dim reversal, names, bounds and refusals on
the CPU (src/gguf/container.rs:162-261, src/gguf/arch.rs:164-270 and the
reference's own container tests, whose tiny-file fixture is rebuilt here);
on the GPU, an engine from a written file against the oracle loading the same
file bytes the way load_f32 does (src/gguf/dequant.rs:538-557), including
the llama q/k permutation (src/gguf/arch.rs:274-286), and against an engine
from the same tensors."""
import struct

import numpy as np
import pytest

import oracle
from oracle.gguf import read_container, read_gguf
from tests.gguf_writer import write_gguf
from lokal_amd import Engine, LokalHipError, gguf_config, synth
from lokal_amd.config import ModelConfig

TINY = ModelConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                   num_key_value_heads=2, vocab_size=300, rms_norm_eps=1e-6, rope_theta=1e6,
                   max_position_embeddings=2048)


def _tiny_fixture(version=3, align=None):
    """One string KV, one Q8_0 tensor of ne=[32, 2] at offset 0 (the shape of
    the reference's tiny_gguf fixture)."""
    kv = b""
    n_kv = 1 + (align is not None)

    def s(x):
        return struct.pack("<Q", len(x)) + x.encode()

    kv += s("general.architecture") + struct.pack("<I", 8) + s("llama")
    if align is not None:
        kv += s("general.alignment") + struct.pack("<II", 4, align)
    info = s("t") + struct.pack("<IQQIQ", 2, 32, 2, 8, 0)
    b = b"GGUF" + struct.pack("<IQQ", version, 1, n_kv) + kv + info
    a = align or 32
    b += b"\0" * ((-len(b)) % a)
    return b + b"\0" * 68


def test_config_and_names_from_a_written_file(tmp_path):
    tensors = synth.synth_model(TINY, synth.Q8_0, 1, tied=True, qkv_bias=True)
    p = tmp_path / "m.gguf"
    write_gguf(p, TINY, tensors, arch="qwen2")
    cfg, n, permuted = gguf_config(p)
    assert (cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers, cfg.num_attention_heads,
            cfg.num_key_value_heads, cfg.vocab_size) == (256, 512, 2, 4, 2, 300)
    assert cfg.rms_norm_eps == pytest.approx(1e-6) and cfg.rope_theta == pytest.approx(1e6)
    assert cfg.max_position_embeddings == 2048
    assert n == len(tensors) and not permuted


def test_llama_arch_is_flagged_permuted_and_alignment_honoured(tmp_path):
    tensors = synth.synth_model(TINY, synth.F16, 2, tied=False)
    p = tmp_path / "l.gguf"
    write_gguf(p, TINY, tensors, arch="llama", align=64, with_tokens=False,
               extra_kv=[("llama.vocab_size", "u32", TINY.vocab_size)])
    cfg, n, permuted = gguf_config(p)
    assert permuted and cfg.vocab_size == 300 and n == len(tensors)


def test_vocab_falls_back_to_the_embedding_rows(tmp_path):
    tensors = synth.synth_model(TINY, synth.F16, 2, tied=True)
    p = tmp_path / "v.gguf"
    write_gguf(p, TINY, tensors, arch="llama", with_tokens=False)
    assert gguf_config(p)[0].vocab_size == 300


@pytest.mark.parametrize("align", [None, 16])
def test_reference_tiny_fixture_parses_then_asks_for_the_config(tmp_path, align):
    p = tmp_path / "t.gguf"
    p.write_bytes(_tiny_fixture(3, align))
    with pytest.raises(LokalHipError, match="llama.embedding_length is missing"):
        gguf_config(p)


@pytest.mark.parametrize("version,align", [(3, None), (2, 64), (3, 16)])
def test_oracle_reads_the_reference_tiny_fixture_as_gguffile_open_does(version, align):
    """The oracle's container walk on the reference's tiny_gguf bytes
    (src/gguf/testutil.rs:9-42) gives what the reference's own tests assert
    of GgufFile::open (src/gguf/container.rs:474-494): the version, one
    tensor, the architecture string, dims [2, 32] (ne reversed to row-major),
    type Q8_0 and 68 data bytes at the alignment boundary."""
    b = _tiny_fixture(version, align)
    v, kv, tensors = read_container(b)
    assert v == version and len(tensors) == 1
    assert kv["general.architecture"] == "llama"
    if align is not None:
        assert kv["general.alignment"] == align
    name, dims, ty, data = tensors[0]
    assert (name, dims, ty, data.size) == ("t", (2, 32), 8, 68)
    # the data section starts at the first alignment boundary after the header
    a = align or 32
    assert len(b) - 68 == -(-(len(b) - 68) // a) * a and not data.any()


def test_oracle_refuses_what_the_reference_tests_refuse():
    """container.rs:496-513: a big-endian version word and a file cut 40 bytes
    short; plus the bad magic and version checks of GgufFile::open."""
    b = bytearray(_tiny_fixture(3, None))
    be = bytearray(b)
    be[4:8] = struct.pack(">I", 3)
    with pytest.raises(ValueError, match="big-endian"):
        read_container(be)
    with pytest.raises(ValueError, match="truncated|run past"):
        read_container(b[:-40])
    with pytest.raises(ValueError, match="bad magic"):
        read_container(b"GGML" + bytes(b[4:]))
    with pytest.raises(ValueError, match="version 1 unsupported"):
        read_container(_tiny_fixture(1, None))


def test_refusals(tmp_path):
    p = tmp_path / "x.gguf"
    p.write_bytes(b"GGML" + b"\0" * 60)
    with pytest.raises(LokalHipError, match="bad magic"):
        gguf_config(p)
    p.write_bytes(_tiny_fixture(version=1))
    with pytest.raises(LokalHipError, match="version 1 unsupported"):
        gguf_config(p)
    p.write_bytes(b"GGUF" + struct.pack(">I", 3) + b"\0" * 16)
    with pytest.raises(LokalHipError, match="big-endian"):
        gguf_config(p)
    p.write_bytes(_tiny_fixture()[:40])
    with pytest.raises(LokalHipError, match="truncated"):
        gguf_config(p)
    with pytest.raises(LokalHipError, match="cannot open"):
        gguf_config(tmp_path / "missing.gguf")


def test_unsupported_types_are_listed_together(tmp_path):
    tensors = synth.synth_model(TINY, synth.Q8_0, 3, tied=True)
    # relabel two matrices as Q2_K / Q4_1 (types the backend does not take)
    # with sizes that fit those types
    out = []
    for t in tensors:
        if t.name.endswith(("layers.0.mlp.down_proj.weight", "layers.1.mlp.down_proj.weight")):
            rows, cols = t.dims
            out.append(synth.Tensor(t.name, 10, t.dims, np.zeros(rows * cols // 256 * 84, np.uint8)))
        elif t.name.endswith("layers.0.mlp.up_proj.weight"):
            rows, cols = t.dims
            out.append(synth.Tensor(t.name, 3, t.dims, np.zeros(rows * cols // 32 * 20, np.uint8)))
        else:
            out.append(t)
    p = tmp_path / "u.gguf"
    write_gguf(p, TINY, out)
    with pytest.raises(LokalHipError, match=r"2 weight type\(s\).*across 3 of .*Q2_K \(2 tensors.*Q4_1 \(1 tensor"):
        gguf_config(p)


def test_unsupported_architecture(tmp_path):
    tensors = synth.synth_model(TINY, synth.F16, 2, tied=True)
    p = tmp_path / "a.gguf"
    write_gguf(p, TINY, tensors, arch="gemma")
    with pytest.raises(LokalHipError, match='"gemma" is not supported'):
        gguf_config(p)


def test_tensor_past_the_end_is_refused(tmp_path):
    tensors = synth.synth_model(TINY, synth.F16, 2, tied=True)
    p = tmp_path / "e.gguf"
    write_gguf(p, TINY, tensors)
    b = p.read_bytes()
    p.write_bytes(b[:-4096])
    with pytest.raises(LokalHipError, match="run past the file"):
        gguf_config(p)


@pytest.mark.gpu
@pytest.mark.parametrize("arch,wtype,bias", [("qwen2", synth.Q8_0, True), ("llama", synth.Q4_K, False),
                                             ("llama", synth.F16, False)])
def test_engine_from_gguf_matches_engine_from_tensors(tmp_path, arch, wtype, bias):
    cfg = TINY if wtype != synth.Q4_K else TINY.with_(hidden_size=512, intermediate_size=1024,
                                                      num_attention_heads=8)
    tensors = synth.synth_model(cfg, wtype, 5, tied=(arch == "qwen2"), qkv_bias=bias)
    p = tmp_path / "g.gguf"
    write_gguf(p, cfg, tensors, arch=arch)
    a = Engine.from_gguf(str(p))
    b = Engine.from_tensors(cfg, tensors)
    assert a.cfg.vocab_size == cfg.vocab_size
    sa, sb = a.session(64), b.session(64)
    for pos, t in enumerate(np.random.default_rng(6).integers(0, cfg.vocab_size, 12)):
        la, lb = sa.forward(int(t), pos), sb.forward(int(t), pos)
        assert np.array_equal(la, lb), (arch, pos)
    sa.close()
    sb.close()
    a.close()
    b.close()


@pytest.mark.parametrize("arch,wtype", [("qwen2", synth.Q8_0), ("llama", synth.Q4_K), ("llama", synth.F16)])
def test_oracle_reads_the_file_as_load_f32_does(tmp_path, arch, wtype):
    """The oracle's reader of the file bytes (oracle/gguf.py) returns the
    written config and tensors under HF names; a llama file's q/k rows come
    back in the converter's order (not the HF order written), and the oracle
    model built from the file with the permutation undone computes the same
    bits as the model built from the HF tensors."""
    cfg = TINY if wtype != synth.Q4_K else TINY.with_(hidden_size=512, intermediate_size=1024,
                                                      num_attention_heads=8)
    tensors = synth.synth_model(cfg, wtype, 11, tied=(arch == "qwen2"), qkv_bias=(arch == "qwen2"))
    p = tmp_path / "o.gguf"
    write_gguf(p, cfg, tensors, arch=arch)
    fcfg, ft, permuted = read_gguf(p)
    assert permuted == (arch == "llama")
    for f in ("hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
              "num_key_value_heads", "vocab_size", "max_position_embeddings"):
        assert getattr(fcfg, f) == getattr(cfg, f), f
    assert np.float32(fcfg.rms_norm_eps) == np.float32(cfg.rms_norm_eps)
    assert np.float32(fcfg.rope_theta) == np.float32(cfg.rope_theta)
    want = {t.name: t for t in tensors}
    assert sorted(t.name for t in ft) == sorted(want)
    for t in ft:
        w = want[t.name]
        assert t.ggml_type == w.ggml_type and tuple(t.dims) == tuple(w.dims), t.name
        same = np.array_equal(t.data, np.asarray(w.data).view(np.uint8).reshape(-1))
        qk = t.name.endswith(("q_proj.weight", "k_proj.weight"))
        assert same != (qk and arch == "llama"), t.name
    a, b = oracle.Model(fcfg, ft, llama_permuted=permuted), oracle.Model(cfg, tensors)
    sa, sb = a.session(16), b.session(16)
    for pos, tok in enumerate((3, 77, 150, 299)):
        assert np.array_equal(sa.forward(tok, pos), sb.forward(tok, pos))
    a.close()
    b.close()


@pytest.mark.gpu
@pytest.mark.parametrize("arch,wtype,bias", [("qwen2", synth.Q8_0, True), ("llama", synth.Q4_K, False),
                                             ("llama", synth.F16, False), ("llama", synth.Q8_0, False)])
def test_engine_from_gguf_matches_oracle_from_the_same_bytes(tmp_path, arch, wtype, bias):
    """GGUF engine (HIP reader, upload-time unpermute) against the oracle built
    from the same file's bytes with load_f32's rule (llama q/k unpermuted):
    logits within 1e-3 over 24 positions (f32 KV caches on both sides) and
    identical greedy ids for 24 steps."""
    cfg = TINY if wtype != synth.Q4_K else TINY.with_(hidden_size=512, intermediate_size=1024,
                                                      num_attention_heads=8)
    tensors = synth.synth_model(cfg, wtype, 13, tied=(arch == "qwen2"), qkv_bias=bias)
    p = tmp_path / "x.gguf"
    write_gguf(p, cfg, tensors, arch=arch)
    del tensors
    fcfg, ft, permuted = read_gguf(p)
    eng = Engine.from_gguf(str(p))
    om = oracle.Model(fcfg, ft, llama_permuted=permuted)
    s, o = eng.session(64, kv_dtype="f32"), om.session(64)
    toks = np.random.default_rng(14).integers(0, cfg.vocab_size, 24)
    for pos, t in enumerate(toks):
        got, want = s.forward(int(t), pos), o.forward(int(t), pos)
        err = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
        assert err < 1e-3, (arch, pos, err)
    first = int(oracle.argmax(want))
    ids = list(s.decode_greedy(first, len(toks), 24))
    cur, ref = first, []
    for i in range(24):
        cur = int(oracle.argmax(o.forward(cur, len(toks) + i)))
        ref.append(cur)
    assert ids == ref
    s.close()
    eng.close()
    om.close()
