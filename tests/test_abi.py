"""The C-ABI library loads and exports exactly what include/lokal_hip.h
declares; host-side refusals work without a GPU."""
import re
from pathlib import Path

import numpy as np
import pytest

from lokal_amd import _lib, synth
from lokal_amd.config import CONFIGS, ModelConfig

HEADER = Path(__file__).resolve().parent.parent / "include" / "lokal_hip.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(lkhip_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared()
    for must in ("lkhip_engine_create_tensors", "lkhip_session_forward", "lkhip_session_prefill",
                 "lkhip_batch_decode_step", "lkhip_q8_0_matvec", "lkhip_q4_k_matvec", "lkhip_dequant_rows",
                 "lkhip_rmsnorm", "lkhip_rope_pairs", "lkhip_swiglu", "lkhip_embed_gather", "lkhip_attn_decode"):
        assert must in names


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing


def test_bindings_cover_the_header():
    assert sorted(_lib.SIGNATURES) == declared()


def test_no_device_here_is_reported_not_crashed():
    L = _lib.lib()
    n = L.lkhip_device_count()
    assert n >= 0
    if n == 0:
        from lokal_amd import Engine, LokalHipError
        cfg = ModelConfig(256, 512, 1, 4, 2, 300, 1e-6)
        with pytest.raises(LokalHipError, match="no HIP device"):
            Engine.from_tensors(cfg, synth.synth_model(cfg, synth.Q8_0, 0))


def test_unknown_backend_refused():
    from lokal_amd import LokalHipError, create
    with pytest.raises(LokalHipError, match='unknown backend "metal"'):
        create("metal", CONFIGS["qwen2.5-0.5b"], [])


def test_synthetic_tensors_are_reproducible_and_sized():
    cfg = ModelConfig(256, 512, 2, 4, 2, 300, 1e-6)
    a = synth.synth_model(cfg, synth.Q8_0, seed=5, qkv_bias=True)
    b = synth.synth_model(cfg, synth.Q8_0, seed=5, qkv_bias=True)
    c = synth.synth_model(cfg, synth.Q8_0, seed=6, qkv_bias=True)
    assert [t.name for t in a] == [t.name for t in b]
    assert all(np.array_equal(x.data, y.data) for x, y in zip(a, b))
    assert not np.array_equal(a[2].data, c[2].data)
    for t in a:
        n = int(np.prod(t.dims))
        rows = t.dims[0] if len(t.dims) == 2 else 1
        assert t.nbytes == rows * synth.row_bytes(t.ggml_type, n // rows)
    q = next(t for t in a if t.name.endswith("q_proj.weight")).data.reshape(-1, 34)
    d = q[:, :2].copy().view(np.float16).astype(np.float32)
    assert (d >= 0).all() and np.isfinite(d).all()
    assert q[:, 2:].view(np.int8).min() >= -127
    k = synth.synth_model(cfg, synth.Q4_K, seed=1)[2].data.reshape(-1, 144)
    dd = k[:, :4].copy().view(np.float16).astype(np.float32)
    assert (dd >= 2.0 ** -10).all() and (dd <= 2.0 ** -6).all()


def test_headline_config_bytes_per_token():
    """Algorithmic Q8_0 bytes of one Qwen2.5-0.5B decode token: 493,961,216 weights x 34/32."""
    c = CONFIGS["qwen2.5-0.5b"]
    h, I, L, V = c.hidden_size, c.intermediate_size, c.num_hidden_layers, c.vocab_size
    per_layer = h * c.q_dim() + 2 * h * c.kv_dim() + c.q_dim() * h + 3 * h * I
    weights = L * per_layer + V * h
    assert weights == 493_961_216
    assert weights * 34 // 32 == 524_833_792


def test_context_window_refused_with_a_reason():
    """The hip arm refuses --context-window as the CPU arm does (src/engine.rs:84-87)."""
    from lokal_amd import LokalHipError, create
    from lokal_amd.engine import check_window
    L = _lib.lib()
    assert L.lkhip_context_window(0, 0) == 0
    assert L.lkhip_context_window(512, 4) == -2
    msg = L.lkhip_last_error().decode()
    assert "--context-window" in msg and "-b metal" in msg and "\n" not in msg
    check_window(None)
    with pytest.raises(LokalHipError, match="context-window"):
        create("hip", CONFIGS["qwen2.5-0.5b"], [], win=(1024, 4))


def test_per_head_qk_norm_refused_before_any_device_work():
    """A Qwen3-style tensor set (self_attn.q_norm / k_norm, src/model.rs:213-222)
    is refused by name, not run without the norm -- also with no GPU present."""
    from lokal_amd import Engine, LokalHipError
    cfg = ModelConfig(256, 512, 1, 4, 2, 300, 1e-6)
    tensors = synth.synth_model(cfg, synth.Q8_0, 0)
    qn = synth.Tensor("model.layers.0.self_attn.q_norm.weight", _lib.LKHIP_F32, (64,),
                      np.ones(64, np.float32))
    with pytest.raises(LokalHipError, match="q_norm.*per-head q/k RMSNorm") as ei:
        Engine.from_tensors(cfg, tensors + [qn])
    assert ei.value.code == -2


def test_dynamic_lds_arrays_are_16_byte_aligned():
    """A kernel's dynamic LDS starts right after its static LDS, at the
    alignment its extern declaration states: one declared without
    __align__(16) in a kernel with a 36-byte static array left every 16-byte
    LDS access of the one-kernel decode step misaligned (364 -> 468 us per
    launch on MI355X).  Every dynamic LDS array of the HIP sources is
    declared 16-byte aligned."""
    src = Path(__file__).resolve().parent.parent / "lokal_amd" / "csrc"
    found = 0
    for f in sorted(src.glob("*.hip")) + sorted(src.glob("*.h")):
        for line in f.read_text().splitlines():
            if re.search(r"\bextern\s+__shared__\b", line):
                found += 1
                assert "__align__(16)" in line, f"{f.name}: {line.strip()}"
    assert found >= 4
