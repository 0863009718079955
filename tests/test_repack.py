"""The host-side repack of GGUF rows into the device layouts
(lokal_amd/csrc/repack.h), on the CPU: every device element, evaluated the way
the kernels evaluate it, equals the oracle's dequant_row_ref value bit for bit
(src/gguf/dequant.rs:191-535) -- on random blocks, on blocks with extreme f16
scales (subnormal, largest finite, negative) and on the reference's hand
vectors.  The header is plain C++, compiled here with g++ into a tiny probe."""
import ctypes as C
import json
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from lokal_amd import synth

ROOT = Path(__file__).resolve().parent.parent
PROBE = r"""
#include "repack.h"
#include <vector>
// device value of element j: Q8_0 form (i8)q * f16 d; Q8_SM form s*q - m
extern "C" int probe(uint32_t t, const uint8_t* s, size_t cols, float* y) {
    const uint32_t dev = lkr::device_type(t);
    if (dev != lkr::G_Q8_0 && dev != lkr::D_Q8_SM) return -1;
    std::vector<uint8_t> d(lkr::data_row_bytes(dev, cols)), a(lkr::aux_row_bytes(dev, cols));
    lkr::repack_row(t, s, cols, d.data(), a.data());
    for (size_t j = 0; j < cols; j++) {
        const float q = (float)(int8_t)d[j];
        if (dev == lkr::G_Q8_0) {
            y[j] = q * lkr::h2f(lkr::u16_at(a.data() + 2 * (j / 32)));
        } else {
            float sm[2];
            memcpy(sm, a.data() + 8 * (j / 16), 8);
            const volatile float p = sm[0] * q;  // rounded before the subtraction
            y[j] = p - sm[1];
        }
    }
    return 0;
}
"""


@pytest.fixture(scope="module")
def probe(tmp_path_factory):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("repack")
    (d / "probe.cpp").write_text(PROBE)
    so = d / "probe.so"
    subprocess.run([gxx, "-O2", "-ffp-contract=off", "-shared", "-fPIC", "-I", str(ROOT / "lokal_amd" / "csrc"),
                    str(d / "probe.cpp"), "-o", str(so)], check=True)
    lib = C.CDLL(str(so))
    lib.probe.argtypes = [C.c_uint32, C.c_void_p, C.c_size_t, C.c_void_p]

    def run(t, raw, n):
        raw = np.ascontiguousarray(raw, np.uint8)
        y = np.zeros(n, np.float32)
        assert lib.probe(t, raw.ctypes.data, n, y.ctypes.data) == 0
        return y
    return run


TYPES = [synth.Q4_0, synth.Q5_0, synth.Q5_K, synth.Q6_K]
# f16 bit patterns for the scale fields: smallest subnormal, a subnormal,
# largest finite, negatives, one, zero
F16_EDGES = [0x0001, 0x03FF, 0x7BFF, 0xFBFF, 0x8001, 0x3C00, 0xBC00, 0x0000]


def f16_offsets(t):
    return {synth.Q4_0: [0], synth.Q5_0: [0], synth.Q5_K: [0, 2], synth.Q6_K: [208]}[t]


def assert_bits(got, want):
    want = np.asarray(want, np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
def test_random_blocks(probe, t):
    e, b = synth.BLK[t]
    raw = synth.gen_weight(t, 11, "repack", 4, 8 * e).data
    n = raw.size // b * e
    assert_bits(probe(t, raw, n), oracle.dequant_row(t, raw.tobytes(), n))


@pytest.mark.parametrize("t", TYPES)
def test_extreme_scales(probe, t):
    e, b = synth.BLK[t]
    rng = np.random.default_rng(t)
    blocks = rng.integers(0, 256, (len(F16_EDGES) ** 2, b), dtype=np.uint8)
    offs = f16_offsets(t)
    for i, (h0, h1) in enumerate((x, y) for x in F16_EDGES for y in F16_EDGES):
        for o, h in zip(offs, (h0, h1)):
            blocks[i, o:o + 2] = (h & 0xFF, h >> 8)
    raw = blocks.reshape(-1)
    n = blocks.shape[0] * e
    assert_bits(probe(t, raw, n), oracle.dequant_row(t, raw.tobytes(), n))


def test_reference_hand_vectors(probe):
    gold = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
    seen = set()
    for v in gold["dequant"]:
        if v["type"] not in TYPES:
            continue
        seen.add(v["type"])
        y = probe(v["type"], np.array(v["bytes"], np.uint8), v["n"])
        for i, want in v["expect"].items():
            assert y[int(i)] == np.float32(want), v["ref"]
    assert seen == set(TYPES)
