"""Measurements of the decode-step kernels on the workloads other than the
headline one (bench.py measures config 3, Qwen2.5-0.5B-shape Q8_0 decode).

    python -m lokal_amd.microbench [--only decode,longctx,layers,attn,gemm,prefill,batch]

Prints one JSON object per measurement:
  decode  configs 1 and 4: SmolLM2-135M-shape F16 (512-token prompt, 128
          greedy tokens) and TinyLlama-1.1B-shape Q4_K (256-token prompt, 256
          tokens), tok/s with the algorithmic weight bytes and % of 8 TB/s;
  layers  config 2: RMSNorm, RoPE-pair rotation, SwiGLU and the f16 embedding
          gather at Qwen2.5-0.5B widths for 1, 8 and 64 rows (latency-bound:
          µs and GB/s, no %-of-peak target);
  attn    config 5: flash-decoding of 4 sequences, one query token each, at
          contexts 4096 / 16384 / 32768 over 24 layers of f16 KV (14 q / 2 kv
          heads), µs per step and HBM GB/s of the KV bytes read once.
  gemm    the multi-row dequant-fused GEMM (lkhip_matmul) on the Qwen2.5-0.5B
          Q8_0 matrices for 1 / 4 / 16 / 64 / 512 activation rows: µs, weight
          GB/s (each weight byte read once per launch) and fp32 TFLOP/s;
  prefill config 3's 512-token prompt through Session::prefill, chunked on
          the GEMM path and as the per-token loop (LKHIP_PREFILL=loop);
  matvec  lkhip_q8_0_matvec (the per-stage dequant-fused matvec) alone at
          the Qwen2.5-0.5B decode shapes 896->896 (q, o_proj), 896->128 (k,
          v), 896->4864 (gate, up), 4864->896 (down), 896->151936 (lm_head):
          a HIP graph of launches that cycle through enough copies of the
          matrix (>= 512 MiB, so the 256 MB Infinity Cache cannot hold them)
          that every launch streams from HBM; µs per launch, GB/s of the
          Q8_0 bytes and % of 8 TB/s;
  mix     a short run of every decode-step kernel family, for profiler
          counter passes (rocprofv3 --pmc): 8 greedy tokens of config 3
          (fused_step_kernel, lm_head_kernel), one config-5 step of 24
          layers at 4096 positions (attn_mfma_kernel), 8
          batched greedy steps of 4 rows (fused_rows_kernel);
  trace   the one-kernel step's per-stage times from every workgroup's
          stage timestamps (config 3, position 528): each stage's duration
          to its slowest workgroup and the spread of its end over workgroups;
  stream  the practical read bandwidth: a plain f32 sum and a device copy
          (ROCm's own kernels through torch) over 145 MB and 1 GiB;
  batch   config 3 served by the Batcher: B sequences (B = 1, 4, 16, 64), each
          with a 512-token prompt, then 64 greedy steps of all B rows on the
          device: aggregate tok/s and weight GB/s (one weight read per step).
Kernel times come from hipEvents around repeated launches on one stream; the
layer kernels are also timed as 200 launches captured in one HIP graph
(us_graph: device time per launch without the per-call host cost).
"""
from __future__ import annotations

import argparse
import json
import sys
import time

import numpy as np

from . import kernels as K
from . import synth
from .engine import Engine

HBM_PEAK_GBS = 8000.0


def _timed(fn, reps: int, stream: K.Stream) -> float:
    """Average ms of fn() over reps launches after two warm-ups."""
    for _ in range(2):
        fn()
    a, b = K.Event(), K.Event()
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    stream.synchronize()
    return a.elapsed_ms(b) / reps


def _hip():
    """The HIP runtime, for stream capture (measurement only)."""
    import ctypes
    h = ctypes.CDLL("libamdhip64.so")
    for f in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
              "hipGraphExecDestroy", "hipGraphDestroy"):
        getattr(h, f).restype = ctypes.c_int
    return h


def _timed_graph_seq(fns, rounds: int, stream: K.Stream) -> float:
    """Average ms per launch of the launches fns, captured `rounds` times in
    order into one HIP graph."""
    it = iter(range(len(fns) * rounds))
    calls = [fns[i % len(fns)] for i in it]
    state = {"i": 0}

    def step():
        calls[state["i"] % len(calls)]()
        state["i"] += 1
    return _timed_graph(step, len(calls), stream)


def _timed_graph(fn, reps: int, stream: K.Stream) -> float:
    """Average ms per launch of fn() captured reps times into one HIP graph
    (device time per kernel without the per-call host launch cost)."""
    import ctypes
    h = _hip()
    fn()  # load the code object outside the capture
    stream.synchronize()
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    if h.hipStreamBeginCapture(stream.ptr, 2):  # hipStreamCaptureModeRelaxed
        raise RuntimeError("hipStreamBeginCapture failed")
    for _ in range(reps):
        fn()
    if h.hipStreamEndCapture(stream.ptr, ctypes.byref(graph)):
        raise RuntimeError("hipStreamEndCapture failed")
    try:
        if h.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)):
            raise RuntimeError("hipGraphInstantiate failed")
        h.hipGraphLaunch(exe, stream.ptr)  # warm-up
        a, b = K.Event(), K.Event()
        a.record(stream)
        if h.hipGraphLaunch(exe, stream.ptr):
            raise RuntimeError("hipGraphLaunch failed")
        b.record(stream)
        stream.synchronize()
        return a.elapsed_ms(b) / reps
    finally:
        if exe:
            h.hipGraphExecDestroy(exe)
        h.hipGraphDestroy(graph)


def decode(name: str, prompt_len: int, steps: int) -> dict:
    cfg, tensors = synth.synth_named(name, 0)
    eng = Engine.from_tensors(cfg, tensors)
    del tensors
    s = eng.session(prompt_len + steps + 16)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, prompt_len).astype(np.uint32)
    lg = s.prefill(prompt)
    tok = int(np.argmax(lg))
    ids = s.decode_greedy(tok, prompt_len, 8)  # warm-up
    t0 = time.perf_counter()
    s.decode_greedy(int(ids[-1]), prompt_len + 8, steps)
    dt = time.perf_counter() - t0
    tok_s = steps / dt
    wbytes = eng.matvec_bytes
    gbs = wbytes * tok_s / 1e9
    s.close()
    eng.close()
    return {"workload": name, "prompt": prompt_len, "decode_tokens": steps, "tok_s": round(tok_s, 1),
            "ms_per_token": round(dt / steps * 1e3, 4), "weight_bytes_per_token": wbytes,
            "weight_gbs": round(gbs, 1), "frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4)}


def stage_trace(name: str = "qwen2.5-0.5b-q8_0", prompt_len: int = 512) -> list[dict]:
    """Per-stage timing of the one-kernel step from every workgroup's stage
    timestamps (lkhip_session_set_trace): for each stage of each layer, the
    end time of every one of the grid's workgroups, relative to the end of the
    previous layer's last workgroup.  Reports, averaged over the layers after
    the first two, each stage's duration as seen by the slowest workgroup and
    the spread (max - min) of its end time over workgroups -- the producer
    skew that the next stage's consumers wait out."""
    cfg, tensors = synth.synth_named(name, 0)
    eng = Engine.from_tensors(cfg, tensors)
    del tensors
    s = eng.session(prompt_len + 64)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, prompt_len).astype(np.uint32)
    tok = int(np.argmax(s.prefill(prompt)))
    ids = s.decode_greedy(tok, prompt_len, 16)
    s.set_trace(0)
    s.decode_greedy(int(ids[-1]), prompt_len + 16, 1)
    t = s.trace_ticks().astype(np.float64)
    s.close()
    eng.close()
    L = cfg.num_hidden_layers
    u = (t - t[:, 0].min()) / 100.0  # 100 MHz ticks -> us
    names = ["qkv", "attn", "merge", "o_proj", "gate_up", "down"]
    dur = np.zeros(6)
    skew = np.zeros(6)
    med = np.zeros(6)
    n = 0
    for layer in range(2, L):
        ref = u[:, 2 + 6 * (layer - 1) + 5].max()
        prev = 0.0
        for k in range(6):
            e = u[:, 2 + 6 * layer + k] - ref
            dur[k] += e.max() - prev
            skew[k] += e.max() - e.min()
            med[k] += np.median(e)
            prev = e.max()
        n += 1
    per_layer = (u[:, 2 + 6 * (L - 1) + 5].max() - u[:, 2 + 6 * 0 + 5].max()) / (L - 1)
    out = [{"workload": "stage-trace", "model": name, "position": prompt_len + 16, "workgroups": int(t.shape[0]),
            "us_per_layer": round(per_layer, 2)}]
    # the launch's start: when the workgroups began (from the first one), when
    # each had the token's embedding, when layer 0 ended, when the last ended
    out.append({"workload": "stage-trace", "part": "start", "start_spread_us": round(u[:, 0].max(), 2),
                "embedding_median_us": round(float(np.median(u[:, 1])), 2), "embedding_max_us": round(u[:, 1].max(), 2),
                "layer0_end_us": round(u[:, 2 + 5].max(), 2), "last_end_us": round(u[:, 2 + 6 * L].max(), 2)})
    for k in range(6):
        out.append({"workload": "stage-trace", "stage": names[k], "us_slowest_workgroup": round(dur[k] / n, 2),
                    "end_median_us": round(med[k] / n, 2), "end_skew_us": round(skew[k] / n, 2)})
    # sub-steps of layer 1 (thread 0 of each workgroup that runs the step),
    # from the end of layer 0's last workgroup
    subs = {15: "S1 x in", 17: "S1 dots", 18: "S1 published", 1: "S2 tile issued", 2: "S2 q arrived",
            3: "S2 scores", 4: "S2 softmax", 5: "S2 P.V", 6: "S2 published", 20: "S3 partials in",
            21: "S3 published", 12: "S4 input in", 13: "S4 published", 14: "S4 rows issued", 8: "S5 input in",
            9: "S5 norm", 10: "S5 held units", 22: "S5 units of the last wave", 7: "S6 input in",
            19: "S6 dot"}
    ref = u[:, 2 + 5].max()
    for k, nm in subs.items():
        v = t[:, 2 + 6 * L + 1 + k]
        m = v > 0
        if m.any():
            w = u[m, 2 + 6 * L + 1 + k] - ref
            out.append({"workload": "stage-trace", "substep": nm, "workgroups": int(m.sum()),
                        "min_us": round(float(w.min()), 2), "median_us": round(float(np.median(w)), 2),
                        "max_us": round(float(w.max()), 2)})
    return out


def layers() -> list[dict]:
    st = K.Stream()
    out = []
    h, nq, inter, vocab = 896, 14, 4864, 151936
    rng = np.random.default_rng(0)
    table = K.Weight(synth.F16, vocab, h, synth.gen_weight(synth.F16, 0, "model.embed_tokens.weight", vocab, h).data)
    for rows in (1, 8, 64):
        x = K.DeviceArray.from_numpy(rng.standard_normal((rows, h)).astype(np.float32))
        g = K.DeviceArray.from_numpy((1 + 0.1 * rng.standard_normal(h)).astype(np.float32))
        y = K.DeviceArray((rows, h))
        f = lambda: K.rmsnorm(x, g, rows, h, 1e-6, y, st.ptr)
        ms, gms = _timed(f, 200, st), _timed_graph(f, 200, st)
        nbytes = rows * h * 4 * 2 + h * 4
        out.append({"kernel": "rmsnorm", "rows": rows, "n": h, "us": round(ms * 1e3, 3), "us_graph": round(gms * 1e3, 3),
                    "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)})
        q = K.DeviceArray.from_numpy(rng.standard_normal((rows, nq * 64)).astype(np.float32))
        pos = K.DeviceArray.from_numpy(rng.integers(0, 32768, rows).astype(np.uint32))
        f = lambda: K.rope_pairs(q, rows, nq * 64, 64, pos, 1e6, st.ptr)
        ms, gms = _timed(f, 200, st), _timed_graph(f, 200, st)
        nbytes = rows * nq * 64 * 4 * 2 + rows * 4
        out.append({"kernel": "rope_pairs", "rows": rows, "n": nq * 64, "us": round(ms * 1e3, 3), "us_graph": round(gms * 1e3, 3),
                    "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)})
        gd = K.DeviceArray.from_numpy(rng.standard_normal(rows * inter).astype(np.float32))
        ud = K.DeviceArray.from_numpy(rng.standard_normal(rows * inter).astype(np.float32))
        od = K.DeviceArray(rows * inter)
        f = lambda: K.swiglu(gd, ud, rows * inter, od, st.ptr)
        ms, gms = _timed(f, 200, st), _timed_graph(f, 200, st)
        nbytes = rows * inter * 4 * 3
        out.append({"kernel": "swiglu", "rows": rows, "n": inter, "us": round(ms * 1e3, 3), "us_graph": round(gms * 1e3, 3),
                    "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)})
        ids = K.DeviceArray.from_numpy(rng.integers(0, vocab, rows).astype(np.uint32))
        eo = K.DeviceArray((rows, h))
        f = lambda: K.embed_gather(table, ids, rows, eo, st.ptr)
        ms, gms = _timed(f, 200, st), _timed_graph(f, 200, st)
        nbytes = rows * h * (2 + 4) + rows * 4
        out.append({"kernel": "embed_gather_f16", "rows": rows, "n": h, "us": round(ms * 1e3, 3), "us_graph": round(gms * 1e3, 3),
                    "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)})
    st.close()
    return out


def attn() -> list[dict]:
    st = K.Stream()
    out = []
    n_seq, nh, nkv, hd, n_layers = 4, 14, 2, 64, 24
    rng = np.random.default_rng(0)
    for ctx in (4096, 16384, 32768):
        # one layer's cache holds N(0,1) f16 values; the 24 layers of a step
        # are 24 distinct caches, so every step reads the full KV once
        kv_elems = n_seq * nkv * ctx * hd
        caches = []
        base = rng.standard_normal(kv_elems).astype(np.float16).view(np.uint16)
        for layer in range(n_layers):
            k = K.DeviceArray.from_numpy(np.roll(base, layer * 7919))
            v = K.DeviceArray.from_numpy(np.roll(base, layer * 104729 + 1))
            caches.append((k, v))
        q = K.DeviceArray.from_numpy(rng.standard_normal((n_seq, nh * hd)).astype(np.float32))
        cl = K.DeviceArray.from_numpy(np.full(n_seq, ctx, np.uint32))
        o = K.DeviceArray((n_seq, nh * hd))

        def step():
            for k, v in caches:
                K.attn_decode(q, k, v, cl, n_seq, nh, nkv, hd, ctx, o, st.ptr)

        ms = _timed(step, 10, st)
        # the same 24 launches captured into a HIP graph, 4 steps' worth
        layer_fns = [(lambda k=k, v=v: K.attn_decode(q, k, v, cl, n_seq, nh, nkv, hd, ctx, o, st.ptr))
                     for k, v in caches]
        gms = _timed_graph_seq(layer_fns, 4, st) * n_layers
        nbytes = n_layers * n_seq * nkv * ctx * hd * 2 * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        ggbs = nbytes / (gms * 1e-3) / 1e9
        out.append({"workload": "attn-4seq", "ctx": ctx, "layers": n_layers, "us_per_step": round(ms * 1e3, 1),
                    "us_per_step_graph": round(gms * 1e3, 1), "kv_bytes_per_step": nbytes, "gbs": round(gbs, 1),
                    "frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4), "frac_of_hbm_graph": round(ggbs / HBM_PEAK_GBS, 4)})
        for k, v in caches:
            k.free()
            v.free()
    st.close()
    return out


def gemm() -> list[dict]:
    """lkhip_matmul on the Qwen2.5-0.5B Q8_0 matrices."""
    st = K.Stream()
    out = []
    rng = np.random.default_rng(0)
    shapes = [("qkv", 1152, 896), ("o_proj", 896, 896), ("gate", 4864, 896), ("down", 896, 4864),
              ("lm_head", 151936, 896)]
    for name, rows, cols in shapes:
        w = K.Weight(synth.Q8_0, rows, cols, synth.gen_weight(synth.Q8_0, 0, name, rows, cols).data)
        for n in (1, 4, 16, 64, 512):
            x = K.DeviceArray.from_numpy(rng.standard_normal((n, cols)).astype(np.float32))
            y = K.DeviceArray((n, rows))
            ms = _timed(lambda: K.matmul(w, x, n, y, stream=st.ptr), 20 if n < 512 else 5, st)
            gbs = w.nbytes / (ms * 1e-3) / 1e9
            out.append({"kernel": "gemm_q8_0", "matrix": name, "rows": rows, "cols": cols, "n_rows": n,
                        "us": round(ms * 1e3, 2), "weight_gbs": round(gbs, 1),
                        "frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4),
                        "tflops": round(2.0 * rows * cols * n / (ms * 1e-3) / 1e12, 2)})
            x.free()
            y.free()
        w.close()
    st.close()
    return out


def prefill() -> list[dict]:
    import os
    cfg, tensors = synth.synth_named("qwen2.5-0.5b-q8_0", 0)
    eng = Engine.from_tensors(cfg, tensors)
    del tensors
    prompt = np.random.default_rng(11).integers(0, cfg.vocab_size, 512).astype(np.uint32)
    out = []
    flops = 2.0 * (eng.matvec_bytes * 32 / 34) * len(prompt)  # every Q8_0 weight, every position
    for mode in ("batched", "loop"):
        if mode == "loop":
            os.environ["LKHIP_PREFILL"] = "loop"
        s = eng.session(len(prompt) + 8)
        s.prefill(prompt[:64])  # warm-up (allocations, graph capture)
        times = []
        for _ in range(5 if mode == "batched" else 1):  # each call prefills positions 0..511 again
            t0 = time.perf_counter()
            s.prefill(prompt)
            times.append(time.perf_counter() - t0)
        dt = sorted(times)[len(times) // 2]
        s.close()
        out.append({"workload": "qwen2.5-0.5b-q8_0 prefill", "mode": mode, "tokens": len(prompt),
                    "ms": round(dt * 1e3, 2), "tok_s": round(len(prompt) / dt, 1),
                    "tflops": round(flops / dt / 1e12, 2)})
    os.environ.pop("LKHIP_PREFILL", None)
    eng.close()
    return out


def batch() -> list[dict]:
    from .engine import BatchRow
    cfg, tensors = synth.synth_named("qwen2.5-0.5b-q8_0", 0)
    eng = Engine.from_tensors(cfg, tensors)
    del tensors
    rng = np.random.default_rng(12)
    out = []
    steps = 64
    import os
    rows_list = [int(v) for v in os.environ.get("LKHIP_MB_ROWS", "1,2,3,4,5,6,7,8,16,32,64").split(",")]
    for B in rows_list:
        bat = eng.batcher(B, 512 + steps + 16)
        first = []
        for slot in range(B):
            lg = bat.prefill(slot, rng.integers(0, cfg.vocab_size, 512).astype(np.uint32))
            first.append(int(np.argmax(lg)))
        rows = [BatchRow(first[s], 512, s) for s in range(B)]
        ids = bat.decode_greedy(rows, 8)  # warm-up: graph capture
        rows = [BatchRow(int(ids[-1, s]), 520, s) for s in range(B)]
        t0 = time.perf_counter()
        bat.decode_greedy(rows, steps)
        dt = time.perf_counter() - t0
        bat.close()
        tok_s = B * steps / dt
        gbs = eng.matvec_bytes * steps / dt / 1e9
        out.append({"workload": "qwen2.5-0.5b-q8_0 batched greedy", "rows": B, "steps": steps,
                    "ms_per_step": round(dt / steps * 1e3, 3), "tok_s": round(tok_s, 1),
                    "weight_gbs": round(gbs, 1), "frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4)})
    eng.close()
    return out


def matvec() -> list[dict]:
    st = K.Stream()
    out = []
    rng = np.random.default_rng(3)
    for name, rows, cols in (("q_proj/o_proj", 896, 896), ("k_proj/v_proj", 128, 896), ("gate/up", 4864, 896),
                             ("down", 896, 4864), ("lm_head", 151936, 896)):
        data = synth.gen_weight(synth.Q8_0, 5, "model.layers.0.mlp.up_proj.weight", rows, cols).data
        nbytes = rows * cols * 34 // 32
        copies = int(min(512, max(2, -(-(512 << 20) // nbytes))))
        ws = [K.Weight(synth.Q8_0, rows, cols, data) for _ in range(copies)]
        x = K.DeviceArray.from_numpy(rng.standard_normal(cols).astype(np.float32))
        y = K.DeviceArray(rows)
        fns = [(lambda w=w: K.q8_0_matvec(w, x, y, stream=st.ptr)) for w in ws]
        rounds = max(1, 256 // copies)
        ms = _timed_graph_seq(fns, rounds, st)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out.append({"bench": "q8_0_matvec", "shape": f"{cols}->{rows}", "matrix": name, "bytes": nbytes,
                    "copies": copies, "resident_bytes": copies * nbytes, "launches": copies * rounds,
                    "us": round(ms * 1e3, 2), "gbs": round(gbs, 1), "frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4)})
        for w in ws:
            w.close()
    return out


def mix() -> list[dict]:
    from .engine import BatchRow
    cfg, tensors = synth.synth_named("qwen2.5-0.5b-q8_0", 0)
    eng = Engine.from_tensors(cfg, tensors)
    del tensors
    rng = np.random.default_rng(21)
    s = eng.session(600)
    tok = int(np.argmax(s.prefill(rng.integers(0, cfg.vocab_size, 512).astype(np.uint32))))
    s.decode_greedy(tok, 512, 8)
    s.close()
    bat = eng.batcher(4, 600)
    rows = []
    for slot in range(4):
        lg = bat.prefill(slot, rng.integers(0, cfg.vocab_size, 512).astype(np.uint32))
        rows.append(BatchRow(int(np.argmax(lg)), 512, slot))
    bat.decode_greedy(rows, 8)
    bat.close()
    eng.close()
    st = K.Stream()
    n_seq, nh, nkv, hd, ctx = 4, 14, 2, 64, 4096
    kv = rng.standard_normal(n_seq * nkv * ctx * hd).astype(np.float16).view(np.uint16)
    k, v = K.DeviceArray.from_numpy(kv), K.DeviceArray.from_numpy(kv[::-1].copy())
    q = K.DeviceArray.from_numpy(rng.standard_normal((n_seq, nh * hd)).astype(np.float32))
    cl = K.DeviceArray.from_numpy(np.full(n_seq, ctx, np.uint32))
    o = K.DeviceArray((n_seq, nh * hd))
    for _ in range(24):
        K.attn_decode(q, k, v, cl, n_seq, nh, nkv, hd, ctx, o, st.ptr)
    st.synchronize()
    k.free()
    v.free()
    st.close()
    # a plain device copy of 256 MiB (read 256, write 256), the reference the
    # FETCH_SIZE / WRITE_SIZE counters of a --pmc pass are scaled by
    n = 256 << 20
    src, dst = K.DeviceArray(n, np.uint8), K.DeviceArray(n, np.uint8)
    K.memset(src, 1)
    K.memcpy_dtod(dst, src)
    K.synchronize()
    src.free()
    dst.free()
    return [{"workload": "mix", "done": True}]


def stream() -> list[dict]:
    """The read bandwidth a plain streaming kernel gets on this device: the
    ROCm library's f32 sum reduction and device copy (through torch, used
    here only as a reference kernel) over 145 MB (the Qwen lm_head's Q8_0
    bytes) and 1 GiB -- the practical ceiling the HBM-bound kernels are
    compared with, beside the 8 TB/s datasheet peak."""
    import torch
    out = []
    for name, nbytes in (("145MB", 144_643_072), ("1GiB", 1 << 30)):
        x = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").uniform_()
        y = torch.empty_like(x)
        for op, fn, moved in (("sum", lambda: x.sum(), nbytes), ("copy", lambda: y.copy_(x), 2 * nbytes)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(20):
                fn()
            b.record()
            torch.cuda.synchronize()
            us = a.elapsed_time(b) / 20 * 1e3
            out.append({"workload": "stream", "op": op, "bytes": nbytes, "us": round(us, 2),
                        "gbs": round(moved / (us * 1e-6) / 1e9, 1),
                        "frac_of_hbm": round(moved / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        del x, y
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", default="decode,layers,attn,gemm,prefill,batch,matvec")
    args = ap.parse_args()
    want = set(args.only.split(","))
    if K.device_count() == 0:
        print("microbench: no HIP device visible", file=sys.stderr)
        return 1
    if "decode" in want:
        print(json.dumps(decode("smollm2-135m", 512, 128)), flush=True)
        print(json.dumps(decode("tinyllama-1.1b-q4_k", 256, 256)), flush=True)
    if "longctx" in want:  # the one-kernel step at long contexts (up to LK_FUSED_MAX_SEQ)
        for p in (4096, 16384, 32000):
            print(json.dumps(decode("qwen2.5-0.5b-q8_0", p, 64)), flush=True)
    if "layers" in want:
        for r in layers():
            print(json.dumps(r), flush=True)
    if "attn" in want:
        for r in attn():
            print(json.dumps(r), flush=True)
    for name, fn in (("gemm", gemm), ("prefill", prefill), ("batch", batch), ("matvec", matvec), ("mix", mix),
                     ("stream", stream), ("trace", stage_trace)):
        if name in want:
            for r in fn():
                print(json.dumps(r), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
