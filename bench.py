"""Decode-step benchmark of the HIP backend (one JSON line on stdout).

Workload: Qwen2.5-0.5B shape, every linear weight in GGUF
Q8_0 (synthetic, seeded), 512-token random prompt prefilled, then greedy decode
of --steps tokens at batch 1, one GPU.  `value` is decode tok/s over exactly
--steps tokens (after --warmup untimed tokens), weights and KV resident in HBM.

The `roofline` object is the dequant-matvec family (every matvec launch of the
decode step, lm_head included): algorithmic Q8_0 weight bytes / summed
hipEvent kernel time, measured live on the session's stream in a second,
event-bracketed pass over --profile-steps tokens, against MI355X's 8 TB/s.
`cpu_baseline` is lokal's CPU path (the C oracle: f32 weights expanded at load,
row-parallel matvec) timed on this host on a bounded sample of the same decode.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402

METRIC = "decode tok/s + % of HBM peak in dequant-matvec, Q8_0 Qwen2.5-0.5B-shape, 1 GPU"
HBM_PEAK_GBS = 8000.0


def cpu_baseline(cfg, tensors, prompt_len: int, budget_s: float) -> dict:
    import oracle
    threads = max(1, min(16, os.cpu_count() or 1))
    oracle.set_threads(threads)
    om = oracle.Model(cfg, tensors)
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, cfg.vocab_size, prompt_len).astype(np.uint32)
    n_max = 64
    s = om.session(prompt_len + n_max + 2)
    lo = s.prefill(prompt)  # untimed, as generate.rs times decode only
    cur = oracle.argmax(lo)
    # one untimed warm-up token, then time tokens until the budget is spent
    lo = s.forward(cur, prompt_len)
    cur = oracle.argmax(lo)
    t0 = time.perf_counter()
    n = 0
    while n < n_max:
        lo = s.forward(cur, prompt_len + 1 + n)
        cur = oracle.argmax(lo)
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    s.close()
    om.close()
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} greedy decode tokens after a {prompt_len}-token prefill and 1 warm-up token, "
                      f"same synthetic Q8_0 weights expanded to f32 (lokal's load_f32 path), "
                      f"{threads} OpenMP threads, {dt:.1f} s"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--profile-steps", type=int, default=32)
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--cpu-prompt", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: lokal's decode step has no multi-GPU path "
              "(sharding is a design note, not built); run with --gpus 1", file=sys.stderr)
        return 2

    from lokal_amd import Engine, _lib, synth

    if _lib.lib().lkhip_device_count() == 0:
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1

    cfg, tensors = synth.synth_named("qwen2.5-0.5b-q8_0", args.seed)
    eng = Engine.from_tensors(cfg, tensors)
    mv_bytes = eng.matvec_bytes
    max_seq = args.prompt + args.warmup + args.steps + args.profile_steps + 2
    sess = eng.session(max_seq)
    prompt = np.random.default_rng(args.seed + 1).integers(0, cfg.vocab_size, args.prompt).astype(np.uint32)

    t0 = time.perf_counter()
    logits = sess.prefill(prompt)
    prefill_s = time.perf_counter() - t0
    tok = int(np.argmax(logits))
    pos = args.prompt

    if args.warmup:
        ids = sess.decode_greedy(tok, pos, args.warmup)
        tok, pos = int(ids[-1]), pos + args.warmup

    t0 = time.perf_counter()
    ids = sess.decode_greedy(tok, pos, args.steps)  # syncs the stream before returning
    dt = time.perf_counter() - t0
    tok, pos = int(ids[-1]), pos + args.steps
    tok_s = args.steps / dt

    # Event-bracketed pass: per-launch kernel times of the same decode step.
    sess.set_profiling(True)
    sess.profile(reset=True)
    sess.decode_greedy(tok, pos, args.profile_steps)
    prof = sess.profile(reset=True)
    sess.set_profiling(False)
    mv_gbs = prof["matvec_bytes"] / (prof["matvec_ms"] * 1e-3) / 1e9
    lm_gbs = prof["lm_head_bytes"] / (prof["lm_head_ms"] * 1e-3) / 1e9 if prof["lm_head_ms"] else None
    n_tok = max(prof["tokens"], 1)

    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0",
        "data": "synthetic",
        "config": {"workload": "qwen2.5-0.5b-q8_0 greedy decode (BASELINE configs[2])", "batch": 1,
                   "prompt_tokens": args.prompt, "decode_tokens": args.steps, "kv_cache": "f16",
                   "accumulate": "f32", "weights": "Q8_0 synthetic, seed %d" % args.seed},
        "roofline": {
            "bound": "hbm",
            "kernel": "dequant-matvec family (QKV, O, gate/up+SwiGLU, down, lm_head+argmax)",
            "achieved": round(mv_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(mv_gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "algorithmic_bytes_per_token": mv_bytes,
            "matvec_us_per_token": round(prof["matvec_ms"] * 1e3 / n_tok, 2),
            "lm_head_gbs": round(lm_gbs, 1) if lm_gbs else None,
            "attn_us_per_token": round(prof["attn_ms"] * 1e3 / n_tok, 2),
            "other_us_per_token": round(prof["other_ms"] * 1e3 / n_tok, 2),
            "profiled_tokens": int(prof["tokens"]),
        },
        "prefill_s": round(prefill_s, 3),
    }
    sess.close()
    eng.close()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, tensors, args.cpu_prompt, args.cpu_budget)
    del tensors
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
