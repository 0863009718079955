"""Decode-step benchmark of the HIP backend (one JSON line on stdout).

Workload: Qwen2.5-0.5B shape, every linear weight in GGUF
Q8_0 (synthetic, seeded), 512-token random prompt prefilled, then greedy decode
of --steps tokens at batch 1, one GPU.  `value` is decode tok/s over exactly
--steps tokens (after --warmup untimed tokens), weights and KV resident in HBM.

A decode step is two launches: the one-kernel layer walk (fused_step_kernel:
QKV, attention, O, gate/up+SwiGLU, down for all 24 layers) and the final
norm + lm_head + argmax (lm_head_kernel).  `roofline` is the dominant kernel,
fused_step_kernel: its algorithmic bytes per launch (the 24 layers' Q8_0
weights, 380,190,720 B) / its average duration, timed live with hipEvents on
the session's stream in a second, event-bracketed pass over --profile-steps
tokens, against MI355X's 8 TB/s.  `roofline.kernels` gives both launches, and
`roofline.matvec_frac` the headline "% of HBM peak in the dequant-matvec
kernels" (all weight bytes / both kernels' time).  `roofline.traffic` is the
HBM bytes per launch that rocprofv3 FETCH_SIZE + WRITE_SIZE counted for the
same command (scaled by the counters' reading for a plain copy of known size;
see --copy-calibration-mb), read from the committed summary under profiles/.
`cpu_baseline` is lokal's CPU path (the C oracle: f32 weights expanded at load,
row-parallel matvec) timed on this host over the same positions the GPU line
times (the window repeated until a bounded budget is spent).
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
TRAFFIC_FILE = ROOT / "profiles" / "fused_step_qwen2.5-0.5b-q8_0_hbm_traffic.txt"


def measured_traffic() -> dict | None:
    """HBM bytes per launch of each kernel, from the committed rocprofv3 --pmc
    summary (lines "traffic <kernel> <bytes>")."""
    if not TRAFFIC_FILE.exists():
        return None
    out = {}
    for line in TRAFFIC_FILE.read_text().splitlines():
        parts = line.split()
        if len(parts) == 3 and parts[0] == "traffic":
            out[parts[1]] = float(parts[2])
    return out or None


def copy_calibration(mb: int) -> None:
    """A plain device copy of known size (read mb MiB, write mb MiB), three
    times, for scaling the FETCH_SIZE / WRITE_SIZE counters of a --pmc run."""
    import ctypes as C
    from lokal_amd._lib import check, lib
    n = mb << 20
    src, dst = C.c_void_p(), C.c_void_p()
    check(lib().lkhip_malloc(C.byref(src), n))
    check(lib().lkhip_malloc(C.byref(dst), n))
    check(lib().lkhip_memset(src, 1, n))
    for _ in range(3):
        check(lib().lkhip_memcpy_dtod(dst, src, n))
    check(lib().lkhip_synchronize())
    check(lib().lkhip_free(src))
    check(lib().lkhip_free(dst))


def host_cpus() -> dict:
    """What this host gives the process: logical CPUs, the ones it may run on,
    the cgroup CPU quota (cores' worth of time), and the CPU model."""
    info = {"nproc": os.cpu_count() or 1, "affinity": len(os.sched_getaffinity(0)), "cgroup_quota": None,
            "model": None}
    try:
        q, per = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            info["cgroup_quota"] = round(int(q) / int(per), 2)
    except (OSError, ValueError):
        pass
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                info["model"] = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return info


def cpu_baseline(cfg, tensors, prompt, p0: int, n_steps: int, budget_s: float) -> dict:
    """lokal's CPU path (the C oracle) over the same positions the GPU line
    times: the same prompt prefilled, greedy decode up to position p0
    untimed, then the window of positions p0 .. p0 + n_steps - 1 timed, and
    repeated from p0 (the same tokens rewrite the same cache rows: identical
    work) until the budget is spent."""
    import oracle
    # the -O3 -mavx2 build of the oracle (bit-identical to the parity build)
    # on every CPU this process may use; a cgroup quota below that caps the
    # threads that can run at once, so the thread count follows the quota
    oracle.select("o3")
    hc = host_cpus()
    threads = hc["affinity"]
    if hc["cgroup_quota"]:
        threads = max(1, min(threads, int(hc["cgroup_quota"])))
    oracle.set_threads(threads)
    om = oracle.Model(cfg, tensors)
    s = om.session(p0 + n_steps + 2)
    lo = s.prefill(prompt)  # untimed, as generate.rs times decode only
    cur = oracle.argmax(lo)
    for p in range(len(prompt), p0):  # the GPU line's warm-up positions, untimed
        cur = oracle.argmax(s.forward(cur, p))
    tok0 = cur
    t0 = time.perf_counter()
    n, reps = 0, 0
    while True:
        cur = tok0
        for i in range(n_steps):
            cur = oracle.argmax(s.forward(cur, p0 + i))
            n += 1
            if time.perf_counter() - t0 > budget_s:
                break
        else:
            reps += 1
            continue
        break
    dt = time.perf_counter() - t0
    s.close()
    om.close()
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "nproc": hc["nproc"], "affinity_cpus": hc["affinity"], "cgroup_cpu_quota": hc["cgroup_quota"],
            "cpu_model": hc["model"], "build": "gcc -O3 -mavx2 -fopenmp -ffp-contract=off (bit-identical to -O2)",
            "sample": f"{n} greedy decode tokens at positions {p0}..{p0 + n_steps - 1} (the GPU line's timed "
                      f"positions; {reps} full passes over the window, then part of one), after a "
                      f"{len(prompt)}-token prefill of the same prompt; same synthetic Q8_0 weights expanded to f32 "
                      f"(lokal's load_f32 path), {threads} OpenMP threads, {dt:.1f} s"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--profile-steps", type=int, default=32)
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="after the run, copy this many MiB on the device three times (counter calibration)")
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
    prefill_first_s = time.perf_counter() - t0
    # again, warm (the first call also allocates the multi-row buffers); it
    # rewrites the same positions with the same values
    t0 = time.perf_counter()
    logits = sess.prefill(prompt)
    prefill_s = time.perf_counter() - t0
    tok = int(np.argmax(logits))
    pos = args.prompt

    if args.warmup:
        ids = sess.decode_greedy(tok, pos, args.warmup)
        tok, pos = int(ids[-1]), pos + args.warmup
    timed_p0 = pos

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
    n_tok = max(prof["tokens"], 1)
    lm_bytes = prof["lm_head_bytes"] / n_tok
    lm_us = prof["lm_head_ms"] * 1e3 / n_tok
    fused_bytes = (prof["matvec_bytes"] - prof["lm_head_bytes"]) / n_tok
    fused_us = (prof["matvec_ms"] - prof["lm_head_ms"]) * 1e3 / n_tok
    fused_gbs = fused_bytes / (fused_us * 1e-6) / 1e9
    lm_gbs = lm_bytes / (lm_us * 1e-6) / 1e9
    all_gbs = (fused_bytes + lm_bytes) / ((fused_us + lm_us) * 1e-6) / 1e9
    traffic = measured_traffic()

    def kern(name, nbytes, us, gbs):
        return {"name": name, "algorithmic_bytes": nbytes, "avg_us": round(us, 2), "achieved_gbs": round(gbs, 1),
                "frac": round(gbs / HBM_PEAK_GBS, 4),
                "traffic": traffic.get(name) if traffic else None}

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
            "kernel": "fused_step_kernel (24 layers: QKV, attention, O, gate/up+SwiGLU, down)",
            "achieved": round(fused_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(fused_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic.get("fused_step_kernel") if traffic else None,
            "kernels": [kern("fused_step_kernel", fused_bytes, fused_us, fused_gbs),
                        kern("lm_head_kernel", lm_bytes, lm_us, lm_gbs)],
            "matvec_frac": round(all_gbs / HBM_PEAK_GBS, 4),
            # each kernel's time is a pair of hipEvents around its launch on
            # the session's stream, so it also spans the launch gap before the
            # kernel; their sum against the timed step shows the gaps'
            # share (rocprofv3's kernel times, under profiles/, exclude them)
            "timing": "hipEvent pairs around each launch (each spans its launch gap)",
            "events_sum_us": round(fused_us + lm_us, 2),
            "step_us": round(dt / args.steps * 1e6, 2),
            "algorithmic_bytes_per_token": mv_bytes,
            "profiled_tokens": int(prof["tokens"]),
        },
        # context, outside the timed decode: the 512-token prompt through
        # Session::prefill (one chunk on the multi-row GEMM path), warm; the
        # first call, which also allocates that path's buffers, beside it
        "prefill": {"tokens": args.prompt, "s": round(prefill_s, 4),
                    "tok_s": round(args.prompt / prefill_s, 1), "first_call_s": round(prefill_first_s, 4)},
    }
    sess.close()
    eng.close()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, tensors, prompt, timed_p0, args.steps, args.cpu_budget)
    del tensors
    print(json.dumps(result), flush=True)
    if args.copy_calibration_mb:
        copy_calibration(args.copy_calibration_mb)
    return 0


if __name__ == "__main__":
    sys.exit(main())
