"""Decode benchmark: TinyLlama-1.1B-shape W8A8 decoder, batch 1, one MI355X.

Workload (the configuration the metric is quoted on): 22 layers, d_model 2048,
32 query / 4 KV heads of 64, SwiGLU 5632, RMSNorm eps 1e-5, RoPE theta 1e4,
vocab 32000, untied FP32 LM head; random-init weights N(0, 0.02) quantized to
INT8 per output row, RMSNorm weights 1; activations quantized per token
(W8A8).  A 512-token random prompt is prefilled, then greedy decode runs;
config.prefill_ms is that first (cold) prefill, config.prefill_warm_p50_ms the
median of ten more on the warm session after the decode.
A "step" is one decode token (one forward of one token plus the device argmax
that feeds the next step).  `value` is decode tokens per second with all
weights and the KV cache resident in HBM.

Beside it:
  roofline      the dominant decode kernel (the persistent decode step; the W8A8
                GEMVs when the multi-launch path runs), algorithmic bytes per
                launch / its HIP-event time, from a second, instrumented pass
                of the same decode steps;
  gemv          standalone W8A8 GEMV at the TinyLlama shapes (M = 1), rotating
                >= 1 GiB of weight copies so the 256 MiB MALL cannot serve them;
  linear_w8a8   the same shapes at M = 4, 16, 128 and 512 tokens (the prefill
                GEMM at 512): us per call, int8 TOPS against the 5.0 POPS peak;
  cpu_baseline  the reference CPU engine (oracle/_ref/leaf_decoder, built from the
                reference sources) on this host, on a bounded sample.
  traffic       HBM bytes per launch of the dominant kernel from two rocprofv3
                counter passes (FETCH_SIZE, WRITE_SIZE), each scaled by what the
                same counter reads for a copy of known size (leaf_amd/bin/hbm_copy);
                derived once with --derive-traffic and kept in profiles/.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
    python bench.py --derive-traffic DIR   # DIR holds the four counter runs (see profiles/)
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, datasheet
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA, datasheet
TRAFFIC_FILE = ROOT / "profiles" / "decode_step_tinyllama_w8a8_traffic.json"
COPY_BYTES = 1 << 30           # hbm_copy 1024: reads and writes this many bytes per launch
PROMPT_TOKENS = 512
SEED = 20261201
METRIC = "decode tok/s + GEMV HBM GB/s (% peak), TinyLlama-shape W8A8, batch 1"


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def artifact_path() -> Path:
    base = Path(os.environ.get("LEAF_BENCH_DIR", Path(tempfile.gettempdir()) / "leaf_bench"))
    base.mkdir(parents=True, exist_ok=True)
    return base / f"tinyllama_w8a8_seed{SEED}.leaf"


def ensure_artifact() -> Path:
    from leaf_amd import models
    from leaf_amd.artifact import write_artifact
    path = artifact_path()
    if not path.exists():
        t = time.perf_counter()
        write_artifact(path, models.tinyllama_w8a8(), seed=SEED)
        log(f"wrote {path} ({path.stat().st_size / 1e9:.2f} GB) in {time.perf_counter() - t:.1f}s")
    return path


def decode_benchmark(path: Path, steps: int, warmup: int, prefill_repeats: int = 10) -> dict:
    from leaf_amd import runtime
    rng = np.random.default_rng(SEED + 1)
    prompt = rng.integers(0, 32000, PROMPT_TOKENS).astype(np.uint32)
    context = PROMPT_TOKENS + 2 * (warmup + steps) + 8
    dec = runtime.Decoder(path, activation_bits=8, max_context=context, max_prefill=PROMPT_TOKENS)
    t = time.perf_counter()
    token = dec.forward_into(prompt, None)
    prefill_ms = (time.perf_counter() - t) * 1e3
    for _ in range(warmup):
        token = dec.forward_into([token], None)
    runtime.synchronize()
    start = time.perf_counter()
    tokens = []
    for _ in range(steps):
        token = dec.forward_into([token], None)
        tokens.append(token)
    runtime.synchronize()
    elapsed = time.perf_counter() - start
    # Same decode steps again with every launch bracketed by HIP events.
    dec.set_profiling(True)
    for _ in range(steps):
        token = dec.forward_into([token], None)
    runtime.synchronize()
    profile = dec.profile()
    dec.set_profiling(False)
    ctx_end = dec.cache_tokens()
    # The same 512-token prefill again on a warm session (cache cleared first).
    warm = []
    for _ in range(prefill_repeats):
        dec.reset()
        runtime.synchronize()
        t = time.perf_counter()
        dec.forward_into(prompt, None)
        runtime.synchronize()
        warm.append((time.perf_counter() - t) * 1e3)
    dec.close()
    return {"elapsed_s": elapsed, "prefill_ms": prefill_ms, "profile": profile, "context_end": ctx_end,
            "prefill_warm_ms": float(np.median(warm)) if warm else None,
            "tokens": tokens[:8]}


def gemv_microbench(repeats: int = 20) -> dict:
    """W8A8 GEMV at M = 1 over >= 1 GiB of rotating weight copies."""
    from leaf_amd import runtime
    from leaf_amd.models import W8A8_LINEAR_SHAPES
    rng = np.random.default_rng(SEED + 2)
    shapes = sorted(set(W8A8_LINEAR_SHAPES))
    layer_bytes = sum(k * n for k, n in W8A8_LINEAR_SHAPES)
    copies = int(np.ceil(1.1 * (1 << 30) / layer_bytes))
    results = {}
    host = {s: (rng.integers(-127, 128, (s[1], s[0]), dtype=np.int8),
                (rng.random(s[1], dtype=np.float32) * 1e-3 + 1e-4).astype(np.float32)) for s in shapes}
    weights = {s: [runtime.DeviceWeight(host[s][0], 8, s[0], host[s][1], s[0]) for _ in range(copies)]
               for s in shapes}
    for (K, N) in shapes:
        x = runtime.DeviceArray.of(rng.standard_normal((1, K), dtype=np.float32))
        y = runtime.DeviceArray((1, N), np.float32)
        ws = weights[(K, N)]
        for w in ws[:4]:
            runtime.linear(w, x, 1, 8, y)
        timer = runtime.Timer()
        launches = 0
        for r in range(repeats):
            for w in ws:
                runtime.linear(w, x, 1, 8, y)
                launches += 1
        ms = timer.stop() / launches
        algorithmic = N * K + 4 * N + K + 4 * N
        results[f"{K}x{N}"] = {"us": round(ms * 1e3, 3), "GBps": round(algorithmic / ms / 1e6, 1),
                               "frac": round(algorithmic / ms / 1e6 / HBM_PEAK_GBS, 3)}
    total_bytes = sum(K * N + 8 * N + K for K, N in W8A8_LINEAR_SHAPES)
    total_us = sum(results[f"{K}x{N}"]["us"] for K, N in W8A8_LINEAR_SHAPES)
    results["layer_set"] = {"GBps": round(total_bytes / total_us / 1e3, 1), "copies": copies,
                            "weight_bytes": copies * layer_bytes}
    for s in weights.values():
        for w in s:
            del w
    return results


def linear_microbench(tokens=(4, 16, 128, 512), repeats: int = 3) -> dict:
    """W8A8 linear at the TinyLlama shapes for M > 1 tokens: per-token int8
    activations (quantized beforehand, as the decoder's norm epilogues leave
    them), per-row int8 weights, the split-K epilogue included, rotating
    >= 1 GiB of weight copies.  Reported per shape as microseconds per call,
    int8 TOPS against the 5.0 POPS dense peak, and the bytes of the call
    (N*K + 8N + M*K + 4M + 4MN) per microsecond."""
    from leaf_amd import runtime
    from leaf_amd.models import W8A8_LINEAR_SHAPES
    rng = np.random.default_rng(SEED + 3)
    shapes = sorted(set(W8A8_LINEAR_SHAPES))
    layer_bytes = sum(k * n for k, n in W8A8_LINEAR_SHAPES)
    copies = int(np.ceil(1.1 * (1 << 30) / layer_bytes))
    weights = {}
    for (K, N) in shapes:
        data = rng.integers(-127, 128, (N, K), dtype=np.int8)
        scales = (rng.random(N, dtype=np.float32) * 1e-3 + 1e-4).astype(np.float32)
        weights[(K, N)] = [runtime.DeviceWeight(data, 8, K, scales, K) for _ in range(copies)]
    out = {}
    for M in tokens:
        row = {}
        for (K, N) in shapes:
            q = runtime.DeviceArray.of(rng.integers(-127, 128, (M, K), dtype=np.int8))
            xs = runtime.DeviceArray.of((rng.random(M, dtype=np.float32) * 1e-2 + 1e-3).astype(np.float32))
            y = runtime.DeviceArray((M, N), np.float32)
            ws = weights[(K, N)]
            for w in ws[:3]:
                runtime.linear_q(w, q, xs, M, y)
            timer = runtime.Timer()
            launches = 0
            for _ in range(repeats):
                for w in ws:
                    runtime.linear_q(w, q, xs, M, y)
                    launches += 1
            ms = timer.stop() / launches
            ops = 2.0 * M * N * K
            traffic = N * K + 8 * N + M * K + 4 * M + 4 * M * N
            row[f"{K}x{N}"] = {"us": round(ms * 1e3, 2), "TOPS": round(ops / ms / 1e9, 1),
                               "frac_mfma": round(ops / ms / 1e9 / INT8_PEAK_TOPS, 4),
                               "GBps": round(traffic / ms / 1e6, 1)}
        out[f"M={M}"] = row
    for s in weights.values():
        s.clear()
    return out


def cpu_baseline(path: Path, budget_s: float = 30.0) -> dict | None:
    """Reference CPU engine (built from the reference sources) on this host."""
    from leaf_amd.artifact import write_tokens
    ref = ROOT / "oracle" / "_ref" / "leaf_decoder"
    cores = min(len(os.sched_getaffinity(0)), 16, 64)
    rng = np.random.default_rng(SEED + 1)
    prompt = rng.integers(0, 32000, PROMPT_TOKENS).astype(np.uint32)
    generate = 9
    with tempfile.TemporaryDirectory() as tmp:
        req = Path(tmp) / "req.bin"
        write_tokens(req, [prompt.tolist()])
        if ref.exists():
            cmd = [str(ref), str(path), str(req), str(Path(tmp) / "l.bin"), str(Path(tmp) / "m.json"),
                   "bench-generate", str(cores), "1", "0", str(generate), "0", "1", "8"]
            t = time.perf_counter()
            run = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
            wall = time.perf_counter() - t
            if run.returncode != 0:
                log("reference CPU baseline failed:", run.stderr.strip())
                return None
            metrics = json.loads((Path(tmp) / "m.json").read_text())
            decode = metrics["decode_samples_ms"]
            return {"value": round(1e3 / float(np.mean(decode)), 3), "unit": "tok/s", "cores": cores,
                    "kind": "reference",
                    "sample": f"leaf_decoder bench-generate, {PROMPT_TOKENS}-token prompt + {generate - 1} decode "
                              f"steps, {cores} threads; prefill {metrics['prefill_p50_ms']:.0f} ms, decode p50 "
                              f"{metrics['decode_p50_ms']:.1f} ms/token; wall {wall:.1f}s"}
    # No reference build here: time the oracle (single-thread restatement).
    from oracle.bindings import oracle
    d = oracle().decoder(path, 8, False)
    t = time.perf_counter()
    d.forward(prompt[:16])
    steps, token = 0, 0
    start = time.perf_counter()
    while time.perf_counter() - start < budget_s / 3 and steps < 8:
        d.forward([token])
        steps += 1
    dt = (time.perf_counter() - start) / steps
    return {"value": round(1.0 / dt, 3), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"oracle decoder, 16-token prompt + {steps} decode steps"}


def _counter_means(csv_path: Path) -> dict:
    """Mean counter value (KiB) per kernel name in one rocprofv3 counter_collection.csv."""
    import csv
    sums: dict = {}
    with open(csv_path, newline="") as f:
        for row in csv.DictReader(f):
            total, count = sums.get(row["Kernel_Name"], (0.0, 0))
            sums[row["Kernel_Name"]] = (total + float(row["Counter_Value"]), count + 1)
    return {name: total / count for name, (total, count) in sums.items()}


def derive_traffic(base: Path, kernel: str = "decode_step_kernel") -> dict:
    """HBM bytes per launch of `kernel` from rocprofv3 --pmc runs under `base`:
    pmc_copy_{FETCH,WRITE}_SIZE (hbm_copy 1024 5) and pmc_step_{FETCH,WRITE}_SIZE
    (the leaf_decoder generation).  Each counter is scaled by the bytes a copy of
    COPY_BYTES moves per unit of that counter."""
    out = {"kernel": kernel}
    total = 0.0
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        copy = _counter_means(next((base / f"pmc_copy_{counter}").glob("*counter_collection.csv")))
        copy_kib = next(v for k, v in copy.items() if "hbm_copy_kernel" in k)
        scale = COPY_BYTES / copy_kib                    # bytes per counted KiB
        step = _counter_means(next((base / f"pmc_step_{counter}").glob("*counter_collection.csv")))
        step_kib = next(v for k, v in step.items() if kernel in k)
        out[counter] = {"kib_per_launch": round(step_kib, 1), "copy_kib": round(copy_kib, 1),
                        "bytes_per_kib": round(scale, 3), "bytes": round(step_kib * scale)}
        total += step_kib * scale
    out["bytes_per_launch"] = round(total)
    return out


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=120)
    parser.add_argument("--warmup", type=int, default=8)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-gemv", action="store_true")
    parser.add_argument("--no-linear", action="store_true")
    parser.add_argument("--derive-traffic", type=Path, default=None)
    args = parser.parse_args()
    if args.derive_traffic is not None:
        traffic = derive_traffic(args.derive_traffic)
        TRAFFIC_FILE.write_text(json.dumps(traffic, indent=1) + "\n")
        print(json.dumps(traffic))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        return 2
    path = ensure_artifact()
    log("decode benchmark ...")
    d = decode_benchmark(path, args.steps, args.warmup)
    value = args.steps / d["elapsed_s"]
    prof = d["profile"]
    # The dominant kernel: the persistent decode step when it ran (one launch
    # per token), else the W8A8 GEMVs of the multi-launch path.
    if prof.get("decode_step", {}).get("launches", 0) > 0:
        g, kernel = prof["decode_step"], ("decode_step_kernel (persistent W8A8 decode step: 22 layers, "
                                          "attention over the cache, FP32 head, argmax)")
    else:
        g = prof.get("gemv_w8a8", {"launches": 0, "ms": 0.0, "bytes": 0.0})
        kernel = "W8A8 decode GEMV (gemv_int_fused_kernel)"
    launches = max(g["launches"], 1)
    avg_ms = g["ms"] / launches
    bytes_per_launch = g["bytes"] / launches
    achieved = bytes_per_launch / avg_ms / 1e6 if avg_ms > 0 else 0.0
    traffic = None
    if TRAFFIC_FILE.exists() and "decode_step" in kernel:
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("bytes_per_launch")
    gemv = None
    if not args.no_gemv:
        log("GEMV microbenchmark ...")
        gemv = gemv_microbench()
    linear = None
    if not args.no_linear:
        log("W8A8 linear microbenchmark ...")
        linear = linear_microbench()
    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline ...")
        cpu = cpu_baseline(path)
    device_ms = {k: round(v["ms"] / args.steps, 4) for k, v in prof.items()}
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(d["elapsed_s"] / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8 (W8A8, int32 acc)",
        "data": "synthetic (random-init N(0,0.02) weights, seeded random prompt)",
        "config": {"workload": "TinyLlama-1.1B-architecture W8A8 decoder, batch 1, 512-token prompt then greedy "
                               "decode", "layers": 22, "hidden": 2048, "heads": 32, "kv_heads": 4, "ffn": 5632,
                   "vocab": 32000, "prompt_tokens": PROMPT_TOKENS, "context_end": d["context_end"],
                   "prefill_ms": round(d["prefill_ms"], 2),
                   "prefill_warm_p50_ms": round(d["prefill_warm_ms"], 3) if d["prefill_warm_ms"] else None},
        "roofline": {"bound": "hbm", "kernel": kernel,
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "avg_launch_us": round(avg_ms * 1e3, 3), "bytes_per_launch": round(bytes_per_launch),
                     "launches": g["launches"]},
        "device_ms_per_step": device_ms,
        "gemv": gemv,
        "linear_w8a8": linear,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
