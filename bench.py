"""Decode benchmark: TinyLlama-1.1B-shape W8A8 decoder, batch 1, one MI355X.

Workload (the configuration the metric is quoted on): 22 layers, d_model 2048,
32 query / 4 KV heads of 64, SwiGLU 5632, RMSNorm eps 1e-5, RoPE theta 1e4,
vocab 32000, untied FP32 LM head; random-init weights N(0, 0.02) quantized to
INT8 per output row, RMSNorm weights 1; activations quantized per token
(W8A8).  The artifact and the 512-token prompt are the seeded ones of the
reference's greedy run in tests/golden/full_configs.json; the prompt is
prefilled, then greedy decode runs.  config.prefill_ms is that first (cold)
prefill, config.prefill_warm_p50_ms the median of ten more on the warm session.
A "step" is one decode token (one forward of one token plus the device argmax
that feeds the next step).  `value` is decode tokens per second with all
weights and the KV cache resident in HBM, with the numerics a W8A8 decoder
runs by default: reference order, every float sum in the CPU engine's order
(bit-exact), on the persistent decode step (config.decode_step: steps it ran,
steps re-run on the memory exchange path after an XCD mismatch, whether the
XCD-local exchange stayed on).

Beside it:
  parity        the reference's whole greedy run (512-token prompt, 128 tokens,
                tests/golden/full_configs.npz) on the default path whatever
                --steps is: identical tokens, bit-equal prefill logits;
  fast_numerics a labelled extra, not the value: the same decode with
                reassociated float sums (numerics "fast", not bit-exact), its
                tok/s and its agreement with the reference;
  roofline      the dominant decode kernel (the persistent decode step; the W8A8
                GEMVs when the multi-launch path runs), algorithmic bytes per
                launch / its HIP-event time, from a second, instrumented pass
                of the same decode steps, against the datasheet and the
                measured (hbm_copy) bandwidth;
  peaks         measured streaming bandwidth (leaf_amd/bin/hbm_copy, 1 GiB) and
                MFMA rates (leaf_amd/bin/mfma_peak) beside the datasheet;
  gemv          standalone W8A8 GEMV at the TinyLlama shapes (M = 1), rotating
                >= 1 GiB of weight copies so the 256 MiB MALL cannot serve them,
                graph-replayed; and one launch over about 1 GiB of rows per
                weight format (W8A8, FP32, BF16, INT4 g32): the streaming rate;
  linear_w8a8   the same shapes at M = 4, 16, 128 and 512 tokens (the prefill
                GEMM at 512): us per call, int8 TOPS against the 5.0 POPS peak;
  configs       the other benchmark configurations at their configured sizes
                (GPT-2 FP32 16 + 32, Qwen INT4 4096 + 256, SmolLM2 BF16-accurate
                2048 + 256): prefill ms and TFLOP/s, decode tok/s, bytes per
                token and GB/s against HBM peak, agreement with the reference;
  cpu_baseline  the reference CPU engine (oracle/_ref/leaf_decoder, built from the
                reference sources) on this host, on bounded samples of the same
                workload (the 512-token prompt, then 8 decode steps): all
                allowed cores (at most 64) and one core, with the host's CPU model.
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
F32_PEAK_TFLOPS = 157.3        # MI355X dense f32 MFMA, datasheet
TRAFFIC_FILE = ROOT / "profiles" / "decode_step_tinyllama_w8a8_traffic.json"
COPY_BYTES = 1 << 30           # hbm_copy 1024: reads and writes this many bytes per launch
GOLDEN = ROOT / "tests" / "golden"
PROMPT_TOKENS = 512
SEED = 20261201                # microbenchmark inputs
METRIC = "decode tok/s + GEMV HBM GB/s (% peak), TinyLlama-shape W8A8, batch 1"


def golden() -> tuple[dict, dict]:
    """The reference's greedy runs at the configured sizes (data only)."""
    meta = json.loads((GOLDEN / "full_configs.json").read_text())
    with np.load(GOLDEN / "full_configs.npz", allow_pickle=False) as data:
        arrays = {k: data[k] for k in data.files}
    return meta, arrays


def config_prompt(meta: dict, vocab: int) -> np.ndarray:
    return np.random.default_rng(meta["prompt_seed"]).integers(0, vocab, meta["prompt_tokens"]).astype(np.uint32)


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def ensure_artifact(family: str = "tinyllama") -> Path:
    """The configuration's seeded artifact, as the reference's greedy run used it."""
    from leaf_amd import models
    from leaf_amd.artifact import write_artifact
    meta = golden()[0][family]
    base = Path(os.environ.get("LEAF_BENCH_DIR", Path(tempfile.gettempdir()) / "leaf_bench"))
    base.mkdir(parents=True, exist_ok=True)
    path = base / f"{family}_seed{meta['artifact_seed']}.leaf"
    if not path.exists():
        t = time.perf_counter()
        write_artifact(path, models.PRESETS[family](), seed=meta["artifact_seed"])
        log(f"wrote {path} ({path.stat().st_size / 1e9:.2f} GB) in {time.perf_counter() - t:.1f}s")
    return path


def rel_error(a, b) -> float:
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def leading_agreement(tokens, reference) -> int:
    return next((i for i, (a, b) in enumerate(zip(tokens, reference)) if a != b), min(len(tokens), len(reference)))


def decode_benchmark(path: Path, steps: int, warmup: int, numerics: str = "default",
                     prefill_repeats: int = 10, details: bool = True) -> dict:
    """Timed greedy decode after the 512-token prefill.  numerics "default" is
    what a W8A8 decoder runs with no option given: reference order (the CPU
    engine's float order, bit-exact); "fast" the reassociated kernels."""
    from leaf_amd import runtime
    meta, arrays = golden()
    prompt = config_prompt(meta["tinyllama"], 32000)
    context = PROMPT_TOKENS + 2 * (warmup + steps) + 8
    dec = runtime.Decoder(path, activation_bits=8, max_context=context, max_prefill=PROMPT_TOKENS,
                          numerics=numerics)
    t = time.perf_counter()
    dec.forward(prompt)
    prefill_ms = (time.perf_counter() - t) * 1e3
    token = int(dec.last_argmax.value)
    for _ in range(warmup):
        token = dec.forward_into([token], None)
    runtime.synchronize()
    before = dec.status()
    start = time.perf_counter()
    for _ in range(steps):
        token = dec.forward_into([token], None)
    runtime.synchronize()
    elapsed = time.perf_counter() - start
    after = dec.status()
    step = {"steps_on_persistent_kernel": after["step_tokens"] - before["step_tokens"],
            "steps_rerun_on_memory_path": after["step_memory_reruns"] - before["step_memory_reruns"],
            "xcd_local_exchange_on": after["xcd_local"]}
    if not details:
        dec.close()
        return {"elapsed_s": elapsed, "step": step, "reference_order": after["reference_order"]}
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
    # One more prefill with every launch bracketed by HIP events: device time,
    # operations and TOPS per kernel class.
    dec.reset()
    dec.set_profiling(True)
    dec.forward_into(prompt, None)
    runtime.synchronize()
    prefill_classes = {}
    for name, v in dec.profile().items():
        entry = {"launches": v["launches"], "ms": round(v["ms"], 4)}
        if v["ops"] > 0 and v["ms"] > 0:
            rate = v["ops"] / v["ms"] / 1e9          # TOPS (or TFLOP/s)
            peak = INT8_PEAK_TOPS if name == "gemm_w8a8" else F32_PEAK_TFLOPS
            entry.update({"T_per_s": round(rate, 1), "frac_peak": round(rate / peak, 4)})
        prefill_classes[name] = entry
    dec.set_profiling(False)
    reference_order = after["reference_order"]
    dec.close()
    return {"elapsed_s": elapsed, "prefill_ms": prefill_ms, "profile": profile, "context_end": ctx_end,
            "prefill_warm_ms": float(np.median(warm)) if warm else None, "step": step,
            "prefill_classes": prefill_classes, "reference_order": reference_order}


def parity_run(path: Path, numerics: str = "default") -> dict:
    """The reference's whole greedy run (512-token prompt, 128 tokens) on the
    GPU, whatever --steps says: prefill logits and every token against the
    reference's (tests/golden/full_configs.npz)."""
    from leaf_amd import runtime
    meta, arrays = golden()
    m = meta["tinyllama"]
    prompt = config_prompt(m, 32000)
    dec = runtime.Decoder(path, activation_bits=8, max_context=len(prompt) + m["generate"] + 8,
                          max_prefill=len(prompt), numerics=numerics)
    first = dec.forward(prompt)
    tokens = [int(dec.last_argmax.value)]
    before = dec.status()
    start = time.perf_counter()
    for _ in range(m["generate"] - 1):
        tokens.append(dec.forward_into([tokens[-1]], None))
    runtime.synchronize()
    elapsed = time.perf_counter() - start
    after = dec.status()
    reference_order = after["reference_order"]
    dec.close()
    reference = arrays["tinyllama_tokens"].tolist()
    want = arrays["tinyllama_prefill_logits"]
    bits = lambda a: np.ascontiguousarray(a, np.float32).view(np.uint32)   # noqa: E731
    return {"numerics": "reference order" if reference_order else "fast",
            "tokens_identical": f"{leading_agreement(tokens, reference)}/{len(reference)}",
            "prefill_logits_bit_equal": bool(np.array_equal(bits(first), bits(want))),
            "prefill_logit_error": float(rel_error(first, want)),
            "decode_steps_on_persistent_kernel": after["step_tokens"] - before["step_tokens"],
            "decode_tok_s": round((len(tokens) - 1) / elapsed, 1)}


def _replayed_us(calls: list, replays: int) -> float:
    """Microseconds per call of `calls` (closures that take a stream), captured
    once into a HIP graph and replayed: the GPU runs them back to back, so the
    figure is device time, not the Python caller's launch rate."""
    from leaf_amd import runtime
    stream = runtime.Stream()
    for call in calls[:3]:
        call(stream.handle)          # any scratch grows before the capture
    stream.synchronize()
    graph = runtime.Graph(stream, lambda: [call(stream.handle) for call in calls])
    graph.launch()
    stream.synchronize()
    timer = runtime.Timer(stream.handle)
    for _ in range(replays):
        graph.launch()
    ms = timer.stop()
    graph.close()
    stream.close()
    return ms * 1e3 / (replays * len(calls))


def gemv_microbench(repeats: int = 20) -> dict:
    """W8A8 GEMV at M = 1 over >= 1 GiB of rotating weight copies, graph-replayed."""
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
        calls = [lambda st, w=w: runtime.linear(w, x, 1, 8, y, stream=st) for w in weights[(K, N)]]
        us = _replayed_us(calls, repeats)
        algorithmic = N * K + 4 * N + K + 4 * N
        results[f"{K}x{N}"] = {"us": round(us, 3), "GBps": round(algorithmic / us / 1e3, 1),
                               "frac": round(algorithmic / us / 1e3 / HBM_PEAK_GBS, 3)}
    total_bytes = sum(K * N + 8 * N + K for K, N in W8A8_LINEAR_SHAPES)
    total_us = sum(results[f"{K}x{N}"]["us"] for K, N in W8A8_LINEAR_SHAPES)
    results["layer_set"] = {"GBps": round(total_bytes / total_us / 1e3, 1), "copies": copies,
                            "weight_bytes": copies * layer_bytes}
    for s in weights.values():
        for w in s:
            del w
    return results


def gemv_streaming(repeats: int = 5) -> dict:
    """One M = 1 GEMV launch over about 1 GiB of weight rows per weight format
    (K = 2048): the kernels' own streaming rate, free of the per-launch
    latency that dominates the 0.5-12 MB matrices of a decoder layer.  Bytes
    per launch: N*K*bits/8 + 4*N*K/group (scales) + activations + outputs."""
    from leaf_amd import runtime
    rng = np.random.default_rng(SEED + 4)
    K = 2048
    out = {}
    # (name, weight bits, activation bits, rows, group)
    formats = [("w8a8", 8, 8, 1 << 19, K), ("fp32", 32, 32, 1 << 17, 0), ("bf16", 16, 32, 1 << 18, 0),
               ("int4_g32", 4, 32, 1 << 19, 32)]
    for name, bits, act_bits, N, group in formats:
        row_bytes = K * bits // 8
        tile = rng.integers(0, 256, (256, row_bytes), dtype=np.uint8)
        if bits == 32:
            tile = (0.02 * rng.standard_normal((256, K))).astype(np.float32).view(np.uint8)
        elif bits == 16:
            tile = ((0.02 * rng.standard_normal((256, K))).astype(np.float32).view(np.uint32) >> 16).astype(
                np.uint16).view(np.uint8)
        data = np.resize(tile, (N, row_bytes))
        scales = None
        if bits in (8, 4):
            scales = (rng.random((N, K // group), dtype=np.float32) * 1e-3 + 1e-4).astype(np.float32)
        w = runtime.DeviceWeight(data, bits, K, scales, group)
        del data
        x = runtime.DeviceArray.of(rng.standard_normal((1, K), dtype=np.float32))
        y = runtime.DeviceArray((1, N), np.float32)
        us = _replayed_us([lambda st: runtime.linear(w, x, 1, act_bits, y, stream=st)], repeats)
        nbytes = N * row_bytes + (4 * N * (K // group) if group else 0) + 4 * K + 4 * N
        out[name] = {"rows": N, "bytes": nbytes, "us": round(us, 2), "GBps": round(nbytes / us / 1e3, 1),
                     "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 3)}
        del w
    return out


def linear_microbench(tokens=(4, 16, 128, 512), repeats: int = 3) -> dict:
    """W8A8 linear at the TinyLlama shapes for M > 1 tokens: per-token int8
    activations (quantized beforehand, as the decoder's norm epilogues leave
    them), per-row int8 weights, the split-K epilogue included, rotating
    >= 1 GiB of weight copies, graph-replayed (device time per call).
    Reported per shape as microseconds per call, int8 TOPS against the 5.0
    POPS dense peak, and the bytes of the call (N*K + 8N + M*K + 4M + 4MN)
    per microsecond."""
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
            calls = [lambda st, w=w: runtime.linear_q(w, q, xs, M, y, stream=st) for w in weights[(K, N)]]
            us = _replayed_us(calls, repeats)
            ops = 2.0 * M * N * K
            traffic = N * K + 8 * N + M * K + 4 * M + 4 * M * N
            row[f"{K}x{N}"] = {"us": round(us, 2), "TOPS": round(ops / us / 1e6, 1),
                               "frac_mfma": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4),
                               "GBps": round(traffic / us / 1e3, 1)}
        out[f"M={M}"] = row
    for s in weights.values():
        s.clear()
    return out


def config_benchmark(family: str, profile_steps: int = 32) -> dict:
    """One benchmark configuration at its configured size, fast kernels: the
    prefill (cold, then the median of three warm), the greedy decode of the
    reference's run (per-step wall time), one more profiled pass of decode
    steps and of the prefill for algorithmic bytes, operations and device time
    per kernel class."""
    from leaf_amd import runtime
    meta_all, arrays = golden()
    m = meta_all[family]
    path = ensure_artifact(family)
    dec = runtime.Decoder(path, m["activation_bits"], m["fp32_math"],
                          max_context=m["prompt_tokens"] + m["generate"] + profile_steps + 8,
                          max_prefill=m["prompt_tokens"])
    vocab = dec.vocabulary_size
    prompt = config_prompt(m, vocab)
    t = time.perf_counter()
    logits = dec.forward(prompt)
    cold_ms = (time.perf_counter() - t) * 1e3
    tokens = [int(dec.last_argmax.value)]
    step_ms = []
    for _ in range(m["generate"] - 1):
        t = time.perf_counter()
        tokens.append(dec.forward_into([tokens[-1]], None))
        step_ms.append((time.perf_counter() - t) * 1e3)
    dec.set_profiling(True)
    token = tokens[-1]
    for _ in range(profile_steps):
        token = dec.forward_into([token], None)
    decode_profile = dec.profile()
    dec.set_profiling(False)
    warm = []
    for _ in range(3):
        dec.reset()
        runtime.synchronize()
        t = time.perf_counter()
        dec.forward_into(prompt, None)
        runtime.synchronize()
        warm.append((time.perf_counter() - t) * 1e3)
    dec.reset()
    dec.set_profiling(True)
    dec.forward_into(prompt, None)
    prefill_profile = dec.profile()
    dec.close()
    decode_ms = float(np.mean(step_ms))
    bytes_per_token = sum(v["bytes"] for v in decode_profile.values()) / profile_steps
    device_ms = sum(v["ms"] for v in decode_profile.values()) / profile_steps
    top = max(decode_profile, key=lambda k: decode_profile[k]["ms"])
    top_gbs = decode_profile[top]["bytes"] / max(decode_profile[top]["ms"], 1e-9) / 1e6
    flops = sum(v["ops"] for v in prefill_profile.values())
    prefill_ms = float(np.median(warm))
    gemm = {k: v for k, v in prefill_profile.items() if k.startswith("gemm")}
    gemm_ms = sum(v["ms"] for v in gemm.values())
    gemm_tflops = sum(v["ops"] for v in gemm.values()) / max(gemm_ms, 1e-9) / 1e9
    reference = arrays[f"{family}_tokens"].tolist()
    return {
        "workload": f"{family}: {m['prompt_tokens']}-token prompt + {m['generate']} greedy tokens, "
                    f"activation bits {m['activation_bits']}, FP32 math {m['fp32_math']}",
        "prefill_ms": round(cold_ms, 2), "prefill_warm_p50_ms": round(prefill_ms, 3),
        "prefill_TFLOPs": round(flops / prefill_ms / 1e9, 2),
        "prefill_gemm": {"ms": round(gemm_ms, 3), "TFLOPs": round(gemm_tflops, 2),
                         "frac_f32_mfma": round(gemm_tflops / F32_PEAK_TFLOPS, 4)},
        "decode_tok_s": round(1e3 / decode_ms, 1), "decode_p50_ms": round(float(np.median(step_ms)), 4),
        "decode_mean_ms": round(decode_ms, 4), "bytes_per_token": round(bytes_per_token),
        "decode_GBps": round(bytes_per_token / decode_ms / 1e6, 1),
        "decode_frac_hbm": round(bytes_per_token / decode_ms / 1e6 / HBM_PEAK_GBS, 4),
        "device_GBps": round(bytes_per_token / device_ms / 1e6, 1),
        "dominant_kernel": {"class": top, "GBps": round(top_gbs, 1), "frac_hbm": round(top_gbs / HBM_PEAK_GBS, 4)},
        "tokens_identical": f"{leading_agreement(tokens, reference)}/{len(reference)}",
        "prefill_logit_error": float(f"{rel_error(logits, arrays[f'{family}_prefill_logits']):.3g}"),
    }


def measured_peaks() -> dict:
    """Streaming bandwidth and MFMA rates measured on this device."""
    out = {"datasheet": {"hbm_GBps": HBM_PEAK_GBS, "int8_mfma_TOPS": INT8_PEAK_TOPS, "bf16_mfma_TFLOPs": 2500.0,
                         "f32_mfma_TFLOPs": F32_PEAK_TFLOPS}}
    copy = ROOT / "leaf_amd" / "bin" / "hbm_copy"
    mfma = ROOT / "leaf_amd" / "bin" / "mfma_peak"
    if copy.exists():
        run = subprocess.run([str(copy), "1024", "10"], capture_output=True, text=True, timeout=120)
        if run.returncode == 0:
            for line in run.stdout.splitlines():
                rate = float(line.split(",")[-1].split()[0])
                out["hbm_copy_GBps" if line.startswith("hbm_copy") else "hbm_read_GBps"] = rate
    if mfma.exists():
        run = subprocess.run([str(mfma)], capture_output=True, text=True, timeout=120)
        if run.returncode == 0:
            out["mfma_TOPS"] = {}
            names = {"int8": "int8_mfma_TOPS", "bf16": "bf16_mfma_TFLOPs", "f32": "f32_mfma_TFLOPs"}
            for line in run.stdout.splitlines():
                kind, instruction = line.split()[1], line.split()[2]
                rate = float(line.split("T/s")[0].split()[-1])
                out["mfma_TOPS"][instruction] = rate
                out[names[kind]] = max(out.get(names[kind], 0.0), rate)
    return out


def host_cpu() -> dict:
    allowed = len(os.sched_getaffinity(0))
    model, flags = "unknown", []
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            if line.startswith("flags") and not flags:
                have = set(line.split(":", 1)[1].split())
                flags = [f for f in ("avx2", "fma", "avx_vnni", "avx512f", "avx512_vnni") if f in have]
    except OSError:
        pass
    return {"allowed_cpus": allowed, "nproc": os.cpu_count(), "model": model, "flags": flags}


def reference_cpu_run(path: Path, prompt: np.ndarray, generate: int, threads: int) -> dict | None:
    """leaf_decoder bench-generate (main_decoder.cpp:278-298) of the reference build."""
    from leaf_amd.artifact import write_tokens
    ref = ROOT / "oracle" / "_ref" / "leaf_decoder"
    if not ref.exists():
        return None
    with tempfile.TemporaryDirectory() as tmp:
        req = Path(tmp) / "req.bin"
        write_tokens(req, [prompt.tolist()])
        cmd = [str(ref), str(path), str(req), str(Path(tmp) / "l.bin"), str(Path(tmp) / "m.json"),
               "bench-generate", str(threads), "1", "0", str(generate), "0", "1", "8"]
        t = time.perf_counter()
        run = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
        wall = time.perf_counter() - t
        if run.returncode != 0:
            log("reference CPU baseline failed:", run.stderr.strip())
            return None
        metrics = json.loads((Path(tmp) / "m.json").read_text())
    decode = metrics["decode_samples_ms"]
    return {"value": round(1e3 / float(np.mean(decode)), 3), "unit": "tok/s", "cores": threads,
            "sample": f"leaf_decoder bench-generate, {len(prompt)}-token prompt + {generate - 1} decode steps, "
                      f"{threads} threads; prefill {metrics['prefill_p50_ms']:.0f} ms, decode p50 "
                      f"{metrics['decode_p50_ms']:.1f} ms/token; wall {wall:.1f}s"}


def cpu_baseline(path: Path, budget_s: float = 30.0) -> dict | None:
    """Reference CPU engine (built from the reference sources) on this host,
    on the 512-token prompt then 8 decode steps: all allowed cores (at most 64,
    the engine's pool limit, host_support.h:119), and one core."""
    host = host_cpu()
    prompt = config_prompt(golden()[0]["tinyllama"], 32000)
    cores = min(host["allowed_cpus"], 64)
    every = reference_cpu_run(path, prompt, 9, cores)
    if every is not None:
        one = reference_cpu_run(path, prompt, 9, 1)
        every.update({"kind": "reference", "one_core": one, "host": host})
        return every
    # No reference build here: time the oracle (single-thread restatement).
    from oracle.bindings import oracle
    d = oracle().decoder(path, 8, False)
    d.forward(prompt[:16])
    steps, token = 0, 0
    start = time.perf_counter()
    while time.perf_counter() - start < budget_s / 3 and steps < 8:
        d.forward([token])
        steps += 1
    dt = (time.perf_counter() - start) / steps
    return {"value": round(1.0 / dt, 3), "unit": "tok/s", "cores": 1, "kind": "port", "host": host,
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


def _db_counters(db: Path) -> list:
    """Per-dispatch counter values of a rocprofv3 --pmc run (rocpd SQLite output),
    in dispatch order: [(kernel name, blocks, {counter: value})]."""
    import sqlite3
    con = sqlite3.connect(str(db))
    rows = con.execute("select dispatch_id, kernel_name, grid_size, workgroup_size, counter_name, value "
                       "from counters_collection order by dispatch_id").fetchall()
    con.close()
    out: dict = {}
    for dispatch, name, grid, group, counter, value in rows:
        entry = out.setdefault(dispatch, (name, grid // max(group, 1), {}))
        entry[2][counter] = entry[2].get(counter, 0.0) + value
    return [out[k] for k in sorted(out)]


# The four W8A8 GEMMs of a TinyLlama prefill layer, in launch order, at 512
# tokens: (name, rows, K).
PREFILL_GEMMS = (("qkv", 2560, 2048), ("o", 2048, 2048), ("gate_up", 11264, 2048), ("down", 2048, 5632))
# Template arguments of the only tile configuration the stacked gate|up
# projection uses (128 rows x 256 tokens, 2 x 4 waves): the label of its dispatches.
GATE_UP_TILE = "<2, 2, 3, 2, 4>"


def derive_prefill_counters(base: Path) -> dict:
    """MFMA utilisation and HBM bytes per prefill GEMM shape from rocprofv3 --pmc
    runs under `base` (each a directory holding one *_results.db):
      mfma/      SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE of the bench
                 (decode + prefills, no microbenchmarks)
      fetch/ write/        FETCH_SIZE / WRITE_SIZE of the same run
      peak/      the same three counters over leaf_amd/bin/mfma_peak (the MFMA issue loop)
      copy_fetch/ copy_write/   FETCH_SIZE / WRITE_SIZE over leaf_amd/bin/hbm_copy 1024
    MFMA busy fractions are scaled so that the int8 32x32x32 issue loop reads
    its measured share of the datasheet rate."""
    def db(name):
        return next((base / name).glob("*.db"))

    def gemms(entries):
        # Label the prefill GEMM dispatches: q|k|v runs 320 blocks of 64 x 64
        # tiles, gate|up 128 x 256 tiles on eight waves; o and down both run 256 blocks and
        # follow q|k|v and gate|up respectively (the last layer, trimmed to
        # one row, runs only its q|k|v as a GEMM).
        out, previous = [], None
        for name, blocks, values in entries:
            if "gemm_w8a8_mfma_kernel" not in name:
                continue
            if GATE_UP_TILE in name:
                label = "gate_up"
            elif blocks == 320:
                label = "qkv"
            elif blocks == 256 and previous in ("qkv", "gate_up"):
                label = "o" if previous == "qkv" else "down"
            else:
                previous = None
                continue
            out.append((label, values))
            previous = label
        return out

    peak = [v for name, _, v in _db_counters(db("peak")) if "mfma_i8_32" in name]
    peak_busy = max(v["SQ_VALU_MFMA_BUSY_CYCLES"] / v["GRBM_GUI_ACTIVE"] for v in peak)
    peak_cu = max(v["SQ_VALU_MFMA_BUSY_CYCLES"] / v["SQ_BUSY_CU_CYCLES"] for v in peak)
    copy = {}
    for counter, sub in (("FETCH_SIZE", "copy_fetch"), ("WRITE_SIZE", "copy_write")):
        vals = [v[counter] for name, _, v in _db_counters(db(sub)) if "hbm_copy_kernel" in name]
        copy[counter] = COPY_BYTES / (sum(vals) / len(vals))
    table = {}
    for label, values in gemms(_db_counters(db("mfma"))):
        t = table.setdefault(label, {"mfma": [], "cu": [], "fetch": [], "write": []})
        t["mfma"].append(values["SQ_VALU_MFMA_BUSY_CYCLES"] / values["GRBM_GUI_ACTIVE"] / peak_busy)
        t["cu"].append(values["SQ_VALU_MFMA_BUSY_CYCLES"] / values["SQ_BUSY_CU_CYCLES"] / peak_cu)
    for counter, sub, key in (("FETCH_SIZE", "fetch", "fetch"), ("WRITE_SIZE", "write", "write")):
        for label, values in gemms(_db_counters(db(sub))):
            table[label][key].append(values[counter] * copy[counter])
    out = {"peak_reference": "leaf_amd/bin/mfma_peak v_mfma_i32_32x32x32_i8 loop", "shapes": {}}
    for name, rows, K in PREFILL_GEMMS:
        t = table[name]
        mean = lambda v: sum(v) / len(v)   # noqa: E731
        out["shapes"][name] = {
            "M": 512, "N": rows, "K": K, "dispatches": len(t["mfma"]),
            "mfma_busy_of_peak_loop_wall": round(mean(t["mfma"]), 4),
            "mfma_busy_of_peak_loop_cu_busy": round(mean(t["cu"]), 4),
            "fetch_bytes": round(mean(t["fetch"])), "write_bytes": round(mean(t["write"])),
            # weights, row scales and biases, int8 activations and their scales; f32 outputs
            "algorithmic_read_bytes": rows * K + 8 * rows + 512 * K + 4 * 512,
            "algorithmic_write_bytes": 4 * 512 * rows}
    return out


def derive_f32_gemm_counters(base: Path) -> dict:
    """MFMA utilisation of the f32 prefill GEMMs of the Qwen INT4 (4096-token)
    and SmolLM2 BF16 (2048-token) prefills, from rocprofv3 --pmc runs under
    `base` with SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE:
      qwen/ smollm2/   leaf_decoder, one prefill of the configuration's prompt,
                       counters on the gemm_f32 kernels only
      peak/            leaf_amd/bin/mfma_peak (its v_mfma_f32_16x16x4_f32 loop)
    Busy fractions are relative to what the same ratios read for that loop."""
    import re

    from leaf_amd import models

    def db(name):
        return next((base / name).glob("*.db"))

    peak = [v for name, _, v in _db_counters(db("peak")) if "mfma_f32_kernel" in name]
    peak_busy = max(v["SQ_VALU_MFMA_BUSY_CYCLES"] / v["GRBM_GUI_ACTIVE"] for v in peak)
    peak_cu = max(v["SQ_VALU_MFMA_BUSY_CYCLES"] / v["SQ_BUSY_CU_CYCLES"] for v in peak)
    meta = golden()[0]
    out = {"peak_reference": "leaf_amd/bin/mfma_peak v_mfma_f32_16x16x4_f32 loop", "configs": {}}
    for family in ("qwen", "smollm2"):
        spec = models.PRESETS[family]()
        M = meta[family]["prompt_tokens"]
        qkv_rows = spec.heads * spec.head_dim + 2 * spec.kv_heads * spec.head_dim
        up_rows = 2 * spec.intermediate if spec.gated else spec.intermediate
        shapes = {"qkv": (qkv_rows, spec.hidden), "o": (spec.hidden, spec.heads * spec.head_dim),
                  "gate_up": (up_rows, spec.hidden), "down": (spec.hidden, spec.intermediate)}
        entries = [(name, blocks, v) for name, blocks, v in _db_counters(db(family)) if "gemm_f32" in name]
        # A layer launches q|k|v, o, gate|up, down in that order; o and down
        # can share a kernel and grid, so they are told apart by what came before.
        keys = [(name, blocks) for name, blocks, _ in entries[:4]]
        table, previous = {}, None
        for name, blocks, v in entries:
            key = (name, blocks)
            label = ("qkv" if key == keys[0] else "gate_up" if key == keys[2]
                     else "o" if key == keys[1] and previous == "qkv"
                     else "down" if key == keys[3] and previous == "gate_up" else None)
            previous = label
            if label is None:
                continue
            kernel = re.sub(r"leafhip::|\(anonymous namespace\)::", "", name).split("(")[0]
            t = table.setdefault(label, {"kernel": kernel, "blocks": blocks, "wall": [], "cu": []})
            t["wall"].append(v["SQ_VALU_MFMA_BUSY_CYCLES"] / v["GRBM_GUI_ACTIVE"] / peak_busy)
            t["cu"].append(v["SQ_VALU_MFMA_BUSY_CYCLES"] / v["SQ_BUSY_CU_CYCLES"] / peak_cu)
        out["configs"][family] = {
            label: {"M": M, "N": shapes[label][0], "K": shapes[label][1], "kernel": t["kernel"],
                    "blocks": t["blocks"], "dispatches": len(t["wall"]),
                    "mfma_busy_of_peak_loop_wall": round(sum(t["wall"]) / len(t["wall"]), 4),
                    "mfma_busy_of_peak_loop_cu_busy": round(sum(t["cu"]) / len(t["cu"]), 4)}
            for label, t in table.items()}
    return out


def summarize_counters(base: Path) -> str:
    """Mean counter values per dispatch, per kernel, over every rocprofv3 --pmc
    run under `base` (each a directory holding one *_results.db)."""
    import re
    per: dict = {}
    for db in sorted(base.glob("*/*_results.db")):
        for name, _, values in _db_counters(db):
            kernel = re.sub(r"leafhip::|\(anonymous namespace\)::", "", name).split("(")[0]
            for counter, value in values.items():
                per.setdefault((kernel, counter), []).append(value)
    lines = ["| Kernel | Counter | Dispatches | Mean per dispatch |", "|---|---|---:|---:|"]
    for (kernel, counter), vals in sorted(per.items()):
        lines.append(f"| `{kernel}` | {counter} | {len(vals)} | {sum(vals) / len(vals):,.1f} |")
    return "\n".join(lines)


def summarize_trace(db: Path, top: int = 25) -> str:
    """Markdown tables from a rocprofv3 --kernel-trace run (rocpd SQLite output):
    the top kernels by total time, and the prefill W8A8 GEMMs by shape (labelled
    as in derive_prefill_counters) with int8 TOPS against the datasheet peak."""
    import re
    import sqlite3
    con = sqlite3.connect(str(db))
    rows = con.execute("select name, grid_x / workgroup_x, duration from kernels order by start").fetchall()
    con.close()
    clean = lambda n: re.sub(r"leafhip::|\(anonymous namespace\)::", "", n).split("(")[0]   # noqa: E731
    totals: dict = {}
    for name, blocks, duration in rows:
        t = totals.setdefault(clean(name), [0, 0.0])
        t[0] += 1
        t[1] += duration
    all_ns = sum(t[1] for t in totals.values())
    lines = ["| Kernel | Calls | Total ms | Average us | % of kernel time |", "|---|---:|---:|---:|---:|"]
    for name, (calls, ns) in sorted(totals.items(), key=lambda kv: -kv[1][1])[:top]:
        lines.append(f"| `{name}` | {calls} | {ns / 1e6:.2f} | {ns / calls / 1e3:.2f} | {100 * ns / all_ns:.1f} |")
    shapes = {g[0]: (g[1], g[2]) for g in PREFILL_GEMMS}
    times: dict = {}
    previous = None
    for name, blocks, duration in rows:
        if "gemm_w8a8_mfma_kernel" not in name:
            continue
        if GATE_UP_TILE in name:
            label = "gate_up"
        elif blocks == 320:
            label = "qkv"
        elif blocks == 256 and previous in ("qkv", "gate_up"):
            label = "o" if previous == "qkv" else "down"
        else:
            previous = None
            continue
        times.setdefault(label, []).append(duration)
        previous = label
    lines += ["", "| Prefill GEMM (512 tokens) | N x K | Dispatches | Average us | int8 TOPS | of 5.0 POPS |",
              "|---|---|---:|---:|---:|---:|"]
    for label, (rows_n, K) in shapes.items():
        d = times.get(label)
        if not d:
            continue
        us = sum(d) / len(d) / 1e3
        tops = 2.0 * 512 * rows_n * K / us / 1e6
        lines.append(f"| {label} | {rows_n} x {K} | {len(d)} | {us:.2f} | {tops:.0f} | {tops / INT8_PEAK_TOPS:.3f} |")
    return "\n".join(lines)


def summarize_config_trace(db: Path) -> str:
    """Markdown tables from a rocprofv3 --kernel-trace run of the configuration
    benchmarks (graph replays traced as plain launches): for one decode step in
    the middle of each configuration's greedy run, every kernel's time per
    token, and the decode attention's read rate over the K and V rows of the
    visible keys.  A step is the kernels after one step's argmax launches up to
    and including the next step's; its configuration is told by the weight
    format of its fused GEMV."""
    import re
    import sqlite3
    from leaf_amd.models import PRESETS
    con = sqlite3.connect(str(db))
    rows = con.execute("select name, duration from kernels order by start").fetchall()
    con.close()
    clean = lambda n: re.sub(r"leafhip::|\(anonymous namespace\)::|void ", "", n).split("(")[0]   # noqa: E731
    meta, _ = golden()
    by_bits = {"<32,": "gpt2", "<4,": "qwen", "<16,": "smollm2"}
    # a step ends with its argmax launches (one, or the chunks and their combine)
    argmax = [i for i, r in enumerate(rows)
              if "argmax" in r[0] and (i + 1 == len(rows) or "argmax" not in rows[i + 1][0])]
    steps: dict = {}
    for a, b in zip(argmax, argmax[1:]):
        names = [clean(rows[i][0]) for i in range(a + 1, b + 1)]
        if any("gemm" in n for n in names) or len(names) < 8:
            continue                                 # a prefill, or not a decode step
        fused = next((n for n in names if n.startswith("gemv_fp_fused_kernel")), "")
        family = next((f for k, f in by_bits.items() if fused.startswith("gemv_fp_fused_kernel" + k)), None)
        if family:
            steps.setdefault(family, []).append((a, b))
    out = []
    for family in ("gpt2", "qwen", "smollm2"):
        if family not in steps:
            continue
        spec, m = PRESETS[family](), meta[family]
        idx = len(steps[family]) // 2
        a, b = steps[family][idx]
        ctx = m["prompt_tokens"] + idx + 1
        per: dict = {}
        for i in range(a + 1, b + 1):
            t = per.setdefault(clean(rows[i][0]), [0, 0.0])
            t[0] += 1
            t[1] += rows[i][1] / 1e3
        total = sum(t[1] for t in per.values())
        kv_bytes = 2 * spec.kv_heads * spec.head_dim * 4 * ctx   # one layer's K and V rows
        out += [f"**{family}** (decode step {idx + 1} of {len(steps[family])} traced, {ctx} keys): "
                f"{total:.1f} us of kernel time per token", "",
                "| Kernel | Calls per token | us per token | us per call |", "|---|---:|---:|---:|"]
        for name, (calls, us) in sorted(per.items(), key=lambda kv: -kv[1][1]):
            out.append(f"| `{name}` | {calls} | {us:.1f} | {us / calls:.2f} |")
        att = per.get("attention_decode_kernel")
        if att:
            gbps = kv_bytes * att[0] / (att[1] * 1e3)
            out += ["", f"Decode attention: {kv_bytes / 1e6:.2f} MB of K and V per layer, "
                    f"{att[1] / att[0]:.2f} us per call: {gbps:.0f} GB/s ({gbps / HBM_PEAK_GBS:.3f} of 8 TB/s)."]
        out.append("")
    return "\n".join(out)


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=120)
    parser.add_argument("--warmup", type=int, default=8)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-gemv", action="store_true")
    parser.add_argument("--no-linear", action="store_true")
    parser.add_argument("--no-configs", action="store_true")
    parser.add_argument("--no-peaks", action="store_true")
    parser.add_argument("--no-fast", action="store_true", help="skip the fast-numerics extra")
    parser.add_argument("--derive-traffic", type=Path, default=None)
    parser.add_argument("--derive-prefill-counters", type=Path, default=None)
    parser.add_argument("--derive-f32-gemm-counters", type=Path, default=None)
    parser.add_argument("--summarize-counters", type=Path, default=None)
    parser.add_argument("--summarize-trace", type=Path, default=None)
    parser.add_argument("--summarize-config-trace", type=Path, default=None)
    args = parser.parse_args()
    if args.summarize_trace is not None:
        print(summarize_trace(args.summarize_trace))
        return 0
    if args.summarize_config_trace is not None:
        print(summarize_config_trace(args.summarize_config_trace))
        return 0
    if args.derive_prefill_counters is not None:
        print(json.dumps(derive_prefill_counters(args.derive_prefill_counters), indent=1))
        return 0
    if args.summarize_counters is not None:
        print(summarize_counters(args.summarize_counters))
        return 0
    if args.derive_f32_gemm_counters is not None:
        print(json.dumps(derive_f32_gemm_counters(args.derive_f32_gemm_counters), indent=1))
        return 0
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
    log("decode benchmark (default numerics) ...")
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
    log("parity: the reference's 128-token greedy run ...")
    parity = parity_run(path)
    fast = None
    if not args.no_fast:
        log("fast numerics (reassociated sums, not bit-exact) ...")
        f = decode_benchmark(path, args.steps, args.warmup, numerics="fast", details=False)
        fast = {"label": "fast numerics: reassociated float sums, not bit-exact with the reference",
                "value": round(args.steps / f["elapsed_s"], 2), "unit": "tok/s", "step": f["step"],
                "parity": parity_run(path, "fast")}
    peaks = None
    if not args.no_peaks:
        log("measured peaks ...")
        peaks = measured_peaks()
    configs = None
    if not args.no_configs:
        configs = {}
        for family in ("gpt2", "qwen", "smollm2"):
            log(f"configuration {family} ...")
            configs[family] = config_benchmark(family)
    gemv = None
    if not args.no_gemv:
        log("GEMV microbenchmark ...")
        gemv = gemv_microbench()
        log("GEMV streaming rate ...")
        gemv["streaming_1GiB"] = gemv_streaming()
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
                               "decode", "numerics": "reference order (bit-exact)" if d["reference_order"] else "fast",
                   "decode_step": d["step"], "layers": 22, "hidden": 2048, "heads": 32, "kv_heads": 4, "ffn": 5632,
                   "vocab": 32000, "prompt_tokens": PROMPT_TOKENS, "context_end": d["context_end"],
                   "prefill_ms": round(d["prefill_ms"], 2),
                   "prefill_warm_p50_ms": round(d["prefill_warm_ms"], 3) if d["prefill_warm_ms"] else None,
                   "prefill_classes": d["prefill_classes"]},
        "roofline": {"bound": "hbm", "kernel": kernel,
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "avg_launch_us": round(avg_ms * 1e3, 3), "bytes_per_launch": round(bytes_per_launch),
                     "launches": g["launches"],
                     "measured_peak": peaks.get("hbm_read_GBps") if peaks else None,
                     "frac_of_measured": round(achieved / peaks["hbm_read_GBps"], 4)
                     if peaks and peaks.get("hbm_read_GBps") else None},
        "parity": parity,
        "fast_numerics": fast,
        "peaks": peaks,
        "configs": configs,
        "device_ms_per_step": device_ms,
        "gemv": gemv,
        "linear_w8a8": linear,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
