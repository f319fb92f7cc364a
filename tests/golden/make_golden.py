"""Write the golden vectors under tests/golden/ from the reference build.

Runs only where the reference checkout exists (it is compiled by
oracle/Makefile into oracle/_ref/: the real leaf_decoder binary and a harness
exposing its kernels).  The fixtures are data: inputs and the reference's
outputs.  Regenerate with

    make -C oracle && python tests/golden/make_golden.py          # kernels, reduced decoders
    make -C oracle && python tests/golden/make_golden.py --full   # configured sizes (minutes)
    make -C oracle && python tests/golden/make_golden.py --features   # artifact and operator features
"""
from __future__ import annotations

import dataclasses
import hashlib
import json
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from leaf_amd import models  # noqa: E402
from leaf_amd.artifact import quantize, round_to_bf16, write_artifact, write_tokens  # noqa: E402
from oracle.bindings import REF_BIN, Reference  # noqa: E402

OUT = Path(__file__).resolve().parent


def activations(rng, M, K):
    """N(0,1) activations with ~0.1% outliers x20 (the W8A8 microbench input)."""
    x = rng.standard_normal((M, K), dtype=np.float32)
    x[rng.random((M, K)) < 0.001] *= np.float32(20)
    return x


def kernel_vectors(ref: Reference) -> dict:
    rng = np.random.default_rng(20261201)
    out = {}
    # W8A8 at TinyLlama widths (K) with reduced output rows, M = 1, 4, 16,
    # plus odd tails and grouped scales.
    cases = [("k2048", 2048, 48, 2048, (1, 4, 16)), ("k5632", 5632, 16, 5632, (1, 4)),
             ("k2048n128", 2048, 128, 2048, (1,)), ("odd", 100, 7, 100, (1, 3, 5)),
             ("g64", 256, 9, 64, (1, 2, 5))]
    for tag, K, N, group, tokens in cases:
        w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        wq, ws = quantize(w, 8, group)
        bias = rng.standard_normal(N, dtype=np.float32) if tag == "odd" else None
        out[f"w8a8_{tag}_w"], out[f"w8a8_{tag}_s"] = wq, ws
        if bias is not None:
            out[f"w8a8_{tag}_b"] = bias
        for M in tokens:
            x = activations(rng, M, K)
            q16, qs = ref.quantize_rows(x)
            out[f"w8a8_{tag}_m{M}_x"] = x
            out[f"w8a8_{tag}_m{M}_q"] = q16.astype(np.int8)
            out[f"w8a8_{tag}_m{M}_qs"] = qs
            # mode 1: quant_tile_avx + quant_dot_avx (fused accumulate); mode 2: quant_dot_avx only
            out[f"w8a8_{tag}_m{M}_y"] = ref.linear_int(8, N, K, group, wq, ws, bias, x, mode=1 if M > 1 else 2)
            if group != K and M > 1 and ref.features & 2:
                out[f"w8a8_{tag}_m{M}_yvnni"] = ref.linear_int(8, N, K, group, wq, ws, bias, x, mode=0)
    # W4A8 grouped
    K, N = 256, 6
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    wq, ws = quantize(w, 4, 32)
    out["w4a8_w"], out["w4a8_s"] = wq, ws
    for M in (1, 3):
        x = activations(rng, M, K)
        out[f"w4a8_m{M}_x"] = x
        out[f"w4a8_m{M}_y"] = ref.linear_int(4, N, K, 32, wq, ws, None, x, mode=2)
    # FP paths: FP32, BF16, W8A32, W4A32 at M = 1..5 and odd widths
    for tag, K, N in (("k768", 768, 16), ("k896", 896, 8), ("odd", 77, 5)):
        w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
        bias = rng.standard_normal(N, dtype=np.float32) * np.float32(0.1)
        out[f"fp_{tag}_w"], out[f"fp_{tag}_b"] = w, bias
        wb = round_to_bf16(w)
        out[f"fp_{tag}_wbf16"] = wb
        forms = [(32, w, None, 0), (16, wb, None, 0), (8, *quantize(w, 8, K), K)]
        if K % 32 == 0:
            forms.append((4, *quantize(w, 4, 32), 32))
        for bits, data, scales, group in forms:
            if bits in (8, 4):
                out[f"fp_{tag}_w{bits}"], out[f"fp_{tag}_s{bits}"] = data, scales
            for M in (1, 2, 5):
                x = rng.standard_normal((M, K), dtype=np.float32)
                out[f"fp_{tag}_b{bits}_m{M}_x"] = x
                out[f"fp_{tag}_b{bits}_m{M}_y"] = ref.linear_fp(bits, N, K, group, data, scales, bias, x)
        x = rng.standard_normal((17, K), dtype=np.float32)
        out[f"acc_{tag}_x"] = x
        out[f"acc_{tag}_y32"] = ref.linear_accurate(32, N, K, w, bias, x)
        out[f"acc_{tag}_y16"] = ref.linear_accurate(16, N, K, wb, bias, x)
    # norms
    for tag, width in (("h2048", 2048), ("h768", 768)):
        x = rng.standard_normal((3, width), dtype=np.float32)
        g = (1 + np.float32(0.1) * rng.standard_normal(width, dtype=np.float32)).astype(np.float32)
        b = rng.standard_normal(width, dtype=np.float32) * np.float32(0.1)
        out[f"norm_{tag}_x"], out[f"norm_{tag}_g"], out[f"norm_{tag}_b"] = x, g, b
        out[f"norm_{tag}_rms"] = ref.norm(x, g, None, 1e-5, 0, False)
        out[f"norm_{tag}_rmsacc"] = ref.norm(x, g, None, 1e-5, 0, True)
        out[f"norm_{tag}_ln"] = ref.norm(x, g, b, 1e-5, 1, False)
    return out


# Reduced models of every family (same operator topology and storage policy as
# the full-size workloads), run through the reference binary.
DECODER_CASES = {
    "gpt2": dict(bias_std=0.05, norm_jitter=0.1),
    "tinyllama": dict(norm_jitter=0.1),
    "qwen": dict(bias_std=0.05),
    "smollm2": dict(),
}


def decoder_spec(family: str):
    return dataclasses.replace(models.PRESETS[family](reduced=True), **DECODER_CASES[family])


def artifact_digest(path: Path) -> str:
    return hashlib.sha256(path.read_bytes()).hexdigest()


def decoder_vectors(tmp: Path) -> tuple[dict, dict]:
    arrays, meta = {}, {}
    for family in DECODER_CASES:
        spec = decoder_spec(family)
        art = tmp / f"{family}.leaf"
        write_artifact(art, spec, seed=101)
        bits, math = models.RUN_POLICY[family]
        prompt = np.random.default_rng(5).integers(0, spec.vocab, 40).astype(np.uint32)
        req = tmp / "req.bin"
        write_tokens(req, [prompt.tolist()])
        logits = tmp / "out.logits"
        # verify in chunks of 13 (exercises the cache), all logits
        cmd = [str(REF_BIN), str(art), str(req), str(logits), str(tmp / "m.json"), "chunked", "1", "1", "0", "16",
               "0", "13", str(bits), f"--fp32-math={math}"]
        subprocess.run(cmd, check=True, capture_output=True)
        all_logits = np.fromfile(logits, np.float32).reshape(-1, spec.vocab)
        cmd = [str(REF_BIN), str(art), str(req), str(logits), str(tmp / "m.json"), "generate", "1", "1", "0", "10",
               "0", "1", str(bits), f"--fp32-math={math}"]
        run = subprocess.run(cmd, check=True, capture_output=True, text=True)
        tokens = [int(line.split()[1]) for line in run.stdout.splitlines() if line.startswith("TOKEN ")]
        arrays[f"{family}_prompt"] = prompt
        arrays[f"{family}_logits_rows"] = all_logits[[0, 12, 13, 26, 39]]
        arrays[f"{family}_tokens"] = np.array(tokens, np.uint32)
        meta[family] = {"artifact_sha256": artifact_digest(art), "activation_bits": bits, "fp32_math": math,
                        "seed": 101, "rows": [0, 12, 13, 26, 39], "chunk": 13,
                        "overrides": DECODER_CASES[family]}
    return arrays, meta


# Operator and storage features beyond the four families, each on a reduced
# model: name -> (preset, overrides, activation bits, FP32 math, prompt tokens,
# chunk, generated tokens).  The reference binary runs the prompt in chunks
# with all logits kept (verify/chunked mode), then the real Decoder's greedy
# loop; the fixture keeps five logit rows and the tokens.
STATIC_FREQUENCIES = tuple(float(np.float32(0.9 / (1 + 3 * i))) for i in range(16))   # in (0, 1]
FEATURE_CASES = {
    # SmoothQuant: calibrated .input_scale factors scale the columns before quantization
    "smoothquant": ("tinyllama", dict(norm_jitter=0.1, smoothquant_alpha=0.5), 8, "fast", 40, 13, 10),
    # INT8 with 64-column scale groups (int8_group_size)
    "int8_group64": ("tinyllama", dict(norm_jitter=0.1, int8_group_size=64), 8, "fast", 40, 13, 10),
    # LEAFDC05: BF16 embedding and head, FP32 elsewhere
    "bf16_io": ("tinyllama", dict(norm_jitter=0.1, bits=32, bf16_io=True, keep_fp32=frozenset()), 32, "fast",
                40, 13, 10),
    # LEAFDC07: per-head Q/K RMSNorm and static RoPE frequencies
    "qk_norm_static_rope": ("tinyllama", dict(norm_jitter=0.1, bits=32, keep_fp32=frozenset(), qk_norm=1,
                                              rope_frequencies=STATIC_FREQUENCIES), 32, "fast", 40, 13, 10),
    # LEAFDC04: several EOS ids, the generation stops on a non-primary one
    # (ids chosen by make_golden from a greedy run, stored in the metadata)
    "multi_eos": ("tinyllama", dict(norm_jitter=0.1), 8, "fast", 40, 13, 16),
    # exact-erf GELU (activation 1), ungated, LayerNorm with biases
    "gelu_erf": ("gpt2", dict(bias_std=0.05, norm_jitter=0.1, activation=1), 32, "fast", 40, 13, 10),
    # ReLU, ungated MLP
    "relu": ("tinyllama", dict(norm_jitter=0.1, bits=32, keep_fp32=frozenset(), activation=3, gated=0), 32,
             "fast", 40, 13, 10),
    # parallel residual, rotary on half of each head, LayerNorm with biases, QKV biases
    "parallel_partial_rotary": ("tinyllama", dict(norm_jitter=0.1, bits=32, keep_fp32=frozenset(),
                                                  parallel_residual=1, rotary_dim=16, norm=1, norm_bias=True,
                                                  attention_bias=True, bias_std=0.05), 32, "fast", 40, 13, 10),
    # learned positions read at an offset, scaled embeddings, ReLU
    "learned_offset_scaled": ("gpt2", dict(bias_std=0.05, norm_jitter=0.1, position_offset=2,
                                           embedding_scale=4.0, activation=3), 32, "fast", 40, 13, 10),
    # no position encoding and no final norm, W8A8
    "no_position_no_final_norm": ("tinyllama", dict(norm_jitter=0.1, position=2, final_norm=0), 8, "fast",
                                  40, 13, 10),
    # LEAFDC03 sliding window of 8 keys, W8A8
    "window8": ("tinyllama", dict(norm_jitter=0.1, sliding_window=8), 8, "fast", 40, 13, 10),
    # 8,300-token context (split-K decode attention beyond 8k keys), INT4 weights
    "long_context": ("qwen", dict(bias_std=0.05, max_positions=8320), 32, "fast", 8300, 1024, 8),
}


def feature_spec(name: str, eos_tokens=None):
    family, overrides, *_ = FEATURE_CASES[name]
    spec = dataclasses.replace(models.PRESETS[family](reduced=True), **overrides)
    if eos_tokens:
        spec = dataclasses.replace(spec, eos=int(eos_tokens[0]), eos_tokens=tuple(int(t) for t in eos_tokens))
    return spec


def feature_rows(prompt_tokens: int, chunk: int) -> list[int]:
    rows = {0, chunk - 1, min(chunk, prompt_tokens - 1), prompt_tokens - 2, prompt_tokens - 1}
    if prompt_tokens > 4352:
        rows |= {4351, 4352, 8191, 8192} & set(range(prompt_tokens))
    return sorted(rows)


def feature_vectors(tmp: Path, ref: Reference, names) -> tuple[dict, dict]:
    arrays, meta = {}, {}
    for name in names:
        family, overrides, bits, math, length, chunk, limit = FEATURE_CASES[name]
        eos = None
        if name == "multi_eos":
            # greedy tokens without EOS, then a stop id that first appears at
            # position >= 3 as the second of three EOS ids
            art = tmp / "probe.leaf"
            write_artifact(art, feature_spec(name), seed=101)
            prompt = np.random.default_rng(7).integers(0, feature_spec(name).vocab, length).astype(np.uint32)
            free, _ = ref.greedy(art, prompt, limit, activation_bits=bits, vocab=feature_spec(name).vocab)
            free = free.tolist()
            stop_at = next(i for i in range(3, len(free)) if free[i] not in free[:i])
            unused = [t for t in range(1, 1000) if t not in free][:2]
            eos = [unused[0], free[stop_at], unused[1]]
        spec = feature_spec(name, eos)
        art = tmp / f"{name}.leaf"
        write_artifact(art, spec, seed=101)
        prompt = np.random.default_rng(7).integers(0, spec.vocab, length).astype(np.uint32)
        req, logits = tmp / "req.bin", tmp / "out.logits"
        write_tokens(req, [prompt.tolist()])
        cmd = [str(REF_BIN), str(art), str(req), str(logits), str(tmp / "m.json"), "chunked", "8", "1", "0", "16",
               "0", str(chunk), str(bits), f"--fp32-math={math}"]
        subprocess.run(cmd, check=True, capture_output=True)
        rows = feature_rows(length, chunk)
        all_logits = np.memmap(logits, np.float32, mode="r").reshape(-1, spec.vocab)
        arrays[f"{name}_logits_rows"] = np.array(all_logits[rows])
        del all_logits
        tokens, _ = ref.greedy(art, prompt, limit, activation_bits=bits, accurate=math == "accurate",
                               vocab=spec.vocab)
        if name == "multi_eos":
            assert len(tokens) == stop_at + 1 and int(tokens[-1]) == eos[1], (tokens, eos)
        arrays[f"{name}_prompt"] = prompt
        arrays[f"{name}_tokens"] = np.asarray(tokens, np.uint32)
        meta[name] = {"artifact_sha256": artifact_digest(art), "activation_bits": bits, "fp32_math": math,
                      "seed": 101, "prompt_seed": 7, "rows": rows, "chunk": chunk, "generate": limit,
                      "eos_tokens": eos, "version": int(art.read_bytes()[7]) - ord("0")}
        print(f"{name}: LEAFDC0{meta[name]['version']}, {len(tokens)} tokens", flush=True)
        art.unlink()
    return arrays, meta


# The benchmark configurations at their configured sizes: (prompt tokens,
# greedy tokens, prompt seed).  Artifacts: models.PRESETS[family]() written
# with FULL_ARTIFACT_SEED.  The real reference Decoder runs the greedy loop;
# the fixture keeps the tokens, and the logits of the prefill (forward 0) and
# of the last single-token forward.
FULL_ARTIFACT_SEED = 20261202
FULL_CASES = {
    "gpt2": (16, 32, 1),
    "tinyllama": (512, 128, 3),
    "qwen": (4096, 256, 4),
    "smollm2": (2048, 256, 5),
}


def full_prompt(family: str) -> np.ndarray:
    length, _, seed = FULL_CASES[family]
    vocab = models.PRESETS[family]().vocab
    return np.random.default_rng(seed).integers(0, vocab, length).astype(np.uint32)


def full_config_vectors(tmp: Path, ref: Reference, families) -> tuple[dict, dict]:
    arrays, meta = {}, {}
    for family in families:
        spec = models.PRESETS[family]()
        art = tmp / f"{family}_full.leaf"
        write_artifact(art, spec, seed=FULL_ARTIFACT_SEED)
        bits, math = models.RUN_POLICY[family]
        length, limit, seed = FULL_CASES[family]
        prompt = full_prompt(family)
        tokens, logits = ref.greedy(art, prompt, limit, activation_bits=bits, accurate=math == "accurate",
                                    keep=(0, limit - 1), vocab=spec.vocab)
        arrays[f"{family}_tokens"] = tokens
        arrays[f"{family}_prefill_logits"] = logits[0]
        arrays[f"{family}_last_logits"] = logits[1]
        meta[family] = {"artifact_sha256": artifact_digest(art), "artifact_seed": FULL_ARTIFACT_SEED,
                        "activation_bits": bits, "fp32_math": math, "prompt_tokens": length,
                        "prompt_seed": seed, "generate": limit, "last_forward": limit - 1}
        print(f"{family}: {len(tokens)} tokens from the reference", flush=True)
        art.unlink()
    return arrays, meta


def main() -> None:
    subprocess.run(["make", "-C", str(ROOT / "oracle"), "-s"], check=True)
    ref = Reference()
    if "--full" in sys.argv:
        # the configured sizes only (minutes: the reference's attention is scalar)
        with tempfile.TemporaryDirectory() as tmp:
            arrays, meta = full_config_vectors(Path(tmp), ref, FULL_CASES)
        np.savez_compressed(OUT / "full_configs.npz", **arrays)
        meta["reference_cpu_features"] = ref.features
        (OUT / "full_configs.json").write_text(json.dumps(meta, indent=2, sort_keys=True) + "\n")
        print("full_configs.npz", (OUT / "full_configs.npz").stat().st_size, "bytes")
        return
    if "--features" in sys.argv:
        with tempfile.TemporaryDirectory() as tmp:
            arrays, meta = feature_vectors(Path(tmp), ref, FEATURE_CASES)
        np.savez_compressed(OUT / "features.npz", **arrays)
        meta["reference_cpu_features"] = ref.features
        (OUT / "features.json").write_text(json.dumps(meta, indent=2, sort_keys=True) + "\n")
        print("features.npz", (OUT / "features.npz").stat().st_size, "bytes")
        return
    kernels = kernel_vectors(ref)
    np.savez_compressed(OUT / "kernels.npz", **kernels)
    with tempfile.TemporaryDirectory() as tmp:
        arrays, meta = decoder_vectors(Path(tmp))
    np.savez_compressed(OUT / "decoders.npz", **arrays)
    meta["reference_cpu_features"] = ref.features
    (OUT / "decoders.json").write_text(json.dumps(meta, indent=2, sort_keys=True) + "\n")
    for f in ("kernels.npz", "decoders.npz"):
        print(f, (OUT / f).stat().st_size, "bytes")


if __name__ == "__main__":
    main()
