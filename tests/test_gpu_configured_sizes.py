"""Every benchmark configuration at the size it names, against the real reference.

tests/golden/full_configs.npz holds, for each configuration, the greedy run of
the real reference Decoder (built from its sources; generate_continuation,
engine/src/main_decoder.cpp:95-113) on the seeded synthetic artifact: the
tokens, the logits of the prefill and the logits of the last single-token
forward.  The GPU writes the same artifact (its SHA-256 is checked) and runs
the same greedy loop.

* TinyLlama-1.1B W8A8, 512-token prompt, 128 greedy tokens; Qwen2.5-0.5B INT4
  (W4A32), 4096-token prompt, 256 tokens: with reference-order numerics the
  prefill and last logits equal the reference's bit for bit and all tokens
  are identical; TinyLlama's 127 decode tokens each run as one launch of the
  persistent decode step.
* GPT-2 small FP32, 16 + 32; Qwen INT4 4096 + 256; SmolLM2-360M BF16 with the
  accurate FP32 policy, 2048 + 256: with the fast kernels, logits within 1e-3
  of the largest |logit| and identical tokens.
* TinyLlama W8A8 with the fast kernels: not bit-exact by design (parallel
  norm and softmax sums move int8 bins); the prefill logits must stay within
  the W8A8 band, and the token agreement is reported.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from leaf_amd import models

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
LOGIT_TOLERANCE = 1e-3      # FP32 / BF16 / weight-only INT4: max-abs error / max |logit|
# W8A8 with the fast kernels: max-abs error and relative RMSE of the prefill
# logits.  At 22 layers the int8 bins a one-ulp change can move compound: the
# oracle itself, with only its RMSNorm square sum taken pairwise instead of
# sequentially, moves these logits by 6-9% of the largest |logit|
# (tests/test_oracle_golden.py measures the same effect on reduced models).
W8A8_FAST_BAND = 1e-1


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN / "full_configs.npz", allow_pickle=False) as data:
        arrays = {k: data[k] for k in data.files}
    return arrays, json.loads((GOLDEN / "full_configs.json").read_text())


@pytest.fixture(scope="module")
def rt():
    from leaf_amd import runtime
    runtime.library()
    return runtime


def rel_error(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def rel_rmse(a, b):
    return float(np.sqrt(np.mean((a - b) ** 2)) / max(np.sqrt(np.mean(b ** 2)), 1e-12))


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32),
                          np.ascontiguousarray(b, np.float32).view(np.uint32))


def prompt_of(family, meta):
    spec = models.PRESETS[family]()
    rng = np.random.default_rng(meta["prompt_seed"])
    return rng.integers(0, spec.vocab, meta["prompt_tokens"]).astype(np.uint32)


def artifact(full_artifacts, family, meta):
    path = full_artifacts(family)
    digest = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 24), b""):
            digest.update(block)
    assert digest.hexdigest() == meta["artifact_sha256"], "the seeded writer no longer reproduces the artifact"
    return path


def greedy(dec, prompt, limit, profile=False):
    """generate_continuation on the GPU: (tokens, prefill logits, last logits,
    decode launches per profiler class when `profile`; profiling keeps graph
    replays off, so the graph-replayed paths run unprofiled)."""
    logits = dec.forward(prompt)
    first = logits
    tokens = []
    dec.set_profiling(profile)
    for i in range(limit):
        tokens.append(int(np.argmax(logits)))   # the first maximum, as std::max_element
        if i + 1 < limit:
            logits = dec.forward([tokens[-1]])
    launches = {k: v["launches"] for k, v in dec.profile().items()}
    return tokens, first, logits, launches


def run(rt, path, meta, prompt, numerics, profile=False):
    dec = rt.Decoder(path, meta["activation_bits"], meta["fp32_math"], numerics=numerics,
                     max_context=len(prompt) + meta["generate"] + 8, max_prefill=len(prompt))
    try:
        return greedy(dec, prompt, meta["generate"], profile)
    finally:
        dec.close()


@pytest.mark.parametrize("family", ["tinyllama", "qwen"])
def test_reference_numerics_equal_the_reference_at_the_configured_size(rt, golden, full_artifacts, family):
    arrays, meta = golden
    m = meta[family]
    prompt = prompt_of(family, m)
    tokens, first, last, launches = run(rt, artifact(full_artifacts, family, m), m, prompt, "reference",
                                        profile=family == "tinyllama")
    want = arrays[f"{family}_tokens"].tolist()
    diverged = next((i for i, (a, b) in enumerate(zip(tokens, want)) if a != b), None)
    print(f"{family} {len(prompt)}+{m['generate']} reference numerics: prefill logits bit-equal "
          f"{bits_equal(first, arrays[f'{family}_prefill_logits'])}, first token difference at {diverged}, "
          f"decode launches {launches}")
    assert bits_equal(first, arrays[f"{family}_prefill_logits"]), "prefill logits differ from the reference"
    assert tokens == want, f"greedy tokens differ from step {diverged}"
    assert bits_equal(last, arrays[f"{family}_last_logits"]), "last-step logits differ from the reference"
    if family == "tinyllama":
        # every decode token ran on the persistent step (a step whose XCD
        # placement check failed runs once more on the memory path)
        steps = m["generate"] - 1
        assert steps <= launches.get("decode_step", 0) <= steps + 4, launches


@pytest.mark.parametrize("family", ["gpt2", "qwen", "smollm2"])
def test_fast_numerics_match_the_reference_at_the_configured_size(rt, golden, full_artifacts, family):
    arrays, meta = golden
    m = meta[family]
    prompt = prompt_of(family, m)
    tokens, first, last, _ = run(rt, artifact(full_artifacts, family, m), m, prompt, "fast")
    e_first = rel_error(first, arrays[f"{family}_prefill_logits"])
    e_last = rel_error(last, arrays[f"{family}_last_logits"])
    want = arrays[f"{family}_tokens"].tolist()
    diverged = next((i for i, (a, b) in enumerate(zip(tokens, want)) if a != b), None)
    print(f"{family} {len(prompt)}+{m['generate']} fast numerics: prefill error {e_first:.2e}, last-step error "
          f"{e_last:.2e}, first token difference at {diverged}")
    assert e_first <= LOGIT_TOLERANCE and e_last <= LOGIT_TOLERANCE
    assert tokens == want, f"greedy tokens differ from step {diverged}"


def test_tinyllama_fast_numerics_stay_within_the_w8a8_band(rt, golden, full_artifacts):
    arrays, meta = golden
    m = meta["tinyllama"]
    prompt = prompt_of("tinyllama", m)
    tokens, first, _, _ = run(rt, artifact(full_artifacts, "tinyllama", m), m, prompt, "fast")
    ref = arrays["tinyllama_prefill_logits"]
    want = arrays["tinyllama_tokens"].tolist()
    same = next((i for i, (a, b) in enumerate(zip(tokens, want)) if a != b), len(want))
    e, r = rel_error(first, ref), rel_rmse(first, ref)
    print(f"tinyllama 512+128 fast numerics: prefill error {e:.2e} (RMSE {r:.2e}); "
          f"tokens identical to the reference for the first {same} of {len(want)}")
    assert e <= W8A8_FAST_BAND and r <= W8A8_FAST_BAND
