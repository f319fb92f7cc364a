"""Artifact and operator features on the GPU against the reference's golden outputs.

Reduced models (tests/golden/make_golden.py FEATURE_CASES) for what the four
benchmark families do not exercise: SmoothQuant `.input_scale` linears,
grouped INT8 scales, LEAFDC05 BF16 embedding/head, LEAFDC07 Q/K RMSNorm with
static RoPE frequencies, LEAFDC04 multi-EOS stop, exact-erf GELU, ReLU,
parallel residual with partial rotary, learned positions at an offset with a
scaled embedding, no positions and no final norm, a LEAFDC03 sliding window,
and an 8,300-token context (decode attention over more than 8k keys).

Fast numerics: the golden logit rows within the tolerance of the family tests
(1e-3 of max |logit|; 2e-2 for W8A8), every generated token identical for
FP activations.  W8A8 in fast numerics can flip a near tie (one int8 bin moves
the logits by up to the band), so there the reference's tokens are fed back
one at a time and each step's argmax must be the reference's token or trail
it by no more than the band.
Reference numerics: the logit rows and tokens equal the reference's bit for
bit; the GELU cases are left out there, the device's erff / tanhf differing
from glibc's in the last bits.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FEATURES = ["smoothquant", "int8_group64", "bf16_io", "qk_norm_static_rope", "multi_eos", "gelu_erf", "relu",
            "parallel_partial_rotary", "learned_offset_scaled", "no_position_no_final_norm", "window8",
            "long_context"]
GELU = {"gelu_erf"}
LOGIT_TOLERANCE = 1e-3
W8A8_LOGIT_TOLERANCE = 2e-2


def rel_error(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def bits_equal(a, b):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module")
def runtime():
    from leaf_amd import runtime
    runtime.library()
    return runtime


def chunked_rows(dec, prompt, chunk, rows):
    """Forward the prompt in chunks with all logits; keep the listed rows."""
    out = []
    for pos in range(0, len(prompt), chunk):
        logits = dec.forward(prompt[pos:pos + chunk], all_logits=True)
        out += [logits[r - pos] for r in rows if pos <= r < pos + len(logits)]
    assert dec.cache_tokens() == len(prompt)
    return np.stack(out)


def reference_mode(meta):
    # the golden outputs come from a host with AVX-VNNI when bit 1 is set
    return "reference-vnni" if meta["reference_cpu_features"] & 2 else "reference-avx2"


@pytest.mark.parametrize("name", FEATURES)
def test_fast_numerics_match_the_reference_golden(runtime, golden_features, feature_artifacts, name):
    arrays, meta = golden_features
    m = meta[name]
    prompt = arrays[f"{name}_prompt"]
    print(f"{name}: LEAFDC0{m['version']}, {len(prompt)} prompt tokens", flush=True)
    dec = runtime.Decoder(feature_artifacts(name), m["activation_bits"], m["fp32_math"], numerics="fast")
    if m["eos_tokens"]:
        assert all(dec.is_eos_token(t) for t in m["eos_tokens"])
    rows = chunked_rows(dec, prompt, m["chunk"], m["rows"])
    err = rel_error(rows, arrays[f"{name}_logits_rows"])
    print(f"{name}: logit rows relative error {err:.2e}")
    assert err <= (W8A8_LOGIT_TOLERANCE if m["activation_bits"] == 8 else LOGIT_TOLERANCE)
    dec.reset()
    want = arrays[f"{name}_tokens"].tolist()
    if m["activation_bits"] != 8:
        tokens, _, _ = dec.generate(prompt, m["generate"])
        assert tokens == want
    else:
        logits = dec.forward(prompt)
        for step, token in enumerate(want):
            best = int(np.argmax(logits))
            gap = float(logits[best] - logits[token])
            assert best == token or gap <= W8A8_LOGIT_TOLERANCE * float(np.max(np.abs(logits))), (step, best, token)
            if step + 1 < len(want):
                logits = dec.forward([token])
    dec.close()


@pytest.mark.parametrize("name", [n for n in FEATURES if n not in GELU])
def test_reference_numerics_equal_the_reference_golden(runtime, golden_features, feature_artifacts, name):
    arrays, meta = golden_features
    m = meta[name]
    prompt = arrays[f"{name}_prompt"]
    print(f"{name}: reference numerics, {len(prompt)} prompt tokens", flush=True)
    dec = runtime.Decoder(feature_artifacts(name), m["activation_bits"], m["fp32_math"],
                          numerics=reference_mode(meta))
    rows = chunked_rows(dec, prompt, m["chunk"], m["rows"])
    want = arrays[f"{name}_logits_rows"]
    if not bits_equal(rows, want):
        diff = np.flatnonzero(rows.view(np.uint32).ravel() != want.view(np.uint32).ravel())
        pytest.fail(f"{diff.size} logits differ, first at {divmod(int(diff[0]), want.shape[1])}, "
                    f"relative error {rel_error(rows, want):.2e}")
    dec.reset()
    tokens, _, _ = dec.generate(prompt, m["generate"])
    assert tokens == arrays[f"{name}_tokens"].tolist()
    dec.close()

