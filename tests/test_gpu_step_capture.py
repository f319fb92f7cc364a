"""The persistent decode step's integer stages, bit for bit against the oracle.

The benchmarked kernel (decode_step_kernel) normalizes, quantizes and takes
its int8 dots itself, with its own reductions.  Its capture variant
(LEAF_DECODE_STEP_CAPTURE) records, for every layer and each of the four
integer linears of one decode step of the full-width TinyLlama W8A8 artifact
(22 x 2048, 32/4 heads, SwiGLU 5632):
  * the f32 vector the phase quantizes -- its own normalized layer input, the
    attention output, its normalized mid vector, the gated activation;
  * the int8 vector and the per-token scale it computed from it;
  * the exact int32 dot of every output row.
The quantization of the step's own vector must equal oracle.quantize_rows
(decoder.cpp:1020-1044, quantize_input_avx :618-627) and every row's int32
dot must equal oracle.int_accumulators (quant_dot_avx, :536-570) on the
artifact's int8 rows.  The f32 vectors themselves come from the step's
parallel reductions and are checked against the oracle only within the
decode-step tolerances elsewhere (tests/test_gpu_decode_step.py).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def read_capture(path):
    raw = np.fromfile(path, np.uint8)
    head = raw[:12].view(np.uint32)
    assert head[0] == 0x4353484C, "not a step capture"
    layers, width = int(head[1]), int(head[2])
    vec = layers * 4 * width
    at = 12
    x = raw[at:at + 4 * vec].view(np.float32).reshape(layers, 4, width)
    at += 4 * vec
    q = raw[at:at + vec].view(np.int8).reshape(layers, 4, width)
    at += vec
    sx = raw[at:at + 16 * layers].view(np.float32).reshape(layers, 4)
    at += 16 * layers
    acc = raw[at:at + 8 * vec].view(np.int32).reshape(layers, 4, 2 * width)
    at += 8 * vec
    return x, q, sx, acc, at


@pytest.mark.parametrize("numerics", ["fast", "reference"])
def test_decode_step_quantization_and_int32_dots_equal_the_oracle(full_artifacts, oracle, tmp_path, monkeypatch,
                                                                   numerics):
    from leaf_amd import models, runtime
    from leaf_amd.artifact import load_tensor
    path = full_artifacts("tinyllama")
    capture = tmp_path / "step.cap"
    monkeypatch.setenv("LEAF_DECODE_STEP_CAPTURE", str(capture))
    dec = runtime.Decoder(path, 8, numerics=numerics)
    prompt = np.random.default_rng(17).integers(0, dec.vocabulary_size, 40).astype(np.uint32)
    token = dec.forward_into(prompt, None)
    dec.set_profiling(True)
    dec.forward([token])
    steps = dec.profile().get("decode_step", {}).get("launches", 0)
    dec.close()
    # one launch, or two when its XCD placement check failed and the host ran
    # the step again on the memory path (the aborted launch records nothing)
    assert steps in (1, 2), "the persistent decode step did not run"
    x, q, sx, acc, size = read_capture(capture)
    assert size == capture.stat().st_size, "one step recorded"
    spec = models.PRESETS["tinyllama"]()
    H, F = spec.hidden, spec.intermediate
    qw = spec.heads * spec.head_dim
    assert x.shape[0] == spec.layers
    checked = 0
    for L in range(spec.layers):
        layer = f"model.layers.{L}."
        mats = [[layer + f"self_attn.{n}_proj.weight" for n in "qkv"], [layer + "self_attn.o_proj.weight"],
                [layer + "mlp.gate_proj.weight", layer + "mlp.up_proj.weight"], [layer + "mlp.down_proj.weight"]]
        for phase, (K, names) in enumerate(zip((H, qw, H, F), mats)):
            xv, qv, s = x[L, phase, :K], q[L, phase, :K], sx[L, phase]
            assert np.isfinite(xv).all() and np.abs(xv).max() > 0, (L, phase)
            oq, os_ = oracle.quantize_rows(xv[None])
            assert np.array_equal(oq[0], qv), f"layer {L} phase {phase}: int8 activations differ"
            assert os_.view(np.uint32)[0] == np.float32(s).view(np.uint32), f"layer {L} phase {phase}: scale differs"
            weights = np.concatenate([load_tensor(path, n)[0] for n in names])
            rows = weights.shape[0]
            want = oracle.int_accumulators(8, rows, K, K, weights, qv[None]).ravel()
            got = acc[L, phase, :rows]
            bad = np.flatnonzero(got != want)
            assert bad.size == 0, f"layer {L} phase {phase}: {bad.size} int32 dots differ, first row {bad[:1]}"
            checked += rows
    print(f"decode step: {spec.layers} layers x 4 phases, {checked} int32 row dots and their int8 inputs bit-exact")
