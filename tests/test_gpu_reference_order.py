"""Reference-order numerics on the GPU, bit for bit against the oracle and the
reference's own outputs.

With LH_NUMERICS_REFERENCE the kernels sum in the CPU path's orders and use
glibc's expf, so every float must be bit-identical: outputs are compared as
uint32 views, no tolerance.  Covered: glibc's expf over a sample of all 2^32
inputs, RMSNorm / accurate RMSNorm / LayerNorm, GQA attention (decode, prefill,
chunks after cached keys, sliding windows), SiLU and ReLU, the dot_avx-order FP
linears (FP32, BF16, W8A32, W4A32 in token groups of four, with column tails),
and whole decoders (reduced W8A8, INT4 and BF16 models against the
reference's golden logits and tokens, plus prompts that trigger the CPU's
final-layer trim).
"""
from __future__ import annotations

import numpy as np
import pytest

from leaf_amd.artifact import quantize, round_to_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from leaf_amd import runtime
    runtime.library()
    runtime.set_kernel_numerics("reference")
    yield runtime
    runtime.set_kernel_numerics("fast")


def bits_equal(a, b):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def first_difference(a, b):
    d = np.flatnonzero(np.ascontiguousarray(a, np.float32).view(np.uint32).ravel()
                       != np.ascontiguousarray(b, np.float32).view(np.uint32).ravel())
    return None if d.size == 0 else (int(d[0]), int(d.size))


def test_expf_equals_glibc_on_a_sample_of_all_floats(rt, oracle):
    # every 251st bit pattern (17.1M inputs of every sign and exponent), plus a
    # dense random sample of the softmax range [-104, 0] and the specials
    patterns = np.arange(0, 1 << 32, 251, dtype=np.uint64).astype(np.uint32)
    rng = np.random.default_rng(31)
    dense = (-104.0 * rng.random(4_000_000)).astype(np.float32)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.72283, 88.72284, -103.97208, -103.97209,
                         32.564632, -63.09946], np.float32)
    x = np.concatenate([patterns.view(np.float32), dense, specials])
    dx, dy = rt.DeviceArray.of(x), rt.DeviceArray(x.shape, np.float32)
    rt.expf(dx, dy)
    got, want = dy.numpy(), oracle.expf(x)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert bits_equal(got[~nan], want[~nan]), first_difference(got[~nan], want[~nan])


@pytest.mark.parametrize("width", [2048, 5632, 960, 896, 64, 7, 100])
def test_norms_bit_exact(rt, oracle, width):
    from leaf_amd.runtime import check, library
    rng = np.random.default_rng(width)
    x = (3 * rng.standard_normal((5, width))).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(width)).astype(np.float32)
    b = (0.1 * rng.standard_normal(width)).astype(np.float32)
    dx, dg, db = rt.DeviceArray.of(x), rt.DeviceArray.of(g), rt.DeviceArray.of(b)
    dy = rt.DeviceArray((5, width), np.float32)
    for accurate in (0, 1):
        check(library().lh_rmsnorm(dx.ptr, 5, width, dg.ptr, np.float32(1e-5), accurate, dy.ptr, None))
        want = oracle.norm(x, g, None, 1e-5, 0, bool(accurate))
        assert bits_equal(dy.numpy(), want), (accurate, first_difference(dy.numpy(), want))
    check(library().lh_layernorm(dx.ptr, 5, width, dg.ptr, db.ptr, np.float32(1e-5), dy.ptr, None))
    want = oracle.norm(x, g, b, 1e-5, 1, False)
    assert bits_equal(dy.numpy(), want), first_difference(dy.numpy(), want)


@pytest.mark.parametrize("tokens,position,window,heads,kv", [
    (1, 640, 0, 32, 4), (1, 4351, 0, 14, 2), (1, 700, 64, 14, 2), (1, 0, 0, 14, 2), (1, 300, 0, 32, 4),
    (1, 9000, 0, 8, 1), (37, 0, 0, 14, 2), (13, 21, 0, 15, 5),
    (16, 5, 7, 14, 2), (512, 0, 0, 32, 4), (200, 300, 0, 32, 4), (130, 100, 64, 14, 2)])
def test_attention_bit_exact(rt, oracle, tokens, position, window, heads, kv):
    from leaf_amd.runtime import check, library
    rng = np.random.default_rng(tokens * 100 + position)
    dim = 64
    total = position + tokens
    cap = total + 70
    q = (2 * rng.standard_normal((heads, tokens, dim))).astype(np.float32)
    keys = (2 * rng.standard_normal((kv, cap, dim))).astype(np.float32)
    values = rng.standard_normal((kv, cap, dim), dtype=np.float32)
    keys[:, total:] = np.nan           # never-written cache rows must not leak
    values[:, total:] = np.nan
    dq, dk, dv = rt.DeviceArray.of(q), rt.DeviceArray.of(keys), rt.DeviceArray.of(values)
    out = rt.DeviceArray((tokens, heads * dim), np.float32)
    check(library().lh_attention(dq.ptr, dk.ptr, dv.ptr, cap, heads, kv, dim, tokens, position, window, out.ptr,
                                 None))
    mask = np.zeros((tokens, total), np.float32)
    for t in range(tokens):
        end = position + t + 1
        begin = end - window if window and end > window else 0
        mask[t, begin:end] = 1
    scale = np.float32(1) / np.sqrt(np.sqrt(np.float32(dim)))
    want = oracle.attention(q, keys, values, mask, heads, kv, tokens, total, cap, dim, float(scale))
    assert bits_equal(out.numpy(), want), first_difference(out.numpy(), want)


def test_activations_bit_exact(rt, oracle):
    from leaf_amd.runtime import check, library
    rng = np.random.default_rng(5)
    tokens, width = 3, 5632
    gate_up = (4 * rng.standard_normal((tokens, 2 * width))).astype(np.float32)
    gate_up[0, :200] = np.linspace(-110, 95, 200, dtype=np.float32)    # exp under- and overflow
    d_in, d_out = rt.DeviceArray.of(gate_up), rt.DeviceArray((tokens, width), np.float32)
    check(library().lh_silu_gate(d_in.ptr, tokens, width, d_out.ptr, None))
    want = oracle.activation(gate_up, tokens, width, True, 0)
    assert bits_equal(d_out.numpy(), want), first_difference(d_out.numpy(), want)
    x = gate_up.ravel()[:20000].copy()
    x[:4] = [0.0, -0.0, -1e-30, 3.0]
    dx, dy = rt.DeviceArray.of(x), rt.DeviceArray(x.shape, np.float32)
    check(library().lh_activation(dx.ptr, x.size, 3, dy.ptr, None))           # ReLU, std::max(x, 0.0f)
    assert bits_equal(dy.numpy(), oracle.activation(x, 1, x.size, False, 3).ravel())


@pytest.mark.parametrize("K,N", [(2048, 40), (896, 24), (100, 9), (36, 5), (960, 17)])
def test_fp_linears_bit_exact(rt, oracle, K, N):
    rng = np.random.default_rng(K + N)
    w = (0.02 * rng.standard_normal((N, K))).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    forms = [(32, w, None, 0), (16, round_to_bf16(w), None, 0), (8, *quantize(w, 8, K), K)]
    if K % 32 == 0:
        forms.append((4, *quantize(w, 4, 32), 32))
    if K % 64 == 0:
        forms.append((8, *quantize(w, 8, 64), 64))
    for bits, data, scales, group in forms:
        dw = rt.DeviceWeight(data, bits, K, scales, group, bias)
        for M in (1, 2, 3, 4, 5, 6, 9, 65, 66, 67, 68, 133):
            x = rng.standard_normal((M, K), dtype=np.float32)
            dx, dy = rt.DeviceArray.of(x), rt.DeviceArray((M, N), np.float32)
            rt.linear(dw, dx, M, 32, dy)
            want = oracle.linear_fp(bits, N, K, group, data, scales, bias, x)
            assert bits_equal(dy.numpy(), want), (bits, group, M, first_difference(dy.numpy(), want))


def test_fp_linears_match_the_reference_golden_vectors(rt, golden_kernels):
    g = golden_kernels
    for tag, K, N in (("k768", 768, 16), ("k896", 896, 8), ("odd", 77, 5)):
        w, bias = g[f"fp_{tag}_w"], g[f"fp_{tag}_b"]
        forms = [(32, w, None, 0), (16, g[f"fp_{tag}_wbf16"], None, 0), (8, g[f"fp_{tag}_w8"], g[f"fp_{tag}_s8"], K)]
        if K % 32 == 0:
            forms.append((4, g[f"fp_{tag}_w4"], g[f"fp_{tag}_s4"], 32))
        for bits, data, scales, group in forms:
            dw = rt.DeviceWeight(data, bits, K, scales, group, bias)
            for M in (1, 2, 5):
                x = g[f"fp_{tag}_b{bits}_m{M}_x"]
                dx, dy = rt.DeviceArray.of(x), rt.DeviceArray((M, N), np.float32)
                rt.linear(dw, dx, M, 32, dy)
                assert bits_equal(dy.numpy(), g[f"fp_{tag}_b{bits}_m{M}_y"]), (tag, bits, M)


def test_norms_match_the_reference_golden_vectors(rt, golden_kernels):
    from leaf_amd.runtime import check, library
    g = golden_kernels
    for tag, width in (("h2048", 2048), ("h768", 768)):
        x, gamma, beta = g[f"norm_{tag}_x"], g[f"norm_{tag}_g"], g[f"norm_{tag}_b"]
        dx, dg, db = rt.DeviceArray.of(x), rt.DeviceArray.of(gamma), rt.DeviceArray.of(beta)
        dy = rt.DeviceArray(x.shape, np.float32)
        check(library().lh_rmsnorm(dx.ptr, x.shape[0], width, dg.ptr, np.float32(1e-5), 0, dy.ptr, None))
        assert bits_equal(dy.numpy(), g[f"norm_{tag}_rms"])
        check(library().lh_rmsnorm(dx.ptr, x.shape[0], width, dg.ptr, np.float32(1e-5), 1, dy.ptr, None))
        assert bits_equal(dy.numpy(), g[f"norm_{tag}_rmsacc"])
        check(library().lh_layernorm(dx.ptr, x.shape[0], width, dg.ptr, db.ptr, np.float32(1e-5), dy.ptr, None))
        assert bits_equal(dy.numpy(), g[f"norm_{tag}_ln"])


# ------------------------------------------------------------ whole decoders
# Families whose arithmetic reference order reproduces exactly: SiLU
# activations and the fast FP32 policy (GPT-2's GELU uses the device's tanhf;
# SmolLM2's accurate policy is rejected, so it runs here with fast FP32 math).
EXACT = {"tinyllama": (8, "fast"), "qwen": (32, "fast"), "smollm2": (32, "fast")}


@pytest.mark.parametrize("family", ["tinyllama", "qwen"])
def test_decoder_logits_and_tokens_equal_the_reference_golden(rt, golden_decoders, artifacts, family):
    arrays, meta = golden_decoders
    m = meta[family]
    assert (m["activation_bits"], m["fp32_math"]) == EXACT[family]
    prompt = arrays[f"{family}_prompt"]
    dec = rt.Decoder(artifacts[family], m["activation_bits"], m["fp32_math"], numerics="reference")
    logits = np.concatenate([dec.forward(prompt[p:p + m["chunk"]], all_logits=True)
                             for p in range(0, len(prompt), m["chunk"])])
    assert bits_equal(logits[m["rows"]], arrays[f"{family}_logits_rows"])
    dec.reset()
    tokens, _, _ = dec.generate(prompt, 10)
    assert tokens == arrays[f"{family}_tokens"].tolist()
    dec.close()


@pytest.mark.parametrize("family", ["tinyllama", "qwen", "smollm2"])
@pytest.mark.parametrize("prompt_tokens", [5, 33, 38])
def test_decoder_steps_equal_the_oracle(rt, oracle, artifacts, family, prompt_tokens):
    # 33 and 38 tokens: the CPU trims its final FP32 layer to the trailing rows
    # (decoder.cpp:1375-1387), keeping the token groups of its linears
    bits, math = EXACT[family]
    dec = rt.Decoder(artifacts[family], bits, math, numerics="reference")
    od = oracle.decoder(artifacts[family], bits, math == "accurate")
    prompt = np.random.default_rng(prompt_tokens).integers(0, dec.vocabulary_size, prompt_tokens).astype(np.uint32)
    a, b = dec.forward(prompt), od.forward(prompt)
    assert bits_equal(a, b), ("prefill", first_difference(a, b))
    for step in range(12):
        tok = int(np.argmax(b))
        assert dec.last_argmax.value == tok
        a, b = dec.forward([tok]), od.forward([tok])
        assert bits_equal(a, b), (step, first_difference(a, b))
    dec.close()
    od.close()


def test_reference_numerics_reject_accurate_math(rt, artifacts):
    from leaf_amd.runtime import LeafError
    with pytest.raises(LeafError, match="accurate"):
        rt.Decoder(artifacts["smollm2"], 32, "accurate", numerics="reference")
