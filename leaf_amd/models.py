"""Architectural presets for the decoder workloads this library is measured on.

Each preset is a :class:`DecoderSpec` carrying the header semantics Leaf's
plan builder would emit for that architecture (tools/decoder_plan.py:157-327)
and the storage policy of the requested artifact.  ``reduced=True`` keeps the
operator topology and precision policy but shrinks widths, depth and vocab so
CPU oracles finish in seconds.
"""
from __future__ import annotations

import dataclasses

from .artifact import (ACT_GELU_TANH, ACT_SILU, NORM_LAYER, NORM_RMS, POS_LEARNED, POS_ROPE,
                       DecoderSpec)


def gpt2_small(reduced: bool = False, **overrides) -> DecoderSpec:
    """GPT-2 small, FP32: LayerNorm(+beta), learned positions, gelu_new, biases, tied head."""
    spec = DecoderSpec(hidden=768, intermediate=3072, heads=12, kv_heads=12, layers=12, vocab=50257,
                       max_positions=1024, head_dim=64, epsilon=1e-5, norm=NORM_LAYER,
                       activation=ACT_GELU_TANH, position=POS_LEARNED, gated=0, final_norm=1,
                       bits=32, tied=True, attention_bias=True, o_bias=True, mlp_bias=True,
                       norm_bias=True)
    if reduced:
        spec = dataclasses.replace(spec, hidden=128, intermediate=512, heads=4, kv_heads=4, layers=2,
                                   vocab=1000, max_positions=256, head_dim=32)
    return dataclasses.replace(spec, **overrides)


def tinyllama_w8a8(reduced: bool = False, **overrides) -> DecoderSpec:
    """TinyLlama-1.1B architecture, INT8 per-row weights, untied FP32 LM head."""
    spec = DecoderSpec(hidden=2048, intermediate=5632, heads=32, kv_heads=4, layers=22, vocab=32000,
                       max_positions=2048, head_dim=64, theta=10000.0, epsilon=1e-5, norm=NORM_RMS,
                       activation=ACT_SILU, position=POS_ROPE, gated=1, bits=8,
                       keep_fp32=frozenset({"lm_head.weight"}))
    if reduced:
        spec = dataclasses.replace(spec, hidden=256, intermediate=704, heads=8, kv_heads=2, layers=2,
                                   vocab=2000, max_positions=512, head_dim=32)
    return dataclasses.replace(spec, **overrides)


def qwen25_int4(reduced: bool = False, **overrides) -> DecoderSpec:
    """Qwen2.5-0.5B architecture, INT4 group-32 weights, QKV bias, tied head."""
    spec = DecoderSpec(hidden=896, intermediate=4864, heads=14, kv_heads=2, layers=24, vocab=151936,
                       max_positions=32768, head_dim=64, theta=1000000.0, epsilon=1e-6,
                       norm=NORM_RMS, activation=ACT_SILU, position=POS_ROPE, gated=1, bits=4,
                       group_size=32, tied=True, attention_bias=True)
    if reduced:
        spec = dataclasses.replace(spec, hidden=224, intermediate=608, heads=7, kv_heads=1, layers=2,
                                   vocab=3000, max_positions=4096, head_dim=32)
    return dataclasses.replace(spec, **overrides)


def smollm2_bf16(reduced: bool = False, **overrides) -> DecoderSpec:
    """SmolLM2-360M architecture, weights stored as BF16 (v6 matrices), tied head."""
    spec = DecoderSpec(hidden=960, intermediate=2560, heads=15, kv_heads=5, layers=32, vocab=49152,
                       max_positions=8192, head_dim=64, theta=100000.0, epsilon=1e-5,
                       norm=NORM_RMS, activation=ACT_SILU, position=POS_ROPE, gated=1, bits=32,
                       source_bf16=True, tied=True)
    if reduced:
        spec = dataclasses.replace(spec, hidden=192, intermediate=512, heads=6, kv_heads=2, layers=2,
                                   vocab=1500, max_positions=1024, head_dim=32)
    return dataclasses.replace(spec, **overrides)


PRESETS = {"gpt2": gpt2_small, "tinyllama": tinyllama_w8a8, "qwen": qwen25_int4, "smollm2": smollm2_bf16}

# How each preset is run: activation bits and FP32 math policy (main_decoder.cpp argv).
RUN_POLICY = {"gpt2": (32, "fast"), "tinyllama": (8, "fast"), "qwen": (32, "fast"),
              "smollm2": (32, "accurate")}

# Standalone W8A8 linear shapes at TinyLlama widths, (K, N): q/o, k/v, gate/up, down.
W8A8_LINEAR_SHAPES = ((2048, 2048), (2048, 256), (2048, 256), (2048, 5632), (2048, 5632), (5632, 2048))
W8A8_LINEAR_TOKENS = (1, 4, 16, 128, 512)
