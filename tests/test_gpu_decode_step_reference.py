"""The persistent single-token decode step in reference-order numerics, bit for bit.

With reference-order numerics (the default for decoders with int8
activations) the one-launch decode step sums every floating-point quantity in
the CPU path's order: the RMSNorm squares in column order (decoder.cpp:706-727),
the attention scores over the dims and the softmax denominator and p.v over the
keys in key order with glibc's expf (transformer.cpp:112-143), SiLU with glibc's
expf (decoder.cpp:983, 1414) and the FP32 head in dot_avx's lane order
(decoder.cpp:355-391).  The oracle is bit-exact against the reference
(tests/test_oracle_golden.py), so every step's logits must equal the oracle's
bit for bit and the greedy tokens must be the oracle's, step after step,
while the profiler shows that every step ran on the persistent kernel.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

from leaf_amd import models
from leaf_amd.artifact import write_artifact

pytestmark = pytest.mark.gpu


def step_spec(**overrides):
    """TinyLlama topology and precision at reduced width (head dim stays 64)."""
    base = dict(hidden=512, intermediate=1408, heads=8, kv_heads=2, layers=3, vocab=3000, max_positions=1024)
    base.update(overrides)
    return dataclasses.replace(models.tinyllama_w8a8(), **base)


@pytest.fixture(scope="module")
def rt():
    from leaf_amd import runtime
    runtime.library()
    return runtime


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    path = tmp_path_factory.mktemp("ref_step") / "small.leaf"
    write_artifact(path, step_spec(), seed=11)
    return path


@pytest.fixture(scope="module")
def wide(tmp_path_factory):
    """Full TinyLlama widths (2048 / 5632 / 32:4 heads / 32000 vocab), two layers."""
    path = tmp_path_factory.mktemp("ref_step") / "wide.leaf"
    write_artifact(path, dataclasses.replace(models.tinyllama_w8a8(), layers=2), seed=12)
    return path


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def ran_every_step(profile, steps):
    # A step whose blocks ran off their XCD (checked inside the kernel) runs
    # again on the memory path; after four such steps in a row the XCD-local
    # path stays off.
    launches = profile.get("decode_step", {}).get("launches", 0)
    return steps <= launches <= steps + 4


def greedy_against_oracle(rt, oracle, path, prompt, steps, status=None):
    """Greedy decode on both sides; every step's logits bit-equal, same tokens.
    status, a list, receives the session's status at the end."""
    dec = rt.Decoder(path, 8, numerics="reference", max_context=len(prompt) + steps + 8)
    od = oracle.decoder(path, 8, False)
    a, b = dec.forward(prompt), od.forward(prompt)
    assert np.array_equal(bits(a), bits(b)), "prefill logits differ from the oracle"
    dec.set_profiling(True)
    tokens = []
    for step in range(steps):
        tok = int(np.argmax(b))
        assert int(dec.last_argmax.value) == tok, f"greedy token differs at step {step}"
        tokens.append(tok)
        a, b = dec.forward([tok]), od.forward([tok])
        diff = np.flatnonzero(bits(a) != bits(b))
        assert diff.size == 0, (f"step {step} (position {len(prompt) + step}): {diff.size} logits differ, "
                                f"first {diff[:3]}, max |diff| {np.max(np.abs(a - b)):.3e}")
    profile = dec.profile()
    if status is not None:
        status.append(dec.status())
    dec.close()
    return tokens, profile


def test_reference_step_is_bit_exact_across_span_boundaries(rt, oracle, small):
    # a 70-token prompt, then 80 steps: 2 -> 3 spans of 64 keys
    prompt = np.random.default_rng(3).integers(0, 3000, 70).astype(np.uint32)
    _, profile = greedy_against_oracle(rt, oracle, small, prompt, 80)
    assert ran_every_step(profile, 80)


@pytest.mark.parametrize("item_heads", [2, 4, 8])
def test_reference_step_with_wider_attention_items(rt, oracle, small, monkeypatch, item_heads):
    # wider items (several query heads per exchange wave) score the same keys
    monkeypatch.setenv("LEAF_DECODE_STEP_ITEM_HEADS", str(item_heads))
    prompt = np.random.default_rng(6).integers(0, 3000, 70).astype(np.uint32)
    _, profile = greedy_against_oracle(rt, oracle, small, prompt, 24)
    assert ran_every_step(profile, 24)


def test_reference_step_at_full_tinyllama_width(rt, oracle, wide):
    prompt = np.random.default_rng(4).integers(0, 32000, 300).astype(np.uint32)
    _, profile = greedy_against_oracle(rt, oracle, wide, prompt, 12)
    assert ran_every_step(profile, 12)


def test_reference_step_from_a_one_token_prompt(rt, oracle, small):
    # the first visible key is the new one: no cached rows at all
    _, profile = greedy_against_oracle(rt, oracle, small, np.array([7], np.uint32), 20)
    assert ran_every_step(profile, 20)


def test_reference_step_with_sliding_window(rt, oracle, tmp_path):
    path = tmp_path / "window.leaf"
    write_artifact(path, step_spec(sliding_window=100, layers=2), seed=13)
    prompt = np.random.default_rng(5).integers(0, 3000, 90).astype(np.uint32)
    _, profile = greedy_against_oracle(rt, oracle, path, prompt, 40)
    assert ran_every_step(profile, 40)


def test_reference_step_xcd_local_and_memory_paths_are_bit_exact(rt, oracle, wide, monkeypatch):
    # Scores travel through one XCD's L2 (LEAF_DECODE_STEP_LOCAL_MERGE) with
    # the q rows (LEAF_DECODE_STEP_LOCAL_Q), or through uncached memory; a
    # host-forced failed XCD check makes every step fall back: four steps run
    # again on the memory path, then the XCD-local exchange stays off, and the
    # session's status says so.  All give the oracle's logits.
    prompt = np.arange(1, 90, dtype=np.uint32) * 11
    for merge, q, force in (("1", "1", "0"), ("1", "0", "0"), ("0", "0", "0"), ("1", "1", "1")):
        monkeypatch.setenv("LEAF_DECODE_STEP_LOCAL_MERGE", merge)
        monkeypatch.setenv("LEAF_DECODE_STEP_LOCAL_Q", q)
        monkeypatch.setenv("LEAF_DECODE_STEP_FORCE_XCD_MISMATCH", force)
        print(f"local merge {merge}, local q {q}, forced mismatch {force}", flush=True)
        status = []
        _, profile = greedy_against_oracle(rt, oracle, wide, prompt, 8, status)
        assert profile.get("decode_step", {}).get("launches", 0) >= 8
        st = status[0]
        assert st["reference_order"] and st["step_tokens"] == 8
        if force == "1":
            assert st["step_memory_reruns"] == 4 and not st["xcd_local"]
        elif merge == "0":
            assert not st["xcd_local"]


def test_reference_step_and_graph_path_agree(rt, small, monkeypatch):
    # the reference-order graph-replayed kernels and the persistent step
    feed = (np.arange(30, dtype=np.uint32) * 97 + 5) % 3000
    runs = []
    for flag in ("1", "0"):
        monkeypatch.setenv("LEAF_DECODE_STEP", flag)
        dec = rt.Decoder(small, 8, numerics="reference")
        dec.set_profiling(True)
        dec.forward(np.arange(1, 41, dtype=np.uint32) * 7)
        rows = [dec.forward([int(tok)]) for tok in feed]
        steps = dec.profile().get("decode_step", {}).get("launches", 0)
        dec.close()
        runs.append(bits(np.stack(rows)))
        assert steps == (30 if flag == "1" else 0)
    assert np.array_equal(runs[0], runs[1])


def test_w8a8_decoders_default_to_reference_numerics(rt, small):
    # no numerics given and LEAF_GPU_NUMERICS unset: the persistent step in
    # reference order, bit-equal to an explicit reference session
    feed = [5, 17, 2999, 0, 1234]
    out = []
    for numerics in ("default", "reference"):
        dec = rt.Decoder(small, 8, numerics=numerics)
        dec.forward(np.arange(10, 30, dtype=np.uint32))
        out.append(bits(np.stack([dec.forward([t]) for t in feed])))
        dec.close()
    assert np.array_equal(out[0], out[1])


def test_reference_session_refuses_more_keys_than_it_holds(rt, tmp_path):
    # One query's keys sit in LDS in reference order (32,448 keys: 159 KiB of
    # LDS less q and one 128-key product buffer, in floats).  A session asked
    # for a longer context is refused when it is created, not at the token
    # that passes the limit; without a requested size the capacity stops at
    # the limit.  The fast kernels take the whole context.
    path = tmp_path / "long.leaf"
    write_artifact(path, step_spec(max_positions=40000, layers=1), seed=14)
    with pytest.raises(rt.LeafError, match="visible keys"):
        rt.Decoder(path, 8, numerics="reference", max_context=32449)
    for numerics, context in (("reference", 32448), ("reference", 0), ("fast", 40000)):
        dec = rt.Decoder(path, 8, numerics=numerics, max_context=context)
        dec.forward(np.arange(1, 20, dtype=np.uint32))
        dec.close()
