"""The persistent single-token decode step in fast numerics against the oracle and the multi-launch path.

(The same step in reference-order numerics, the default for W8A8 decoders,
is bit-exact against the oracle: tests/test_gpu_decode_step_reference.py.)
Single-token W8A8 forwards of TinyLlama-shape decoders (RMSNorm, RoPE, gated
SiLU MLP, head dim 64, per-row INT8 matrices, FP32 head) run as one
cooperative launch.  The runs are teacher-forced: the oracle's greedy token is
fed to both sides at every step.  Each step's logits must match the oracle
within W8A8_LOGIT_TOLERANCE of the largest |logit| and W8A8_RMSE_TOLERANCE
relative RMSE (the bound and its source are given beside the constants); the
greedy choice must match whenever the oracle's top-2 margin is wider than
twice the 2e-2 band of an order-only change (inside it, a single int8
rounding flip upstream -- the reference's own AVX2 and scalar W8A8 builds
differ by such flips -- can reorder near-tied logits); and the kernel must
actually have run (profiler class "decode_step").
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

from leaf_amd import models
from leaf_amd.artifact import write_artifact

pytestmark = pytest.mark.gpu

# W8A8 logits: no logit further than 5e-2 of the largest |logit| from the
# oracle's, and relative RMSE (as Leaf's quality() defines it,
# tools/decoder_validation.py:222-253) within 5e-2.  GPU and CPU sum the RMSNorm
# squares in different orders; some activations then land on the other side
# of an int8 rounding boundary and each flip moves every logit.  The oracle
# alone shows the size of this band: changing only its norm summation order
# moves these models' logits by 1.2-1.9e-2 at reduced width
# (tests/test_oracle_golden.py) and by up to 3.6e-2 at TinyLlama width.
W8A8_LOGIT_TOLERANCE = 5e-2
W8A8_RMSE_TOLERANCE = 5e-2


def rel_error(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def rel_rmse(a, b):
    return float(np.sqrt(np.mean((a - b) ** 2)) / max(np.sqrt(np.mean(b ** 2)), 1e-12))


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
    path = tmp_path_factory.mktemp("step") / "small.leaf"
    write_artifact(path, step_spec(), seed=11)
    return path


@pytest.fixture(scope="module")
def wide(tmp_path_factory):
    """Full TinyLlama widths (2048 / 5632 / 32:4 heads / 32000 vocab), two layers."""
    path = tmp_path_factory.mktemp("step") / "wide.leaf"
    write_artifact(path, dataclasses.replace(models.tinyllama_w8a8(), layers=2), seed=12)
    return path


def decisive(reference, tolerance=2e-2):
    """Whether the reference's top-2 margin exceeds twice the typical movement
    (2e-2 of the largest |logit|) of an order-only change."""
    top = np.sort(reference)[-2:]
    return top[1] - top[0] > 2 * tolerance * np.max(np.abs(reference))


def run_steps(rt, oracle, path, prompt_tokens, steps, seed, **decoder_args):
    dec = rt.Decoder(path, 8, numerics="fast", **decoder_args)
    od = oracle.decoder(path, 8, False)
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, dec.vocabulary_size, prompt_tokens).astype(np.uint32)
    a, b = dec.forward(prompt), od.forward(prompt)
    assert rel_error(a, b) <= W8A8_LOGIT_TOLERANCE
    dec.set_profiling(True)
    worst, tokens, checked, rmse = 0.0, [], 0, 0.0
    for step in range(steps):
        tok = int(np.argmax(b))
        assert int(dec.last_argmax.value) == int(np.argmax(a)), "device argmax differs from the logits it returned"
        if decisive(b):
            assert int(np.argmax(a)) == tok, f"greedy token differs at step {step} with a decisive margin"
            checked += 1
        tokens.append(tok)
        a, b = dec.forward([tok]), od.forward([tok])
        worst = max(worst, rel_error(a, b))
        rmse = max(rmse, rel_rmse(a, b))
        assert rmse <= W8A8_RMSE_TOLERANCE, f"relative logit RMSE {rmse:.2e} at step {step}"
    profile = dec.profile()
    dec.close()
    print(f"greedy choice compared at {checked} of {steps} steps (the rest within the tolerance band); "
          f"worst relative RMSE {rmse:.2e}")
    assert checked >= steps // 5
    return worst, tokens, profile


def ran_every_step(profile, steps):
    # Every step ran on the persistent decode step; a step whose blocks ran
    # off their XCD (checked inside the kernel) runs again on the memory path,
    # and after four such steps in a row the XCD-local path stays off.
    launches = profile.get("decode_step", {}).get("launches", 0)
    return steps <= launches <= steps + 4


def test_step_matches_oracle_across_span_boundaries(rt, oracle, small):
    # a 70-token prompt, then 80 steps: 2 -> 3 spans of 64 keys
    worst, _, profile = run_steps(rt, oracle, small, 70, 80, seed=3)
    print(f"decode step: worst relative logit error {worst:.2e}")
    assert worst <= W8A8_LOGIT_TOLERANCE
    assert ran_every_step(profile, 80)


@pytest.mark.parametrize("item_heads", [2, 4, 8])
def test_step_with_wider_attention_items(rt, oracle, small, monkeypatch, item_heads):
    # Long contexts give each attention item more query heads (fewer, wider
    # items when heads x spans outgrow the grid); forced here at a short one.
    monkeypatch.setenv("LEAF_DECODE_STEP_ITEM_HEADS", str(item_heads))
    worst, _, profile = run_steps(rt, oracle, small, 70, 30, seed=6)
    assert worst <= W8A8_LOGIT_TOLERANCE
    assert ran_every_step(profile, 30)


def test_step_at_full_tinyllama_width(rt, oracle, wide):
    worst, _, profile = run_steps(rt, oracle, wide, 300, 12, seed=4)
    print(f"decode step (2048/5632/32:4): worst relative logit error {worst:.2e}")
    assert worst <= W8A8_LOGIT_TOLERANCE
    assert ran_every_step(profile, 12)


def test_step_with_sliding_window(rt, oracle, tmp_path):
    path = tmp_path / "window.leaf"
    write_artifact(path, step_spec(sliding_window=100, layers=2), seed=13)
    worst, _, profile = run_steps(rt, oracle, path, 90, 40, seed=5)
    assert worst <= W8A8_LOGIT_TOLERANCE
    assert ran_every_step(profile, 40)


def test_step_and_graph_paths_agree(rt, small, monkeypatch):
    # the same token sequence through both single-token paths
    feed = (np.arange(30, dtype=np.uint32) * 97 + 5) % 3000
    runs = []
    for flag in ("1", "0"):
        monkeypatch.setenv("LEAF_DECODE_STEP", flag)
        dec = rt.Decoder(small, 8, numerics="fast")
        dec.set_profiling(True)
        dec.forward(np.arange(1, 41, dtype=np.uint32) * 7)
        rows = [dec.forward([int(tok)]) for tok in feed]
        steps = dec.profile().get("decode_step", {}).get("launches", 0)
        dec.close()
        runs.append(np.stack(rows))
        assert steps == (30 if flag == "1" else 0)
    assert rel_error(runs[0], runs[1]) <= W8A8_LOGIT_TOLERANCE
    assert rel_rmse(runs[0], runs[1]) <= W8A8_RMSE_TOLERANCE


def test_xcd_local_attention_matches_the_memory_path(rt, wide, oracle, monkeypatch):
    # At TinyLlama widths the span partials of each head pair go through one
    # XCD's L2 (LEAF_DECODE_STEP_LOCAL_MERGE), and so do the q rows of the
    # pair, with the new key folded into its span after the cached keys
    # (LEAF_DECODE_STEP_LOCAL_Q).  The local merge moves the same words: with
    # it alone the logits equal those of the memory path, and so do those of
    # a run whose (host-forced) failed XCD check makes the first step abort
    # and every step fall back.  The late fold sums in another order: those
    # logits stay within the decode step's bounds of the oracle.
    feed = (np.arange(12, dtype=np.uint32) * 131 + 7) % 32000
    prompt = np.arange(1, 90, dtype=np.uint32) * 11
    runs = []
    for merge, q, force in (("1", "0", "0"), ("0", "0", "0"), ("1", "1", "1"), ("1", "1", "0")):
        monkeypatch.setenv("LEAF_DECODE_STEP_LOCAL_MERGE", merge)
        monkeypatch.setenv("LEAF_DECODE_STEP_LOCAL_Q", q)
        monkeypatch.setenv("LEAF_DECODE_STEP_FORCE_XCD_MISMATCH", force)
        dec = rt.Decoder(wide, 8, numerics="fast")
        dec.set_profiling(True)
        dec.forward(prompt)
        rows = [dec.forward([int(tok)]) for tok in feed]
        steps = dec.profile().get("decode_step", {}).get("launches", 0)
        dec.close()
        runs.append(np.stack(rows))
        assert steps >= len(feed)
    assert np.array_equal(runs[0], runs[1])
    assert np.array_equal(runs[2], runs[1])
    od = oracle.decoder(wide, 8, False)
    od.forward(prompt)
    ref = np.stack([od.forward([int(tok)]) for tok in feed])
    for got in runs[3], runs[1]:
        assert max(rel_error(x, y) for x, y in zip(got, ref)) <= W8A8_LOGIT_TOLERANCE
        assert max(rel_rmse(x, y) for x, y in zip(got, ref)) <= W8A8_RMSE_TOLERANCE


def test_step_is_deterministic_across_reset(rt, small):
    dec = rt.Decoder(small, 8, numerics="fast")
    prompt = np.arange(3, 53, dtype=np.uint32)
    outs = []
    for _ in range(2):
        dec.reset()
        tok = dec.forward_into(prompt, None)
        rows = []
        for _ in range(20):
            rows.append(dec.forward([tok]))
            tok = int(dec.last_argmax.value)
        outs.append(np.stack(rows))
    dec.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
