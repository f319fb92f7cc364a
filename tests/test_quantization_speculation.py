"""The rule by which the reference-order decode step quantizes a normalized
vector before its exact RMSNorm sum is known, checked on the CPU.

The persistent step's weight waves quantize y~ = x * gamma (no RMSNorm scale)
while the exchange waves still form the column-order square sum, and take
their int8 dots with those values.  When the sum lands they confirm them: an
element whose t~ = y~ / (max|y~| / 127) lies more than 4e-4 from a rounding
boundary keeps its int8 value, the nearer ones are quantized again with the
exact scale, and the exact per-token scale is the largest exact |y| among the
candidates |y~| >= max|y~| (1 - 1e-6) (one per 64-lane wave lane at most).
This file restates that rule in float32 numpy and checks it against the
oracle's own quantization of the exact normalized vector
(oracle.quantize_rows, decoder.cpp:1020-1044 on y = ((x - 0) * s) * gamma + 0,
decoder.cpp:706-727): every confirmed speculation must give the oracle's
int8 values and scale bit for bit, whatever the two scales are.  A planted
mistake (no re-quantization of the near elements) must be caught.
"""
from __future__ import annotations

import numpy as np

f32 = np.float32
MARGIN = f32(4e-4)
CANDIDATE = f32(1.0 - 1e-6)


def quantize(y, multiplier):
    return np.clip(np.rint((y * multiplier).astype(f32)), -127, 127).astype(np.int8)


def per_token_scale(amax):
    return max(f32(amax / f32(127.0)), f32(1e-12))


def lanes_of(n):
    # lane l of a wave holds the 16-element chunks l, l + 64, ...
    return (np.arange(n) // 16) % 64


def speculate_and_confirm(x, gamma, scale, margin=MARGIN):
    """The device rule: (accepted, int8 values, per-token scale) or (False, ...)."""
    n = x.size
    ys = (x * gamma).astype(f32)
    amax_s = f32(np.max(np.abs(ys)))
    mult_s = f32(1.0) / per_token_scale(amax_s)
    t = (ys * mult_s).astype(f32)
    qs = quantize(ys, mult_s)
    near = np.abs(t - np.rint(t)) > f32(0.5) - margin
    cand = np.abs(ys) >= f32(amax_s * CANDIDATE)
    if np.bincount(lanes_of(n)[cand], minlength=64).max() > 1:
        return False, None, None
    ye = lambda idx: (((x[idx] - f32(0.0)) * scale).astype(f32) * gamma[idx] + f32(0.0)).astype(f32)
    amax_e = f32(np.max(np.abs(ye(cand))))
    sx = per_token_scale(amax_e)
    mult_e = f32(1.0) / sx
    if np.any(quantize(ye(near), mult_e) != qs[near]):
        return False, None, None
    if not (amax_s / f32(127.0) > f32(1e-11) and amax_e / f32(127.0) > f32(1e-11) and np.isfinite(amax_e)):
        return False, None, None
    return True, qs, sx


def vectors(seed, trials):
    rng = np.random.default_rng(seed)
    for _ in range(trials):
        n = int(rng.choice([512, 2048]))
        x = (rng.standard_normal(n) * rng.choice([0.01, 1.0, 30.0])).astype(f32)
        gamma = (rng.standard_normal(n) * 0.2 + 1.0).astype(f32)
        sq = np.cumsum(np.square(x, dtype=f32), dtype=f32)[-1]          # the column-order sum
        scale = f32(1.0) / np.sqrt(f32(sq / f32(n) + f32(1e-5)), dtype=f32)
        # the rule must hold whatever the scale: perturb it well past any sum's error
        scale = f32(scale * f32(rng.choice([1.0, 1.0 + 1e-3, 0.5, 2.0])))
        yield x, gamma, scale


def exact(oracle, x, gamma, scale):
    y = ((((x - f32(0.0)) * scale).astype(f32)) * gamma + f32(0.0)).astype(f32)
    q, s = oracle.quantize_rows(y[None])
    return q[0], f32(s[0])


def test_confirmed_speculation_equals_the_oracle_quantization(oracle):
    accepted = 0
    trials = 400
    for x, gamma, scale in vectors(5, trials):
        ok, q, sx = speculate_and_confirm(x, gamma, scale)
        if not ok:
            continue
        accepted += 1
        want_q, want_s = exact(oracle, x, gamma, scale)
        assert np.array_equal(q, want_q), "a confirmed speculation changed an int8 value"
        assert f32(sx).view(np.uint32) == want_s.view(np.uint32), "the confirmed scale differs"
    # the slow path stays rare
    assert accepted >= 0.95 * trials, accepted


def test_the_speculation_moves_t_by_less_than_the_margin():
    worst = 0.0
    for x, gamma, scale in vectors(6, 300):
        ys = (x * gamma).astype(f32)
        ye = ((((x - f32(0.0)) * scale).astype(f32)) * gamma + f32(0.0)).astype(f32)
        ts = ys * (f32(1.0) / per_token_scale(f32(np.max(np.abs(ys)))))
        te = ye * (f32(1.0) / per_token_scale(f32(np.max(np.abs(ye)))))
        worst = max(worst, float(np.max(np.abs(te.astype(np.float64) - ts.astype(np.float64)))))
    # 127 * 12 * 2^-24 bounds the move; the margin leaves a factor of four
    assert worst < 127 * 12 * 2.0 ** -24 < MARGIN / 4, worst


def tie_vector(rng, n=2048):
    """A vector with one element whose speculative t~ is exactly 10.5, a
    rounding tie: any move of the exact t decides the int8 value."""
    x = (rng.standard_normal(n)).astype(f32)
    gamma = np.ones(n, f32)
    ys = x * gamma
    mult = f32(1.0) / per_token_scale(f32(np.max(np.abs(ys))))
    j = int(np.argmin(np.abs(x)))          # not the maximum
    y = f32(10.5) / mult
    for _ in range(64):                     # walk to the float whose product rounds to 10.5
        t = f32(y * mult)
        if t == f32(10.5):
            break
        y = np.nextafter(y, f32(np.inf) if t < f32(10.5) else f32(-np.inf), dtype=f32)
    x[j] = y
    return x, gamma, j


def test_without_the_near_elements_check_a_wrong_value_would_pass(oracle):
    # planted mistake: no element counts as near a rounding boundary
    rng = np.random.default_rng(8)
    wrong = 0
    for _ in range(50):
        x, gamma, j = tie_vector(rng)
        scale = f32(rng.uniform(0.5, 2.0))
        ok, q, _ = speculate_and_confirm(x, gamma, scale, margin=f32(-1.0))
        if ok and not np.array_equal(q, exact(oracle, x, gamma, scale)[0]):
            wrong += 1
        # the rule as the step runs it never accepts a wrong value
        ok, q, _ = speculate_and_confirm(x, gamma, scale)
        if ok:
            assert np.array_equal(q, exact(oracle, x, gamma, scale)[0])
    assert wrong > 0, "the near-element check never mattered: the test would not see it missing"
