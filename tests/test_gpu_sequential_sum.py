"""The column-order float sum of the reference-order decode step, formed in parallel.

norm() sums a row's squares and attention_impl its softmax denominator one
element after another in float (decoder.cpp:716-718, transformer.cpp:127-130).
The decode step forms that sum with one wave (wave_sequential_sum in
leaf_amd/csrc/sequential_sum.h; the softmax denominator) or two
(wave_pair_sequential_sum; the RMSNorm squares): runs of steps whose rounding
cannot depend on the running sum are added as exact jumps and only the others
are taken one by one.  Here it must equal numpy's float32 accumulate -- a plain loop, one
rounding per element -- bit for bit, on the shapes it serves (2048 and 5632
squares, a few hundred to 4,096 softmax terms) and on inputs built to defeat
it: ties at every step, powers of two, two scales 2^30 apart, zeros, one
element, subnormal terms (summed like any other), and infinite, NaN or
negative terms and totals past 2^126 (which take the plain chain).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from leaf_amd import runtime
    runtime.library()
    return runtime


def column_sums(x):
    return np.add.accumulate(np.asarray(x, np.float32), axis=1, dtype=np.float32)[:, -1]


def gpu_sums(rt, x, method=0):
    x = np.ascontiguousarray(x, np.float32)
    count, n = x.shape
    dx = rt.DeviceArray.of(x)
    out = rt.DeviceArray((count,), np.float32)
    cycles = rt.DeviceArray((count,), np.int64)
    rt.sequential_sum(dx, n, count, out, cycles, method)
    rt.synchronize()
    return out.numpy(), cycles.numpy()


def cases(n, rng):
    count = 64
    g = rng.standard_normal((count, n)).astype(np.float32)
    scale = np.ldexp(np.float32(1), rng.integers(-40, 40, (count, 1))).astype(np.float32)
    yield "squares", (g * scale) ** 2
    out = g * (np.where(rng.random((count, n)) < 0.001, 20, 1)).astype(np.float32)
    yield "squares with outliers", out * out
    yield "softmax terms", np.exp(-rng.random((count, n)) * 8).astype(np.float32)
    yield "zeros and ones", (rng.random((count, n)) < 0.5).astype(np.float32)
    yield "small integers (ties)", rng.integers(0, 16, (count, n)).astype(np.float32) * scale
    yield "powers of two", np.ldexp(np.float32(1), rng.integers(0, 20, (count, n))).astype(np.float32) * scale
    two = rng.random((count, n)).astype(np.float32) * scale
    two[:, : n // 2] *= np.float32(2.0 ** -30)
    yield "two scales", two
    yield "heavy tail", np.abs(g) * np.where(rng.random((count, n)) < 0.01, 1e6, 1).astype(np.float32)
    yield "all zero", np.zeros((count, n), np.float32)
    yield "softmax tail (subnormal terms)", np.exp(-rng.random((count, n)) * 110).astype(np.float32)
    yield "subnormal terms", rng.integers(0, 1 << 23, (count, n)).astype(np.uint32).view(np.float32)
    yield "squares near the subnormal range", (g * np.float32(1e-20)) ** 2
    zeros_first = (g * scale) ** 2
    zeros_first[:, : n // 3] = 0
    yield "leading zeros", zeros_first


@pytest.mark.parametrize("method", [0, 2], ids=["one wave", "two waves"])
@pytest.mark.parametrize("n", [1, 7, 33, 64, 256, 257, 600, 640, 760, 1000, 2047, 2048, 4096, 5632])
def test_parallel_column_sum_equals_the_chain(rt, n, method):
    rng = np.random.default_rng(n)
    for name, x in cases(n, rng):
        got, _ = gpu_sums(rt, x, method)
        want = column_sums(x)
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, f"{name}, n={n}: {bad.size} of {len(want)} sums differ (row {bad[0]})"


@pytest.mark.parametrize("method", [0, 2], ids=["one wave", "two waves"])
def test_unusual_terms(rt, method):
    # a subnormal term and -0 are summed like any other; infinite, NaN and
    # negative terms and a total past 2^126 take the plain chain
    x = np.abs(np.random.default_rng(1).standard_normal((7, 2048))).astype(np.float32)
    x[0, 100] = np.float32(1e-40)
    x[1, 5] = np.inf
    x[2, 7] = np.nan
    x[3, :] *= np.float32(2.0 ** 110)
    x[4, 9] = np.float32(-0.0)
    x[5, 11] = np.float32(-1.5)
    x[6, :] = np.float32(1e-40)
    got, _ = gpu_sums(rt, x, method)
    want = column_sums(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_matches_a_python_float32_loop(rt):
    x = (np.random.default_rng(2).standard_normal((1, 777)) ** 2).astype(np.float32)
    s = np.float32(0)
    for v in x[0]:
        s = np.float32(s + v)
    got, _ = gpu_sums(rt, x)
    assert got.view(np.uint32)[0] == np.float32(s).view(np.uint32)


def test_parallel_sum_is_faster_than_the_chain(rt):
    rng = np.random.default_rng(3)
    for n in (600, 2048):
        x = (rng.standard_normal((256, n)) ** 2).astype(np.float32)
        fast, c0 = gpu_sums(rt, x, 0)
        pair, c2 = gpu_sums(rt, x, 2)
        slow, c1 = gpu_sums(rt, x, 1)
        assert np.array_equal(fast.view(np.uint32), slow.view(np.uint32))
        assert np.array_equal(pair.view(np.uint32), slow.view(np.uint32))
        print(f"n={n}: one wave {np.median(c0):.0f} cycles, two waves {np.median(c2):.0f}, "
              f"chain {np.median(c1):.0f}")
        assert np.median(c0) < np.median(c1) and np.median(c2) < np.median(c1)
