"""lh_linear_noalloc: the allocation-free linear, through the C ABI.

Its output and int32 accumulators must equal lh_linear's bit for bit, on two
calls in a row where the second is smaller (the fixed scratch array keeps the
first call's contents), on the GEMM path (split-K sums in the array), the
multi-token GEMV path (quantized input in the array) and the fused single-token
GEMV, for W8A8 at TinyLlama shapes and W4A8.  A call whose quantized input
would not fit the array is refused before any launch.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from leaf_amd.artifact import quantize

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from leaf_amd import runtime
    runtime.library()
    return runtime


def run(rt, entry, dw, x, bits):
    M, K = x.shape
    dx = rt.DeviceArray.of(x)
    dy = rt.DeviceArray((M, dw.rows), np.float32)
    dacc = rt.DeviceArray((M, dw.rows, K // dw.desc.group), np.int32) if bits == 8 else None
    rt.check(entry(C.byref(dw.desc), dx.ptr, M, bits, dy.ptr, dacc.ptr if dacc else None, None))
    return dy.numpy(), dacc.numpy() if dacc else None


@pytest.mark.parametrize("K,N,group,bits,sizes", [
    (2048, 2048, 2048, 8, (512, 16)),        # GEMM with split-K sums, then a smaller GEMM
    (5632, 2048, 5632, 8, (128, 4)),         # GEMM, then the 4-token GEMV on the quantized input
    (2048, 5632, 2048, 8, (64, 1)),          # GEMM, then the fused single-token GEMV
    (256, 96, 32, 4, (40, 3)),               # W4A8 grouped scales
])
def test_noalloc_linear_equals_linear(rt, K, N, group, bits, sizes):
    rng = np.random.default_rng(K + N + bits)
    w = (0.02 * rng.standard_normal((N, K))).astype(np.float32)
    data, scales = quantize(w, bits, group)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    dw = rt.DeviceWeight(data, bits, K, scales, group, bias)
    lib = rt.library()
    for M in sizes:
        x = rng.standard_normal((M, K), dtype=np.float32)
        x[rng.random((M, K)) < 0.001] *= np.float32(20)
        want_y, want_acc = run(rt, lib.lh_linear, dw, x, 8)
        got_y, got_acc = run(rt, lib.lh_linear_noalloc, dw, x, 8)
        assert np.array_equal(got_y.view(np.uint32), want_y.view(np.uint32)), (M, "outputs differ")
        assert np.array_equal(got_acc, want_acc), (M, "int32 accumulators differ")


def test_noalloc_linear_fp_path_equals_linear(rt):
    rng = np.random.default_rng(3)
    w = (0.02 * rng.standard_normal((300, 896))).astype(np.float32)
    dw = rt.DeviceWeight(w, 32, 896)
    lib = rt.library()
    for M in (9, 2):
        x = rng.standard_normal((M, 896), dtype=np.float32)
        want, _ = run(rt, lib.lh_linear, dw, x, 32)
        got, _ = run(rt, lib.lh_linear_noalloc, dw, x, 32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_linear_refuses_inputs_beyond_its_scratch(rt):
    K, N = 5632, 16
    limit = 32 << 20
    tokens = limit // (K + 4) + 1        # its quantized input alone exceeds the array
    w = np.ones((N, K), np.int8)
    dw = rt.DeviceWeight(w, 8, K, np.ones((N, 1), np.float32), K)
    dx = rt.DeviceArray((1,), np.float32)            # never read: the call is refused first
    dy = rt.DeviceArray((1,), np.float32)
    lib = rt.library()
    status = lib.lh_linear_noalloc(C.byref(dw.desc), dx.ptr, tokens, 8, dy.ptr, None, None)
    assert status == 1 and b"too large" in lib.lh_last_error()
