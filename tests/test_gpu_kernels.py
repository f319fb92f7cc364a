"""GPU kernels through the C ABI against the oracle, on the same seeded inputs.

Integer work (activation quantization, int32 accumulators, the W8A8 / W4A8
epilogue) must be bit-exact.  Floating-point paths are checked against the
oracle and an FP64 restatement with the stated tolerances.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from leaf_amd.artifact import quantize, round_to_bf16  # noqa: E402
from leaf_amd.models import W8A8_LINEAR_SHAPES  # noqa: E402


@pytest.fixture(scope="module")
def rt():
    from leaf_amd import runtime
    runtime.library()
    return runtime


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def activations(rng, M, K):
    x = rng.standard_normal((M, K), dtype=np.float32)
    x[rng.random((M, K)) < 0.001] *= np.float32(20)
    return x


def run_int_linear(rt, w, s, b, x, bits, group, acc=True):
    M, K = x.shape
    N = w.shape[0]
    dw = rt.DeviceWeight(w, bits, K, s, group, b)
    dx = rt.DeviceArray.of(x)
    dy = rt.DeviceArray((M, N), np.float32)
    dacc = rt.DeviceArray((M, N, K // group), np.int32) if acc else None
    rt.linear(dw, dx, M, 8, dy, dacc)
    return dy.numpy(), (dacc.numpy() if acc else None)


def test_quantize_rows_bit_exact(rt, oracle):
    rng = np.random.default_rng(1)
    for M, K in ((1, 2048), (7, 5632), (3, 100)):
        x = activations(rng, M, K)
        dx = rt.DeviceArray.of(x)
        q, s = rt.DeviceArray((M, K), np.int8), rt.DeviceArray((M,), np.float32)
        rt.quantize_rows(dx, M, K, q, s)
        oq, os_ = oracle.quantize_rows(x)
        assert np.array_equal(q.numpy(), oq) and bits_equal(s.numpy(), os_)


@pytest.mark.parametrize("K,N", sorted(set(W8A8_LINEAR_SHAPES)))
def test_w8a8_decode_gemv_bit_exact_at_tinyllama_shapes(rt, oracle, K, N):
    rng = np.random.default_rng(K * 7 + N)
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    wq, ws = quantize(w, 8, K)
    x = activations(rng, 1, K)
    y, acc = run_int_linear(rt, wq, ws, None, x, 8, K)
    q, qs = oracle.quantize_rows(x)
    assert np.array_equal(acc, oracle.int_accumulators(8, N, K, K, wq, q)), "int32 accumulators differ"
    assert bits_equal(y, oracle.linear_int(8, N, K, K, wq, ws, None, x)), "dequantized outputs differ"


@pytest.mark.parametrize("M", [2, 4, 16, 128])
def test_w8a8_multi_token_bit_exact(rt, oracle, M):
    rng = np.random.default_rng(M)
    K, N = 2048, 256
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    wq, ws = quantize(w, 8, K)
    b = rng.standard_normal(N, dtype=np.float32)
    x = activations(rng, M, K)
    y, acc = run_int_linear(rt, wq, ws, b, x, 8, K)
    q, _ = oracle.quantize_rows(x)
    assert np.array_equal(acc, oracle.int_accumulators(8, N, K, K, wq, q))
    assert bits_equal(y, oracle.linear_int(8, N, K, K, wq, ws, b, x))


@pytest.mark.parametrize("K,N", sorted(set(W8A8_LINEAR_SHAPES)))
@pytest.mark.parametrize("M", [4, 16, 128, 512])
def test_w8a8_config_grid_bit_exact(rt, oracle, K, N, M):
    # The W8A8 microbenchmark configuration at every shape and token count:
    # weights N(0, 0.02) quantized per output row, activations N(0, 1) with
    # ~0.1% outliers x20 quantized per token; int32 accumulators and the
    # dequantized outputs against quant_dot / quant_tile / quant_vnni_tile
    # (decoder.cpp:536-702) as the oracle restates them.
    rng = np.random.default_rng(20261201 + K * 13 + N * 7 + M)
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    wq, ws = quantize(w, 8, K)
    x = activations(rng, M, K)
    y, acc = run_int_linear(rt, wq, ws, None, x, 8, K)
    q, _ = oracle.quantize_rows(x)
    assert np.array_equal(acc, oracle.int_accumulators(8, N, K, K, wq, q)), "int32 accumulators differ"
    assert bits_equal(y, oracle.linear_int(8, N, K, K, wq, ws, None, x)), "dequantized outputs differ"


def test_w8a8_prefill_gemm_512_tokens_bit_exact(rt, oracle):
    rng = np.random.default_rng(512)
    M, K, N = 512, 2048, 320
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    wq, ws = quantize(w, 8, K)
    x = activations(rng, M, K)
    y, acc = run_int_linear(rt, wq, ws, None, x, 8, K)
    q, _ = oracle.quantize_rows(x)
    assert np.array_equal(acc, oracle.int_accumulators(8, N, K, K, wq, q))
    assert bits_equal(y, oracle.linear_int(8, N, K, K, wq, ws, None, x))


@pytest.mark.parametrize("M,K,N", [(300, 5632, 200), (130, 2048, 2560), (512, 2048, 1408), (17, 768, 129),
                                   (300, 256, 16448), (512, 2048, 11264)])
def test_w8a8_tiled_gemm_edges_bit_exact(rt, oracle, M, K, N):
    # Tiles cut by the token and row counts, K from 256 to 5632: 64 x 64 tiles
    # (with split K for the short inputs), and 128 rows x 256 tokens for the
    # large outputs (16448 rows: 129 row tiles, the last one partial; 11264:
    # the stacked gate|up projection of a 512-token TinyLlama prefill)
    rng = np.random.default_rng(M * 31 + N)
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    wq, ws = quantize(w, 8, K)
    b = rng.standard_normal(N, dtype=np.float32)
    x = activations(rng, M, K)
    y, acc = run_int_linear(rt, wq, ws, b, x, 8, K)
    q, _ = oracle.quantize_rows(x)
    assert np.array_equal(acc, oracle.int_accumulators(8, N, K, K, wq, q))
    assert bits_equal(y, oracle.linear_int(8, N, K, K, wq, ws, b, x))


@pytest.mark.parametrize("bits,group,K,N,M", [(8, 64, 256, 9, 1), (8, 64, 256, 9, 5), (8, 64, 512, 70, 67),
                                              (8, 2, 100, 7, 3), (4, 32, 256, 6, 1), (4, 32, 896, 40, 3),
                                              (4, 896, 896, 40, 1), (8, 100, 100, 7, 1), (4, 2, 64, 3, 2)])
def test_grouped_and_odd_integer_paths_bit_exact(rt, oracle, bits, group, K, N, M):
    rng = np.random.default_rng(bits * 1000 + K + M)
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    wq, ws = quantize(w, bits, group)
    b = rng.standard_normal(N, dtype=np.float32)
    x = activations(rng, M, K)
    y, acc = run_int_linear(rt, wq, ws, b, x, bits, group)
    q, _ = oracle.quantize_rows(x)
    assert np.array_equal(acc, oracle.int_accumulators(bits, N, K, group, wq, q))
    oracle.set_vnni_policy(0)
    assert bits_equal(y, oracle.linear_int(bits, N, K, group, wq, ws, b, x))


def test_golden_w8a8_vectors_on_gpu(rt, golden_kernels):
    # the reference's own outputs (tests/golden/kernels.npz), straight on the GPU
    g = golden_kernels
    for tag, group, tokens in (("k2048", 2048, (1, 4, 16)), ("k5632", 5632, (1, 4)), ("odd", 100, (1, 3, 5)),
                               ("g64", 64, (1, 2, 5))):
        w, s, b = g[f"w8a8_{tag}_w"], g[f"w8a8_{tag}_s"], g.get(f"w8a8_{tag}_b")
        for M in tokens:
            y, _ = run_int_linear(rt, w, s, b, g[f"w8a8_{tag}_m{M}_x"], 8, group, acc=False)
            assert bits_equal(y, g[f"w8a8_{tag}_m{M}_y"]), (tag, M)


def test_grouped_int8_sums_follow_the_cpu_form(rt, oracle, golden_kernels):
    # Over several tokens the CPU sums INT8 scale groups with fused
    # multiply-adds (quant_tile_avx) or, on AVX-VNNI hosts, with a multiply and
    # an add (quant_vnni_tile); the kernel-level numerics pin either form.
    g = golden_kernels
    try:
        for mode, policy, key in (("reference-vnni", 1, "yvnni"), ("reference-avx2", 0, "y")):
            rt.set_kernel_numerics(mode)
            w, s = g["w8a8_g64_w"], g["w8a8_g64_s"]
            for M in (2, 5):
                y, _ = run_int_linear(rt, w, s, None, g[f"w8a8_g64_m{M}_x"], 8, 64, acc=False)
                assert bits_equal(y, g[f"w8a8_g64_m{M}_{key}"]), (mode, M)
            # tokens 2..4 run the generic kernel, 67 the grouped MFMA GEMM
            rng = np.random.default_rng(64)
            for M, K, N in ((3, 256, 9), (67, 512, 70)):
                wq, ws = quantize(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02), 8, 64)
                b = rng.standard_normal(N, dtype=np.float32)
                x = activations(rng, M, K)
                y, _ = run_int_linear(rt, wq, ws, b, x, 8, 64, acc=False)
                oracle.set_vnni_policy(policy)
                assert bits_equal(y, oracle.linear_int(8, N, K, 64, wq, ws, b, x)), (mode, M)
    finally:
        rt.set_kernel_numerics("fast")
        oracle.set_vnni_policy(0)


def fp_case(bits, w, K):
    if bits == 32:
        return w, None, 0
    if bits == 16:
        return round_to_bf16(w), None, 0
    group = K if bits == 8 else 32
    q, s = quantize(w, bits, group)
    return q, s, group


@pytest.mark.parametrize("bits", [32, 16, 8, 4])
@pytest.mark.parametrize("M", [1, 2, 4, 17, 64])
def test_fp_linear_within_tolerance(rt, oracle, bits, M):
    rng = np.random.default_rng(bits + M)
    K, N = 768, 130
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    data, scales, group = fp_case(bits, w, K)
    b = rng.standard_normal(N, dtype=np.float32) * np.float32(0.1)
    x = rng.standard_normal((M, K), dtype=np.float32)
    dw = rt.DeviceWeight(data, bits, K, scales, group, b)
    dx = rt.DeviceArray.of(x)
    dy = rt.DeviceArray((M, N), np.float32)
    rt.linear(dw, dx, M, 32, dy)
    y = dy.numpy()
    ref = oracle.linear_fp(bits, N, K, group, data, scales, b, x)
    # FP64 restatement of the same dequantized weights
    if bits == 32:
        wd = data.astype(np.float64)
    elif bits == 16:
        wd = (data.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    else:
        if bits == 4:
            un = np.empty((N, K), np.int8)
            un[:, ::2] = data & 15
            un[:, 1::2] = data >> 4
            un[un >= 8] -= 16
        else:
            un = data
        wd = un.astype(np.float64) * np.repeat(scales.astype(np.float64), group, axis=1)
    e = x.astype(np.float64) @ wd.T + b
    # test_decode_gemv.cpp:36-42 bound against FP64, twice that against the CPU path
    assert np.all(np.abs(y - e) <= 2e-5 * (1 + np.abs(e)))
    assert np.all(np.abs(y - ref) <= 4e-5 * (1 + np.abs(ref)))


@pytest.mark.parametrize("bits,K", [(32, 3072), (16, 5632), (32, 1028)])
def test_fp_single_token_long_rows_within_tolerance(rt, oracle, bits, K):
    # One token over rows of 9-16 chunks per lane (GPT-2's 3072-wide MLP
    # output projection, BF16 at 5632) and a width with a partial last chunk
    # pass: the fused GEMV's one-row-per-wave variant, against the oracle.
    rng = np.random.default_rng(bits + K)
    N = 300
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    data, scales, group = fp_case(bits, w, K)
    b = rng.standard_normal(N, dtype=np.float32) * np.float32(0.1)
    x = rng.standard_normal((1, K), dtype=np.float32)
    dw = rt.DeviceWeight(data, bits, K, scales, group, b)
    dx = rt.DeviceArray.of(x)
    dy = rt.DeviceArray((1, N), np.float32)
    rt.linear(dw, dx, 1, 32, dy)
    ref = oracle.linear_fp(bits, N, K, group, data, scales, b, x)
    y = dy.numpy()
    assert np.all(np.abs(y - ref) <= 4e-5 * (1 + np.abs(ref)))


@pytest.mark.parametrize("bits", [32, 16, 8, 4])
def test_f32_gemm_tiles_agree_bit_exactly(rt, oracle, monkeypatch, bits):
    # The LDS-staged f32 GEMM runs the same MFMA sequence per output in every
    # tile shape, so all four tiles must give the same bits, on ragged token
    # and row counts (partial tiles at both edges), and stay within the FP
    # linear tolerance of the oracle.
    rng = np.random.default_rng(700 + bits)
    M, K, N = 300, 896, 200
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    data, scales, group = fp_case(bits, w, K)
    b = rng.standard_normal(N, dtype=np.float32) * np.float32(0.1)
    x = rng.standard_normal((M, K), dtype=np.float32)
    dw = rt.DeviceWeight(data, bits, K, scales, group, b)
    dx = rt.DeviceArray.of(x)
    outs = {}
    for tile in ("128x64", "64x128", "128x128", "64x64"):
        monkeypatch.setenv("LEAF_F32_GEMM_TILE", tile)
        dy = rt.DeviceArray((M, N), np.float32)
        rt.linear(dw, dx, M, 32, dy)
        outs[tile] = dy.numpy()
    monkeypatch.delenv("LEAF_F32_GEMM_TILE")
    first = outs["128x64"]
    for tile, y in outs.items():
        assert np.array_equal(y.view(np.uint32), first.view(np.uint32)), tile
    ref = oracle.linear_fp(bits, N, K, group, data, scales, b, x)
    assert np.all(np.abs(first - ref) <= 4e-5 * (1 + np.abs(ref)))


def test_norms_within_tolerance(rt, oracle):
    from leaf_amd.runtime import check, library
    rng = np.random.default_rng(9)
    for width in (2048, 768, 77):
        x = rng.standard_normal((3, width), dtype=np.float32)
        g = (1 + 0.1 * rng.standard_normal(width)).astype(np.float32)
        b = (0.1 * rng.standard_normal(width)).astype(np.float32)
        dx, dg, db = rt.DeviceArray.of(x), rt.DeviceArray.of(g), rt.DeviceArray.of(b)
        dy = rt.DeviceArray((3, width), np.float32)
        for accurate in (0, 1):
            check(library().lh_rmsnorm(dx.ptr, 3, width, dg.ptr, np.float32(1e-5), accurate, dy.ptr, None))
            np.testing.assert_allclose(dy.numpy(), oracle.norm(x, g, None, 1e-5, 0, bool(accurate)), rtol=2e-6,
                                       atol=2e-6)
        check(library().lh_layernorm(dx.ptr, 3, width, dg.ptr, db.ptr, np.float32(1e-5), dy.ptr, None))
        np.testing.assert_allclose(dy.numpy(), oracle.norm(x, g, b, 1e-5, 1, False), rtol=2e-6, atol=2e-6)


def test_rope_kv_matches_reference_formula(rt, oracle):
    from leaf_amd.runtime import check, library
    rng = np.random.default_rng(11)
    heads, kv, dim, rot, M, pos, cap = 4, 2, 64, 32, 3, 5, 16
    qkv = rng.standard_normal((M, (heads + 2 * kv) * dim), dtype=np.float32)
    freq = oracle.rope_frequencies(10000.0, rot)
    cos, sin = oracle.rope_tables(freq, rot, 0, cap)
    dq = rt.DeviceArray.of(qkv)
    dcos, dsin = rt.DeviceArray.of(cos), rt.DeviceArray.of(sin)
    qh = rt.DeviceArray((heads, M, dim), np.float32)
    keys, values = rt.DeviceArray((kv, cap, dim), np.float32).zero(), rt.DeviceArray((kv, cap, dim), np.float32).zero()
    check(library().lh_rope_kv(dq.ptr, M, heads, kv, dim, rot, pos, dcos.ptr, dsin.ptr, qh.ptr, keys.ptr, values.ptr,
                               cap, None))
    half = rot // 2
    q = qkv[:, :heads * dim].reshape(M, heads, dim).transpose(1, 0, 2).copy()
    c, s = cos[pos:pos + M][None, :, :], sin[pos:pos + M][None, :, :]
    a, bb = q[..., :half].copy(), q[..., half:rot].copy()
    q[..., :half] = a * c - bb * s
    q[..., half:rot] = bb * c + a * s
    assert bits_equal(qh.numpy(), q)
    k = qkv[:, heads * dim:(heads + kv) * dim].reshape(M, kv, dim).transpose(1, 0, 2).copy()
    a, bb = k[..., :half].copy(), k[..., half:rot].copy()
    k[..., :half] = a * c - bb * s
    k[..., half:rot] = bb * c + a * s
    assert bits_equal(keys.numpy()[:, pos:pos + M], k)
    v = qkv[:, (heads + kv) * dim:].reshape(M, kv, dim).transpose(1, 0, 2)
    assert bits_equal(values.numpy()[:, pos:pos + M], v)


@pytest.mark.parametrize("tokens,position,window,heads,kv", [
    (1, 640, 0, 14, 2), (1, 4351, 0, 14, 2), (1, 700, 64, 14, 2), (37, 0, 0, 14, 2), (13, 21, 0, 14, 2),
    (16, 5, 7, 14, 2),
    # prefill sizes: the TinyLlama prompt, a chunk after cached keys, a window
    (512, 0, 0, 32, 4), (200, 300, 0, 32, 4), (130, 100, 64, 14, 2)])
def test_attention_matches_oracle(rt, oracle, tokens, position, window, heads, kv):
    from leaf_amd.runtime import check, library
    rng = np.random.default_rng(tokens * 100 + position)
    dim = 64
    total = position + tokens
    cap = total + 70
    q = rng.standard_normal((heads, tokens, dim), dtype=np.float32)
    keys = rng.standard_normal((kv, cap, dim), dtype=np.float32)
    values = rng.standard_normal((kv, cap, dim), dtype=np.float32)
    # cache rows past the visible keys were never written: NaN must not leak
    keys[:, total:] = np.nan
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
    ref = oracle.attention(q, keys, values, mask, heads, kv, tokens, total, cap, dim, float(scale))
    got = out.numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=2e-6)


def test_argmax_first_maximum(rt):
    from leaf_amd.runtime import check, library
    x = np.zeros((3, 50257), np.float32)
    x[0, 7] = x[0, 9000] = 3.0
    x[1] = -1.0
    x[2, 50256] = 1.0
    dx = rt.DeviceArray.of(x)
    out = rt.DeviceArray((3,), np.uint32)
    check(library().lh_argmax(dx.ptr, 3, 50257, out.ptr, None))
    assert out.numpy().tolist() == [7, 0, 50256]
