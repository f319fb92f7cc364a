"""ctypes bindings for the CPU oracle (liboracle.so) and the reference harness.

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and bench.py's
CPU-baseline leg.  ``reference()`` returns the harness compiled from the
reference sources (oracle/_ref/libleafref.so) or None where it was not built.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_SO = HERE / "_ref" / "libleafref.so"
REF_BIN = HERE / "_ref" / "leaf_decoder"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i16p = np.ctypeslib.ndpointer(np.int16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_sz = C.c_size_t

_oracle = None
_reference = None


def build(quiet: bool = True) -> None:
    """Compile liboracle.so (and the reference builds when the checkout exists)."""
    subprocess.run(["make", "-C", str(HERE), "-s"], check=True,
                   stdout=subprocess.DEVNULL if quiet else None)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Oracle:
    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            build()
        lib = C.CDLL(str(path))
        self.lib = lib
        lib.oracle_quantize_rows.argtypes = [_f32p, _sz, _sz, _i8p, _f32p]
        lib.oracle_set_vnni_policy.argtypes = [C.c_int]
        lib.oracle_set_norm_order.argtypes = [C.c_int]
        lib.oracle_int_accumulators.argtypes = [C.c_uint, _sz, _sz, _sz, C.c_void_p, _i8p, _sz, _i32p]
        for name in ("oracle_linear_int", "oracle_linear_fp"):
            getattr(lib, name).argtypes = [C.c_uint, _sz, _sz, _sz, C.c_void_p, C.c_void_p, C.c_void_p,
                                           _f32p, _sz, _f32p]
        lib.oracle_linear_int_q.argtypes = [C.c_uint, _sz, _sz, _sz, C.c_void_p, C.c_void_p, C.c_void_p,
                                            _i8p, _f32p, _sz, _f32p]
        lib.oracle_linear_accurate.argtypes = [C.c_uint, _sz, _sz, C.c_void_p, C.c_void_p, _f32p, _sz, _f32p]
        lib.oracle_norm.argtypes = [_f32p, _sz, _sz, _f32p, C.c_void_p, C.c_float, C.c_uint, C.c_int, _f32p]
        lib.oracle_rope_frequencies.argtypes = [C.c_float, C.c_uint, _f32p]
        lib.oracle_rope_tables.argtypes = [_f32p, C.c_uint, _sz, _sz, _f32p, _f32p]
        lib.oracle_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz, _sz,
                                         C.c_float]
        lib.oracle_activate.argtypes = [C.c_uint, C.c_float]
        lib.oracle_activate.restype = C.c_float
        lib.oracle_activation.argtypes = [_f32p, _sz, _sz, C.c_int, C.c_uint, _f32p]
        lib.oracle_expf.argtypes = [_f32p, _sz, _f32p]
        lib.oracle_quantize_weights.argtypes = [_f32p, _sz, _sz, C.c_uint, _sz, _u8p, _f32p]
        lib.oracle_decoder_open.argtypes = [C.c_char_p, C.c_uint, C.c_int, C.c_char_p, _sz]
        lib.oracle_decoder_open.restype = C.c_void_p
        lib.oracle_decoder_close.argtypes = [C.c_void_p]
        lib.oracle_decoder_reset.argtypes = [C.c_void_p]
        lib.oracle_decoder_forward.argtypes = [C.c_void_p, _u32p, _sz, C.c_int, _f32p, C.c_char_p, _sz]
        lib.oracle_decoder_cache_tokens.argtypes = [C.c_void_p]
        lib.oracle_decoder_cache_tokens.restype = _sz
        lib.oracle_decoder_vocab.argtypes = [C.c_void_p]
        lib.oracle_decoder_vocab.restype = C.c_uint32
        lib.oracle_decoder_generate.argtypes = [C.c_void_p, _u32p, _sz, C.c_uint, _u32p, C.POINTER(_sz),
                                                C.c_char_p, _sz]

    # -- kernels ------------------------------------------------------------
    def set_norm_order(self, order: int) -> None:
        """0: sequential square sums (the reference); 1: pairwise."""
        self.lib.oracle_set_norm_order(order)

    def set_vnni_policy(self, policy: int) -> None:
        """0: fused grouped-W8A8 epilogue (default), 1: VNNI tile form, -1: this CPU's choice."""
        self.lib.oracle_set_vnni_policy(policy)

    def quantize_rows(self, x):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        q, s = np.empty((M, K), np.int8), np.empty(M, np.float32)
        self.lib.oracle_quantize_rows(x, M, K, q, s)
        return q, s

    def int_accumulators(self, bits, rows, cols, group, data, q):
        q = np.ascontiguousarray(q, np.int8)
        acc = np.empty((q.shape[0], rows, cols // group), np.int32)
        self.lib.oracle_int_accumulators(bits, rows, cols, group, _ptr(data), q, q.shape[0], acc)
        return acc

    def linear_int(self, bits, rows, cols, group, data, scales, bias, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty((x.shape[0], rows), np.float32)
        self.lib.oracle_linear_int(bits, rows, cols, group, _ptr(data), _ptr(scales), _ptr(bias), x, x.shape[0], y)
        return y

    def linear_int_q(self, bits, rows, cols, group, data, scales, bias, q, qscale):
        y = np.empty((q.shape[0], rows), np.float32)
        self.lib.oracle_linear_int_q(bits, rows, cols, group, _ptr(data), _ptr(scales), _ptr(bias),
                                     np.ascontiguousarray(q, np.int8), np.ascontiguousarray(qscale, np.float32),
                                     q.shape[0], y)
        return y

    def linear_fp(self, bits, rows, cols, group, data, scales, bias, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty((x.shape[0], rows), np.float32)
        self.lib.oracle_linear_fp(bits, rows, cols, group, _ptr(data), _ptr(scales), _ptr(bias), x, x.shape[0], y)
        return y

    def linear_accurate(self, bits, rows, cols, data, bias, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty((x.shape[0], rows), np.float32)
        self.lib.oracle_linear_accurate(bits, rows, cols, _ptr(data), _ptr(bias), x, x.shape[0], y)
        return y

    def norm(self, x, gamma, beta, eps, kind, accurate=False):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.lib.oracle_norm(x, x.shape[0], x.shape[1], np.ascontiguousarray(gamma, np.float32), _ptr(beta),
                             eps, kind, int(accurate), y)
        return y

    def rope_frequencies(self, theta, rotary_dim):
        f = np.empty(rotary_dim // 2, np.float32)
        self.lib.oracle_rope_frequencies(theta, rotary_dim, f)
        return f

    def rope_tables(self, freq, rotary_dim, position, tokens):
        c = np.empty((tokens, rotary_dim // 2), np.float32)
        s = np.empty_like(c)
        self.lib.oracle_rope_tables(np.ascontiguousarray(freq, np.float32), rotary_dim, position, tokens, c, s)
        return c, s

    def attention(self, q_heads, keys, values, mask, heads, kv_heads, tokens, total, stride, dim, scale):
        out = np.zeros((tokens, heads * dim), np.float32)
        self.lib.oracle_attention(np.ascontiguousarray(q_heads, np.float32), np.ascontiguousarray(keys, np.float32),
                                  np.ascontiguousarray(values, np.float32), np.ascontiguousarray(mask, np.float32),
                                  out, heads, kv_heads, tokens, total, stride, dim, scale)
        return out

    def activate(self, code, x):
        return np.array([self.lib.oracle_activate(code, float(v)) for v in np.asarray(x, np.float32).ravel()],
                        np.float32).reshape(np.shape(x))

    def activation(self, gate_up, tokens, width, gated, code):
        gate_up = np.ascontiguousarray(gate_up, np.float32)
        act = np.empty((tokens, width), np.float32)
        self.lib.oracle_activation(gate_up, tokens, width, int(gated), code, act)
        return act

    def expf(self, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.lib.oracle_expf(x, x.size, y)
        return y

    def quantize_weights(self, w, bits, group):
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = w.shape
        packed = np.empty((rows, cols if bits == 8 else cols // 2), np.uint8)
        scales = np.empty((rows, cols // group), np.float32)
        self.lib.oracle_quantize_weights(w, rows, cols, bits, group, packed, scales)
        return (packed.view(np.int8) if bits == 8 else packed), scales

    def decoder(self, path, activation_bits=32, accurate=False):
        return OracleDecoder(self, path, activation_bits, accurate)


class OracleDecoder:
    def __init__(self, oracle: Oracle, path, activation_bits=32, accurate=False):
        self.lib = oracle.lib
        err = C.create_string_buffer(512)
        self.handle = self.lib.oracle_decoder_open(str(path).encode(), activation_bits, int(accurate), err, 512)
        if not self.handle:
            raise RuntimeError(err.value.decode())
        self.vocab = self.lib.oracle_decoder_vocab(self.handle)

    def close(self):
        if self.handle:
            self.lib.oracle_decoder_close(self.handle)
            self.handle = None

    __del__ = close

    def reset(self):
        self.lib.oracle_decoder_reset(self.handle)

    @property
    def cache_tokens(self):
        return self.lib.oracle_decoder_cache_tokens(self.handle)

    def forward(self, ids, all_logits=False):
        ids = np.ascontiguousarray(ids, np.uint32)
        out = np.empty((len(ids) if all_logits else 1) * self.vocab, np.float32)
        err = C.create_string_buffer(512)
        if self.lib.oracle_decoder_forward(self.handle, ids, len(ids), int(all_logits), out, err, 512):
            raise RuntimeError(err.value.decode())
        return out.reshape(-1, self.vocab) if all_logits else out

    def generate(self, prompt, limit):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(max(limit, 1), np.uint32)
        n = _sz(0)
        err = C.create_string_buffer(512)
        if self.lib.oracle_decoder_generate(self.handle, prompt, len(prompt), limit, out, C.byref(n), err, 512):
            raise RuntimeError(err.value.decode())
        return out[:n.value].tolist()


class Reference:
    """Harness around the real reference kernels (oracle/ref_harness.cpp)."""

    def __init__(self, path: Path = REF_SO):
        lib = C.CDLL(str(path))
        self.lib = lib
        lib.ref_quantize_rows.argtypes = [_f32p, _sz, _sz, _i16p, _f32p]
        lib.ref_linear_int.argtypes = [C.c_uint, _sz, _sz, _sz, C.c_void_p, C.c_void_p, C.c_void_p, _f32p, _sz,
                                       C.c_int, _f32p]
        lib.ref_linear_fp.argtypes = [C.c_uint, _sz, _sz, _sz, C.c_void_p, C.c_void_p, C.c_void_p, _f32p, _sz, _f32p]
        lib.ref_linear_accurate.argtypes = [C.c_uint, _sz, _sz, C.c_void_p, C.c_void_p, _f32p, _sz, _f32p]
        lib.ref_norm.argtypes = [_f32p, _sz, _sz, _f32p, C.c_void_p, C.c_float, C.c_uint, C.c_int, _f32p]
        lib.ref_decoder_greedy.argtypes = [C.c_char_p, C.c_uint, C.c_uint, C.c_int, _u32p, _sz, C.c_uint, _u32p,
                                           C.POINTER(C.c_uint), _sz, _f32p, C.c_char_p, _sz]
        lib.ref_decoder_greedy.restype = C.c_int
        self.features = lib.ref_cpu_features()

    def greedy(self, path, prompt, limit, activation_bits=32, accurate=False, keep=(0,), threads=8, vocab=None):
        """The real Decoder's greedy run: (tokens, logits of the forwards in `keep`)."""
        prompt = np.ascontiguousarray(prompt, np.uint32)
        keep_arr = (C.c_uint * len(keep))(*keep)
        tokens = np.empty(max(limit, 1), np.uint32)
        logits = np.empty((len(keep), vocab), np.float32)
        err = C.create_string_buffer(512)
        n = self.lib.ref_decoder_greedy(str(path).encode(), threads, activation_bits, int(accurate), prompt,
                                        len(prompt), limit, tokens, keep_arr, len(keep), logits, err, 512)
        if n < 0:
            raise RuntimeError(err.value.decode())
        return tokens[:n], logits

    def quantize_rows(self, x):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        q, s = np.empty((M, K), np.int16), np.empty(M, np.float32)
        self.lib.ref_quantize_rows(x, M, K, q, s)
        return q, s

    def linear_int(self, bits, rows, cols, group, data, scales, bias, x, mode=0):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty((x.shape[0], rows), np.float32)
        rc = self.lib.ref_linear_int(bits, rows, cols, group, _ptr(data), _ptr(scales), _ptr(bias), x,
                                     x.shape[0], mode, y)
        if rc < 0:
            raise RuntimeError("reference integer path unavailable on this CPU")
        return y

    def linear_fp(self, bits, rows, cols, group, data, scales, bias, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty((x.shape[0], rows), np.float32)
        if self.lib.ref_linear_fp(bits, rows, cols, group, _ptr(data), _ptr(scales), _ptr(bias), x, x.shape[0], y):
            raise RuntimeError("reference AVX2 path unavailable on this CPU")
        return y

    def linear_accurate(self, bits, rows, cols, data, bias, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty((x.shape[0], rows), np.float32)
        if self.lib.ref_linear_accurate(bits, rows, cols, _ptr(data), _ptr(bias), x, x.shape[0], y):
            raise RuntimeError("reference AVX2 path unavailable on this CPU")
        return y

    def norm(self, x, gamma, beta, eps, kind, accurate=False):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.lib.ref_norm(x, x.shape[0], x.shape[1], np.ascontiguousarray(gamma, np.float32), _ptr(beta),
                          eps, kind, int(accurate), y)
        return y


def oracle() -> Oracle:
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle


def reference() -> Reference | None:
    global _reference
    if _reference is None and REF_SO.exists():
        _reference = Reference()
    return _reference
