"""Python binding of libleafhip's C ABI (include/leafhip.h) via ctypes.

``Decoder`` mirrors leaf::runtime::Decoder (engine/include/leaf/runtime/decoder.h:15-50):
constructor policy arguments, ``reset``, ``forward``/``forward_into`` and the
accessors, with errors raised as RuntimeError("Leaf decoder: ...") like the
reference.  ``DeviceArray`` and the kernel helpers expose the kernel-level
entry points for parity tests and microbenchmarks.  No PyTorch involved: the
library owns device memory and streams.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
from pathlib import Path

import numpy as np

PACKAGE = Path(__file__).resolve().parent
LIBRARY = PACKAGE / "libleafhip.so"

LH_OK = 0
STATUS_NAMES = {1: "invalid argument", 2: "artifact", 3: "device", 4: "out of memory", 5: "state", 6: "unsupported"}


class LeafError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class ModelInfo(C.Structure):
    _fields_ = [(name, C.c_uint32) for name in (
        "version", "hidden", "intermediate", "heads", "kv_heads", "layers", "vocab", "max_positions", "eos",
        "head_dim", "sliding_window")] + [("theta", C.c_float), ("epsilon", C.c_float)] + [
        (name, C.c_uint32) for name in ("norm_kind", "activation", "position_kind", "gated", "parallel_residual",
                                        "rotary_dim", "position_offset", "final_norm")] + [
        ("embedding_scale", C.c_float), ("qk_norm", C.c_uint32), ("eos_count", C.c_uint32),
        ("source_bf16_tensors", C.c_uint32), ("quantized_tensors", C.c_uint32),
        ("artifact_bytes", C.c_uint64), ("device_bytes", C.c_uint64)]


class ProfileEntry(C.Structure):
    _fields_ = [("name", C.c_char * 24), ("launches", C.c_uint64), ("milliseconds", C.c_double),
                ("bytes", C.c_double), ("operations", C.c_double)]


class SessionOptions(C.Structure):
    _fields_ = [("max_context", C.c_uint32), ("max_prefill", C.c_uint32), ("numerics", C.c_uint32)]


# Floating-point order of a session or of kernel-level calls (include/leafhip.h).
NUMERICS = {"default": 0, "fast": 1, "reference": 2, "reference-avx2": 3, "reference-vnni": 4}


class Weight(C.Structure):
    _fields_ = [("data", C.c_void_p), ("scales", C.c_void_p), ("bias", C.c_void_p),
                ("rows", C.c_uint32), ("cols", C.c_uint32), ("bits", C.c_uint32), ("group", C.c_uint32)]


_lib = None
_exiting = False


def _mark_exiting() -> None:
    # Objects still alive at interpreter exit are not released through the
    # library: finalizers then run in no fixed order, possibly after the HIP
    # runtime (or a profiler attached to it) has begun shutting down.  Close
    # them explicitly to release device memory earlier.
    global _exiting
    _exiting = True


atexit.register(_mark_exiting)


def library(path: Path | None = None) -> C.CDLL:
    """Load libleafhip.so; fails loudly when the HIP build is missing."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(path or os.environ.get("LEAFHIP_LIBRARY", LIBRARY))
    if not path.exists():
        raise RuntimeError(f"{path} is missing: build it with `python -m leaf_amd.build`")
    lib = C.CDLL(str(path))
    vp, sz, u32, i32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_int
    sigs = {
        "lh_last_error": ([], C.c_char_p), "lh_version": ([], C.c_char_p),
        "lh_context_create": ([i32, C.POINTER(vp)], i32), "lh_context_destroy": ([vp], i32),
        "lh_model_load_file": ([vp, C.c_char_p, u32, u32, C.POINTER(vp)], i32),
        "lh_model_load": ([vp, vp, sz, u32, u32, C.POINTER(vp)], i32),
        "lh_model_get_info": ([vp, C.POINTER(ModelInfo)], i32),
        "lh_artifact_check": ([vp, sz, u32, u32], i32),
        "lh_model_eos_tokens": ([vp, vp, sz, C.POINTER(sz)], i32),
        "lh_model_destroy": ([vp], i32),
        "lh_session_create": ([vp, C.POINTER(SessionOptions), C.POINTER(vp)], i32),
        "lh_session_destroy": ([vp], i32), "lh_reset": ([vp], i32),
        "lh_cache_tokens": ([vp, C.POINTER(sz)], i32),
        "lh_forward": ([vp, vp, sz, i32, vp, sz, vp], i32),
        "lh_generate": ([vp, vp, sz, u32, vp, C.POINTER(sz), vp, vp], i32),
        "lh_session_logits_device": ([vp, C.POINTER(vp), C.POINTER(sz)], i32),
        "lh_session_set_profiling": ([vp, i32], i32),
        "lh_session_profile": ([vp, vp, sz, C.POINTER(sz)], i32),
        "lh_session_status": ([vp, C.POINTER(C.c_int), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                               C.POINTER(C.c_int)], i32),
        "lh_device_alloc": ([sz, C.POINTER(vp)], i32), "lh_device_free": ([vp], i32),
        "lh_copy_to_device": ([vp, vp, sz], i32), "lh_copy_to_host": ([vp, vp, sz], i32),
        "lh_memset_device": ([vp, i32, sz], i32), "lh_synchronize": ([], i32),
        "lh_stream_create": ([C.POINTER(vp)], i32), "lh_stream_destroy": ([vp], i32),
        "lh_stream_synchronize": ([vp], i32),
        "lh_timer_start": ([vp, C.POINTER(vp)], i32), "lh_timer_stop": ([vp, vp, C.POINTER(C.c_double)], i32),
        "lh_stream_begin_capture": ([vp], i32), "lh_stream_end_capture": ([vp, C.POINTER(vp)], i32),
        "lh_graph_launch": ([vp, vp], i32), "lh_graph_destroy": ([vp], i32),
        "lh_quantize_rows_i8": ([vp, sz, sz, vp, vp, vp], i32),
        "lh_linear": ([C.POINTER(Weight), vp, sz, u32, vp, vp, vp], i32),
        "lh_linear_q": ([C.POINTER(Weight), vp, vp, sz, vp, vp, vp], i32),
        "lh_linear_noalloc": ([C.POINTER(Weight), vp, sz, u32, vp, vp, vp], i32),
        "lh_gemv_f32": ([C.POINTER(Weight), vp, sz, vp, vp], i32),
        "lh_gemv_bf16": ([C.POINTER(Weight), vp, sz, vp, vp], i32),
        "lh_gemv_w8a32": ([C.POINTER(Weight), vp, sz, vp, vp], i32),
        "lh_gemv_w4a32": ([C.POINTER(Weight), vp, sz, vp, vp], i32),
        "lh_gemv_w8a8": ([C.POINTER(Weight), vp, sz, vp, vp, vp], i32),
        "lh_gemv_w4a8": ([C.POINTER(Weight), vp, sz, vp, vp, vp], i32),
        "lh_gemm_w8a8": ([C.POINTER(Weight), vp, sz, vp, vp, vp], i32),
        "lh_gemm_f32": ([C.POINTER(Weight), vp, sz, vp, vp], i32),
        "lh_rmsnorm": ([vp, sz, sz, vp, C.c_float, i32, vp, vp], i32),
        "lh_layernorm": ([vp, sz, sz, vp, vp, C.c_float, vp, vp], i32),
        "lh_rope_kv": ([vp, sz, u32, u32, u32, u32, sz, vp, vp, vp, vp, vp, sz, vp], i32),
        "lh_attention": ([vp, vp, vp, sz, u32, u32, u32, sz, sz, u32, vp, vp], i32),
        "lh_silu_gate": ([vp, sz, sz, vp, vp], i32),
        "lh_activation": ([vp, sz, u32, vp, vp], i32),
        "lh_argmax": ([vp, sz, sz, vp, vp], i32),
        "lh_set_kernel_numerics": ([u32], i32),
        "lh_expf": ([vp, sz, vp, vp], i32),
        "lh_sequential_sum": ([vp, sz, sz, vp, vp, u32, vp], i32),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = args, res
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != LH_OK:
        message = library().lh_last_error().decode()
        raise LeafError(status, message or f"leafhip error {status} ({STATUS_NAMES.get(status, '?')})")


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- devices ---
class DeviceArray:
    """A device allocation holding one numpy-shaped array."""

    def __init__(self, shape, dtype):
        self.shape = tuple(np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        check(library().lh_device_alloc(max(self.nbytes, 1), C.byref(p)))
        self.ptr = p.value

    @classmethod
    def of(cls, array: np.ndarray) -> "DeviceArray":
        array = np.ascontiguousarray(array)
        d = cls(array.shape, array.dtype)
        check(library().lh_copy_to_device(d.ptr, _ptr(array), array.nbytes))
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(library().lh_copy_to_host(_ptr(out), self.ptr, self.nbytes))
        return out

    def zero(self) -> "DeviceArray":
        check(library().lh_memset_device(self.ptr, 0, self.nbytes))
        return self

    def free(self):
        if getattr(self, "ptr", None):
            library().lh_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        if not _exiting:
            self.free()


class DeviceWeight:
    """A LEAFDC matrix (payload, optional scales and bias) resident on the device."""

    def __init__(self, data: np.ndarray, bits: int, cols: int, scales: np.ndarray | None = None,
                 group: int = 0, bias: np.ndarray | None = None):
        rows = data.shape[0]
        self.data = DeviceArray.of(data)
        self.scales = DeviceArray.of(np.ascontiguousarray(scales, np.float32)) if scales is not None else None
        self.bias = DeviceArray.of(np.ascontiguousarray(bias, np.float32)) if bias is not None else None
        self.desc = Weight(self.data.ptr, self.scales.ptr if self.scales else None,
                           self.bias.ptr if self.bias else None, rows, cols, bits,
                           group if bits in (8, 4) else 0)
        self.rows, self.cols, self.bits, self.group = rows, cols, bits, group


def synchronize():
    check(library().lh_synchronize())


# ----------------------------------------------------------------- decoder ---
class Decoder:
    """leaf::runtime::Decoder on one MI355X (engine/include/leaf/runtime/decoder.h:15-50)."""

    def __init__(self, artifact: str | os.PathLike, activation_bits: int = 32, fp32_math: str = "fast",
                 device: int = 0, max_context: int = 0, max_prefill: int = 0, numerics: str = "default"):
        lib = library()
        if fp32_math not in ("fast", "accurate"):
            raise RuntimeError("Leaf decoder: invalid FP32 math policy")
        self._ctx = C.c_void_p()
        check(lib.lh_context_create(device, C.byref(self._ctx)))
        self._model = C.c_void_p()
        self._session = C.c_void_p()
        try:
            check(lib.lh_model_load_file(self._ctx, str(artifact).encode(), activation_bits,
                                         1 if fp32_math == "accurate" else 0, C.byref(self._model)))
            options = SessionOptions(max_context, max_prefill, NUMERICS[numerics])
            check(lib.lh_session_create(self._model, C.byref(options), C.byref(self._session)))
        except Exception:
            self.close()
            raise
        self.info = ModelInfo()
        check(lib.lh_model_get_info(self._model, C.byref(self.info)))
        n = C.c_size_t()
        check(lib.lh_model_eos_tokens(self._model, None, 0, C.byref(n)))
        eos = np.empty(max(n.value, 1), np.uint32)
        check(lib.lh_model_eos_tokens(self._model, _ptr(eos), eos.size, C.byref(n)))
        self._eos = set(eos[:n.value].tolist())
        self.activation_bits = activation_bits
        self.fp32_math = fp32_math

    def close(self):
        lib = library()
        if getattr(self, "_session", None) and self._session.value:
            lib.lh_session_destroy(self._session)
            self._session = C.c_void_p()
        if getattr(self, "_model", None) and self._model.value:
            lib.lh_model_destroy(self._model)
            self._model = C.c_void_p()
        if getattr(self, "_ctx", None) and self._ctx.value:
            lib.lh_context_destroy(self._ctx)
            self._ctx = C.c_void_p()

    def __del__(self):
        if not _exiting:
            self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- reference API ---------------------------------------------------------
    def reset(self) -> None:
        check(library().lh_reset(self._session))

    def forward(self, tokens, all_logits: bool = False) -> np.ndarray:
        ids = np.ascontiguousarray(tokens, np.uint32)
        rows = len(ids) if all_logits else 1
        out = np.empty(max(rows, 1) * self.vocabulary_size, np.float32)
        self.last_argmax = C.c_uint32()
        check(library().lh_forward(self._session, _ptr(ids), len(ids), int(all_logits), _ptr(out), out.size,
                                   C.byref(self.last_argmax)))
        return out.reshape(rows, -1) if all_logits else out

    def forward_into(self, tokens, logits: np.ndarray | None, all_logits: bool = False) -> int:
        """Writes logits into a caller-owned float32 buffer; returns the argmax of the last row."""
        ids = np.ascontiguousarray(tokens, np.uint32)
        argmax = C.c_uint32()
        check(library().lh_forward(self._session, _ptr(ids), len(ids), int(all_logits),
                                   _ptr(logits) if logits is not None else None,
                                   0 if logits is None else logits.size, C.byref(argmax)))
        return argmax.value

    def generate(self, prompt, limit: int):
        """Greedy continuation (main_decoder.cpp:95-113); returns (tokens, prefill_ms, decode_ms list)."""
        ids = np.ascontiguousarray(prompt, np.uint32)
        tokens = np.empty(max(limit, 1), np.uint32)
        produced = C.c_size_t()
        prefill = C.c_double()
        decode = np.zeros(max(limit, 1), np.float64)
        check(library().lh_generate(self._session, _ptr(ids), len(ids), limit, _ptr(tokens), C.byref(produced),
                                    C.byref(prefill), _ptr(decode)))
        n = produced.value
        return tokens[:n].tolist(), prefill.value, decode[:max(n - 1, 0)].tolist()

    def set_profiling(self, enable: bool) -> None:
        check(library().lh_session_set_profiling(self._session, int(enable)))

    def profile(self) -> dict:
        """Per-kernel-class device time since the last call: {name: {launches, ms, bytes, ops}}."""
        entries = (ProfileEntry * 16)()
        n = C.c_size_t()
        check(library().lh_session_profile(self._session, C.cast(entries, C.c_void_p), 16, C.byref(n)))
        return {e.name.decode(): {"launches": e.launches, "ms": e.milliseconds, "bytes": e.bytes,
                                  "ops": e.operations} for e in entries[:n.value]}

    def status(self) -> dict:
        """The session's numerics and the persistent decode step's record since the
        session began: tokens it produced, steps re-run on the memory exchange path
        after an XCD mismatch, and whether the XCD-local exchange is still on."""
        ref, tokens, reruns, local = C.c_int(), C.c_uint64(), C.c_uint64(), C.c_int()
        check(library().lh_session_status(self._session, C.byref(ref), C.byref(tokens), C.byref(reruns),
                                          C.byref(local)))
        return {"reference_order": bool(ref.value), "step_tokens": tokens.value,
                "step_memory_reruns": reruns.value, "xcd_local": bool(local.value)}

    @property
    def vocabulary_size(self) -> int:
        return self.info.vocab

    def eos_token(self) -> int:
        return self.info.eos

    def is_eos_token(self, token: int) -> bool:
        return token in self._eos

    def cache_tokens(self) -> int:
        n = C.c_size_t()
        check(library().lh_cache_tokens(self._session, C.byref(n)))
        return n.value

    def weight_bytes(self) -> int:
        return self.info.artifact_bytes

    def source_bf16_tensors(self) -> int:
        return self.info.source_bf16_tensors

    def uses_accurate_fp32(self) -> bool:
        return self.fp32_math == "accurate"


# ------------------------------------------------------------ kernel calls ---
def linear(weight: DeviceWeight, x: DeviceArray, tokens: int, activation_bits: int, y: DeviceArray,
           acc: DeviceArray | None = None, stream=None) -> None:
    check(library().lh_linear(C.byref(weight.desc), x.ptr, tokens, activation_bits, y.ptr,
                              acc.ptr if acc is not None else None, stream))


def linear_q(weight: DeviceWeight, q: DeviceArray, scales: DeviceArray, tokens: int, y: DeviceArray,
             acc: DeviceArray | None = None, stream=None) -> None:
    check(library().lh_linear_q(C.byref(weight.desc), q.ptr, scales.ptr, tokens, y.ptr,
                                acc.ptr if acc is not None else None, stream))


def artifact_check(artifact: bytes, activation_bits: int = 32, fp32_math: str = "fast") -> str | None:
    """Validates LEAFDC bytes on the host: None when accepted, else the error text."""
    lib = library()
    buf = C.create_string_buffer(bytes(artifact), len(artifact))
    status = lib.lh_artifact_check(buf, len(artifact), activation_bits, 1 if fp32_math == "accurate" else 0)
    return None if status == LH_OK else lib.lh_last_error().decode()


def set_kernel_numerics(numerics: str) -> None:
    """Numerics of this thread's kernel-level calls: "fast", "reference", "reference-avx2" or "reference-vnni"."""
    check(library().lh_set_kernel_numerics(NUMERICS[numerics]))


def expf(x: DeviceArray, y: DeviceArray, stream=None) -> None:
    check(library().lh_expf(x.ptr, int(np.prod(x.shape)), y.ptr, stream))


def sequential_sum(x: DeviceArray, n: int, count: int, sums: DeviceArray, cycles: DeviceArray | None = None,
                   method: int = 0, stream=None) -> None:
    """sums[i] = the float32 sum of row i in column order (lh_sequential_sum)."""
    check(library().lh_sequential_sum(x.ptr, n, count, sums.ptr, cycles.ptr if cycles is not None else None,
                                      method, stream))


def quantize_rows(x: DeviceArray, rows: int, cols: int, q: DeviceArray, scales: DeviceArray, stream=None) -> None:
    check(library().lh_quantize_rows_i8(x.ptr, rows, cols, q.ptr, scales.ptr, stream))


class Stream:
    """A library-created HIP stream (needed for graph capture)."""

    def __init__(self):
        self.handle = C.c_void_p()
        check(library().lh_stream_create(C.byref(self.handle)))

    def synchronize(self):
        check(library().lh_stream_synchronize(self.handle))

    def close(self):
        if getattr(self, "handle", None) and self.handle.value:
            library().lh_stream_destroy(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        if not _exiting:
            self.close()


class Graph:
    """Work captured from a stream and replayed as one HIP graph."""

    def __init__(self, stream: Stream, record):
        check(library().lh_stream_begin_capture(stream.handle))
        try:
            record()
        finally:
            self.handle = C.c_void_p()
            status = library().lh_stream_end_capture(stream.handle, C.byref(self.handle))
        check(status)
        self.stream = stream

    def launch(self):
        check(library().lh_graph_launch(self.handle, self.stream.handle))

    def close(self):
        if getattr(self, "handle", None) and self.handle.value:
            library().lh_graph_destroy(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        if not _exiting:
            self.close()


class Timer:
    """HIP-event timing of work on a stream (None = default stream)."""

    def __init__(self, stream=None):
        self.stream = stream
        self._t = C.c_void_p()
        check(library().lh_timer_start(stream, C.byref(self._t)))

    def stop(self) -> float:
        ms = C.c_double()
        check(library().lh_timer_stop(self._t, self.stream, C.byref(ms)))
        return ms.value
