"""The LEAFDC validator against the real reference loader, on mutated artifacts.

Valid artifacts of every edition (LEAFDC02 W8A8 and INT4, 03 sliding window,
04 multi-EOS, 05 BF16 I/O, 06 BF16 matrices, 07 Q/K norm with static RoPE
frequencies, and a SmoothQuant-calibrated W8A8) are mutated one field at a
time: every header field, the magic and version, truncations at many lengths,
the v7 operator block, the EOS list, tensor descriptors (rank, shape, bits,
group, offsets, sizes, scale metadata, names), quantization scales and
calibrated input scales.  Each mutant goes to the reference build
(oracle/_ref/leaf_decoder, verify mode on one token: Decoder::Impl::Impl,
engine/src/decoder.cpp:787-933, and the first use of every tensor) and to
lh_artifact_check.  Both must accept it, or both reject it with the same
message.  Runs on the CPU; skipped where the reference build is absent.
"""
from __future__ import annotations

import concurrent.futures
import dataclasses
import resource
import struct
import subprocess
import tempfile
from pathlib import Path

import numpy as np
import pytest

from leaf_amd import models
from leaf_amd.artifact import DESCRIPTOR, HEADER, write_artifact, write_tokens

ROOT = Path(__file__).resolve().parents[1]
REFERENCE = ROOT / "oracle" / "_ref" / "leaf_decoder"

pytestmark = pytest.mark.skipif(not REFERENCE.exists(), reason="reference build (oracle/_ref) not present")

HEADER_FIELDS = ["version", "count", "base", "hidden", "intermediate", "heads", "kv_heads", "layers", "vocab",
                 "max_positions", "eos", "head_dim", "sliding_window", "theta", "epsilon", "norm_kind", "activation",
                 "position_kind", "gated", "parallel", "rotary_dim", "position_offset", "final_norm",
                 "embedding_scale"]


def header_offsets():
    """(name, byte offset, struct format) of every field after the magic."""
    out, at = [], 8
    for name in HEADER_FIELDS:
        fmt = "<Q" if name == "base" else "<f" if name in ("theta", "epsilon", "embedding_scale") else "<I"
        out.append((name, at, fmt))
        at += struct.calcsize(fmt)
    assert at == HEADER.size
    return out


def bases():
    tiny = models.PRESETS["tinyllama"](reduced=True)
    qwen = models.PRESETS["qwen"](reduced=True)
    return {
        "w8a8": (tiny, 8),
        "int4": (dataclasses.replace(qwen, bias_std=0.05), 32),
        "window": (dataclasses.replace(tiny, sliding_window=8), 8),
        "eos": (dataclasses.replace(tiny, eos=5, eos_tokens=(5, 9, 11)), 8),
        "bf16io": (dataclasses.replace(tiny, bits=32, bf16_io=True, keep_fp32=frozenset()), 32),
        "bf16": (models.PRESETS["smollm2"](reduced=True), 32),
        "v7": (dataclasses.replace(tiny, bits=32, keep_fp32=frozenset(), qk_norm=1,
                                   rope_frequencies=tuple(float(f) for f in 0.5 ** np.arange(tiny.head_dim // 2))),
               32),
        "smooth": (dataclasses.replace(tiny, smoothquant_alpha=0.5), 8),
    }


@dataclasses.dataclass
class Layout:
    meta_end: int          # end of the version block and EOS list
    base: int
    descriptors: list      # (name, name_offset, fields_offset, rows, cols, bits, group, offset, size, soff, scount)


def layout(blob: bytes, version: int) -> Layout:
    (_, _, count, base, *_rest) = HEADER.unpack_from(blob, 0)
    at = HEADER.size
    if version == 7:
        _, _, n = struct.unpack_from("<3I", blob, at)
        at += 12 + 4 * n
    if version >= 4:
        (n,) = struct.unpack_from("<I", blob, at)
        at += 4 + 4 * n
    meta_end = at
    descriptors = []
    for _ in range(count):
        (length,) = struct.unpack_from("<I", blob, at)
        name = blob[at + 4:at + 4 + length].decode()
        fields = at + 4 + length
        rank, rows, cols, bits, group, off, size, soff, scount = DESCRIPTOR.unpack_from(blob, fields)
        descriptors.append((name, at, fields, rows, cols, bits, group, off, size, soff, scount))
        at = fields + DESCRIPTOR.size
    return Layout(meta_end, base, descriptors)


def put(blob: bytearray, at: int, fmt: str, value) -> bytearray:
    out = bytearray(blob)
    struct.pack_into(fmt, out, at, value)
    return out


def mutants(blob: bytes, version: int, full: bool):
    """(label, mutated bytes) pairs."""
    lay = layout(blob, version)
    out = []
    if full:
        for name, at, fmt in header_offsets():
            (orig,) = struct.unpack_from(fmt, blob, at)
            if fmt == "<f":
                values = [0.0, -1.0, float("nan"), float("inf"), orig * 2]
            elif fmt == "<Q":
                values = [0, 1, orig + 1, orig + 64, len(blob) + 64, 1 << 40]
            else:
                values = sorted({0, 1, 2, (orig + 1) & 0xFFFFFFFF, max(orig - 1, 0), 0xFFFFFFFF, 0x80000000})
            out += [(f"header {name}={v}", put(blob, at, fmt, v)) for v in values]
        for magic in (b"LEAFDC02", b"LEAFDC03", b"LEAFDC04", b"LEAFDC05", b"LEAFDC06", b"LEAFDC07", b"LEAFDC08",
                      b"XEAFDC02"):
            mutated = bytearray(blob)
            mutated[:8] = magic
            out.append((f"magic {magic!r}", mutated))
        cuts = [5, 8, 11, 12, 20, 30, 60, 107, 108, 110, lay.meta_end + 2, (lay.meta_end + lay.base) // 2,
                lay.base - 1, lay.base, lay.base + 100, len(blob) - 1]
        out += [(f"truncated at {n}", blob[:n]) for n in sorted(set(c for c in cuts if 0 < c < len(blob)))]
    if version == 7:
        at = HEADER.size
        for v in (1, 5, 6, 7):
            out.append((f"v7 storage={v}", put(blob, at, "<I", v)))
        out.append(("v7 qk=2", put(blob, at + 4, "<I", 2)))
        out.append(("v7 qk=0 and no frequencies", put(put(blob, at + 4, "<I", 0), at + 8, "<I", 0)))
        (n,) = struct.unpack_from("<I", blob, at + 8)
        for v in (n + 1, n - 1, 1 << 30):
            out.append((f"v7 frequencies={v}", put(blob, at + 8, "<I", v)))
        for f in (0.0, float("nan"), 2.0, -1.0):
            out.append((f"v7 frequency[0]={f}", put(blob, at + 12, "<f", f)))
    if version >= 4:
        eos_at = lay.meta_end - 4 * struct.unpack_from("<I", blob, HEADER.size + (12 + 4 * struct.unpack_from(
            "<I", blob, HEADER.size + 8)[0] if version == 7 else 0))[0] - 4
        (n,) = struct.unpack_from("<I", blob, eos_at)
        for v in (0, 1, 2, 1025, 1 << 30):
            out.append((f"eos count={v}", put(blob, eos_at, "<I", v)))
        if n >= 1:
            vocab = HEADER.unpack_from(blob, 0)[9]
            out.append(("eos token out of range", put(blob, eos_at + 4, "<I", vocab)))
        if n >= 2:
            (second,) = struct.unpack_from("<I", blob, eos_at + 8)
            out.append(("eos token duplicate", put(blob, eos_at + 4, "<I", second)))
        out.append(("eos primary mismatch", put(blob, 52, "<I", 3)))
    picks = [lay.descriptors[0], lay.descriptors[len(lay.descriptors) // 2], lay.descriptors[-1]]
    quantized = [d for d in lay.descriptors if d[5] in (8, 4)]
    if quantized:
        picks.append(quantized[0])
    scales_in = [d for d in lay.descriptors if d[0].endswith(".input_scale")]
    if scales_in:
        picks.append(scales_in[0])
    for d in picks:
        name, name_at, f, rows, cols, bits, group, off, size, soff, scount = d
        label = f"tensor {name}"
        for i, v in ((0, 1), (0, 3), (1, 0), (1, rows + 1), (2, 0), (2, cols + 1), (3, 16), (3, 7), (3, 4), (3, 8),
                     (3, 32), (4, 0), (4, group + 1), (4, 2 * group if group else 64)):
            out.append((f"{label} field{i}={v}", put(blob, f + 4 * i, "<I", v)))
        for i, v in ((0, off + 1), (0, off + 64), (0, 1 << 40), (1, size + 1), (1, max(size - 1, 0)),
                     (2, soff + 4), (2, soff + 64), (2, 1 << 40), (3, scount + 1), (3, 0)):
            out.append((f"{label} q{i}={v}", put(blob, f + 20 + 8 * i, "<Q", v)))
        out.append((f"{label} name length huge", put(blob, name_at, "<I", 1 << 30)))
        other = lay.descriptors[0][0] if name != lay.descriptors[0][0] else lay.descriptors[1][0]
        if len(other) == len(name):
            mutated = bytearray(blob)
            mutated[name_at + 4:name_at + 4 + len(name)] = other.encode()
            out.append((f"{label} renamed to {other}", mutated))
        mutated = bytearray(blob)
        mutated[name_at + 4] = ord("X")
        out.append((f"{label} renamed", mutated))
        if bits in (8, 4) and scount:
            for v in (0.0, float("nan"), -1.0, float("inf")):
                out.append((f"{label} scale[0]={v}", put(blob, lay.base + soff, "<f", v)))
        if name.endswith(".input_scale"):
            for v in (0.0, float("nan"), -2.0):
                out.append((f"{label} value[0]={v}", put(blob, lay.base + off, "<f", v)))
    return out


def with_extra_tensor(blob: bytes, version: int, name: str, rows: int, cols: int, bits: int,
                      size: int = 0) -> bytes:
    """The artifact with one more tensor descriptor (rank 2, no group or scales,
    data at offset 0) after the others; the payload moves with the data base."""
    lay = layout(blob, version)
    last = lay.descriptors[-1]
    end = last[2] + DESCRIPTOR.size
    entry = struct.pack("<I", len(name)) + name.encode() + DESCRIPTOR.pack(2, rows, cols, bits, 0, 0, size, 0, 0)
    base = (end + len(entry) + 63) & ~63
    out = bytearray(blob[:end] + entry)
    out += bytes(base - len(out))
    out += blob[lay.base:]
    (count,) = struct.unpack_from("<I", blob, 12)
    struct.pack_into("<I", out, 12, count + 1)
    struct.pack_into("<Q", out, 16, base)
    return bytes(out)


def reference_verdict(tmp: Path, blob: bytes, bits: int, tag: str = "m") -> str | None:
    """None when the reference loads the artifact and runs a one-token forward,
    else its error line (kept verbatim: messages may end in a space)."""
    art, req = tmp / f"{tag}.leaf", tmp / "req.bin"
    art.write_bytes(blob)
    if not req.exists():
        write_tokens(req, [[0]])
    run = subprocess.run([str(REFERENCE), str(art), str(req), str(tmp / f"{tag}.bin"), str(tmp / f"{tag}.json"),
                          "verify", "1", "1", "0", "1", "0", "1", str(bits)], capture_output=True, text=True,
                         timeout=60, preexec_fn=lambda: resource.setrlimit(resource.RLIMIT_AS, (4 << 30, 4 << 30)))
    art.unlink()
    if run.returncode == 0:
        return None
    return run.stderr.rstrip("\n").splitlines()[-1]


@pytest.mark.parametrize("base", list(bases()))
def test_validator_matches_the_reference_loader(base):
    from leaf_amd import runtime
    spec, bits = bases()[base]
    with tempfile.TemporaryDirectory() as d:
        tmp = Path(d)
        report = write_artifact(tmp / "base.leaf", spec, seed=11)
        blob = (tmp / "base.leaf").read_bytes()
        assert reference_verdict(tmp, blob, bits) is None, "the reference rejects the unmutated artifact"
        assert runtime.artifact_check(blob, bits) is None
        cases = mutants(blob, report["version"], full=base in ("w8a8", "v7", "eos"))
        write_tokens(tmp / "req.bin", [[0]])
        with concurrent.futures.ThreadPoolExecutor(8) as pool:
            verdicts = list(pool.map(lambda item: reference_verdict(tmp, bytes(item[1][1]), bits, f"m{item[0]}"),
                                     enumerate(cases)))
        differences = []
        for (label, mutated), want in zip(cases, verdicts):
            got = runtime.artifact_check(bytes(mutated), bits)
            if want is None:
                ok = got is None
            else:
                ok = got is not None and want == "Leaf decoder: " + got
            if not ok:
                differences.append(f"{label}: reference {want!r}, here {got!r}")
        print(f"{base} (LEAFDC0{report['version']}): {len(cases)} mutants, {len(differences)} differences")
        assert not differences, "\n".join(differences[:20])


def test_a_shape_whose_byte_count_wraps_passes_the_loader_rules():
    """rows·cols·bits/8 is computed in 64 bits by the reference's loader
    (decoder.cpp:875-877), so an extra tensor of 2^31 x 2^28 FP32 elements
    and 0 stored bytes passes it, and lh_artifact_check agrees.  The GPU load
    path rechecks the shape without wrapping
    (tests/test_gpu_decoder.py::test_gpu_load_rejects_a_wrapping_tensor_shape)."""
    from leaf_amd import runtime
    spec, bits = bases()["w8a8"]
    with tempfile.TemporaryDirectory() as d:
        tmp = Path(d)
        report = write_artifact(tmp / "base.leaf", spec, seed=11)
        blob = with_extra_tensor((tmp / "base.leaf").read_bytes(), report["version"], "model.extra.weight",
                                 1 << 31, 1 << 28, 32)
        assert reference_verdict(tmp, blob, bits) is None
        assert runtime.artifact_check(blob, bits) is None
        unwrapped = with_extra_tensor((tmp / "base.leaf").read_bytes(), report["version"], "model.extra.weight",
                                      1 << 20, 1 << 20, 32)
        want = reference_verdict(tmp, unwrapped, bits)
        assert want is not None and want == "Leaf decoder: " + runtime.artifact_check(unwrapped, bits)
