"""LEAFDC02..07 decoder artifacts: writer for seeded synthetic models, and reader.

The byte layout is Leaf's (writer: tools/export_decoder.py:22-25, 213-420;
reader: engine/src/decoder.cpp:787-933).  It has to be identical, because the
reference CPU decoder and this library's GPU decoder must load the very same
file.  Weights are drawn from a seeded numpy generator instead of a Hugging
Face snapshot: there is no network here, and the tests and benchmarks need
models of exact architectural shape with random-init weights.

Quantization follows export_decoder.quantize (tools/export_decoder.py:91-105):
symmetric, ``s = max(absmax_group / limit, 1e-12)`` in float32,
``q = clip(rint(w / s), -limit, limit)``; INT4 packs the even column in the low
nibble.  Every payload starts on a 64-byte boundary relative to ``data_base``.
"""
from __future__ import annotations

import dataclasses
import struct
from pathlib import Path
from typing import Iterable

import numpy as np

HEADER = struct.Struct("<8sIIQ10Iff8If")        # export_decoder.py:23, read at decoder.cpp:795-808
OPERATOR_METADATA = struct.Struct("<3I")        # export_decoder.py:24, read at decoder.cpp:823-838
DESCRIPTOR = struct.Struct("<5I4Q")             # export_decoder.py:25, read at decoder.cpp:858-890
NO_EOS = 0xFFFFFFFF

NORM_RMS, NORM_LAYER = 0, 1
ACT_SILU, ACT_GELU_ERF, ACT_GELU_TANH, ACT_RELU = 0, 1, 2, 3
POS_ROPE, POS_LEARNED, POS_NONE = 0, 1, 2

LAYER_MATRICES = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                  "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


@dataclasses.dataclass
class DecoderSpec:
    """Header semantics plus storage policy of one decoder artifact."""
    hidden: int
    intermediate: int
    heads: int
    kv_heads: int
    layers: int
    vocab: int
    max_positions: int
    head_dim: int
    eos: int = NO_EOS
    sliding_window: int = 0
    theta: float = 10000.0
    epsilon: float = 1e-5
    norm: int = NORM_RMS
    activation: int = ACT_SILU
    position: int = POS_ROPE
    gated: int = 1
    parallel_residual: int = 0
    rotary_dim: int | None = None
    position_offset: int = 0
    final_norm: int = 1
    embedding_scale: float = 1.0
    eos_tokens: tuple[int, ...] = ()
    qk_norm: int = 0
    rope_frequencies: tuple[float, ...] = ()
    # storage policy
    bits: int = 32                  # 32, 8 or 4 for ".weight" matrices with rows > 1
    group_size: int = 64            # INT4 group (min(group, cols))
    int8_group_size: int = 0        # 0 = one scale per row
    keep_fp32: frozenset = frozenset()
    source_bf16: bool = False       # v6: matrices stored as original BF16 bits
    bf16_io: bool = False           # v5: embedding and head stored as BF16 bits, the rest FP32
    smoothquant_alpha: float = 0.0  # > 0: SmoothQuant-calibrated linears with ".input_scale" tensors
    tied: bool = False              # lm_head shares the embedding payload
    attention_bias: bool = False    # q/k/v(/o) projection biases
    o_bias: bool = False
    mlp_bias: bool = False
    norm_bias: bool = False         # LayerNorm beta tensors
    # random init
    std: float = 0.02
    bias_std: float = 0.0
    norm_jitter: float = 0.0        # 0 keeps gamma = 1 exactly

    @property
    def rotary(self) -> int:
        """Rotated width per head: the whole head for RoPE unless set explicitly."""
        if self.rotary_dim is not None:
            return self.rotary_dim
        return self.head_dim if self.position == POS_ROPE else 0

    @property
    def qwidth(self) -> int:
        return self.heads * self.head_dim

    @property
    def kvwidth(self) -> int:
        return self.kv_heads * self.head_dim

    def header_values(self) -> tuple:
        return (self.hidden, self.intermediate, self.heads, self.kv_heads, self.layers, self.vocab,
                self.max_positions, self.eos, self.head_dim, self.sliding_window,
                float(self.theta), float(self.epsilon),
                self.norm, self.activation, self.position, self.gated, self.parallel_residual,
                self.rotary, self.position_offset, self.final_norm, float(self.embedding_scale))


def tensor_shapes(spec: DecoderSpec) -> dict[str, tuple[int, int]]:
    """Canonical tensors (tools/decoder_plan.py:408-427) plus the spec's biases."""
    h, f = spec.hidden, spec.intermediate
    shapes = {"model.embed_tokens.weight": (spec.vocab, h), "lm_head.weight": (spec.vocab, h)}
    if spec.final_norm:
        shapes["model.norm.weight"] = (1, h)
    if spec.position == POS_LEARNED:
        shapes["model.position_embeddings.weight"] = (spec.max_positions + spec.position_offset, h)
    for i in range(spec.layers):
        p = f"model.layers.{i}."
        shapes.update({p + "input_layernorm.weight": (1, h), p + "post_attention_layernorm.weight": (1, h),
                       p + "self_attn.q_proj.weight": (spec.qwidth, h),
                       p + "self_attn.k_proj.weight": (spec.kvwidth, h),
                       p + "self_attn.v_proj.weight": (spec.kvwidth, h),
                       p + "self_attn.o_proj.weight": (h, spec.qwidth),
                       p + "mlp.up_proj.weight": (f, h), p + "mlp.down_proj.weight": (h, f)})
        if spec.gated:
            shapes[p + "mlp.gate_proj.weight"] = (f, h)
        if spec.qk_norm:
            shapes[p + "self_attn.q_norm.weight"] = (1, spec.head_dim)
            shapes[p + "self_attn.k_norm.weight"] = (1, spec.head_dim)
    biases = {}
    if spec.norm_bias and spec.final_norm:
        biases["model.norm.bias"] = (1, h)
    for i in range(spec.layers):
        p = f"model.layers.{i}."
        if spec.norm_bias:
            biases[p + "input_layernorm.bias"] = (1, h)
            biases[p + "post_attention_layernorm.bias"] = (1, h)
        roles = []
        if spec.attention_bias:
            roles += ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"]
        if spec.o_bias:
            roles.append("self_attn.o_proj")
        if spec.mlp_bias:
            roles += (["mlp.gate_proj"] if spec.gated else []) + ["mlp.up_proj", "mlp.down_proj"]
        for role in roles:
            biases[p + role + ".bias"] = (1, shapes[p + role + ".weight"][0])
    shapes.update(biases)
    return shapes


def quantize(array: np.ndarray, bits: int, group: int) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric per-group quantization (tools/export_decoder.py:91-105)."""
    rows, cols = array.shape
    if cols % group:
        raise ValueError(f"input width {cols} is not divisible by group size {group}")
    grouped = array.reshape(rows, cols // group, group)
    limit = (1 << (bits - 1)) - 1
    scales = np.maximum(np.max(np.abs(grouped), axis=-1) / limit, 1e-12).astype("<f4")
    values = np.clip(np.rint(grouped / scales[..., None]), -limit, limit).astype(np.int8).reshape(rows, cols)
    if bits == 4:
        nibbles = values.astype(np.uint8) & 15
        values = nibbles[:, 0::2] | (nibbles[:, 1::2] << 4)
    return np.ascontiguousarray(values), np.ascontiguousarray(scales)


def round_to_bf16(array: np.ndarray) -> np.ndarray:
    """Round float32 to BF16 bits (round-to-nearest-even), returned as uint16."""
    bits = np.ascontiguousarray(array, dtype=np.float32).view(np.uint32)
    rounded = bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))
    return (rounded >> np.uint32(16)).astype("<u2")


def _bf16_matrix(name: str, rows: int, layers: int) -> bool:
    """Tensor roles v6 may store as BF16 (decoder.cpp:93-115)."""
    if rows <= 1:
        return False
    if name in ("lm_head.weight", "model.embed_tokens.weight", "model.position_embeddings.weight"):
        return True
    if not name.startswith("model.layers."):
        return False
    rest = name[len("model.layers."):]
    index, _, role = rest.partition(".")
    return index.isdigit() and int(index) < layers and role.removesuffix(".weight") in LAYER_MATRICES \
        and role.endswith(".weight")


def _precision(spec: DecoderSpec, name: str, rows: int) -> int:
    # export_decoder.py:312-314
    if spec.source_bf16 and _bf16_matrix(name, rows, spec.layers) and name not in spec.keep_fp32:
        return 16
    if spec.bf16_io and name in ("model.embed_tokens.weight", "lm_head.weight"):
        return 16
    if name.endswith(".input_scale"):
        return 32
    if name.endswith(".weight") and rows > 1 and name not in spec.keep_fp32:
        return spec.bits
    return 32


def _version(spec: DecoderSpec) -> tuple[int, bytes]:
    eos_list = list(spec.eos_tokens)
    if spec.eos != NO_EOS and not eos_list:
        eos_list = [spec.eos]
    version = 4 if len(eos_list) > 1 else 3 if spec.sliding_window else 2
    meta = struct.pack(f"<{len(eos_list) + 1}I", len(eos_list), *eos_list) if version == 4 else b""
    storage = 0
    if spec.bf16_io:
        version = storage = 5
        meta = struct.pack(f"<{len(eos_list) + 1}I", len(eos_list), *eos_list)
    if spec.source_bf16:
        version = storage = 6
        meta = struct.pack(f"<{len(eos_list) + 1}I", len(eos_list), *eos_list)
    if spec.qk_norm or spec.rope_frequencies:
        ext = OPERATOR_METADATA.pack(storage, spec.qk_norm, len(spec.rope_frequencies))
        version = 7
        meta = (ext + struct.pack(f"<{len(spec.rope_frequencies)}f", *spec.rope_frequencies)
                + struct.pack(f"<{len(eos_list) + 1}I", len(eos_list), *eos_list))
    return version, meta


def _calibrated(spec: DecoderSpec, name: str, rows: int) -> bool:
    """The linears a SmoothQuant export calibrates: quantized matrices other
    than the embeddings (export_decoder.py:285-296)."""
    return bool(spec.smoothquant_alpha) and name.endswith(".weight") and rows > 1 and \
        name not in spec.keep_fp32 and spec.bits in (8, 4) and \
        not name.startswith(("model.embed_tokens.", "model.position_embeddings."))


def channel_factors(weight: np.ndarray, activation_max: np.ndarray, alpha: float) -> np.ndarray:
    """SmoothQuant per-input-channel factors s_j = max|X_j|^alpha / max|W_j|^(1-alpha)
    (Xiao et al., 2022), bounded to [1e-4, 1e4]; the export multiplies W by s and
    stores 1/s as the layer's ".input_scale" (export_decoder.py:108-118, 372-384)."""
    weight_max = np.maximum(np.max(np.abs(weight), axis=0), 1e-5)
    return np.clip(np.maximum(activation_max, 1e-5) ** alpha / weight_max ** (1 - alpha), 1e-4, 1e4).astype(np.float32)


def synthetic_activation_max(seed: int, name: str, cols: int) -> np.ndarray:
    """Seeded stand-in for calibration statistics: |N(0,1)| * 2 + 0.5 per input
    channel, with 1% outlier channels x 20."""
    key = sum((i + 1) * b for i, b in enumerate(name.encode())) % (1 << 31)
    rng = np.random.default_rng([seed, key, 7])
    maxima = np.abs(rng.standard_normal(cols)) * 2 + 0.5
    maxima[rng.random(cols) < 0.01] *= 20
    return maxima


class _Init:
    """Seeded per-tensor generator: the same (seed, name) always yields the same data."""

    def __init__(self, spec: DecoderSpec, seed: int):
        self.spec, self.seed = spec, seed

    def blocks(self, name: str, rows: int, cols: int, block_elements: int = 1 << 22):
        """Yield (first_row, array) blocks of the tensor; one random stream per tensor,
        so the values do not depend on the block size."""
        spec = self.spec
        digest = np.frombuffer(name.encode(), dtype=np.uint8).astype(np.uint64)
        key = int((digest * (np.arange(digest.size, dtype=np.uint64) + 1)).sum() % (1 << 31))
        rng = np.random.Generator(np.random.PCG64([self.seed, key, len(name)]))
        step = max(1, min(rows, block_elements // max(cols, 1)))
        buffer = np.empty((step, cols), np.float32)
        for first in range(0, rows, step):
            out = buffer[:min(step, rows - first)]
            if name.endswith("norm.weight"):
                if spec.norm_jitter:
                    rng.standard_normal(out.shape, dtype=np.float32, out=out)
                    out *= np.float32(spec.norm_jitter)
                    out += np.float32(1)
                else:
                    out.fill(1)
            elif name.endswith(".bias"):
                if spec.bias_std:
                    rng.standard_normal(out.shape, dtype=np.float32, out=out)
                    out *= np.float32(spec.bias_std)
                else:
                    out.fill(0)
            else:
                rng.standard_normal(out.shape, dtype=np.float32, out=out)
                out *= np.float32(spec.std)
            yield first, out

    def __call__(self, name: str, rows: int, cols: int) -> np.ndarray:
        out = np.empty((rows, cols), np.float32)
        for first, block in self.blocks(name, rows, cols):
            out[first:first + len(block)] = block
        return out


def write_artifact(path: str | Path, spec: DecoderSpec, seed: int = 0) -> dict:
    """Write a seeded random-init decoder artifact; returns a small report."""
    path = Path(path)
    version, meta = _version(spec)
    shapes = tensor_shapes(spec)
    init = _Init(spec, seed)
    # SmoothQuant: W * s is stored for each calibrated linear, 1/s as its input scale
    smoothing = {}
    for name, (rows, cols) in list(shapes.items()):
        if _calibrated(spec, name, rows):
            factors = channel_factors(init(name, rows, cols), synthetic_activation_max(seed, name, cols),
                                      spec.smoothquant_alpha)
            smoothing[name] = factors
            shapes[name.removesuffix(".weight") + ".input_scale"] = (1, cols)
    descriptors, shared, offset = [], {}, 0
    for name, (rows, cols) in shapes.items():
        precision = _precision(spec, name, rows)
        group = (spec.int8_group_size or cols) if precision == 8 else \
            min(spec.group_size, cols) if precision == 4 else 0
        if precision == 8 and cols % group:
            raise ValueError(f"INT8 group {group} must divide {cols}")
        if precision == 4 and (cols % group or group % 2):
            raise ValueError(f"INT4 group {group} must divide even width {cols}")
        source = "model.embed_tokens.weight" if (spec.tied and name == "lm_head.weight") else name
        identity = (source, rows, cols, precision, group)
        if identity in shared:
            descriptors.append((name, rows, cols, precision, group, *shared[identity], None))
            continue
        size = rows * cols * precision // 8
        offset = (offset + 63) & ~63
        data_offset = offset
        offset += size
        scales = rows * (cols // group) if precision in (4, 8) else 0
        offset = (offset + 63) & ~63
        scale_offset = offset
        offset += scales * 4
        shared[identity] = (data_offset, size, scale_offset, scales)
        descriptors.append((name, rows, cols, precision, group, data_offset, size, scale_offset, scales, source))
    metadata = HEADER.size + len(meta) + sum(4 + len(d[0].encode()) + DESCRIPTOR.size for d in descriptors)
    base = (metadata + 63) & ~63
    magic = f"LEAFDC0{version}".encode()
    tmp = path.with_suffix(path.suffix + ".partial")
    path.parent.mkdir(parents=True, exist_ok=True)
    with tmp.open("wb") as out:
        out.write(HEADER.pack(magic, version, len(descriptors), base, *spec.header_values()))
        out.write(meta)
        for name, rows, cols, precision, group, start, size, scale_start, scales, _ in descriptors:
            encoded = name.encode()
            out.write(struct.pack("<I", len(encoded)) + encoded)
            out.write(DESCRIPTOR.pack(2, rows, cols, precision, group, start, size, scale_start, scales))
        end = base + offset
        for name, rows, cols, precision, group, start, size, scale_start, scales, source in descriptors:
            if source is None:
                continue
            row_bytes = cols * precision // 8
            groups = cols // group if group else 0
            if name.endswith(".input_scale"):
                inverse = (1.0 / smoothing[name.removesuffix(".input_scale") + ".weight"]).astype("<f4")
                out.seek(base + start)
                out.write(memoryview(np.ascontiguousarray(inverse)).cast("B"))
                continue
            for first, array in init.blocks(source, rows, cols):
                if source in smoothing:
                    array = array * smoothing[source][None, :]
                if precision == 32:
                    payload, scale_array = array, None
                elif precision == 16:
                    payload, scale_array = round_to_bf16(array), None
                else:
                    payload, scale_array = quantize(array, precision, group)
                out.seek(base + start + first * row_bytes)
                out.write(memoryview(np.ascontiguousarray(payload)).cast("B"))
                if scales:
                    out.seek(base + scale_start + first * groups * 4)
                    out.write(memoryview(scale_array).cast("B"))
        out.truncate(max(end, out.tell()))
    tmp.replace(path)
    return {"version": version, "tensor_count": len(descriptors), "bytes": path.stat().st_size,
            "data_base": base}


@dataclasses.dataclass
class TensorInfo:
    name: str
    rows: int
    cols: int
    bits: int
    group: int
    offset: int
    size: int
    scale_offset: int
    scale_count: int


def read_tensor_table(path: str | Path) -> tuple[dict, dict[str, TensorInfo], int]:
    """Parse the header and tensor table (no validation beyond structure)."""
    blob = Path(path).read_bytes()[:1 << 24]
    fields = HEADER.unpack_from(blob)
    magic, version, count, base = fields[:4]
    keys = ("hidden", "intermediate", "heads", "kv_heads", "layers", "vocab", "max_positions", "eos",
            "head_dim", "sliding_window", "theta", "epsilon", "norm", "activation", "position", "gated",
            "parallel_residual", "rotary_dim", "position_offset", "final_norm", "embedding_scale")
    header = dict(zip(keys, fields[4:]))
    header["version"] = version
    pos = HEADER.size
    if version == 7:
        storage, qk, nfreq = OPERATOR_METADATA.unpack_from(blob, pos)
        pos += 12
        header.update(storage=storage, qk_norm=qk,
                      rope_frequencies=list(struct.unpack_from(f"<{nfreq}f", blob, pos)))
        pos += 4 * nfreq
    if version >= 4:
        (n,) = struct.unpack_from("<I", blob, pos)
        header["eos_tokens"] = list(struct.unpack_from(f"<{n}I", blob, pos + 4))
        pos += 4 + 4 * n
    tensors = {}
    for _ in range(count):
        (length,) = struct.unpack_from("<I", blob, pos)
        name = blob[pos + 4:pos + 4 + length].decode()
        pos += 4 + length
        rank, rows, cols, bits, group, off, size, soff, scount = DESCRIPTOR.unpack_from(blob, pos)
        pos += DESCRIPTOR.size
        tensors[name] = TensorInfo(name, rows, cols, bits, group, off, size, soff, scount)
    return header, tensors, base


def load_tensor(path: str | Path, name: str) -> tuple[np.ndarray, np.ndarray | None, TensorInfo]:
    """Raw payload and scales of one tensor (memory-mapped)."""
    _, tensors, base = read_tensor_table(path)
    info = tensors[name]
    raw = np.memmap(path, dtype=np.uint8, mode="r", offset=base + info.offset, shape=(info.size,))
    dtype = {32: "<f4", 16: "<u2", 8: np.int8, 4: np.uint8}[info.bits]
    data = np.asarray(raw).view(dtype)
    data = data.reshape(info.rows, -1)
    scales = None
    if info.scale_count:
        scales = np.asarray(np.memmap(path, dtype="<f4", mode="r", offset=base + info.scale_offset,
                                      shape=(info.scale_count,))).reshape(info.rows, -1)
    return data, scales, info


def write_tokens(path: str | Path, requests: Iterable[Iterable[int]]) -> None:
    """tokens.bin request file: u32 count, then {u32 len, u32 ids[len]} (main_decoder.cpp:196-210)."""
    requests = [list(r) for r in requests]
    with Path(path).open("wb") as out:
        out.write(struct.pack("<I", len(requests)))
        for ids in requests:
            out.write(struct.pack(f"<I{len(ids)}I", len(ids), *ids))
