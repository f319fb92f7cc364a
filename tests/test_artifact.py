"""The synthetic LEAFDC writer: layout, quantization and acceptance by the reference reader."""
from __future__ import annotations

import dataclasses
import subprocess

import numpy as np
import pytest

from leaf_amd import models
from leaf_amd.artifact import (HEADER, load_tensor, quantize, read_tensor_table, round_to_bf16, write_artifact,
                               write_tokens)
from oracle.bindings import REF_BIN


def test_layout_alignment_and_tied_payloads(tmp_path):
    spec = models.qwen25_int4(reduced=True)
    path = tmp_path / "q.leaf"
    write_artifact(path, spec, seed=3)
    header, tensors, base = read_tensor_table(path)
    assert base % 64 == 0 and header["version"] == 2
    for t in tensors.values():
        assert t.offset % 64 == 0
        assert t.size == t.rows * t.cols * t.bits // 8
    assert tensors["lm_head.weight"].offset == tensors["model.embed_tokens.weight"].offset
    assert tensors["model.layers.0.self_attn.q_proj.weight"].bits == 4
    assert tensors["model.layers.0.self_attn.q_proj.bias"].bits == 32
    data, scales, info = load_tensor(path, "model.layers.1.mlp.down_proj.weight")
    assert scales.shape == (info.rows, info.cols // 32)


def test_bf16_rounding_is_nearest_even():
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0e38], np.float32)
    b = round_to_bf16(x)
    back = (b.astype(np.uint32) << 16).view(np.float32)
    assert back[0] == 1.0 and back[1] == 1.0 and back[2] == 1.015625 and back[3] == -2.5


@pytest.mark.skipif(not REF_BIN.exists(), reason="reference build (oracle/_ref) not present")
@pytest.mark.parametrize("family", list(models.PRESETS))
def test_reference_reader_accepts_every_family(tmp_path, family):
    spec = models.PRESETS[family](reduced=True)
    path = tmp_path / "m.leaf"
    write_artifact(path, spec, seed=1)
    write_tokens(tmp_path / "t.bin", [[1, 2, 3]])
    bits, math = models.RUN_POLICY[family]
    run = subprocess.run([str(REF_BIN), str(path), str(tmp_path / "t.bin"), str(tmp_path / "l.bin"),
                          str(tmp_path / "m.json"), "verify", "1", "1", "0", "1", "0", "1", str(bits),
                          f"--fp32-math={math}"], capture_output=True, text=True)
    assert run.returncode == 0, run.stderr


def test_versions_follow_the_exporter(tmp_path):
    base = models.tinyllama_w8a8(reduced=True)
    for overrides, version in ((dict(), 2), (dict(sliding_window=4), 3), (dict(eos=5, eos_tokens=(5, 6)), 4),
                               (dict(qk_norm=1, heads=4, head_dim=32, bits=32, keep_fp32=frozenset()), 7)):
        path = tmp_path / f"v{version}.leaf"
        write_artifact(path, dataclasses.replace(base, **overrides), seed=1)
        magic, v = HEADER.unpack_from(path.read_bytes())[:2]
        assert magic == f"LEAFDC0{version}".encode() and v == version
