"""The leaf_decoder process protocol (engine/src/main_decoder.cpp:116-363) of the
MI355X binary, and the launcher that drives it the way `leaf run` does.

CPU tests: identity (--runtime-info, accepted by leaf/runtime_check.py's rule)
and argument rejection before any device work.  GPU tests: verify / chunked
logits, generate TOKEN lines and bench-generate metrics against the oracle and
the reference's golden outputs.
"""
from __future__ import annotations

import json
import subprocess

import numpy as np
import pytest

from leaf_amd import launcher
from leaf_amd.artifact import write_tokens

BIN = launcher.BUNDLED


def run(*args, timeout=120):
    return subprocess.run([str(BIN), *map(str, args)], capture_output=True, text=True, timeout=timeout)


def test_runtime_info_passes_the_launchers_identity_check():
    assert BIN.exists(), "leaf_decoder is not built (python -m leaf_amd.build)"
    info = launcher.runtime_info(BIN)
    assert info["runtime"] == "leaf_decoder" and info["artifact_versions"] == [2, 3, 4, 5, 6, 7]
    assert "accurate" in info["fp32_math_modes"] and info["source_bf16_matrices_supported"] is True


@pytest.mark.parametrize("extra,message", [
    (["nomode"], "unknown decoder mode"),
    (["generate", "1", "0"], "runs and chunk must be positive"),
    (["generate", "1", "1", "0", "4", "0", "1", "8", "--fp32-math=exact"], "FP32 math must be fast or accurate"),
    (["generate", "1", "1", "0", "4", "0", "1", "8", "--fp32-math=fast", "--fp32-math=fast"],
     "duplicate FP32 math policy"),
    (["generate", "1", "1", "0", "4", "0", "1", "8", "--fp32-math=fast", "0,1"],
     "worker CPU list must precede named decoder options"),
    (["generate", "1", "1", "0", "4", "0", "1", "8", "1,,2"], "worker CPUs must be comma-separated"),
    (["generate", "1", "1", "0", "4", "0", "1", "8", "--bogus"], "unknown decoder option: --bogus"),
    (["generate", "1", "1", "0", "4", "0", "1", "8", "--benchmark-counters"], "benchmark counters require bench mode"),
])
def test_arguments_are_rejected_before_device_work(tmp_path, extra, message):
    write_tokens(tmp_path / "t.bin", [[1, 2]])
    r = run(tmp_path / "none.leaf", tmp_path / "t.bin", tmp_path / "l.bin", tmp_path / "m.json", *extra)
    assert r.returncode == 1 and r.stderr.startswith("Leaf decoder: ") and message in r.stderr, r.stderr


@pytest.mark.parametrize("payload,message", [(b"", "truncated token request"),
                                             (b"\x00\x00\x00\x00", "invalid request count"),
                                             (b"\x01\x00\x00\x00\x00\x00\x00\x00", "invalid token count"),
                                             (b"\x01\x00\x00\x00\x01\x00\x00\x00\x05\x00\x00\x00\x09",
                                              "trailing token request bytes")])
def test_malformed_token_requests(tmp_path, payload, message):
    (tmp_path / "t.bin").write_bytes(payload)
    r = run(tmp_path / "none.leaf", tmp_path / "t.bin", tmp_path / "l.bin", tmp_path / "m.json", "generate")
    assert r.returncode == 1 and message in r.stderr, r.stderr


def test_launcher_selects_the_configured_binary(monkeypatch, tmp_path):
    monkeypatch.setenv("LEAF_DECODER_BIN", str(tmp_path / "missing"))
    with pytest.raises(FileNotFoundError, match="LEAF_DECODER_BIN"):
        launcher.executable()
    monkeypatch.delenv("LEAF_DECODER_BIN")
    assert launcher.executable() == BIN


@pytest.mark.gpu
@pytest.mark.parametrize("family", ["gpt2", "tinyllama"])
def test_verify_and_chunked_logits_match_the_oracle(tmp_path, oracle, golden_decoders, artifacts, family):
    arrays, meta = golden_decoders
    m = meta[family]
    prompt = arrays[f"{family}_prompt"][:20]
    write_tokens(tmp_path / "t.bin", [prompt.tolist()])
    od = oracle.decoder(artifacts[family], m["activation_bits"], m["fp32_math"] == "accurate")
    vocab = od.vocab
    tol = 2e-2 if m["activation_bits"] == 8 else 1e-3
    for mode, chunk in (("verify", 1), ("chunked", 7)):
        r = run(artifacts[family], tmp_path / "t.bin", tmp_path / "l.bin", tmp_path / "m.json", mode, 1, 1, 0, 1,
                0, chunk, m["activation_bits"], f"--fp32-math={m['fp32_math']}")
        assert r.returncode == 0, r.stderr
        logits = np.fromfile(tmp_path / "l.bin", np.float32).reshape(-1, vocab)
        od.reset()
        step = len(prompt) if mode == "verify" else chunk
        ref = np.concatenate([od.forward(prompt[p:p + step], all_logits=True) for p in range(0, len(prompt), step)])
        assert logits.shape == ref.shape
        assert float(np.max(np.abs(logits - ref)) / np.max(np.abs(ref))) <= tol
        assert json.loads((tmp_path / "m.json").read_text())["fp32_math"] == m["fp32_math"]


@pytest.mark.gpu
@pytest.mark.parametrize("family", ["gpt2", "tinyllama", "qwen", "smollm2"])
def test_generate_streams_the_reference_tokens(golden_decoders, artifacts, family):
    arrays, meta = golden_decoders
    m = meta[family]
    metrics = {}
    tokens = list(launcher.generate(artifacts[family], arrays[f"{family}_prompt"].tolist(), 10, m["activation_bits"],
                                    m["fp32_math"], metrics=metrics))
    assert tokens == arrays[f"{family}_tokens"].tolist()
    assert metrics["generated_tokens"] == tokens and len(metrics["decode_samples_ms"]) == 9
    assert metrics["activation_bits"] == m["activation_bits"] and metrics["time_to_first_token_ms"] > 0


@pytest.mark.gpu
def test_bench_generate_repeats_identical_greedy_runs(tmp_path, golden_decoders, artifacts):
    arrays, _ = golden_decoders
    write_tokens(tmp_path / "t.bin", [arrays["tinyllama_prompt"].tolist()])
    r = run(artifacts["tinyllama"], tmp_path / "t.bin", tmp_path / "l.bin", tmp_path / "m.json", "bench-generate",
            1, 3, 1, 8, 0, 1, 8)
    assert r.returncode == 0, r.stderr
    metrics = json.loads((tmp_path / "m.json").read_text())
    assert metrics["generated_tokens"] == arrays["tinyllama_tokens"].tolist()[:8]
    assert len(metrics["generation_samples_ms"]) == 3 and len(metrics["decode_samples_ms"]) == 3 * 7
    assert metrics["decode_p50_ms"] > 0
    r = run(artifacts["tinyllama"], tmp_path / "t.bin", tmp_path / "l.bin", tmp_path / "m.json", "bench", 1, 2, 0,
            1, 0, 1, 8)
    assert r.returncode == 0, r.stderr
    assert len(json.loads((tmp_path / "m.json").read_text())["decode_samples_ms"]) == 2
