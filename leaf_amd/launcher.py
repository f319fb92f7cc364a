"""The `leaf run` side of the process boundary, for token ids.

Leaf's launcher (leaf/cli.py:426-510) writes a one-request ``tokens.bin``,
spawns ``leaf_decoder ... generate``, streams ``TOKEN <id>`` lines and merges
``metrics.json``; the binary is chosen by ``LEAF_DECODER_BIN`` (cli.py:36-45)
and checked with ``--runtime-info`` (leaf/runtime_check.py:8-41).  This module
does the same against the MI355X ``leaf_decoder`` built in this package.
Tokenization and model download stay with Leaf: callers pass token ids.

    python -m leaf_amd.launcher model.leaf 1 2 3 --max-tokens 16 --activation-bits 8
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import tempfile
import time
from pathlib import Path
from typing import Iterator, Sequence

from .artifact import write_tokens

PACKAGE = Path(__file__).resolve().parent
BUNDLED = PACKAGE / "bin" / "leaf_decoder"
ACCEPTED_VERSIONS = ([2, 3, 4, 5], [2, 3, 4, 5, 6], [2, 3, 4, 5, 6, 7])


def executable() -> Path:
    """LEAF_DECODER_BIN when set (it must exist), else the bundled GPU binary."""
    configured = os.environ.get("LEAF_DECODER_BIN")
    if configured:
        path = Path(configured)
        if not path.is_file():
            raise FileNotFoundError(f"LEAF_DECODER_BIN does not point to an executable: {path}")
        return path.resolve()
    if BUNDLED.is_file():
        return BUNDLED
    raise RuntimeError(f"{BUNDLED} is missing: build it with `python -m leaf_amd.build`")


def runtime_info(runtime: Path) -> dict:
    """--runtime-info identity check with the reference's acceptance rule."""
    try:
        result = subprocess.run([str(runtime), "--runtime-info"], capture_output=True, text=True, timeout=15)
    except subprocess.TimeoutExpired as error:
        raise RuntimeError(f"Runtime startup timed out: {runtime}") from error
    try:
        info = json.loads(result.stdout)
        if result.returncode or info.get("runtime") != "leaf_decoder" or \
                info.get("artifact_versions") not in ACCEPTED_VERSIONS:
            raise ValueError("unexpected runtime identity or artifact support")
    except (ValueError, AttributeError) as error:
        raise RuntimeError(f"Runtime check failed for {runtime}") from error
    return dict(path=str(runtime.resolve()), **info)


def generate(artifact: str | os.PathLike, ids: Sequence[int], max_tokens: int, activation_bits: int = 32,
             fp32_math: str = "fast", runtime: Path | None = None, metrics: dict | None = None) -> Iterator[int]:
    """Yields greedy token ids as the child prints them; fills `metrics` at the end."""
    if not ids:
        raise ValueError("Prompt produced no tokens")
    if fp32_math not in ("fast", "accurate"):
        raise ValueError("--fp32-math must be fast or accurate")
    runtime = runtime or executable()
    start = time.perf_counter()
    with tempfile.TemporaryDirectory(prefix="leaf_run_") as temp:
        folder = Path(temp)
        write_tokens(folder / "tokens.bin", [list(ids)])
        command = [str(runtime), str(artifact), str(folder / "tokens.bin"), str(folder / "logits.bin"),
                   str(folder / "metrics.json"), "generate", "1", "1", "0", str(max_tokens), "0", "1",
                   str(activation_bits)]
        if fp32_math == "accurate":
            command.append("--fp32-math=accurate")
        process = subprocess.Popen(command, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, bufsize=1)
        first_token_ms = None
        count = 0
        for line in process.stdout:
            if line.startswith("TOKEN "):
                if first_token_ms is None:
                    first_token_ms = (time.perf_counter() - start) * 1000
                count += 1
                yield int(line.split()[1])
        error = process.stderr.read()
        if process.wait():
            raise RuntimeError(error.strip())
        result = json.loads((folder / "metrics.json").read_text())
        if fp32_math == "accurate" and result.get("fp32_math") != "accurate":
            raise RuntimeError("Native FP32 math policy differs from the requested accurate execution")
    result.update(time_to_first_token_ms=first_token_ms, end_to_end_ms=(time.perf_counter() - start) * 1000,
                  tokens=count)
    if metrics is not None:
        metrics.update(result)


def main(argv: Sequence[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description="Greedy generation on one MI355X through leaf_decoder")
    parser.add_argument("artifact")
    parser.add_argument("ids", nargs="+", type=int)
    parser.add_argument("--max-tokens", type=int, default=16)
    parser.add_argument("--activation-bits", type=int, default=32, choices=(8, 32))
    parser.add_argument("--fp32-math", default="fast", choices=("fast", "accurate"))
    parser.add_argument("--metrics", type=Path)
    args = parser.parse_args(argv)
    metrics: dict = {}
    for token in generate(args.artifact, args.ids, args.max_tokens, args.activation_bits, args.fp32_math,
                          metrics=metrics):
        print(token, flush=True)
    if args.metrics:
        args.metrics.write_text(json.dumps(metrics, indent=2) + "\n")
    print(f"Leaf: {metrics.get('tokens')} tokens, decode p50 {metrics.get('decode_p50_ms', 0):.3f} ms",
          file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
