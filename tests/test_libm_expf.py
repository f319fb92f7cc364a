"""The glibc expf restatement of leaf_amd/csrc/libm_expf.h, pinned on the CPU.

The reference's softmax and SiLU call std::exp(float), i.e. glibc's expf
(engine/src/kernels/transformer.cpp:134, engine/src/decoder.cpp:983).  The
reference-order GPU kernels compute it with the same double-precision
algorithm.  These checks pin that restatement:
  * its 32-entry table follows from the definition T[i] = nearest double to
    2^(i/32), less i << 47 (recomputed here in 60-digit decimal arithmetic);
  * compiled for the host, it returns this machine's expf bit for bit for all
    2^32 float inputs (tests/native/expf_exhaustive.cpp);
  * a planted mistake (z rounded before its two uses, the unfused form) is
    caught by the same exhaustive run.
"""
from __future__ import annotations

import re
import shutil
import struct
import subprocess
from decimal import Decimal, getcontext
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "leaf_amd" / "csrc" / "libm_expf.h"
CHECKER = ROOT / "tests" / "native" / "expf_exhaustive.cpp"


def header_table() -> list[int]:
    text = HEADER.read_text()
    block = text[text.index("kExp2Table32[32] = {"):]
    block = block[:block.index("};")]
    return [int(v, 16) for v in re.findall(r"0x([0-9a-f]{16})ull", block)]


def test_exp2_table_follows_from_its_definition():
    getcontext().prec = 60
    ln2 = Decimal(2).ln()
    table = header_table()
    assert len(table) == 32
    for i, stored in enumerate(table):
        nearest = float((ln2 * i / 32).exp())          # correctly rounded to double
        bits = struct.unpack("<Q", struct.pack("<d", nearest))[0]
        assert stored == (bits - (i << 47)) % (1 << 64), i


def build_checker(tmp: Path, header: Path) -> Path:
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ is not installed")
    source = tmp / "expf_exhaustive.cpp"
    source.write_text(CHECKER.read_text().replace('"../../leaf_amd/csrc/libm_expf.h"', f'"{header}"'))
    exe = tmp / "expf_exhaustive"
    subprocess.run([gxx, "-std=c++17", "-O2", "-ffp-contract=off", "-mfma", "-pthread", str(source), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    return exe


def test_expf_equals_libm_for_every_float(tmp_path):
    exe = build_checker(tmp_path, HEADER)
    out = subprocess.run([str(exe), "8"], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("mismatches 0 "), out.stdout


def test_exhaustive_check_catches_a_rounded_z(tmp_path):
    # Plant the mistake a restatement is most likely to make: round
    # z = x * 32/ln2 once and reuse it, as the source reads without contraction.
    text = HEADER.read_text()
    fused = "double kd = __builtin_fma(inv_ln2_n, xd, shift);"
    assert fused in text
    planted = text.replace(fused, "const double z = inv_ln2_n * xd;\n    double kd = z + shift;")
    planted = planted.replace("const double r = __builtin_fma(inv_ln2_n, xd, -kd);", "const double r = z - kd;")
    header = tmp_path / "libm_expf_planted.h"
    header.write_text(planted)
    exe = build_checker(tmp_path, header)
    out = subprocess.run([str(exe), "8"], capture_output=True, text=True, timeout=600)
    assert out.returncode == 1 and out.stdout.startswith("mismatches 2 "), out.stdout
