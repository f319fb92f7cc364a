"""Build libleafhip.so (and the leaf_decoder and hbm_copy executables) for gfx950 with hipcc.

    python -m leaf_amd.build            # compile everything in-tree

Outputs land next to the sources' package (leaf_amd/libleafhip.so,
leaf_amd/bin/leaf_decoder) so they travel with the tree.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libleafhip.so"
EXECUTABLE = PACKAGE / "bin" / "leaf_decoder"
ARCH = os.environ.get("LEAF_HIP_ARCH", "gfx950")

SOURCES = ["kernels.hip", "gemm_w8a8.hip", "gemm_f32.hip", "decode_step.hip", "reference_order.hip", "artifact_format.cpp", "runtime.cpp",
           "session.cpp", "capi.cpp"]

# -ffp-contract=off: every FMA in the kernels is explicit (fmaf), so the integer
# epilogues keep the CPU path's separate roundings.  Packed FP32 instructions
# are disabled (-packed-fp32-ops).
HIPFLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-ffp-contract=off",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wno-unused-command-line-argument", "-I", str(ROOT / "include")]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (ROCm is required to build libleafhip)")


def _compile(source: str) -> Path:
    src = CSRC / source
    obj = BUILD / (source + ".o")
    cmd = [hipcc(), *HIPFLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"compiling {source} failed:\n{result.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    workers = min(len(SOURCES), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(_compile, SOURCES))
    tmp = LIBRARY.with_suffix(".so.tmp")
    link = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(link, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking libleafhip.so failed:\n{result.stderr}")
    tmp.replace(LIBRARY)
    if (CSRC / "main_decoder.cpp").exists():
        EXECUTABLE.parent.mkdir(exist_ok=True)
        exe_tmp = EXECUTABLE.with_suffix(".tmp")
        cmd = ["g++", "-std=c++17", "-O2", "-I", str(ROOT / "include"), str(CSRC / "main_decoder.cpp"),
               "-L", str(PACKAGE), "-lleafhip", f"-Wl,-rpath,$ORIGIN/..", "-o", str(exe_tmp)]
        result = subprocess.run(cmd, capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError(f"building leaf_decoder failed:\n{result.stderr}")
        exe_tmp.replace(EXECUTABLE)
    # hbm_copy: the copy of known size that calibrates the profiler's byte
    # counters and measures streaming bandwidth; mfma_peak: matrix-core rates
    for tool in ("hbm_copy", "mfma_peak"):
        if not (CSRC / f"{tool}.hip").exists():
            continue
        probe = PACKAGE / "bin" / tool
        probe.parent.mkdir(exist_ok=True)
        cmd = [hipcc(), *HIPFLAGS, str(CSRC / f"{tool}.hip"), "-o", str(probe.with_suffix(".tmp"))]
        result = subprocess.run(cmd, capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError(f"building {tool} failed:\n{result.stderr}")
        probe.with_suffix(".tmp").replace(probe)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
