"""Build recipe of libfattn.so: hand-written HIP for gfx950 only.

It plays the part of the reference's build.rs (build.rs:5-30), which compiles
kernels/fused_attn.cu to PTX with nvcc: here hipcc compiles the kernels and the C-ABI layer
into one shared library holding a gfx950 code object (no PTX, no JIT, no other target).

Usage: ``python candle-fused-attn_amd/build.py`` (or ``build()`` from Python).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "lib"
LIB = LIB_DIR / "libfattn.so"
SOURCES = [CSRC / "fattn_kernels.hip", CSRC / "fattn_api.cpp"]
HEADERS = [REPO / "include" / "fattn.h", CSRC / "fattn_internal.h"]
# The C++ op layer over the C ABI (the reference's src/lib.rs ops for C++ callers), linked
# against libfattn.so, and its test program (links the CPU oracle; test infrastructure).
HOST = PKG_DIR / "host"
HOST_LIB = LIB_DIR / "libcandle_fused_attn.so"
HOST_TEST_SRC = REPO / "tests" / "cpp" / "parity_host.cpp"
HOST_TEST = REPO / "tests" / "cpp" / "parity_host"
ORACLE_DIR = REPO / "oracle"

# gfx950 only. Packed fp32 ALU instructions are disabled (-packed-fp32-ops); the host pass warns
# that it does not know that target feature, which is harmless.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libfattn.so")
    return path


def command(out: Path = LIB) -> list[str]:
    return [hipcc(), *HIPCC_FLAGS, f"-I{REPO / 'include'}", f"-I{CSRC}",
            *[str(s) for s in SOURCES], "-o", str(out)]


def _run(cmd: list[str], tmp: Path, out: Path, verbose: bool) -> Path:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> Path:
    """Compile libfattn.so in-tree (always; the caller decides when to rebuild)."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    return _run(command(tmp), tmp, LIB, verbose)


def host_command(out: Path = HOST_LIB) -> list[str]:
    return [hipcc(), "-x", "hip", *HIPCC_FLAGS, f"-I{REPO / 'include'}", f"-I{HOST}",
            str(HOST / "candle_fused_attn.cpp"), f"-L{LIB_DIR}", "-lfattn",
            "-Wl,-rpath,$ORIGIN", "-o", str(out)]


def build_host(verbose: bool = False) -> Path:
    """Compile libcandle_fused_attn.so (the C++ op layer; needs libfattn.so built first)."""
    tmp = HOST_LIB.with_suffix(".so.tmp")
    return _run(host_command(tmp), tmp, HOST_LIB, verbose)


STEP_BENCH_SRC = HOST / "step_bench.cpp"
STEP_BENCH = LIB_DIR / "cfa_step_bench"


def step_bench_command(out: Path = STEP_BENCH) -> list[str]:
    return [hipcc(), "-O2", "-std=c++17", "-Wall", f"-I{HOST}", str(STEP_BENCH_SRC),
            f"-L{LIB_DIR}", "-lcandle_fused_attn", "-lfattn", "-Wl,-rpath,$ORIGIN",
            "-o", str(out)]


def build_step_bench(verbose: bool = False) -> Path:
    """Compile lib/cfa_step_bench (times steps through the C++ op layer; needs
    libcandle_fused_attn.so built first)."""
    tmp = STEP_BENCH.with_name(STEP_BENCH.name + ".tmp")
    return _run(step_bench_command(tmp), tmp, STEP_BENCH, verbose)


def host_test_command(out: Path = HOST_TEST) -> list[str]:
    rpath = "$ORIGIN/../../candle-fused-attn_amd/lib:$ORIGIN/../../oracle"
    return [hipcc(), "-O2", "-std=c++17", "-Wall", f"-I{HOST}", str(HOST_TEST_SRC),
            f"-L{LIB_DIR}", "-lcandle_fused_attn", "-lfattn", f"-L{ORACLE_DIR}", "-loracle",
            f"-Wl,-rpath,{rpath}", "-o", str(out)]


def build_host_test(verbose: bool = False) -> Path:
    """Compile tests/cpp/parity_host (needs libcandle_fused_attn.so and oracle/liboracle.so)."""
    tmp = HOST_TEST.with_name(HOST_TEST.name + ".tmp")
    return _run(host_test_command(tmp), tmp, HOST_TEST, verbose)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    print(build_host(verbose="-v" in sys.argv))
    print(build_step_bench(verbose="-v" in sys.argv))
