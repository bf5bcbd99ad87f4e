"""Builds libpace_kv.so (the HIP kernels and their C ABI) in-tree for gfx950.

Usage: ``python -m paceserve_amd.build``.  The library is written next to this
file so that it travels with the source tree; ``paceserve_amd._native`` loads
it from there and never builds on import.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC_DIR = PKG_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
LIB_NAME = "libpace_kv.so"
LIB_PATH = PKG_DIR / LIB_NAME

SOURCES = ["kv_copy.hip", "kv_stage.hip", "kv_plan.cpp", "kv_append.hip", "kv_channel.cpp"]
HEADERS = ["internal.h"]

# Packed-FP32 instructions are disabled for every HIP translation unit.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc_path() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def build_library(verbose: bool = False) -> Path:
    """Compiles every HIP source into LIB_PATH (always recompiles)."""
    srcs = [str(CSRC_DIR / s) for s in SOURCES]
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc_path(), *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}", "-o", str(tmp), *srcs]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "packed-fp32-ops"
    msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if noise not in ln]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


C_ABI_DIR = REPO_DIR / "tests" / "c_abi"
C_CHECK_SRC = C_ABI_DIR / "pace_kv_check.c"
C_CHECK_BIN = C_CHECK_SRC.with_suffix("")
# promote latency timed from C (no Python in the loop); bench.py runs it
C_LATENCY_SRC = C_ABI_DIR / "pace_kv_promote_latency.c"
C_LATENCY_BIN = C_LATENCY_SRC.with_suffix("")


def build_c_program(src: Path, verbose: bool = False) -> Path:
    """Compiles a plain-C user of the ABI (tests/c_abi/*.c) against the built
    library; the binary, written next to its source, finds the library
    through its rpath ($ORIGIN-relative) and the HIP runtime under
    ROCM_PATH."""
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    out = src.with_suffix("")
    rel = os.path.relpath(PKG_DIR, out.parent)
    cmd = [os.environ.get("CC", "gcc"), "-std=c99", "-O2", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{rocm / 'include'}", f"-I{INCLUDE_DIR}", str(src), "-o", str(out),
           f"-L{PKG_DIR}", "-lpace_kv", f"-L{rocm / 'lib'}", "-lamdhip64",
           f"-Wl,-rpath,$ORIGIN/{rel}", f"-Wl,-rpath,{rocm / 'lib'}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{src.name} build failed:\n" + proc.stdout + proc.stderr)
    return out


def build_c_check(verbose: bool = False) -> Path:
    """Builds the C programs of tests/c_abi; returns the ABI check's path."""
    build_c_program(C_LATENCY_SRC, verbose)
    return build_c_program(C_CHECK_SRC, verbose)


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)
    print(build_c_check(verbose="-v" in sys.argv))
    print(C_LATENCY_BIN)
