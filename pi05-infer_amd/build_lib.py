"""Build the gfx950 libraries with hipcc (in-tree, next to the Python package) and the C-ABI
benchmark driver ``denoise_bench``.

* ``libpi05_denoise.so``: the denoise engine (include/pi05_denoise.h), hand-written kernels only;
* ``libpi05_prefix.so``: the prefix prefill and the vision tower (include/pi05_prefill.h,
  include/pi05_siglip.h), whose plain GEMMs run on hipBLASLt -- the only library that links it, so
  a denoise-only process never loads hipBLASLt.

    python pi05-infer_amd/build_lib.py [--verbose]
    python pi05-infer_amd/build_lib.py --stamps   (the profiling build phase_stamps.py reads)
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OUT = os.path.join(HERE, "pi05_infer", "libpi05_denoise.so")
SOURCES = ["pi05_kernels.hip", "pi05_persistent.hip", "pi05_persistent_batched.hip", "pi05_persistent_grouped.hip", "pi05_engine.hip"]
PREFIX_OUT = os.path.join(HERE, "pi05_infer", "libpi05_prefix.so")
PREFIX_SOURCES = ["pi05_prefill.hip", "pi05_siglip.hip"]
PREFIX_LIBS = ["-lhipblaslt"]  # the plain GEMMs of the prefill and the vision tower
STAMPS_OUT = os.path.join(HERE, "pi05_infer", "stamps", "libpi05_denoise.so")  # profiling build (phase_stamps.py)
BENCH_SRC = "denoise_bench.hip"
BENCH_OUT = os.path.join(HERE, "pi05_infer", "denoise_bench")

HIPCC_FLAGS = [
    "-O3",
    "--offload-arch=gfx950",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # keep hipcc from forming packed-fp32 (v_pk_*_f32) instructions on gfx950
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs))


def build(verbose: bool = False) -> str:
    _run([hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", *[os.path.join(CSRC, s) for s in SOURCES], "-o",
          OUT + ".tmp"], verbose)
    os.replace(OUT + ".tmp", OUT)
    _run([hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", *[os.path.join(CSRC, s) for s in PREFIX_SOURCES], *PREFIX_LIBS,
          "-o", PREFIX_OUT + ".tmp"], verbose)
    os.replace(PREFIX_OUT + ".tmp", PREFIX_OUT)
    bench_flags = [f for f in HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    _run([hipcc(), *bench_flags, f"-I{INCLUDE}", os.path.join(CSRC, BENCH_SRC), f"-L{os.path.dirname(OUT)}", "-lpi05_denoise",
          "-Wl,-rpath,$ORIGIN", "-o", BENCH_OUT + ".tmp"], verbose)
    os.replace(BENCH_OUT + ".tmp", BENCH_OUT)
    return OUT


def build_stamps(verbose: bool = False) -> str:
    """The denoise library with per-phase s_memrealtime stamps (-DPI05_PHASE_TIMESTAMPS, ~1 % slower;
    exports pi05_debug_phase_timestamps), next to the package in pi05_infer/stamps/ -- a profiling
    build that phase_stamps.py loads instead of the product library."""
    os.makedirs(os.path.dirname(STAMPS_OUT), exist_ok=True)
    _run([hipcc(), *HIPCC_FLAGS, "-DPI05_PHASE_TIMESTAMPS", f"-I{INCLUDE}", f"-I{CSRC}", *[os.path.join(CSRC, s) for s in SOURCES],
          "-o", STAMPS_OUT + ".tmp"], verbose)
    os.replace(STAMPS_OUT + ".tmp", STAMPS_OUT)
    return STAMPS_OUT


if __name__ == "__main__":
    if "--stamps" in sys.argv:
        print(build_stamps(verbose="--verbose" in sys.argv))
    else:
        print(build(verbose="--verbose" in sys.argv))
