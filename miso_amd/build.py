"""Build the product library libmiso_attn.so (gfx950) in-tree with hipcc.

    python -m miso_amd.build            # or: python miso_amd/build.py

The shared library lands in miso_amd/lib/ and is what miso_amd.attention, the GPU tests,
__graft_entry__.smoke() and bench.py load. No JIT and no site-packages install: the built file
travels with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libmiso_attn.so"
SOURCES = [PKG / "csrc" / "miso_attn_capi.hip"]
# bench.py's eager timing loops (host code over the C ABI above); not part of the product.
BENCH_LIB = LIB_DIR / "libmiso_bench.so"
BENCH_SOURCES = [PKG / "csrc" / "miso_bench.cpp"]
HEADERS = sorted((PKG / "kernels").glob("*.hpp")) + [ROOT / "include" / "miso_attn.h"]

# Packed FP32 VALU forms are disabled for all device code built here.
HIP_FLAGS = [
    "-O3",
    "-std=c++20",
    "--offload-arch=gfx950",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wextra",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wl,-Bsymbolic",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False) -> Path:
    """Compile libmiso_attn.so for gfx950, then libmiso_bench.so over it (always recompiles)."""
    _compile(SOURCES, LIB, verbose)
    _compile(BENCH_SOURCES, BENCH_LIB, verbose,
             ["-L", str(LIB_DIR), "-lmiso_attn", "-Wl,-rpath,$ORIGIN"])
    return LIB


def _compile(sources, lib: Path, verbose: bool, extra=()) -> None:
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIP_FLAGS, "-I", str(PKG / "kernels"), "-I", str(ROOT / "include"),
           *map(str, sources), *extra, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is expected.
    noise = ("packed-fp32-ops", "not a recognized feature")
    err = "\n".join(l for l in res.stderr.splitlines() if not any(n in l for n in noise))
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, lib)


if __name__ == "__main__":
    print(build(verbose=True))
