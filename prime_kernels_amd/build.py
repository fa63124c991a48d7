"""Build the native library `_lib/libprime_decode.so` with hipcc for gfx950.

Usage: python -m prime_kernels_amd.build   (also called by __graft_entry__.build()).
The library is built in-tree so it travels with the source tree; nothing is JIT-compiled at
run time, and the Python wrappers fail loudly when it is missing.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB_DIR = PKG / "_lib"
LIB = LIB_DIR / "libprime_decode.so"
SOURCES = [PKG / "csrc" / "decode_megakernel.hip", PKG / "csrc" / "decode_sr.hip", PKG / "csrc" / "lossless_bf16.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed-fp32 ops are kept out of generated code on this target (known-unstable forms)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-inline-asm", f"-I{ROOT / 'include'}",
    # every symbol the library uses must be defined in it
    "-Wl,--no-undefined",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False) -> Path:
    LIB_DIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *map(str, SOURCES), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
