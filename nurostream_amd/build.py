"""Compile the HIP library (libnsx.so) for gfx950, in tree.

    python -m nurostream_amd.build

The library is plain C ABI (include/nurostream_amd.h); Python binds it with
ctypes (nurostream_amd/_native.py), so no torch extension machinery is used.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libnsx.so"
SOURCES = ("quant.hip", "moe.hip", "attn.hip", "reader.hip")
HEADERS = ("nsx_common.h", "raw_dot.h")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-pthread",
    # never let the compiler emit packed fp32 arithmetic (v_pk_fma_f32 & co.)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    # kernel arguments preloaded into SGPRs at wave launch (gfx950), not fetched by the first instructions
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    # one-lane atomics stay one atomic: the optimizer's wave-wide rewrite reads the result at once, a wait on
    # every load issued before it (the grouped gate/up kernel takes its next unit while its weights load)
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into nurostream_amd/libnsx.so (always rebuilds)."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", str(tmp), *(str(CSRC / s) for s in SOURCES)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in line and "unknown CPU feature" not in line
                    and "is not a recognized feature" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    p = build(verbose=True)
    print(f"built {p} ({p.stat().st_size / 1e6:.1f} MB)")
    sys.exit(0)
