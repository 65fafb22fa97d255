"""Build of the gfx950 HIP library (libei_attn.so) in-tree with hipcc.

The library holds the kernels and the C ABI of include/ei_attn.h.  It is built here on the
CPU (hipcc cross-compiles for gfx950) and travels with the source tree; nothing is
compiled at import time on the GPU host.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libei_attn.so"
SOURCES = ["csrc/prologue.hip", "csrc/decode.hip", "csrc/prefill.hip", "csrc/project.hip", "csrc/capi.cpp",
           "host/hip_attention.cpp", "host/gguf_index.cpp", "host/qwen3_schema.cpp"]
HEADERS = ["common.h", "launch.h"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    "-Wall",
    # packed fp32 VALU ops are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libei_attn.so)")


def build(verbose: bool = False) -> Path:
    """Compile every source for gfx950 into exactinfer_amd/libei_attn.so (always rebuilds)."""
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(ROOT / "include"),
           *[str(PKG / s) for s in SOURCES], "-o", str(LIB) + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(str(LIB) + ".tmp", LIB)
    return LIB


def inputs() -> list[Path]:
    """Every file the library is built from: the sources, the private headers and the ABI header."""
    return ([PKG / s for s in SOURCES] + [CSRC / h for h in HEADERS] + [PKG / "host" / h for h in ("gguf_index.h", "hip_attention.h")] +
            [ROOT / "include" / h for h in ("ei_attn.h", "ei_gguf.h")])


def is_stale() -> bool:
    """True when the library is absent or older than any file it is built from."""
    if not LIB.exists():
        return True
    built = LIB.stat().st_mtime
    return any(p.stat().st_mtime > built for p in inputs())


def ensure_built() -> Path:
    """Build the library when it is absent or older than a source or header (the entry scripts'
    convenience: tests, smoke and the bench load what is built; the library loader itself never
    builds and fails loudly)."""
    return build() if is_stale() else LIB


if __name__ == "__main__":
    print(build(verbose=True))
