"""Builds libkvpath.so (the gfx950 HIP kernels behind include/kvpath.h) in-tree.

Run as ``python -m kavor_amd._build``; ``__graft_entry__.build()`` calls
:func:`build_library`.  The library is written next to this file so that it travels
with the source tree, and is loaded by :mod:`kavor_amd._lib`.
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
LIB_PATH = PKG_DIR / "libkvpath.so"
SOURCES = ["capi.hip", "kv_append.hip", "paged_decode.hip", "varlen_prefill.hip", "norm_rope.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    # Packed-FP32 VALU forms are kept out of every kernel: plain fp32 code only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libkvpath.so")


def build_library(verbose: bool = False) -> Path:
    """Compiles every kernel source into ``kavor_amd/libkvpath.so`` (always rebuilds)."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}",
           *[str(CSRC_DIR / s) for s in SOURCES], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that is harmless.
    noise = "'-packed-fp32-ops' is not a recognized feature for this target"
    msgs = [ln for ln in (proc.stderr or "").splitlines() if noise not in ln and "(ignoring feature)" not in ln]
    if proc.returncode != 0:
        raise RuntimeError("building libkvpath.so failed:\n" + "\n".join(msgs))
    if verbose and any(m.strip() for m in msgs):
        print("\n".join(msgs), file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
