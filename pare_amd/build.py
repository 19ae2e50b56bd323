"""Builds libpare_amd.so in-tree with hipcc for gfx950.

Usage: ``python -m pare_amd.build`` (or ``pare_amd.build.build()``).
The library is written next to this file so it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libpare_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME

SOURCES = ["capi.hip", "w4a16_gemv.hip", "w4a16_gemm.hip", "w4a16_gemm64.hip", "w4a16_skinny.hip",
           "w4a16_layout.hip", "decode_ops.hip", "gptq.hip"]

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "--offload-arch=gfx950",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 arithmetic is kept out of the generated code on purpose.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden",
    # No implicit contraction: hipcc would otherwise fold (f16)(a * b) into one
    # v_fma_mixlo_f16 (a single rounding) where the reference rounds to fp32
    # first and then to fp16. Wanted fusions are written as fmaf().
    "-ffp-contract=off",
    # MFMA results in ordinary VGPRs: the accumulators feed VALU every group,
    # and AGPR operands would cost one v_accvgpr_read per value.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; cannot build libpare_amd.so")


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compiles every HIP source into ``pare_amd/libpare_amd.so`` (always rebuilds)."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), *HIPCC_FLAGS, *(extra_flags or []), f"-I{REPO_DIR / 'include'}",
           *[str(CSRC / s) for s in SOURCES], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
