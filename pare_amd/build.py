"""Builds libpare_amd.so in-tree with hipcc for gfx950.

Usage: ``python -m pare_amd.build`` (or ``pare_amd.build.build()``);
``python -m pare_amd.build sanitized`` builds the host-sanitized C ABI for
CPU tests (``build_sanitized()``).
The library is written next to this file so it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libpare_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME

SOURCES = ["capi.hip", "w4a16_gemv.hip", "w4a16_gemm.hip", "w4a16_gemm64.hip", "w4a16_skinny.hip",
           "w4a16_layout.hip", "decode_ops.hip", "gptq.hip", "probes.hip",
           "w4a16_tgemm.hip", "w4a16_bgemm.hip"]

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


def _run(cmd: list[str], verbose: bool) -> str:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    return res.stderr


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compiles every HIP source into ``pare_amd/libpare_amd.so`` (always rebuilds).

    Each source is compiled to an object of its own in parallel (``_build/``
    at the repository root, ignored by git), then the objects are linked."""
    hipcc = _hipcc()
    obj_dir = REPO_DIR / "_build"
    obj_dir.mkdir(exist_ok=True)
    flags = [f for f in HIPCC_FLAGS if f != "-shared"] + list(extra_flags or [])
    inc = f"-I{REPO_DIR / 'include'}"
    jobs = []
    for src in SOURCES:
        obj = obj_dir / (Path(src).stem + ".o")
        jobs.append((obj, [hipcc, *flags, inc, "-c", str(CSRC / src), "-o", str(obj)]))
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", "0") or 0) or os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        logs = list(pool.map(lambda j: _run(j[1], verbose), jobs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    logs.append(_run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC",
                      *[str(o) for o, _ in jobs], "-o", str(tmp)], verbose))
    if verbose:
        for log in logs:
            if log.strip():
                print(log, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer for the C ABI's
# argument validation (capi.hip): every -fsanitize goes to the host pass only
# (-Xarch_host), the device code is built exactly as in build().
SANITIZE_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                  "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]
SANITIZED_DIR = REPO_DIR / "_build" / "sanitized"


def asan_runtime() -> Path:
    """The clang AddressSanitizer runtime of the ROCm toolchain (to LD_PRELOAD
    into an uninstrumented python that loads the sanitized library)."""
    for cand in sorted(Path("/opt/rocm/llvm/lib/clang").glob("*/lib/linux/libclang_rt.asan-x86_64.so")):
        return cand
    raise RuntimeError("libclang_rt.asan-x86_64.so not found under /opt/rocm/llvm/lib/clang")


def build_sanitized(verbose: bool = False) -> Path:
    """Builds ``_build/sanitized/libpare_amd.so``: capi.hip (the C ABI and its
    host-side validation) with ASan and UBSan in the host pass, linked with the
    other sources' objects from build() (compiled first if missing). For CPU
    tests of the C ABI; the GPU box never loads it."""
    hipcc = _hipcc()
    obj_dir = REPO_DIR / "_build"
    SANITIZED_DIR.mkdir(parents=True, exist_ok=True)
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    inc = f"-I{REPO_DIR / 'include'}"
    objs = []
    for src in SOURCES:
        if src == "capi.hip":
            obj = SANITIZED_DIR / "capi.o"
            _run([hipcc, *flags, *SANITIZE_FLAGS, inc, "-c", str(CSRC / src), "-o", str(obj)], verbose)
        else:
            obj = obj_dir / (Path(src).stem + ".o")
            if not obj.exists():
                obj_dir.mkdir(exist_ok=True)
                _run([hipcc, *flags, inc, "-c", str(CSRC / src), "-o", str(obj)], verbose)
        objs.append(str(obj))
    out = SANITIZED_DIR / LIB_NAME
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address",
          "-Xarch_host", "-fsanitize=undefined", *objs, "-o", str(out)], verbose)
    return out


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "sanitized":
        print(build_sanitized(verbose=True))
    else:
        print(build(verbose=True))
