"""Code-generation checks of the MFMA GEMM (CPU only: hipcc cross-compiles gfx950).

The GEMM keeps its operands in flight as buffer->LDS copies and waits for them
with explicit vmcnt counts. If the compiler cannot tell a ring slot's LDS reads
apart from the copies still landing in other slots (lost alias information), it
inserts `s_waitcnt vmcnt(0)` in the steady-state loop: every step then waits a
full memory round trip and the kernel runs about twice as slow, with correct
results. These tests read the AMD assembly of our own build and fail on that.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from pare_amd import build as B

GEMM = B.CSRC / "w4a16_gemm.hip"


def _hipcc() -> str | None:
    try:
        return B._hipcc()
    except RuntimeError:
        return None


@pytest.fixture(scope="module")
def gemm_asm(tmp_path_factory) -> str:
    cc = _hipcc()
    if cc is None or shutil.which(cc) is None and not Path(cc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "gemm.s"
    flags = [f for f in B.HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    cmd = [cc, *flags, f"-I{B.REPO_DIR / 'include'}", "--cuda-device-only", "-S", str(GEMM),
           "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def _kernels(asm: str) -> dict[str, str]:
    """Body of every w4a16_gemm_kernel instantiation, by mangled name."""
    out = {}
    for m in re.finditer(r"^(_ZN\S*w4a16_gemm_kernel\S*):", asm, re.M):
        end = asm.find("s_endpgm", m.end())
        out[m.group(1)] = asm[m.end():end]
    return out


def _loops(body: str) -> list[str]:
    """Text of each innermost loop: from its header label to the branch back to it."""
    loops = []
    for m in re.finditer(r"^(\.LBB\w+):\s*;\s*=>This Inner Loop Header", body, re.M):
        label = m.group(1)
        back = re.search(rf"s_cbranch\w*\s+{re.escape(label)}\s*$", body[m.end():], re.M)
        assert back, f"no back-branch to {label}"
        loops.append(body[m.end():m.end() + back.start()])
    return loops


def test_every_gemm_variant_compiled(gemm_asm):
    names = _kernels(gemm_asm)
    # MT in {1, 2, 4} x {fp32 zeros, u8 zeros, group-major scales/zeros}
    assert len(names) == 9, sorted(names)


def test_gemm_steady_loop_never_drains_the_copy_queue(gemm_asm):
    for name, body in _kernels(gemm_asm).items():
        loops = _loops(body)
        assert loops, f"{name}: no steady-state loop found"
        for text in loops:
            waits = re.findall(r"s_waitcnt\s+vmcnt\((\d+)\)", text)
            assert waits, f"{name}: steady-state loop has no vmcnt wait"
            assert "0" not in waits, f"{name}: vmcnt(0) inside the steady-state loop"
            assert "s_barrier" in text, f"{name}: steady-state loop lost its barrier"

