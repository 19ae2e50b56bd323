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
    """Text of each innermost loop, gathered from the compiler's block
    annotations ("=>This Inner Loop Header" and "in Loop: Header=BBx_y"),
    whatever order the blocks were laid out in."""
    loops: dict[str, list[str]] = {}
    current = None
    for line in body.splitlines():
        m = re.match(r"^(?:\.L(BB\w+):|; %bb\.\d+:)(.*)$", line)
        if m:
            note = m.group(2)
            if "Inner Loop Header" in note and m.group(1):
                current = m.group(1)
            else:
                h = re.search(r"in Loop: Header=(BB\w+)", note)
                current = h.group(1) if h else None
        if current is not None:
            loops.setdefault(current, []).append(line)
    return ["\n".join(v) for v in loops.values()]


def test_every_gemm_variant_compiled(gemm_asm):
    names = _kernels(gemm_asm)
    # MT in {1, 2, 4} x {fp32 zeros, u8 zeros, group-major scales/zeros} with
    # 128-row weight tiles (NT = 4), and MT = 4 again with 64-row tiles (NT = 2)
    tiles = sorted(re.search(r"gemm_kernelILi(\d)ELb(\d)ELb(\d)ELi(\d)E", n).groups() for n in names)
    expect = sorted([(mt, z, g, "4") for mt in "124" for z, g in (("0", "0"), ("1", "0"), ("1", "1"))]
                    + [("4", z, g, "2") for z, g in (("0", "0"), ("1", "0"), ("1", "1"))])
    assert tiles == expect, sorted(names)


def test_gemm_compute_loop_never_waits_for_copies(gemm_asm):
    """The compute waves issue no copies, so their loop (the one with the MFMAs)
    must hold no vmcnt wait at all; the producer loops wait for their own
    copies only. Every loop crosses one barrier per step."""
    for name, body in _kernels(gemm_asm).items():
        loops = _loops(body)
        mfma_loops = [t for t in loops if "v_mfma" in t]
        assert len(mfma_loops) == 1, f"{name}: expected one compute loop, found {len(mfma_loops)}"
        assert not re.search(r"s_waitcnt[^\n]*vmcnt", mfma_loops[0]), \
            f"{name}: the compute loop waits on the copy queue"
        assert "s_barrier" in mfma_loops[0], f"{name}: the compute loop lost its barrier"
        assert any("buffer_load" in t and "s_barrier" in t for t in loops), \
            f"{name}: no producer loop"


# --- split-K GEMV -----------------------------------------------------------

GEMV = B.CSRC / "w4a16_gemv.hip"


@pytest.fixture(scope="module")
def gemv_asm(tmp_path_factory) -> str:
    cc = _hipcc()
    if cc is None or shutil.which(cc) is None and not Path(cc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "gemv.s"
    flags = [f for f in B.HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    cmd = [cc, *flags, f"-I{B.REPO_DIR / 'include'}", "--cuda-device-only", "-S", str(GEMV),
           "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def _gemv_kernels(asm: str) -> dict[tuple, str]:
    """Body of every w4a16_gemv_kernel<MT, U, D, SPW, XM, ZU8> instantiation,
    keyed by (MT, U, D, SPW, XM, ZU8, mangled name). XM: 0 plain activations,
    1 act_order gather from global memory, 2 silu(gate) * up, 3 residual add +
    RMSNorm, 4 act_order gather from activations staged in LDS, 5 RMSNorm with
    sum(x^2) from a residual launch's partials. The body runs to the function's
    end label, not its first s_endpgm: the early return of one-slice launches
    can be laid out ahead of the streaming loop."""
    out = {}
    pat = r"^(_ZN\S*w4a16_gemv_kernelILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d)ELb(\d)E\S*):"
    for m in re.finditer(pat, asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        key = tuple(int(m.group(i)) for i in range(2, 8)) + (m.group(1),)
        out[key] = asm[m.end():end]
    return out


def test_gemv_ring_never_drains_before_the_stream(gemv_asm):
    """A ring variant (D >= 2) enters its streaming loop with D - 1 batches in
    flight. Any full wait (vmcnt(0)) before the loop header drains them, which
    cost 1-1.5 us per gate/up launch when the compiler once masked the
    loop-carried zero-point registers there. Left out: the in-kernel
    act_order gather (XM = 1), which must wait for its permutation loads before
    it can gather, and lanes holding more than four activation-row slices
    (M >= 3 with K > 16384), which spill registers."""
    kernels = _gemv_kernels(gemv_asm)
    rings = {k: v for k, v in kernels.items() if k[2] >= 2 and k[4] != 1 and k[0] * k[3] <= 4}
    assert len(rings) >= 16, sorted(kernels)
    for key, body in rings.items():
        name = key[-1]
        head = body.split("Inner Loop Header", 1)[0]
        assert "Inner Loop Header" in body, f"{name}: no streaming loop"
        assert not re.search(r"s_waitcnt[^\n]*vmcnt\(0\)", head), \
            f"{name}: waits for every load before the streaming loop"


def test_gemv_no_spill_on_the_common_variants(gemv_asm):
    """One and two activation rows with one slice per lane and u8 zero points
    (every Llama and Qwen decode shape up to K = 16384) must not touch scratch
    memory."""
    checked = 0
    for key, body in _gemv_kernels(gemv_asm).items():
        mt, u, d, spw, xm, zu8, name = key
        if mt <= 2 and spw == 1 and zu8 == 1:
            checked += 1
            assert "scratch_store" not in body, f"{name}: spills to scratch"
    assert checked >= 8
