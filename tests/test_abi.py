"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/pare_amd.h declares with the arity the ctypes binding uses, and the
host-side validation rejects malformed calls before anything is launched
(pare/kernels/matmul_int4.py:208-217 and pare/core/pack.py:113 raise there)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from pare_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "pare_amd.h"


def _declared():
    text = HEADER.read_text()
    decls = {}
    for m in re.finditer(r"PMI_API\s+[\w\s\*]+?\b(pmi_\w+)\s*\(([^)]*)\)", text, re.S):
        args = m.group(2).strip()
        decls[m.group(1)] = 0 if args in ("", "void") else len(args.split(","))
    return decls


@pytest.fixture(scope="module")
def L():
    return _lib.lib()


def test_header_declares_entry_points():
    d = _declared()
    assert {"pmi_matmul_w4a16", "pmi_repack_int4_for_kernel", "pmi_dequant_w4a16",
            "pmi_rtn_quantize", "pmi_zeros_to_u8", "pmi_last_error"} <= set(d)


def test_every_declared_symbol_is_exported_and_bound(L):
    for name, arity in _declared().items():
        assert hasattr(L, name), f"{name} not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
        assert len(_lib.SIGNATURES[name][1]) == arity, f"{name}: arity mismatch"


def test_version(L):
    assert L.pmi_abi_version() == _lib.ABI_VERSION == 16


def test_kernel_choice(L):
    # the tiled-weight GEMM, for callers that pass the tiled copy
    assert L.pmi_matmul_kernel_choice(16, 14336, 4096, 128, 1) == 5
    assert L.pmi_matmul_kernel_choice(3, 14336, 4096, 128, 1) == 5
    assert L.pmi_matmul_kernel_choice(4, 4096, 4096, 128, 1) == 5
    assert L.pmi_matmul_kernel_choice(2, 14336, 4096, 128, 1) == 5
    assert L.pmi_matmul_kernel_choice(2, 6144, 4096, 128, 1) == 1     # GEMV at 2 rows below N = 8192
    assert L.pmi_matmul_kernel_choice(1, 14336, 4096, 128, 1) == 1    # GEMV at 1 row
    assert L.pmi_matmul_kernel_choice(64, 14336, 4096, 128, 1) == 5   # 64-row blocks
    assert L.pmi_matmul_kernel_choice(2048, 4096, 4096, 128, 1) == 6  # big tiles: 16 x 16 workgroups
    assert L.pmi_matmul_kernel_choice(2048, 4096, 4096, 128, 0) != 6  # ... only with the tiled copy
    assert L.pmi_matmul_kernel_choice(2048, 4096, 4096, 64, 1) != 6   # gs 64: not the big tiles
    assert L.pmi_matmul_kernel_choice(65, 14336, 4096, 128, 1) != 5   # past 64 rows
    assert L.pmi_matmul_kernel_choice(64, 28672, 4096, 128, 1) != 5   # more than one pass
    assert L.pmi_matmul_kernel_choice(256, 1024, 4096, 128, 1) == 5   # narrow: 64-row blocks, one pass
    assert L.pmi_matmul_kernel_choice(512, 512, 3584, 128, 1) == 5
    assert L.pmi_matmul_kernel_choice(512, 1024, 4096, 128, 1) != 5   # two passes
    assert L.pmi_matmul_kernel_choice(96, 3584, 3584, 128, 1) != 5
    assert L.pmi_matmul_kernel_choice(128, 1024, 14336, 128, 1) != 5  # K > 8192
    assert L.pmi_matmul_kernel_choice(8, 28672, 4096, 128, 1) == 5
    assert L.pmi_matmul_kernel_choice(64, 4096, 4096, 64, 1) == 5    # gs 64: tiled GEMM past 4 rows
    assert L.pmi_matmul_kernel_choice(512, 4096, 4096, 32, 1) == 5
    assert L.pmi_matmul_kernel_choice(4, 4096, 4096, 64, 1) == 5
    assert L.pmi_matmul_kernel_choice(64, 4096, 4096, 64, 0) == 1    # without the copy: GEMV
    assert L.pmi_matmul_kernel_choice(8, 4096, 4096, 128, 1) == 5
    assert L.pmi_matmul_kernel_choice(32, 6144, 4096, 32, 1) == 5
    assert L.pmi_matmul_kernel_choice(16, 4096, 14336, 128, 1) == 5   # long rows: K split, 64-row tiles
    assert L.pmi_matmul_kernel_choice(2, 4096, 14336, 128, 1) == 5
    assert L.pmi_matmul_kernel_choice(1, 4096, 14336, 128, 1) == 1    # one row: GEMV
    assert L.pmi_matmul_kernel_choice(17, 4096, 14336, 128, 1) != 5   # past 16 rows
    assert L.pmi_matmul_kernel_choice(16, 14336, 14336, 128, 1) != 5  # 224 panels: no room to split
    assert L.pmi_matmul_kernel_choice(16, 1024, 4096, 128, 1) == 5    # narrow layers too
    assert L.pmi_matmul_kernel_choice(8, 512, 3584, 128, 1) == 5
    assert L.pmi_matmul_kernel_choice(4, 1024, 4096, 128, 1) == 1     # narrow at 4 rows: GEMV
    assert L.pmi_matmul_kernel_choice(16, 28672, 4096, 128, 1) != 5   # more than one pass at 16 rows
    assert L.pmi_matmul_kernel_choice(16, 18944, 3584, 128, 1) == 5   # tile ranges: one pass
    assert L.pmi_matmul_kernel_choice(16, 18944, 3584, 128, 3) == 5
    # act_order (PMI_CHOICE_PERM): the in-kernel gather up to 16 rows where X
    # and the perm table fit LDS
    TP = _lib.PMI_CHOICE_TILED | _lib.PMI_CHOICE_PERM
    assert L.pmi_matmul_kernel_choice(4, 512, 3584, 128, TP) == 5
    assert L.pmi_matmul_kernel_choice(2, 512, 3584, 128, TP) == 1     # GEMV at 2 narrow rows
    assert L.pmi_matmul_kernel_choice(2, 3584, 3584, 128, TP) == 5
    assert L.pmi_matmul_kernel_choice(16, 3584, 3584, 128, TP) == 5
    assert L.pmi_matmul_kernel_choice(1, 3584, 3584, 128, TP) == 1
    assert L.pmi_matmul_kernel_choice(4, 512, 3584, 128, _lib.PMI_CHOICE_PERM) == 1  # no copy
    assert L.pmi_matmul_kernel_choice(16, 3584, 18944, 128, TP) == 5  # long rows, X gathered first
    assert L.pmi_matmul_kernel_choice(2, 3584, 18944, 128, TP) == 5
    # GEMV for M <= 2 (M <= 4 for N < 8192); skinny MFMA kernel up to M = 16 for
    # N <= 8192 while the activations fit the LDS budget; MFMA GEMM otherwise
    assert L.pmi_matmul_kernel_choice(1, 4096, 4096, 128, 0) == 1
    assert L.pmi_matmul_kernel_choice(4, 4096, 4096, 128, 0) == 1
    assert L.pmi_matmul_kernel_choice(8, 4096, 3072, 128, 0) == 3
    assert L.pmi_matmul_kernel_choice(8, 4096, 4096, 128, 0) == 2   # 64.1 KiB of padded activations
    assert L.pmi_matmul_kernel_choice(8, 4096, 18944, 128, 0) == 2   # 296 KiB of activations
    assert L.pmi_matmul_kernel_choice(16, 4096, 4096, 128, 0) == 2   # 128 KiB of activations
    assert L.pmi_matmul_kernel_choice(4, 4096, 14336, 128, 0) == 2   # long rows: MFMA GEMM
    assert L.pmi_matmul_kernel_choice(3, 3584, 18944, 128, 0) == 2
    assert L.pmi_matmul_kernel_choice(4, 6144, 4096, 128, 0) == 1    # GEMV
    assert L.pmi_matmul_kernel_choice(3, 4096, 8192, 128, 0) == 1
    assert L.pmi_matmul_kernel_choice(1, 4096, 4096, 64, 0) == 1     # group size not % 128
    assert L.pmi_matmul_kernel_choice(64, 14336, 4096, 256, 0) == 2
    assert L.pmi_matmul_kernel_choice(64, 4096, 4096, 64, 0) == 1
    # register-streamed GEMM: from M = 128, and at M = 33..64 when its 128-row
    # blocks fill the CUs without a K split (fused gate/up, N = 28672)
    assert L.pmi_matmul_kernel_choice(64, 14336, 4096, 128, 0) == 2
    assert L.pmi_matmul_kernel_choice(64, 28672, 4096, 128, 0) == 4
    assert L.pmi_matmul_kernel_choice(32, 28672, 4096, 128, 0) == 2
    assert L.pmi_matmul_kernel_choice(128, 14336, 4096, 128, 0) == 4
    assert L.pmi_matmul_kernel_choice(512, 4096, 14336, 128, 0) == 4
    assert L.pmi_matmul_kernel_choice(128, 4096, 4096, 256, 0) == 2   # group size 256: MFMA GEMM
    assert L.pmi_matmul_kernel_choice(32, 4096, 384, 128, 0) == 1     # odd group count: GEMV
    assert L.pmi_matmul_kernel_choice(2, 14336, 4096, 128, 0) == 1    # GEMV up to M = 2
    assert L.pmi_matmul_kernel_choice(3, 14336, 4096, 128, 0) == 2    # large N: GEMM from M = 3
    assert L.pmi_matmul_kernel_choice(4, 28672, 4096, 128, 0) == 2
    assert L.pmi_matmul_kernel_choice(4, 28672, 4096, 64, 0) == 1     # no GEMM for gs 64
    assert L.pmi_matmul_kernel_choice(8, 14336, 2048, 128, 0) == 2    # skinny only for N <= 8192
    assert L.pmi_matmul_kernel_choice(5, 4096, 2048, 128, 0) == 3
    assert L.pmi_matmul_workspace_bytes(32, 4096, 384, 128, 0) == 0


def test_tgemm_splits(L):
    # K ranges of the tiled GEMM up to 16 rows where its workgroups fill at most
    # a quarter of the 256 CUs: 4 (fewer only where K has fewer unit quads)
    assert L.pmi_tgemm_splits(16, 512, 3584, 128, 0) == 4    # 32 workgroups
    assert L.pmi_tgemm_splits(16, 512, 3584, 128, 1) == 4    # act_order (in-kernel gather)
    assert L.pmi_tgemm_splits(16, 1024, 4096, 128, 0) == 4   # 64 workgroups
    assert L.pmi_tgemm_splits(12, 2048, 4096, 128, 0) == 1   # 128 workgroups: unsplit
    assert L.pmi_tgemm_splits(16, 2048, 4096, 128, 0) == 4   # 13-16 rows: four tiles per workgroup
    assert L.pmi_tgemm_splits(16, 3584, 3584, 128, 0) == 4
    assert L.pmi_tgemm_splits(16, 3584, 3584, 128, 1) == 1   # not with the act_order gather
    assert L.pmi_tgemm_splits(16, 6144, 4096, 128, 0) == 1   # 96 panels: more than a quarter
    assert L.pmi_tgemm_splits(16, 512, 1536, 128, 0) == 3    # 3 quads
    assert L.pmi_tgemm_splits(9, 200, 8192, 32, 0) == 4
    assert L.pmi_tgemm_splits(8, 512, 3584, 128, 0) == 4     # 8 rows too
    assert L.pmi_tgemm_splits(8, 3584, 3584, 128, 0) == 1    # 224 workgroups at 8 rows: unsplit
    assert L.pmi_tgemm_splits(17, 512, 3584, 128, 0) == 1    # past 16 rows: unsplit
    assert L.pmi_tgemm_splits(16, 512, 1000, 128, 0) == 1    # not a tiled GEMM shape
    assert L.pmi_tgemm_splits(4, 4096, 14336, 128, 0) == 4   # long rows: 64 workgroups of 4 tiles
    assert L.pmi_tgemm_splits(16, 3584, 18944, 128, 1) == 4
    assert L.pmi_tgemm_splits(16, 14336, 14336, 128, 0) == 1
    # the workspace covers the partial tiles (1 KiB per workgroup and split)
    # after the counter block
    assert L.pmi_matmul_workspace_bytes(16, 512, 3584, 128, 0) >= 64 * 1024 + 32 * 4 * 1024
    assert L.pmi_matmul_workspace_bytes(16, 1024, 4096, 128, 1) >= 64 * 1024 + 64 * 4 * 1024


def test_kernel_override(L):
    try:
        assert L.pmi_set_kernel_override(1) == 0
        assert L.pmi_matmul_kernel_choice(1, 4096, 4096, 128, 0) == 1
        assert L.pmi_set_kernel_override(7) == _lib.PMI_ERR_INVALID
        assert "unknown kernel" in _lib.last_error()
        assert L.pmi_set_kernel_override(3) == 1
        # forced skinny on a shape it cannot run: rejected before any launch
        assert _mm(L, M=32, N=256, K=256) == _lib.PMI_ERR_UNSUPPORTED
        assert "skinny" in _lib.last_error()
    finally:
        L.pmi_set_kernel_override(0)
    assert L.pmi_matmul_kernel_choice(1, 4096, 4096, 128, 0) == 1


FAKE = 0x10000  # 64 KiB-aligned non-null address; never dereferenced by invalid calls


def _mm(L, M=1, N=256, K=256, gs=128, x=FAKE, w=FAKE, s=FAKE, z=FAKE, zdt=_lib.PMI_F32,
        perm=None, perm16=None, y=FAKE, xdt=_lib.PMI_F16, ydt=_lib.PMI_F16, s_gm=None, z_gm=None):
    return L.pmi_matmul_w4a16(x, xdt, w, s, z, zdt, perm, perm16, s_gm, z_gm, None, y, ydt, M, N,
                              K, gs, None, 0, None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(K=200), _lib.PMI_ERR_INVALID, "divisible"),
    (dict(gs=48, K=96), _lib.PMI_ERR_UNSUPPORTED, "multiple of 32"),
    (dict(gs=0), _lib.PMI_ERR_INVALID, "group_size > 0"),
    (dict(M=-1), _lib.PMI_ERR_INVALID, "M < 0"),
    (dict(xdt=_lib.PMI_F32), _lib.PMI_ERR_UNSUPPORTED, "fp16"),
    (dict(zdt=_lib.PMI_F16), _lib.PMI_ERR_INVALID, "zero dtype"),
    (dict(x=None), _lib.PMI_ERR_INVALID, "null"),
    (dict(s=None), _lib.PMI_ERR_INVALID, "null"),
    (dict(x=FAKE + 2), _lib.PMI_ERR_INVALID, "x must be 16-byte aligned"),
    (dict(w=FAKE + 4), _lib.PMI_ERR_INVALID, "weight must be 16-byte aligned"),
    (dict(z=FAKE + 1), _lib.PMI_ERR_INVALID, "fp32 zeros"),
    (dict(s_gm=FAKE), _lib.PMI_ERR_INVALID, "together"),
    (dict(z_gm=FAKE), _lib.PMI_ERR_INVALID, "together"),
    (dict(s_gm=FAKE + 2, z_gm=FAKE), _lib.PMI_ERR_INVALID, "4-byte aligned"),
    (dict(perm16=FAKE), _lib.PMI_ERR_INVALID, "perm16 is given with perm"),
    (dict(perm=FAKE, perm16=FAKE + 8), _lib.PMI_ERR_INVALID, "16-byte alignment"),
    (dict(perm=FAKE, perm16=FAKE, K=65536 + 128), _lib.PMI_ERR_INVALID, "K <= 65536"),
])
def test_matmul_validation(L, kw, code, msg):
    rc = _mm(L, **kw)
    assert rc == code
    assert msg in _lib.last_error()


def test_matmul_empty_is_noop(L):
    assert _mm(L, M=0, x=None, w=None, s=None, z=None, y=None) == _lib.PMI_OK
    assert _mm(L, N=0, x=None, w=None, s=None, z=None, y=None) == _lib.PMI_OK
    assert _lib.last_error() == ""


def test_sz_group_major_validation(L):
    rc = L.pmi_sz_group_major(FAKE, FAKE, _lib.PMI_F16, FAKE, FAKE, None, 4, 2, None)
    assert rc == _lib.PMI_ERR_INVALID and "zero dtype" in _lib.last_error()
    rc = L.pmi_sz_group_major(FAKE, FAKE, _lib.PMI_U8, FAKE, FAKE, None, 4, 0, None)
    assert rc == _lib.PMI_ERR_INVALID and "G > 0" in _lib.last_error()
    rc = L.pmi_sz_group_major(FAKE, None, _lib.PMI_U8, FAKE, FAKE, None, 4, 2, None)
    assert rc == _lib.PMI_ERR_INVALID and "null" in _lib.last_error()
    assert L.pmi_sz_group_major(None, None, _lib.PMI_U8, None, None, None, 0, 2, None) == _lib.PMI_OK


def test_perm_u16_validation(L):
    rc = L.pmi_perm_u16(FAKE, FAKE, None, 65537, None)
    assert rc == _lib.PMI_ERR_INVALID and "K <= 65536" in _lib.last_error()
    rc = L.pmi_perm_u16(FAKE, FAKE + 8, None, 256, None)
    assert rc == _lib.PMI_ERR_INVALID and "16-byte aligned" in _lib.last_error()
    rc = L.pmi_perm_u16(FAKE + 2, FAKE, None, 256, None)
    assert rc == _lib.PMI_ERR_INVALID and "4-byte aligned" in _lib.last_error()
    rc = L.pmi_perm_u16(None, FAKE, None, 256, None)
    assert rc == _lib.PMI_ERR_INVALID and "null" in _lib.last_error()
    assert L.pmi_perm_u16(None, None, None, 0, None) == _lib.PMI_OK


def test_repack_validation(L):
    rc = L.pmi_repack_int4_for_kernel(FAKE, FAKE * 2, None, 8, 200, 128, None)
    assert rc == _lib.PMI_ERR_INVALID and "divisible" in _lib.last_error()
    rc = L.pmi_repack_int4_for_kernel(FAKE, FAKE, None, 8, 256, 128, None)
    assert rc == _lib.PMI_ERR_INVALID and "in-place" in _lib.last_error()
    assert L.pmi_repack_int4_for_kernel(None, None, None, 0, 256, 128, None) == _lib.PMI_OK


def test_dequant_validation(L):
    rc = L.pmi_dequant_w4a16(FAKE, 7, FAKE, FAKE, _lib.PMI_F32, None, FAKE, _lib.PMI_F16,
                             4, 256, 128, None)
    assert rc == _lib.PMI_ERR_INVALID and "layout" in _lib.last_error()
    rc = L.pmi_dequant_w4a16(FAKE, 0, FAKE, FAKE, _lib.PMI_F32, None, FAKE, _lib.PMI_U8,
                             4, 256, 128, None)
    assert rc == _lib.PMI_ERR_INVALID and "out dtype" in _lib.last_error()


def test_rtn_validation(L):
    rc = L.pmi_rtn_quantize(FAKE, _lib.PMI_F32, FAKE, FAKE, FAKE, 4, 100, 128, 0, None)
    assert rc == _lib.PMI_ERR_INVALID and "divisible" in _lib.last_error()
    rc = L.pmi_rtn_quantize(FAKE, _lib.PMI_F32, FAKE, FAKE, FAKE, 4, 256, 128, 3, None)
    assert rc == _lib.PMI_ERR_INVALID and "sym" in _lib.last_error()


def test_error_message_is_thread_local(L):
    import threading

    _mm(L, K=200)
    seen = {}

    def other():
        seen["msg"] = _lib.last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "divisible" in _lib.last_error()


def test_pmi_error_maps_to_runtime_error():
    with pytest.raises(RuntimeError, match="PMI_ERR_INVALID"):
        _lib.call("pmi_repack_int4_for_kernel", FAKE, FAKE * 2, None, 8, 200, 128, None)
