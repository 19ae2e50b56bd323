"""The tiled weight layout and the tiled-weight GEMM (2..64 activation rows, more on narrow layers).

Layout: pmi_tile_w4a16 is checked byte for byte against a numpy restatement of
its documented mapping, written from the quantisation codes (not from the
kernel layout it reads), for every group size it takes and for act_order
(permuted) weights. GEMM: outputs against the fp32-accumulated oracle at
rtol = atol = 1e-2 (the bar of the other kernels), across row counts,
shapes (ragged N included), group sizes, act_order and the module path.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import pare_amd as P
from oracle import pare_oracle as O
from pare_amd import _lib
from pare_amd.kernels import force_kernel, tgemm_splits

DEV = "cuda"
RTOL = ATOL = 1e-2


def tiled_from_codes(q: np.ndarray) -> np.ndarray:
    """Tiled bytes of INT4 codes q (uint8 [N, K], values 0..15): block (panel p,
    unit u) is 4 tiles x 64 lanes x 16 bytes; lane n + 16 h of tile j holds row
    64 p + 4 n + j, byte b < 8 columns 128 u + 8 h + b (low nibble) and + 64
    (high nibble), byte b >= 8 columns 128 u + 32 + 8 h + (b - 8) and + 64;
    rows past N are zero."""
    N, K = q.shape
    P_, U = (N + 63) // 64, K // 128
    qp = np.zeros((P_ * 64, K), dtype=np.uint8)
    qp[:N] = q
    out = np.zeros((P_, U, 4, 4, 16, 16), dtype=np.uint8)  # p, u, j, h, n, b
    b = np.arange(16)
    for h in range(4):
        cols = np.where(b < 8, 8 * h + b, 32 + 8 * h + (b - 8))  # [16] within a unit
        for j in range(4):
            rows = np.arange(P_)[:, None] * 64 + 4 * np.arange(16)[None, :] + j  # [P, 16]
            for u in range(U):
                lo = qp[rows][:, :, 128 * u + cols]        # [P, 16(n), 16(b)]
                hi = qp[rows][:, :, 128 * u + cols + 64]
                out[:, u, j, h] = lo | (hi << 4)
    return out.reshape(-1)


def codes_storage(packed: np.ndarray) -> np.ndarray:
    """INT4 codes [N, K] of a storage-layout (pack_int4) weight."""
    return O.unpack_int4(packed)


def _cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _layer(N, K, gs, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy().astype(np.float32)
    return O.rtn_quantize(w, gs)


# ---- CPU: the restatement itself ------------------------------------------------

def test_tiled_restatement_places_every_code_once():
    """Brute force on a small layer: each code appears exactly once, in the
    slot the documented formula names (found by searching the tiled bytes for a
    marker)."""
    N, K = 70, 256
    q = np.zeros((N, K), dtype=np.uint8)
    t = tiled_from_codes(q)
    assert t.size == ((N + 63) // 64) * 64 * K // 2
    for row, col in [(0, 0), (5, 9), (63, 127), (64, 128), (69, 255), (17, 70), (2, 200)]:
        q[:] = 0
        q[row, col] = 7
        t = tiled_from_codes(q)
        nz = np.flatnonzero(t)
        assert nz.size == 1
        byte = t[nz[0]]
        hi = col % 128 >= 64
        assert byte == (7 << 4 if hi else 7)
        i = nz[0]
        b, L = i % 16, (i // 16) % 64
        j, pu = (i // 1024) % 4, i // 4096
        u, p = pu % (K // 128), pu // (K // 128)
        n, h = L % 16, L // 16
        assert row == 64 * p + 4 * n + j
        c = col % 128 - (64 if hi else 0)
        assert c == (8 * h + b if b < 8 else 32 + 8 * h + b - 8)
        assert col // 128 == u



# ---- GPU: layout -----------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("N,K,gs", [(64, 512, 128), (200, 1024, 32), (130, 1536, 64),
                                    (256, 2048, 256), (96, 512, 512), (4096, 4096, 128)])
def test_tile_bitexact(N, K, gs):
    packed, s, z = _layer(N, K, gs, seed=N + K)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs)
    wt = P.tile_w4a16(wk, gs).cpu().numpy()
    assert np.array_equal(wt, tiled_from_codes(codes_storage(packed)))


@pytest.mark.gpu
def test_tile_act_order_bitexact():
    N, K, gs = 128, 1024, 128
    packed, s, z = _layer(N, K, gs, seed=5)
    perm = torch.randperm(K, generator=torch.Generator().manual_seed(3)).to(torch.int32)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs, perm=perm.to(DEV))
    wt = P.tile_w4a16(wk, gs).cpu().numpy()
    q = codes_storage(packed)[:, perm.numpy()]
    assert np.array_equal(wt, tiled_from_codes(q))


@pytest.mark.gpu
def test_tile_rejects():
    L = _lib.lib()
    assert L.pmi_tile_w4a16(0x10000, 0x20000, 64, 200, 100, None) != 0  # K % gs
    assert L.pmi_tile_w4a16(0x10000, 0x20000, 64, 320, 160, None) != 0  # gs 160
    assert L.pmi_tile_w4a16(0x10000, 0x20000, 64, 192, 64, None) != 0   # K % 128
    assert L.pmi_tiled_bytes(70, 256) == 128 * 128


# ---- GPU: GEMM ---------------------------------------------------------------------

def _abi_no_workspace(x, wk, s, zu8, sz, wt, perm, gs):
    """pmi_matmul_w4a16 with no workspace at all (null, 0 bytes)."""
    M, K = x.shape
    N = wk.shape[0]
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV)
    L = _lib.lib()
    rc = L.pmi_matmul_w4a16(x.data_ptr(), _lib.PMI_F16, wk.data_ptr(), s.data_ptr(), zu8.data_ptr(),
                            _lib.PMI_U8, perm.data_ptr() if perm is not None else None, None,
                            sz[0].data_ptr(), sz[1].data_ptr(), wt.data_ptr(), y.data_ptr(),
                            _lib.PMI_F16, M, N, K, gs, None, 0,
                            torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.last_error()
    return y


def _tgemm_case(M, N, K, gs, seed, kernel="tgemm", act_order=False, no_workspace=False):
    if act_order:
        g0 = torch.Generator().manual_seed(seed)
        w = (torch.randn(N, K, generator=g0) * 0.02).numpy().astype(np.float32)
        packed, s, z, g_idx = O.rtn_quantize_act_order(w, np.random.default_rng(seed).permutation(K), gs)
        perm = P.perm_from_g_idx(_cuda(g_idx), gs)
        wk = P.repack_int4_for_kernel(_cuda(packed), gs, perm=perm)
        ref_w = O.dequantize_gidx(O.unpack_int4(packed), s, z, g_idx)
    else:
        packed, s, z = _layer(N, K, gs, seed)
        perm = None
        wk = P.repack_int4_for_kernel(_cuda(packed), gs)
        ref_w = O.dequantize_packed(packed, s, z)
    zu8 = P.zeros_to_u8(_cuda(z))
    sz = P.sz_group_major(_cuda(s), zu8)
    wt = P.tile_w4a16(wk, gs)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(M, K, generator=g).to(torch.float16)
    with force_kernel(kernel):
        if no_workspace:
            y = _abi_no_workspace(x.to(DEV), wk, _cuda(s).contiguous(), zu8.contiguous(), sz, wt,
                                  perm, gs)
        else:
            y = P.matmul_w4a16(x.to(DEV), wk, _cuda(s), zu8, gs, sz_gm=sz, w_tiled=wt, perm=perm)
    torch.cuda.synchronize()
    ref = O.linear_fp32(x.float().numpy(), ref_w)
    yy = y.float().cpu().numpy()
    err = np.abs(yy - ref)
    print(f"[parity] tgemm M={M} N={N} K={K} gs={gs} act_order={act_order}: "
          f"max_abs={err.max():.3e}", flush=True)
    assert np.isfinite(yy).all()
    assert (err <= ATOL + RTOL * np.abs(ref)).all(), f"max_abs={err.max():.4e}"
    return y


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 16, 17, 24, 32, 33, 47, 64, 65, 100])
def test_tgemm_rows(M):
    _tgemm_case(M, 1024, 2048, 128, seed=10 + M)


SPLIT_CASES = [
    # (M, N, K, gs, act_order): narrow layers up to 16 rows, K split over
    # workgroups (even and uneven quads per split, one quad per split, ragged
    # N, gs 32 / 64 / 256 and act_order with the in-kernel gather)
    (16, 512, 3584, 128, False), (16, 512, 3584, 128, True), (16, 1024, 4096, 128, False),
    (16, 1024, 3584, 128, True), (8, 1024, 4096, 128, False), (9, 512, 1536, 128, False),
    (12, 200, 2048, 32, False), (16, 1024, 3072, 64, False), (10, 512, 3584, 256, False),
    (16, 520, 8192, 128, False), (4, 512, 3584, 128, True), (13, 1024, 4096, 128, True),
    (5, 512, 8192, 128, False), (3, 200, 1536, 128, True),
    # long rows (K > 8192): four 16-row tiles per workgroup, K split four ways;
    # act_order gathered into the workspace first (the in-kernel gather stops at
    # K = 8192), one row included
    (4, 1024, 14336, 128, False), (16, 3584, 18944, 128, False), (2, 512, 18944, 128, True),
    (7, 1024, 18944, 128, True), (1, 512, 14336, 128, True), (16, 3584, 18944, 128, True),
    # 13-16 rows, 1024 < N <= 4096: four tiles per workgroup, K split four ways
    (16, 2048, 4096, 128, False), (13, 4036, 2048, 128, False)]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,gs,act_order", SPLIT_CASES)
def test_tgemm_split_k(M, N, K, gs, act_order):
    """The K split of narrow layers against the oracle; the same call twice
    gives the same bits (partials added in split order, whatever the arrival
    order), and the unsplit run (no workspace) agrees to the tolerance."""
    assert tgemm_splits(M, N, K, gs, perm=act_order) > 1
    y = _tgemm_case(M, N, K, gs, seed=M * 7 + N, act_order=act_order)
    y2 = _tgemm_case(M, N, K, gs, seed=M * 7 + N, act_order=act_order)
    assert torch.equal(y, y2)
    # without a workspace act_order needs the in-kernel gather (K <= 8192, X and
    # the perm table within the kernel's LDS)
    if not act_order or (K <= 8192 and M * (2 * K + 16) + 4 * K <= 159 * 1024):
        _tgemm_case(M, N, K, gs, seed=M * 7 + N, act_order=act_order, no_workspace=True)


@pytest.mark.gpu
def test_tgemm_split_k_counters_reset():
    """Calls of different split counts and workgroup counts alternate on one
    stream and one workspace: every call leaves the counters at zero."""
    shapes = [(16, 512, 3584), (16, 1024, 4096), (12, 2048, 4096), (16, 512, 1536), (8, 200, 2048)]
    for M, N, K in shapes + shapes[::-1]:
        _tgemm_case(M, N, K, 128, seed=M + N + K)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,act_order", [(256, 1024, 4096, False), (512, 512, 3584, False),
                                             (129, 1024, 4096, True), (200, 520, 3584, False)])
def test_tgemm_narrow_many_rows(M, N, K, act_order):
    """Narrow layers past 64 rows, where dispatch picks the tiled GEMM while its
    64-row blocks take one pass over the CUs (act_order: X[:, perm] gathered
    into the workspace first)."""
    assert P.kernel_choice(M, N, K, 128, tiled=True, perm=act_order) == "tgemm"
    _tgemm_case(M, N, K, 128, seed=M + N, kernel="auto", act_order=act_order)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 4096), (6144, 4096), (3584, 3584),
                                 (1028, 1536), (200, 2560), (4100, 2048)])
@pytest.mark.parametrize("M", [4, 16, 32, 64])
def test_tgemm_shapes(M, N, K):
    _tgemm_case(M, N, K, 128, seed=N % 97 + M)


@pytest.mark.gpu
@pytest.mark.parametrize("N", [14336, 28672])
@pytest.mark.parametrize("M", [2, 8])
def test_tgemm_gate_rows_2_and_8(M, N):
    """The plain tiled GEMM (unsplit, no act_order) at 2 and 8 rows on gate_proj
    and the fused gate/up shape."""
    assert tgemm_splits(M, N, 4096, 128) == 1
    _tgemm_case(M, N, 4096, 128, seed=N % 89 + M)


@pytest.mark.gpu
@pytest.mark.parametrize("gs", [32, 64, 256, "channel"])
@pytest.mark.parametrize("M", [5, 20])
def test_tgemm_group_sizes(gs, M):
    K = 2048
    _tgemm_case(M, 2048, K, K if gs == "channel" else gs, seed=7 + M)


@pytest.mark.gpu
@pytest.mark.parametrize("gs", [32, 64])
@pytest.mark.parametrize("M", [33, 64, 100])
def test_tgemm_small_groups_many_rows(gs, M):
    """Group sizes 32 and 64 past 32 rows: activation blocks of 32 rows, chosen
    automatically when the tiled copy is there."""
    assert P.kernel_choice(M, 4096, 4096, gs, tiled=True) == "tgemm"
    _tgemm_case(M, 4096, 4096, gs, seed=M + gs, kernel="auto")


@pytest.mark.gpu
@pytest.mark.parametrize("M", [3, 16, 29])
def test_tgemm_act_order(M):
    _tgemm_case(M, 3584, 3584, 128, seed=40 + M, act_order=True)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,gs", [
    (1, 512, 3584, 128), (2, 1024, 1536, 128), (7, 4096, 4096, 128), (16, 4096, 4096, 128),
    (16, 512, 3584, 128), (8, 2048, 7680, 128), (16, 200, 2048, 32), (11, 1028, 3072, 64),
    (16, 18944, 3584, 128)])
def test_tgemm_act_order_in_kernel_gather(M, N, K, gs):
    """Up to 16 rows the tiled GEMM gathers X[:, perm] itself from LDS (no
    workspace, no gather launch): every row count, group size and the largest
    K its LDS takes at 8 and 16 rows."""
    _tgemm_case(M, N, K, gs, seed=M * 31 + N % 89, act_order=True, no_workspace=True)


@pytest.mark.gpu
def test_tgemm_automatic_dispatch_and_determinism():
    """Gate_proj at 16 rows with the tiled copy runs on the tiled GEMM by
    itself, gives the same bits on every call, and agrees with the MFMA GEMM
    within the parity bar."""
    assert P.kernel_choice(16, 14336, 4096, 128, tiled=True) == "tgemm"
    assert P.kernel_choice(16, 14336, 4096, 128) != "tgemm"
    y0 = _tgemm_case(16, 14336, 4096, 128, seed=3, kernel="auto")
    y1 = _tgemm_case(16, 14336, 4096, 128, seed=3, kernel="auto")
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    y2 = _tgemm_case(16, 14336, 4096, 128, seed=3, kernel="gemm")
    assert torch.allclose(y0.float(), y2.float(), rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
def test_tgemm_needs_tiled_copy_when_forced():
    N, K, gs = 1024, 2048, 128
    packed, s, z = _layer(N, K, gs, 1)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs)
    x = torch.randn(8, K, device=DEV, dtype=torch.float16)
    with force_kernel("tgemm"), pytest.raises(RuntimeError, match="tiled GEMM"):
        P.matmul_w4a16(x, wk, _cuda(s), P.zeros_to_u8(_cuda(z)), gs)


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [2, 16, 32])
def test_module_builds_tiled_copy(rows):
    """QuantizedLinear builds the tiled copy on its first forward whose row
    count runs on the tiled GEMM (not at 2 rows for N = 6144) and matches its
    own dequant path."""
    torch.manual_seed(0)
    lin = torch.nn.Linear(4096, 6144, bias=False).half()
    q = P.QuantizedLinear.from_linear(lin.to(DEV), P.QuantConfig()).to(DEV)
    q.use_kernel = True
    x = torch.randn(rows, 4096, device=DEV, dtype=torch.float16)
    y = q(x)
    assert (getattr(q, "_packed_weight_tiled", None) is not None) == (rows >= 3)
    q.use_kernel = False
    ref = q(x)
    torch.cuda.synchronize()
    assert torch.allclose(y.float(), ref.float(), rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(16, 512, 3584), (5, 3584, 3584), (16, 4096, 4096), (2, 1024, 1536)])
def test_tgemm_in_kernel_gather_equals_pregathered(M, N, K):
    """The in-kernel gather of X[:, perm] gives the same bits as the tiled GEMM
    on X[:, perm] gathered beforehand (same A operands, same order of sums)."""
    gs = 128
    g0 = torch.Generator().manual_seed(M + N)
    w = (torch.randn(N, K, generator=g0) * 0.02).numpy().astype(np.float32)
    packed, s, z, g_idx = O.rtn_quantize_act_order(w, np.random.default_rng(K).permutation(K), gs)
    perm = P.perm_from_g_idx(_cuda(g_idx), gs)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs, perm=perm)
    zu8 = P.zeros_to_u8(_cuda(z))
    sz = P.sz_group_major(_cuda(s), zu8)
    wt = P.tile_w4a16(wk, gs)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(3)).to(torch.float16).to(DEV)
    with force_kernel("tgemm"):
        y_in = _abi_no_workspace(x, wk, _cuda(s).contiguous(), zu8.contiguous(), sz, wt, perm, gs)
        y_pre = _abi_no_workspace(x[:, perm.long()].contiguous(), wk, _cuda(s).contiguous(),
                                  zu8.contiguous(), sz, wt, None, gs)
    torch.cuda.synchronize()
    assert torch.equal(y_in.view(torch.int16), y_pre.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,act_order", [
    (16, 18944, 3584, False), (5, 18944, 3584, False), (16, 18944, 3584, True), (3, 18944, 3584, True),
    (8, 28672, 4096, False), (12, 20004, 1536, False), (16, 16448, 2048, False), (7, 16448, 2048, True)])
def test_tgemm_tile_ranges(M, N, K, act_order):
    """Up to 16 rows with more 64-row panels than CUs, each workgroup takes a
    range of 5-8 consecutive 16-row tiles (ragged N, and the in-kernel act_order
    gather, included)."""
    _tgemm_case(M, N, K, 128, seed=N % 101 + M, act_order=act_order, no_workspace=True)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,gs", [(16, 3584, 3584, 128), (16, 512, 3584, 128),
                                      (8, 18944, 3584, 128), (4, 1024, 4096, 128),
                                      (1, 2048, 8192, 128), (13, 4096, 2048, 128),
                                      (8, 1024, 2048, 64), (4, 512, 2048, 32),
                                      (16, 2048, 4096, 256)])
def test_tgemm_gather_perm16_equals_int32(M, N, K, gs):
    """The in-kernel act_order gather reading the 16-bit copy of the permutation
    (pack.perm_u16) instead of the int32 table: plain, K-split (k_v) and
    tile-range (18944 rows) launches, group sizes 32 to 256, give identical bits,
    within tolerance of the oracle."""
    seed = N % 89 + M
    g0 = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g0) * 0.02).numpy().astype(np.float32)
    packed, s, z, g_idx = O.rtn_quantize_act_order(w, np.random.default_rng(seed).permutation(K), gs)
    perm = P.perm_from_g_idx(_cuda(g_idx), gs)
    p16 = P.perm_u16(perm)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs, perm=perm)
    zu8 = P.zeros_to_u8(_cuda(z))
    sz = P.sz_group_major(_cuda(s), zu8)
    wt = P.tile_w4a16(wk, gs)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(seed + 1)).to(torch.float16)
    print(f"[case] tgemm gather perm16 M={M} N={N} K={K}", flush=True)
    with force_kernel("tgemm"):
        y32 = P.matmul_w4a16(x.to(DEV), wk, _cuda(s), zu8, gs, sz_gm=sz, w_tiled=wt, perm=perm)
        y16 = P.matmul_w4a16(x.to(DEV), wk, _cuda(s), zu8, gs, sz_gm=sz, w_tiled=wt, perm=perm,
                             perm16=p16)
    torch.cuda.synchronize()
    assert torch.equal(y16.view(torch.int16), y32.view(torch.int16))
    ref = O.linear_fp32(x.float().numpy(), O.dequantize_gidx(O.unpack_int4(packed), s, z, g_idx))
    err = np.abs(y16.float().cpu().numpy() - ref)
    assert (err <= ATOL + RTOL * np.abs(ref)).all(), f"max_abs={err.max():.4e}"


# ---- the big-tile variant (kernel 6): many activation rows ------------------------

BGEMM_CASES = [
    # (M, N, K): 16 x 16 tiles, a partial last activation block, a last band of
    # three panels, a last panel of 28 rows, long rows, gs 256
    (2048, 4096, 4096, 128), (1000, 4096, 4096, 128), (640, 14272, 4096, 128),
    (700, 14300, 2048, 128), (1536, 4096, 14336, 128), (1024, 4096, 4096, 256)]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,gs", BGEMM_CASES)
def test_bgemm_against_oracle(M, N, K, gs):
    """The big-tile variant against the oracle (forced, and automatic where
    dispatch picks it); the same call twice gives the same bits."""
    y = _tgemm_case(M, N, K, gs, seed=M + N % 97, kernel="bgemm")
    y2 = _tgemm_case(M, N, K, gs, seed=M + N % 97, kernel="bgemm")
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


@pytest.mark.gpu
def test_bgemm_b_operand_is_the_reference_dequant():
    """B = fp16((q - z) * s) with the reference's roundings: with x one-hot
    rows, each output is one dequantised weight times 1, so y equals the
    reference's fp16 dequantisation (pare/core/functional.py:91, then
    .to(fp16)) bit for bit, including scales whose products round to fp16
    ties."""
    N, K, gs = 512, 2048, 128
    g = torch.Generator().manual_seed(4)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy().astype(np.float32)
    packed, s, z = O.rtn_quantize(w, gs)
    # scales with many fp32 product bits: products land near fp16 ties
    s = (s * np.float32(1.0009765625) + np.float32(3e-9)).astype(np.float32)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs)
    zu8 = P.zeros_to_u8(_cuda(z))
    sz = P.sz_group_major(_cuda(s), zu8)
    wt = P.tile_w4a16(wk, gs)
    M = 256
    cols = np.arange(M) * 7 % K
    x = torch.zeros(M, K, dtype=torch.float16)
    x[torch.arange(M), torch.from_numpy(cols)] = 1.0
    with force_kernel("bgemm"):
        y = P.matmul_w4a16(x.to(DEV), wk, _cuda(s), zu8, gs, sz_gm=sz, w_tiled=wt)
    torch.cuda.synchronize()
    ref = O.dequantize_packed(packed, s, z).astype(np.float16)   # [N, K]
    assert np.array_equal(y.cpu().numpy().view(np.uint16), ref[:, cols].T.view(np.uint16))


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(2048, 4096, 4096), (512, 14336, 4096), (2048, 28672, 4096)])
def test_bgemm_automatic_dispatch(M, N, K):
    assert P.kernel_choice(M, N, K, 128, tiled=True) == "bgemm"
    _tgemm_case(M, N, K, 128, seed=N % 89 + M, kernel="auto")


@pytest.mark.gpu
def test_bgemm_act_order_gathered():
    """act_order past 64 rows: X[:, perm] gathered into the workspace, then the
    big-tile GEMM."""
    assert P.kernel_choice(2048, 4096, 4096, 128, tiled=True, perm=True) == "bgemm"
    _tgemm_case(2048, 4096, 4096, 128, seed=11, kernel="auto", act_order=True)


@pytest.mark.gpu
def test_bgemm_forced_on_unsupported_shape_raises():
    N, K, gs = 1024, 2048, 64
    packed, s, z = _layer(N, K, gs, 1)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs)
    zu8 = P.zeros_to_u8(_cuda(z))
    sz = P.sz_group_major(_cuda(s), zu8)
    wt = P.tile_w4a16(wk, gs)
    x = torch.randn(256, K, device=DEV, dtype=torch.float16)
    with force_kernel("bgemm"), pytest.raises(RuntimeError, match="big-tile"):
        P.matmul_w4a16(x, wk, _cuda(s), zu8, gs, sz_gm=sz, w_tiled=wt)
