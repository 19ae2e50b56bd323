"""pmi_matmul_w4a16_noalloc (the allocation-free entry point) against
pmi_matmul_w4a16 with a caller workspace, through the C ABI: identical bits
on two calls in a row, the second with a smaller input, for the split-K MFMA
GEMM and for act_order (X gathered into the scratch); and a clear error for a
shape whose scratch need exceeds the library's fixed array."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import pare_amd as P
from oracle import pare_oracle as O
from pare_amd import _lib

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
GS = 128


def _layer(N, K, seed, act_order=False):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    perm = None
    if act_order:
        perm = np.random.default_rng(seed).permutation(K).astype(np.int32)
        packed, s, z = O.rtn_quantize(w[:, perm], GS)
        perm_t = torch.from_numpy(perm).to(DEV)
    else:
        packed, s, z = O.rtn_quantize(w, GS)
        perm_t = None
    wk = P.repack_int4_for_kernel(torch.from_numpy(packed).to(DEV), GS)
    s_t = torch.from_numpy(s.reshape(N, -1)).to(DEV).contiguous()
    z_t = P.zeros_to_u8(torch.from_numpy(z.reshape(N, -1)).to(DEV)).contiguous()
    return wk, s_t, z_t, perm_t


def _tiled(layer):
    """The group-major scale/zero copies and the tiled weight copy of a layer."""
    wk, s, z, _ = layer
    s_gm, z_gm = P.sz_group_major(s, z)
    return s_gm, z_gm, P.tile_w4a16(wk, GS)


def _call(fn, x, layer, N, K, ws=None, tiled=None):
    wk, s, z, perm = layer
    M = x.shape[0]
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV)
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    s_gm, z_gm, w_t = (t.data_ptr() for t in tiled) if tiled is not None else (None, None, None)
    p16 = P.perm_u16(perm) if perm is not None else None  # the act_order GEMV reads it
    common = (x.data_ptr(), _lib.PMI_F16, wk.data_ptr(), s.data_ptr(), z.data_ptr(), _lib.PMI_U8,
              perm.data_ptr() if perm is not None else None,
              p16.data_ptr() if p16 is not None else None, s_gm, z_gm, w_t, y.data_ptr(),
              _lib.PMI_F16, M, N, K, GS)
    if fn == "noalloc":
        rc = L.pmi_matmul_w4a16_noalloc(*common, stream)
    else:
        rc = L.pmi_matmul_w4a16(*common, ws.data_ptr() if ws is not None else None,
                                ws.numel() if ws is not None else 0, stream)
    return rc, y


@pytest.mark.parametrize("N,K,Ms,act_order", [
    (4096, 4096, (16, 8), False),      # split-K MFMA GEMM: counters + partial tiles in scratch
    (1024, 4096, (64, 40), False),     # split-K, other tiling
    (3584, 3584, (16, 1), True),       # act_order GEMM gather, then the GEMV
    (512, 3584, (32, 5), True),
])
def test_noalloc_equals_workspace_path(N, K, Ms, act_order):
    layer = _layer(N, K, seed=N + K, act_order=act_order)
    L = _lib.lib()
    for M in Ms:   # two calls in a row, the second smaller
        x = torch.randn(M, K, generator=torch.Generator(device=DEV).manual_seed(M), device=DEV).half()
        need = L.pmi_matmul_workspace_bytes(M, N, K, GS, int(act_order))
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=DEV) if need else None
        rc, want = _call("workspace", x, layer, N, K, ws)
        assert rc == 0, _lib.last_error()
        rc, got = _call("noalloc", x, layer, N, K)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        print(f"[noalloc] N={N} K={K} M={M} act_order={act_order} need={need} "
              f"kernel={P.kernel_choice(M, N, K, GS)}", flush=True)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (M, N, K)


@pytest.mark.parametrize("N,K,Ms,act_order", [
    (14336, 4096, (16, 8), False),     # tiled-weight GEMM, no scratch
    (3584, 3584, (24, 5), True),       # tiled-weight GEMM on X[:, perm] gathered into the scratch
])
def test_noalloc_tiled_equals_workspace_path(N, K, Ms, act_order):
    layer = _layer(N, K, seed=N + 3, act_order=act_order)
    tiled = _tiled(layer)
    L = _lib.lib()
    for M in Ms:   # two calls in a row, the second smaller
        assert P.kernel_choice(M, N, K, GS, tiled=True) == "tgemm"
        x = torch.randn(M, K, generator=torch.Generator(device=DEV).manual_seed(M), device=DEV).half()
        need = L.pmi_matmul_workspace_bytes(M, N, K, GS, int(act_order))
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=DEV) if need else None
        rc, want = _call("workspace", x, layer, N, K, ws, tiled)
        assert rc == 0, _lib.last_error()
        rc, got = _call("noalloc", x, layer, N, K, tiled=tiled)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        print(f"[noalloc] tiled N={N} K={K} M={M} act_order={act_order} need={need}", flush=True)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (M, N, K)


def test_noalloc_rejects_oversized_scratch():
    """M = 2048 act_order on K = 18944 needs its gathered X (74 MiB) in the
    scratch: refused with PMI_ERR_UNSUPPORTED before anything is launched."""
    L = _lib.lib()
    M, N, K = 2048, 3584, 18944
    assert L.pmi_matmul_workspace_bytes(M, N, K, GS, 1) > (16 << 20)
    dummy = torch.zeros(16, dtype=torch.uint8, device=DEV)
    p = dummy.data_ptr()
    rc = L.pmi_matmul_w4a16_noalloc(p, _lib.PMI_F16, p, p, p, _lib.PMI_U8, p, None, None, None,
                                    None, p, _lib.PMI_F16, M, N, K, GS,
                                    torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.PMI_ERR_UNSUPPORTED
    assert "scratch" in _lib.last_error() and "16777216" in _lib.last_error()
