"""Bounded determinism soak of the cross-workgroup combines.

Five kernels finish with a last-workgroup combine: the split-K MFMA GEMM, the
register-streamed GEMM and the tiled GEMM's K split of narrow layers (partial
tiles + a per-tile counter), the split decode attention (per-split max/sum/P.V partials) and the argmax (per-chunk
maxima). Each combine adds its partials in a fixed order, so every call must
give the same bits. Here 320 calls over mixed shapes, interleaved so that one
workspace serves them all in turn, are each compared bit for bit with the
first result of their case; the test stops at the first mismatch. Every call
is bounded (no kernel waits on another workgroup), so a failure is a wrong
value, never a hang.
"""

from __future__ import annotations

import pytest
import torch

import pare_amd as P
from pare_amd import _lib
from pare_amd.decoder import argmax_into, decode_attention
from pare_amd.kernels import force_kernel, tgemm_splits

pytestmark = pytest.mark.gpu

DEV = "cuda"
GS = 128
ROUNDS = 40


def _layer(N, K, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(N, K, generator=g, device=DEV) * 0.02
    packed, s, z = P.rtn_quantize(w, GS)
    return P.repack_int4_for_kernel(packed, GS), s.reshape(N, -1), P.zeros_to_u8(z).reshape(N, -1)


def _matmul_case(kernel, M, N, K, seed):
    wk, s, z = _layer(N, K, seed)
    x = torch.randn(M, K, generator=torch.Generator(device=DEV).manual_seed(seed + 1),
                    device=DEV).half()
    sz = P.sz_group_major(s, z)
    L = _lib.lib()
    with force_kernel(kernel):
        need = L.pmi_matmul_workspace_bytes(M, N, K, GS, 0)
    assert need > 0, f"{kernel} M={M} N={N} K={K} must split K (a combine to soak)"

    def run():
        with force_kernel(kernel):
            return P.matmul_w4a16(x, wk, s, z, GS, sz_gm=sz)
    return f"{kernel} M={M} N={N} K={K}", run


def _tgemm_split_case(M, N, K, seed):
    wk, s, z = _layer(N, K, seed)
    x = torch.randn(M, K, generator=torch.Generator(device=DEV).manual_seed(seed + 1),
                    device=DEV).half()
    sz = P.sz_group_major(s, z)
    wt = P.tile_w4a16(wk, GS)
    assert tgemm_splits(M, N, K, GS) > 1, f"tgemm M={M} N={N} K={K} must split K"

    def run():
        with force_kernel("tgemm"):
            return P.matmul_w4a16(x, wk, s, z, GS, sz_gm=sz, w_tiled=wt)
    return f"tgemm split M={M} N={N} K={K}", run


def _attention_case(B, H, KV, L, p, seed):
    D = 128
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(B, H, 1, D, generator=g, device=DEV).half()
    ck = torch.randn(B, KV, L, D, generator=g, device=DEV).half()
    cv = torch.randn(B, KV, L, D, generator=g, device=DEV).half()
    pos = torch.full((1,), p, dtype=torch.long, device=DEV)
    return (f"attention B={B} H={H} KV={KV} L={L} p={p}",
            lambda: decode_attention(q, ck, cv, pos, 1 / D ** 0.5))


def _argmax_case(rows, n, seed):
    x = torch.randn(rows, n, generator=torch.Generator(device=DEV).manual_seed(seed),
                    device=DEV).half()
    out = torch.empty(rows, 1, dtype=torch.long, device=DEV)

    def run():
        argmax_into(x, out)
        return out.clone()
    return f"argmax rows={rows} n={n}", run


def test_combines_are_deterministic_under_repetition():
    cases = [
        _matmul_case("gemm", 16, 4096, 4096, 1),
        _matmul_case("gemm", 64, 1024, 4096, 2),
        _matmul_case("gemm64", 64, 4096, 4096, 3),
        _tgemm_split_case(16, 512, 3584, 7),
        _tgemm_split_case(8, 1024, 4096, 8),
        _attention_case(4, 32, 8, 640, 639, 4),
        _attention_case(1, 32, 8, 2048, 1500, 5),
        _argmax_case(4, 128256, 6),
    ]
    first = {}
    for rnd in range(ROUNDS):
        for name, run in cases:
            y = run()
            torch.cuda.synchronize()
            if rnd == 0:
                first[name] = y.clone()
                print(f"[soak] {name}: reference taken", flush=True)
                continue
            same = torch.equal(y.view(torch.int16) if y.dtype == torch.float16 else y,
                               first[name].view(torch.int16) if y.dtype == torch.float16 else first[name])
            assert same, f"round {rnd}: {name} differs from its first result"
    print(f"[soak] {ROUNDS * len(cases)} calls, every result identical to its first", flush=True)
