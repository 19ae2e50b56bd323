"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Bars:
  - integer/byte work (repack, RTN codes, zero conversion): bit-exact;
  - dequantised weights: bit-exact with the reference dequant path in fp32,
    fp16 and bf16;
  - layer outputs: |y - y_ref| <= atol + rtol * |y_ref| with rtol = atol = 1e-2
    in fp16 against the fp32-accumulated oracle; max-abs error is printed.
Mirrors the reference's kernel tests (pare tests/test_triton_kernel.py:108-245)
and widens them to the BASELINE shapes, group sizes and act_order.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import pare_amd as P
from oracle import pare_oracle as O
from pare_amd import _lib
from pare_amd.kernels import force_kernel



pytestmark = pytest.mark.gpu

RTOL = 1e-2
ATOL = 1e-2
KAT = json.loads((Path(__file__).parent / "golden" / "kat_int4.json").read_text())
DEV = "cuda"


def _w(N, K, seed, std=0.02):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, K, generator=g) * std).numpy().astype(np.float32)


def _x(M, K, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).to(torch.float16)


def _layer(N, K, gs, seed):
    w = _w(N, K, seed)
    packed, s, z = O.rtn_quantize(w, gs)
    return packed, s, z


def _cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _check_out(y_gpu, y_ref, what):
    y = y_gpu.float().cpu().numpy()
    err = np.abs(y - y_ref)
    bound = ATOL + RTOL * np.abs(y_ref)
    print(f"[parity] {what}: max_abs={err.max():.3e} max_rel_excess={(err - bound).max():.3e}",
          flush=True)
    assert np.isfinite(y).all(), f"{what}: non-finite output"
    assert (err <= bound).all(), f"{what}: max_abs={err.max():.4e}"


def _matmul_case(M, N, K, gs, seed, zero_u8=False, kernel="auto", gm=False):
    packed, s, z = _layer(N, K, gs, seed)
    x = _x(M, K, seed + 1000)
    w_k = P.repack_int4_for_kernel(_cuda(packed), gs)
    zz = _cuda(z)
    if zero_u8:
        zz = P.zeros_to_u8(zz)
    sz_gm = P.sz_group_major(_cuda(s), zz) if gm else None
    with force_kernel(kernel):
        name = P.kernel_choice(M, N, K, gs)
        print(f"[case] M={M} N={N} K={K} gs={gs} u8={zero_u8} gm={gm} kernel={name}", flush=True)
        y = P.matmul_w4a16(x.to(DEV), w_k, _cuda(s), zz, gs, sz_gm=sz_gm)
    torch.cuda.synchronize()
    ref = O.linear_fp32(x.float().numpy(), O.dequantize_packed(packed, s, z))
    _check_out(y, ref, f"M={M} N={N} K={K} gs={gs} u8={zero_u8} gm={gm} kernel={name}")


def test_device_is_supported():
    assert P.kernel_available(), "libpare_amd.so did not load or the device is not gfx950"


# ---------------------------------------------------------------------------
# integer / byte work: bit-exact
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K,gs", [(8, 256, 128), (16, 4096, 128), (7, 512, 32),
                                    (5, 512, 64), (3, 1024, 256), (4, 384, 384)])
def test_repack_bitexact(N, K, gs):
    q = np.random.default_rng(N * K + gs).integers(0, 16, (N, K))
    packed = O.pack_int4(q)
    got = P.repack_int4_for_kernel(_cuda(packed), gs).cpu().numpy()
    assert (got == O.repack_int4_for_kernel(packed, gs)).all()


def test_repack_golden_pattern():
    k = KAT["repack_pattern"]
    got = P.repack_int4_for_kernel(_cuda(np.array(k["storage"], dtype=np.uint8)), k["group_size"])
    assert got.cpu().tolist() == k["kernel"]


def test_repack_with_perm_bitexact():
    rng = np.random.default_rng(11)
    N, K, gs = 6, 512, 128
    q = rng.integers(0, 16, (N, K))
    perm = rng.permutation(K).astype(np.int32)
    packed = O.pack_int4(q)
    got = P.repack_int4_for_kernel(_cuda(packed), gs, perm=_cuda(perm)).cpu().numpy()
    want = O.repack_int4_for_kernel(O.permute_columns_packed(packed, perm), gs)
    assert (got == want).all()


@pytest.mark.parametrize("gs", [32, 64, 128, 256, "channel"])
@pytest.mark.parametrize("wdtype", [torch.float32, torch.float16, torch.bfloat16])
def test_rtn_producer_bitexact(gs, wdtype):
    N, K = 48, 512
    w = torch.from_numpy(_w(N, K, 21)).to(wdtype)
    wf = w.float().numpy()
    if gs == "channel":
        packed, s, z = P.rtn_quantize(w.to(DEV), granularity="per_channel")
        rp, rs, rz = O.rtn_quantize(wf, granularity="per_channel")
    else:
        packed, s, z = P.rtn_quantize(w.to(DEV), gs)
        rp, rs, rz = O.rtn_quantize(wf, gs)
    assert (packed.cpu().numpy() == rp).all()
    assert (s.cpu().numpy().view(np.uint32) == rs.view(np.uint32)).all()
    assert (z.cpu().numpy() == rz).all()


def test_rtn_producer_sym_bitexact():
    w = _w(16, 256, 5)
    packed, s, z = P.rtn_quantize(_cuda(w), 128, sym=True)
    rp, rs, rz = O.rtn_quantize(w, 128, sym=True)
    assert (packed.cpu().numpy() == rp).all()
    assert (s.cpu().numpy().view(np.uint32) == rs.view(np.uint32)).all()
    assert (z.cpu().numpy() == 0).all()


@pytest.mark.parametrize("name", ["scale_zero_asym", "scale_zero_neg", "scale_zero_flat"])
def test_rtn_golden(name):
    k = KAT[name]
    w = np.array(k["w"], dtype=np.float32)
    packed, s, z = P.rtn_quantize(_cuda(w), k["group_size"])
    assert s.item() == np.float32(k["scale"]) and z.item() == k["zero"]
    q = O.unpack_int4(packed.cpu().numpy())
    if "q" in k:
        assert q.tolist() == k["q"]
    else:
        assert q.reshape(-1)[-1] == k["q_last"]


def test_rtn_golden_sym_quirk():
    k = KAT["sym_unsigned_quirk"]
    packed, s, z = P.rtn_quantize(_cuda(np.array(k["w"], dtype=np.float32)), 128, sym=True)
    assert s.item() == np.float32(k["scale"])
    assert O.unpack_int4(packed.cpu().numpy()).reshape(-1)[:4].tolist() == k["q_head"]


def test_zeros_to_u8():
    z = np.random.default_rng(3).integers(0, 16, (64, 8, 1)).astype(np.float32)
    got = P.zeros_to_u8(_cuda(z)).cpu().numpy()
    assert got.dtype == np.uint8 and (got == z.reshape(64, 8)).all()
    bad = z.copy()
    bad[0, 0, 0] = 3.5
    bad[1, 1, 0] = 16.0
    with pytest.raises(ValueError, match="2 zero points"):
        P.zeros_to_u8(_cuda(bad))


# ---------------------------------------------------------------------------
# dequantised weights: bit-exact
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("layout", ["storage", "kernel"])
@pytest.mark.parametrize("gs", [32, 128, 256])
def test_dequant_bitexact(layout, gs):
    N, K = 40, 1024
    packed, s, z = _layer(N, K, gs, 31)
    ref32 = O.dequantize_packed(packed, s, z)
    src = _cuda(packed) if layout == "storage" else P.repack_int4_for_kernel(_cuda(packed), gs)
    for dt, view in ((torch.float32, np.uint32), (torch.float16, np.uint16)):
        got = P.dequantize_int4(src, _cuda(s), _cuda(z), gs, dtype=dt, layout=layout).cpu()
        want = ref32 if dt == torch.float32 else ref32.astype(np.float16)
        assert (got.numpy().view(view) == want.view(view)).all(), f"{layout} {dt}"
    got = P.dequantize_int4(src, _cuda(s), _cuda(z), gs, dtype=torch.bfloat16, layout=layout).cpu()
    want = torch.from_numpy(ref32).to(torch.bfloat16)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_dequant_pow2_golden():
    k = KAT["dequant_pow2"]
    # pad the 4 golden columns to one 128-column group
    q = np.zeros((1, 128), dtype=np.int32)
    q[0, :4] = k["q"][0]
    packed = O.pack_int4(q)
    s = np.full((1, 1, 1), k["scale"], dtype=np.float32)
    z = np.full((1, 1, 1), k["zero"], dtype=np.float32)
    got = P.dequantize_int4(_cuda(packed), _cuda(s), _cuda(z), 128, dtype=torch.float16)
    assert got.float().cpu().numpy()[0, :4].tolist() == k["w"][0]


@pytest.mark.parametrize("layout", ["storage", "kernel"])
def test_dequant_f16_double_rounding_ties(layout):
    """fp32 product then fp16 cast (two roundings), not one fused rounding."""
    cases = KAT["dequant_f16_ties"]
    n = len(cases)
    q = np.zeros((2 * n, 128), dtype=np.int32)
    s = np.zeros((2 * n, 1, 1), dtype=np.float32)
    z = np.zeros((2 * n, 1, 1), dtype=np.float32)
    want = np.zeros(2 * n, dtype=np.uint16)
    for i, c in enumerate(cases):
        sv = np.array([c["scale_bits"]], dtype=np.uint32).view(np.float32)[0]
        q[2 * i, 0], s[2 * i], z[2 * i], want[2 * i] = c["d"], sv, 0, c["w16"]
        q[2 * i + 1, 0], s[2 * i + 1], z[2 * i + 1] = 15 - c["d"], sv, 15
        want[2 * i + 1] = c["w16"] | 0x8000
    packed = O.pack_int4(q)
    src = _cuda(packed) if layout == "storage" else P.repack_int4_for_kernel(_cuda(packed), 128)
    got = P.dequantize_int4(src, _cuda(s), _cuda(z), 128, dtype=torch.float16, layout=layout)
    assert (got.cpu().numpy()[:, 0].view(np.uint16) == want).all()


def test_dequant_gidx_bitexact():
    rng = np.random.default_rng(41)
    N, K, gs = 24, 768, 128
    w = _w(N, K, 41)
    perm = rng.permutation(K)
    packed, s, z, g = O.rtn_quantize_act_order(w, perm, gs)
    ref = O.dequantize_gidx(O.unpack_int4(packed), s, z, g)
    got = P.dequantize_int4(_cuda(packed), _cuda(s), _cuda(z), gs, g_idx=_cuda(g)).cpu().numpy()
    assert (got.view(np.uint32) == ref.view(np.uint32)).all()
    # kernel layout with the permutation derived from g_idx reproduces the same weights
    pm = P.perm_from_g_idx(_cuda(g), gs)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs, perm=pm)
    got_k = P.dequantize_int4(wk, _cuda(s), _cuda(z), gs, layout="kernel", perm=pm).cpu().numpy()
    assert (got_k.view(np.uint32) == ref.view(np.uint32)).all()


# ---------------------------------------------------------------------------
# matmul: tolerance vs fp32-accumulated oracle
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m", [1, 4, 16, 64])
def test_matches_dequant_on_the_fly_256(m):
    """test_triton_kernel.py:127-143 shape, stricter tolerance."""
    _matmul_case(m, 256, 256, 128, 1)


def test_non_divisible_m():
    """test_triton_kernel.py:154-167."""
    for m in [1, 3, 7, 31]:
        _matmul_case(m, 256, 256, 128, 7)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 16, 17, 32, 33, 64, 65, 128])
def test_matmul_m_sweep(M):
    _matmul_case(M, 1040, 1024, 128, 100 + M)


@pytest.mark.parametrize("M", [3, 4, 8])
def test_matmul_large_n_small_m(M):
    """N >= 8192: the automatic choice moves to the MFMA GEMM from M = 3."""
    _matmul_case(M, 9000, 1024, 128, 300 + M, zero_u8=True)


@pytest.mark.parametrize("N,K", [(1024, 4096), (4096, 4096), (520, 3584), (96, 18944),
                                 (4096, 14336)])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_matmul_shapes(M, N, K):
    _matmul_case(M, N, K, 128, N + K + M)


@pytest.mark.parametrize("gs", [32, 64, 256, "channel"])
@pytest.mark.parametrize("M", [1, 3, 20])
def test_matmul_group_sizes(gs, M):
    K = 1024
    _matmul_case(M, 272, K, K if gs == "channel" else gs, 7 * M)


# Every kernel on the shapes it supports, forced explicitly (the automatic
# choice sends most small-M shapes to the skinny kernel).
KERNEL_CASES = [
    ("gemv", 1, 4096, 4096, 128), ("gemv", 3, 520, 3584, 128), ("gemv", 4, 96, 18944, 128),
    ("gemv", 2, 272, 1024, 64), ("gemv", 6, 300, 2048, 128),
    ("skinny", 1, 4096, 4096, 128), ("skinny", 2, 1040, 1024, 128), ("skinny", 4, 520, 3584, 128),
    ("skinny", 5, 272, 2048, 256), ("skinny", 13, 400, 1024, 128), ("skinny", 16, 272, 1024, 128),
    ("skinny", 1, 200, 18944, 128), ("skinny", 1, 1024, 14336, 128), ("skinny", 3, 64, 512, 512),
    ("gemm", 5, 1040, 1024, 128), ("gemm", 16, 4096, 4096, 128), ("gemm", 64, 520, 3584, 128),
    ("gemm", 17, 272, 2048, 256), ("gemm", 48, 1040, 14336, 128), ("gemm", 96, 300, 4096, 128),
    ("gemv", 32, 200, 384, 128),
]


@pytest.mark.parametrize("kernel,M,N,K,gs", KERNEL_CASES)
def test_each_kernel(kernel, M, N, K, gs):
    _matmul_case(M, N, K, gs, M * 131 + N + K, kernel=kernel)


# The register-streamed GEMM (group size 128): one and two 32-row tiles,
# ragged M inside a 64-row block and across blocks, ragged N, short and long
# K including an odd number of groups (the two K waves then differ by one
# stage), K split over up to 16 workgroups (small N) or none (large N), fp32
# and u8 zero points, with and without the group-major scale/zero copies.
GEMM64_CASES = [(1, 64, 512, False, False), (5, 272, 2048, True, False),
                (17, 100, 4096, False, False), (32, 1040, 1024, True, True),
                (33, 520, 3584, True, True), (48, 1040, 14336, False, False),
                (64, 4096, 4096, True, True), (64, 300, 18944, True, False),
                (65, 272, 2048, True, True), (100, 130, 1024, False, False),
                (128, 1040, 4096, True, True), (64, 14336, 4096, True, True),
                (40, 200, 384, True, False), (64, 128, 1152, False, True),
                (20, 36000, 640, True, True)]


@pytest.mark.parametrize("M,N,K,zero_u8,gm", GEMM64_CASES)
def test_gemm64(M, N, K, zero_u8, gm):
    _matmul_case(M, N, K, 128, M * 13 + N + K, zero_u8=zero_u8, kernel="gemm64", gm=gm)


def test_gemm64_rejects_other_group_sizes():
    packed, s, z = _layer(64, 1024, 256, 3)
    w_k = P.repack_int4_for_kernel(_cuda(packed), 256)
    with force_kernel("gemm64"), pytest.raises(RuntimeError, match="group_size == 128"):
        P.matmul_w4a16(_x(16, 1024, 4).to(DEV), w_k, _cuda(s), _cuda(z), 256)


@pytest.mark.parametrize("zero_u8", [False, True])
def test_sz_group_major_bitexact(zero_u8):
    N, K, gs = 300, 1024, 128
    _, s, z = _layer(N, K, gs, 5)
    zz = P.zeros_to_u8(_cuda(z)) if zero_u8 else _cuda(z)
    s_gm, z_gm = P.sz_group_major(_cuda(s), zz)
    torch.cuda.synchronize()
    G = K // gs
    assert s_gm.shape == (G, N) and z_gm.shape == (G, N) and z_gm.dtype == torch.uint8
    s2, z2 = s.reshape(N, G), z.reshape(N, G)
    assert (s_gm.cpu().numpy().view(np.uint32) == s2.T.view(np.uint32)).all()
    assert (z_gm.cpu().numpy() == z2.T.astype(np.uint8)).all()


def test_sz_group_major_rejects_bad_zeros():
    s = torch.ones(8, 2, device=DEV)
    z = torch.full((8, 2), 3.0, device=DEV)
    z[5, 1] = 16.0
    with pytest.raises(ValueError, match="1 zero points"):
        P.sz_group_major(s, z)


# The MFMA GEMM with the group-major scales and zeros: split and unsplit tiles,
# ragged N and M, multi-unit groups; N % 4 != 0 takes the [N, G] path.
GM_CASES = [(5, 1040, 1024, 128), (16, 4096, 4096, 128), (33, 520, 3584, 128),
            (64, 14336, 4096, 128), (64, 4096, 14336, 128), (128, 1040, 2048, 128),
            (17, 272, 2048, 256), (64, 300, 1024, 512), (40, 1042, 1024, 128)]


@pytest.mark.parametrize("M,N,K,gs", GM_CASES)
def test_gemm_group_major(M, N, K, gs):
    _matmul_case(M, N, K, gs, M * 7 + N + K, zero_u8=True, kernel="gemm", gm=True)


@pytest.mark.parametrize("kernel", ["gemv", "skinny"])
@pytest.mark.parametrize("M", [1, 4])
def test_each_kernel_u8_zeros(kernel, M):
    _matmul_case(M, 1024, 4096, 128, 77 + M, zero_u8=True, kernel=kernel)


@pytest.mark.parametrize("M", [1, 2, 16, 64])
def test_matmul_u8_zeros(M):
    _matmul_case(M, 512, 2048, 128, 3 + M, zero_u8=True)


def test_zero_input_gives_zero_output():
    packed, s, z = _layer(128, 256, 128, 2)
    w = P.repack_int4_for_kernel(_cuda(packed), 128)
    for m in (1, 8):
        y = P.matmul_w4a16(torch.zeros(m, 256, dtype=torch.float16, device=DEV), w, _cuda(s),
                           _cuda(z), 128)
        assert y.abs().max().item() == 0.0


@pytest.mark.parametrize("kernel", ["auto", "gemv", "gemm", "skinny", "gemm64"])
def test_deterministic(kernel):
    packed, s, z = _layer(4096, 4096, 128, 9)
    w = P.repack_int4_for_kernel(_cuda(packed), 128)
    for m in ((1, 4) if kernel in ("gemv", "skinny") else (1, 64)):
        x = _x(m, 4096, 10).to(DEV)
        with force_kernel(kernel):
            a = P.matmul_w4a16(x, w, _cuda(s), _cuda(z), 128)
            b = P.matmul_w4a16(x, w, _cuda(s), _cuda(z), 128)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_scales_shapes_accepted():
    packed, s, z = _layer(64, 256, 128, 12)
    w = P.repack_int4_for_kernel(_cuda(packed), 128)
    x = _x(2, 256, 13).to(DEV)
    y3 = P.matmul_w4a16(x, w, _cuda(s), _cuda(z), 128)
    y2 = P.matmul_w4a16(x, w, _cuda(s.reshape(64, 2)), _cuda(z.reshape(64, 2)), 128)
    assert torch.equal(y3, y2)


def test_matmul_rejects_bad_zeros():
    packed, s, z = _layer(64, 256, 128, 12)
    w = P.repack_int4_for_kernel(_cuda(packed), 128)
    zb = z.copy()
    zb[3, 1, 0] = 2.5
    with pytest.raises(ValueError, match="integers"):
        P.matmul_w4a16(_x(1, 256, 1).to(DEV), w, _cuda(s), _cuda(zb), 128)


def test_matmul_reference_errors():
    packed, s, z = _layer(64, 256, 128, 12)
    w = P.repack_int4_for_kernel(_cuda(packed), 128)
    with pytest.raises(RuntimeError):
        P.matmul_w4a16(_x(1, 256, 1), w, _cuda(s), _cuda(z), 128)  # CPU x
    with pytest.raises(AssertionError):
        P.matmul_w4a16(_x(1, 256, 1).to(DEV).float(), w, _cuda(s), _cuda(z), 128)
    with pytest.raises(AssertionError):
        P.matmul_w4a16(_x(2, 512, 1).to(DEV)[:, ::2], w, _cuda(s), _cuda(z), 128)


@pytest.mark.parametrize("kernel", ["auto", "gemv", "gemm", "gemm64"])
@pytest.mark.parametrize("M", [1, 16])
@pytest.mark.parametrize("N,K", [(512, 3584), (3584, 3584), (200, 18944)])
def test_matmul_act_order(M, N, K, kernel):
    """Qwen2.5-7B-style act_order: g_idx from a seeded permutation."""
    gs = 128
    rng = np.random.default_rng(N + K)
    w = _w(N, K, N + K)
    perm_np = rng.permutation(K)
    packed, s, z, g = O.rtn_quantize_act_order(w, perm_np, gs)
    x = _x(M, K, 5)
    pm = P.perm_from_g_idx(_cuda(g), gs)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs, perm=pm)
    with force_kernel(kernel):
        name = P.kernel_choice(M, N, K, gs)
        y = P.matmul_w4a16(x.to(DEV), wk, _cuda(s), _cuda(z), gs, perm=pm)
    ref = O.linear_fp32(x.float().numpy(), O.dequantize_gidx(O.unpack_int4(packed), s, z, g))
    _check_out(y, ref, f"act_order M={M} N={N} K={K} kernel={name}")


@pytest.mark.parametrize("M,N,K", [(1, 3584, 3584), (2, 3584, 3584), (1, 3584, 18944),
                                   (1, 512, 3584), (4, 4096, 8192)])
def test_gemv_act_order_lds_gather_equals_pregathered(M, N, K):
    """Where the activation rows fit 64 KiB of LDS, every GEMV workgroup stages X
    there and gathers X[:, perm] from it. Against the same GEMV on X[:, perm]
    gathered beforehand: same products, same order, identical bits."""
    gs = 128
    rng = np.random.default_rng(M + N + K)
    w = _w(N, K, M + 7)
    packed, s, z, g = O.rtn_quantize_act_order(w, rng.permutation(K), gs)
    x = _x(M, K, 11).to(DEV)
    pm = P.perm_from_g_idx(_cuda(g), gs)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs, perm=pm)
    print(f"[case] act_order gemv lds M={M} N={N} K={K}", flush=True)
    with force_kernel("gemv"):
        y = P.matmul_w4a16(x, wk, _cuda(s), _cuda(z), gs, perm=pm)
        y_pre = P.matmul_w4a16(x.index_select(1, pm.long()).contiguous(), wk, _cuda(s), _cuda(z), gs)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_pre.view(torch.int16))
    ref = O.linear_fp32(x.float().cpu().numpy(), O.dequantize_gidx(O.unpack_int4(packed), s, z, g))
    _check_out(y, ref, f"act_order gemv lds M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K,gs", [(1, 3584, 3584, 128), (2, 3584, 3584, 128),
                                      (3, 512, 3584, 128), (4, 4096, 8192, 128),
                                      (1, 3584, 18944, 128), (1, 512, 3584, 128),
                                      (1, 256, 32768, 128), (1, 512, 4096, 32),
                                      (2, 1024, 2048, 64), (1, 768, 4096, 256)])
def test_gemv_act_order_perm16_equals_int32(M, N, K, gs):
    """The GEMV's LDS gather reading the 16-bit copy of the permutation
    (pack.perm_u16): the same columns as through the int32 table, so identical
    bits, and within tolerance of the oracle. K = 32768 is the longest row the
    one-row gather stages (64 KiB); group sizes 32 to 256 move the lanes' column
    offsets within a group."""
    rng = np.random.default_rng(M + N + K + 1)
    w = _w(N, K, M + 17)
    packed, s, z, g = O.rtn_quantize_act_order(w, rng.permutation(K), gs)
    x = _x(M, K, 13).to(DEV)
    pm = P.perm_from_g_idx(_cuda(g), gs)
    p16 = P.perm_u16(pm)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs, perm=pm)
    print(f"[case] act_order gemv perm16 M={M} N={N} K={K}", flush=True)
    with force_kernel("gemv"):
        y32 = P.matmul_w4a16(x, wk, _cuda(s), _cuda(z), gs, perm=pm)
        y16 = P.matmul_w4a16(x, wk, _cuda(s), _cuda(z), gs, perm=pm, perm16=p16)
    torch.cuda.synchronize()
    assert torch.equal(y16.view(torch.int16), y32.view(torch.int16))
    ref = O.linear_fp32(x.float().cpu().numpy(), O.dequantize_gidx(O.unpack_int4(packed), s, z, g))
    _check_out(y16, ref, f"act_order gemv perm16 M={M} N={N} K={K}")


def test_perm_u16_copy_and_clamp():
    """pmi_perm_u16 copies every entry of a permutation into 16 bits (values up
    to 65535 at K = 65536), and entries outside [0, K) become 0 and are counted,
    the clamp the kernels apply to the int32 table at use: a malformed table
    gives the same GEMV bits through either copy. K > 65536 has no copy."""
    K = 65536
    perm = torch.randperm(K, generator=torch.Generator(device=DEV).manual_seed(3),
                          device=DEV).to(torch.int32)
    p16 = P.perm_u16(perm)
    assert torch.equal(p16.cpu().view(torch.uint16).to(torch.int32), perm.cpu())
    assert P.perm_u16(torch.arange(K + 128, dtype=torch.int32, device=DEV)) is None
    with pytest.raises(ValueError, match="outside"):
        P.perm_u16(torch.tensor([0, 1, 5, 2], dtype=torch.int32, device=DEV))
    # a malformed table through the C ABI: clamped and counted, same GEMV bits
    N, K, gs = 512, 3584, 128
    bad = torch.randperm(K, generator=torch.Generator(device=DEV).manual_seed(4),
                         device=DEV).to(torch.int32)
    bad[5], bad[700], bad[3000] = -1, K, K + 9
    out = torch.empty(K, dtype=torch.int16, device=DEV)
    cnt = torch.zeros(1, dtype=torch.int32, device=DEV)
    L = _lib.lib()
    assert L.pmi_perm_u16(bad.data_ptr(), out.data_ptr(), cnt.data_ptr(), K,
                          torch.cuda.current_stream().cuda_stream) == 0, _lib.last_error()
    torch.cuda.synchronize()
    assert int(cnt.item()) == 3
    assert torch.equal(out.cpu().view(torch.uint16).to(torch.int32),
                       torch.where((bad >= 0) & (bad < K), bad, 0).cpu())
    packed, s, z = O.rtn_quantize(_w(N, K, 21), gs)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs)
    x = _x(1, K, 22).to(DEV)
    with force_kernel("gemv"):
        y32 = P.matmul_w4a16(x, wk, _cuda(s), _cuda(z), gs, perm=bad)
        y16 = P.matmul_w4a16(x, wk, _cuda(s), _cuda(z), gs, perm=bad, perm16=out)
    torch.cuda.synchronize()
    assert torch.equal(y16.view(torch.int16), y32.view(torch.int16))


@pytest.mark.parametrize("M", [1, 3, 6])
def test_gemv_act_order_gathered_equals_in_kernel_gather(M):
    """With a workspace the GEMV reads X[:, perm] gathered once; without one each
    wave gathers its own columns (from LDS at M = 1, where the row fits 64 KiB;
    from global memory at M = 3 and 6, where four rows do not). Same products,
    same order: identical bits."""
    N, K, gs = 3584, 18944, 128
    rng = np.random.default_rng(M + 40)
    w = _w(N, K, M + 41)
    packed, s, z, g = O.rtn_quantize_act_order(w, rng.permutation(K), gs)
    x = _x(M, K, 9).to(DEV)
    pm = P.perm_from_g_idx(_cuda(g), gs)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs, perm=pm)
    zu8 = P.zeros_to_u8(_cuda(z))
    sd = _cuda(s).reshape(N, K // gs).contiguous()
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    need = L.pmi_matmul_workspace_bytes(M, N, K, gs, 1)
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    outs = []
    with force_kernel("gemv"):
        print(f"[case] act_order gemv gather M={M}", flush=True)
        for wsp, nb in ((ws.data_ptr(), need), (None, 0)):
            y = torch.empty(M, N, dtype=torch.float16, device=DEV)
            rc = L.pmi_matmul_w4a16(x.data_ptr(), _lib.PMI_F16, wk.data_ptr(), sd.data_ptr(),
                                    zu8.data_ptr(), _lib.PMI_U8, pm.data_ptr(), None, None, None,
                                    None, y.data_ptr(), _lib.PMI_F16, M, N, K, gs, wsp, nb, stream)
            assert rc == 0, _lib.last_error()
            outs.append(y)
    torch.cuda.synchronize()
    assert int(ws[:65536].count_nonzero()) == 0, "the counter block must stay zero"
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    ref = O.linear_fp32(x.float().cpu().numpy(), O.dequantize_gidx(O.unpack_int4(packed), s, z, g))
    _check_out(outs[0], ref, f"act_order gemv gathered M={M}")


@pytest.mark.parametrize("M", [16, 64])
def test_matmul_act_order_group_major(M):
    N, K, gs = 3584, 3584, 128
    rng = np.random.default_rng(M)
    w = _w(N, K, M + 1)
    packed, s, z, g = O.rtn_quantize_act_order(w, rng.permutation(K), gs)
    x = _x(M, K, 6)
    pm = P.perm_from_g_idx(_cuda(g), gs)
    wk = P.repack_int4_for_kernel(_cuda(packed), gs, perm=pm)
    zu8 = P.zeros_to_u8(_cuda(z))
    with force_kernel("gemm"):
        print(f"[case] act_order gm M={M}", flush=True)
        y = P.matmul_w4a16(x.to(DEV), wk, _cuda(s), zu8, gs, perm=pm,
                           sz_gm=P.sz_group_major(_cuda(s), zu8))
    ref = O.linear_fp32(x.float().numpy(), O.dequantize_gidx(O.unpack_int4(packed), s, z, g))
    _check_out(y, ref, f"act_order gm M={M}")


def test_gemm_workspace_reused_across_shapes():
    """One workspace serves split-K GEMMs of different tile counts and act_order
    gathers in any order; each result matches the oracle and the split-K
    counter block is zero again after every call."""
    L = _lib.lib()
    gs = 128
    cases = [(64, 14336, 4096, False), (16, 512, 3584, True), (48, 4096, 4096, False),
             (64, 3584, 3584, True), (17, 1024, 4096, False), (128, 2048, 4096, False)]
    need = max(L.pmi_matmul_workspace_bytes(M, N, K, gs, int(pm)) for M, N, K, pm in cases)
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    for rep in range(2):
        for i, (M, N, K, use_perm) in enumerate(cases):
            seed = 50 + i
            w = _w(N, K, seed)
            if use_perm:
                perm_np = np.random.default_rng(seed).permutation(K)
                packed, s, z, g = O.rtn_quantize_act_order(w, perm_np, gs)
                pm = P.perm_from_g_idx(_cuda(g), gs)
                ref_w = O.dequantize_gidx(O.unpack_int4(packed), s, z, g)
            else:
                packed, s, z = O.rtn_quantize(w, gs)
                pm = None
                ref_w = O.dequantize_packed(packed, s, z)
            wk = P.repack_int4_for_kernel(_cuda(packed), gs, perm=pm)
            x = _x(M, K, seed + 1)
            xd = x.to(DEV)
            sd = _cuda(s).reshape(N, K // gs).contiguous()
            zd = P.zeros_to_u8(_cuda(z))
            y = torch.empty(M, N, dtype=torch.float16, device=DEV)
            with force_kernel("gemm"):
                rc = L.pmi_matmul_w4a16(xd.data_ptr(), _lib.PMI_F16, wk.data_ptr(), sd.data_ptr(),
                                        zd.data_ptr(), _lib.PMI_U8,
                                        pm.data_ptr() if pm is not None else None, None, None, None,
                                        None, y.data_ptr(), _lib.PMI_F16, M, N, K, gs, ws.data_ptr(),
                                        ws.numel(), stream)
            assert rc == 0, _lib.last_error()
            torch.cuda.synchronize()
            assert int(ws[:65536].count_nonzero()) == 0, "split-K counters not reset"
            _check_out(y, O.linear_fp32(x.float().numpy(), ref_w),
                       f"shared workspace rep={rep} M={M} N={N} K={K} perm={use_perm}")


# ---------------------------------------------------------------------------
# QuantizedLinear integration (test_triton_kernel.py:174-245)
# ---------------------------------------------------------------------------

def _ql(N, K, seed=0, bias=False):
    torch.manual_seed(seed)
    lin = torch.nn.Linear(K, N, bias=bias)
    return P.QuantizedLinear.from_linear(lin, P.QuantConfig(bits=4, scheme="rtn", group_size=128)), lin


def test_from_linear_buffers_match_oracle():
    ql, lin = _ql(64, 256)
    rp, rs, rz = O.rtn_quantize(lin.weight.detach().numpy(), 128)
    assert (ql.packed_weight.cpu().numpy() == rp).all()
    assert (ql.scale.cpu().numpy() == rs).all() and (ql.zero.cpu().numpy() == rz).all()
    assert ql.packed_weight.shape == (64, 128) and ql.packed_weight.dtype == torch.uint8


def test_use_kernel_flag_and_matches_dequant_path():
    ql, _ = _ql(256, 256, seed=3)
    ql = ql.cuda()
    x = torch.randn(8, 256, device=DEV, dtype=torch.float16)
    with torch.no_grad():
        y_std = ql(x).float()
        ql.use_kernel = True
        y_k = ql(x).float()
    assert y_k.shape == (8, 256) and not y_k.isnan().any()
    assert (y_std - y_k).abs().max().item() < 0.05


def test_module_dequantize_bitexact():
    ql, _ = _ql(128, 512, seed=4)
    ql = ql.cuda()
    ref = O.dequantize_packed(ql.packed_weight.cpu().numpy(), ql.scale.cpu().numpy(),
                              ql.zero.cpu().numpy())
    got = ql.dequantize().cpu().numpy()
    assert (got.view(np.uint32) == ref.view(np.uint32)).all()


def test_lazy_repack_cached():
    ql, _ = _ql(128, 256)
    ql.use_kernel = True
    ql = ql.cuda()
    x = torch.randn(2, 256, device=DEV, dtype=torch.float16)
    assert not hasattr(ql, "_packed_weight_kernel")
    with torch.no_grad():
        ql(x)
    assert hasattr(ql, "_packed_weight_kernel")
    buf = id(ql._packed_weight_kernel)
    with torch.no_grad():
        ql(x)
    assert id(ql._packed_weight_kernel) == buf


def test_3d_input_and_bias():
    ql, lin = _ql(256, 256, bias=True)
    ql.use_kernel = True
    ql = ql.cuda()
    x = torch.randn(2, 64, 256, device=DEV, dtype=torch.float16)
    with torch.no_grad():
        y = ql(x)
    assert y.shape == (2, 64, 256)
    w16 = ql.dequantize(torch.float16).float()
    ref = x.float() @ w16.T + ql.bias.float()
    assert (y.float() - ref).abs().max().item() < 0.05


def test_bf16_input_round_trip_dtype():
    ql, _ = _ql(128, 256)
    ql.use_kernel = True
    ql = ql.cuda()
    x = torch.randn(3, 256, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        y = ql(x)
    assert y.dtype == torch.bfloat16
    ref = x.to(torch.float16).float() @ ql.dequantize(torch.float16).float().T
    assert (y.float() - ref).abs().max().item() < 0.05


def test_cpu_input_raises_instead_of_fallback():
    ql, _ = _ql(64, 128)
    ql.use_kernel = True
    with pytest.raises(RuntimeError, match="HIP device"):
        ql(torch.randn(4, 128))


def test_from_tensors_without_use_kernel_attr():
    ql, _ = _ql(64, 256)
    ql2 = P.QuantizedLinear.from_tensors(ql.packed_weight, None, ql.scale, ql.zero, ql.config,
                                         None, 256, 64).cuda()
    del ql2.use_kernel  # a layer object that never had the flag (linear.py:166-202)
    with torch.no_grad():
        y = ql2(torch.randn(2, 256, device=DEV, dtype=torch.float16))
    assert y.shape == (2, 64)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_act_order_module(M):
    """An act_order layer through the module: it builds the permutation from
    g_idx and its 16-bit copy once, and the forward matches the oracle."""
    rng = np.random.default_rng(8)
    N, K, gs = 96, 512, 128
    w = _w(N, K, 8)
    perm = rng.permutation(K)
    packed, s, z, g = O.rtn_quantize_act_order(w, perm, gs)
    ql = P.QuantizedLinear(_cuda(packed), _cuda(s), _cuda(z), P.QuantConfig(group_size=gs), None,
                           K, N, use_kernel=True, g_idx=_cuda(g))
    x = _x(M, K, 2)
    with torch.no_grad():
        y = ql(x.to(DEV))
    pm = P.perm_from_g_idx(_cuda(g), gs)
    assert torch.equal(ql._perm16.cpu().view(torch.uint16).to(torch.int32), pm.cpu())
    ref = O.linear_fp32(x.float().numpy(), O.dequantize_gidx(O.unpack_int4(packed), s, z, g))
    _check_out(y, ref, f"act_order module M={M}")


@pytest.mark.parametrize("M", [1, 4, 16, 64])
def test_fused_linears_match_each_layer(M):
    """q/k/v-style fusion: one launch over concatenated buffers gives every
    layer's own output (within tolerance of each layer's oracle), bias included."""
    K, gs = 512, 128
    sizes = [256, 64, 96]
    layers, refs_w, biases = [], [], []
    for i, N in enumerate(sizes):
        packed, s, z = _layer(N, K, gs, 70 + i)
        b = (torch.arange(N, dtype=torch.float32) / N - 0.5) if i != 1 else None
        layers.append(P.QuantizedLinear(_cuda(packed), _cuda(s), _cuda(z),
                                        P.QuantConfig(group_size=gs),
                                        b.to(DEV) if b is not None else None, K, N, use_kernel=True))
        refs_w.append(O.dequantize_packed(packed, s, z))
        biases.append(b)
    fused = P.FusedQuantizedLinear(layers)
    x = _x(M, K, 9)
    with torch.no_grad():
        outs = fused(x.to(DEV))
    assert [o.shape[-1] for o in outs] == sizes
    for i, (o, wref, b) in enumerate(zip(outs, refs_w, biases)):
        ref = O.linear_fp32(x.float().numpy(), wref)
        if b is not None:
            ref = ref + b.numpy()
        _check_out(o.contiguous(), ref, f"fused layer {i} M={M}")


# ---------------------------------------------------------------------------
# BASELINE full sizes
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_llama_decode_layers_full_size(N, K):
    """Llama-3.1-8B decode layers at M=1 (and the M=64 crossover side)."""
    for M in (1, 64):
        _matmul_case(M, N, K, 128, 10 + N // 1024 + M)


# ---- native bf16 activations (extension: the reference casts to fp16) -------------

def _bf16_ref(x: torch.Tensor, w_hat: np.ndarray) -> np.ndarray:
    """The oracle in bf16: the dequantised weight rounded to bf16 (nearest
    even), then x @ W^T accumulated in fp32."""
    wb = torch.from_numpy(np.ascontiguousarray(w_hat, dtype=np.float32)).bfloat16().float()
    return (x.float().cpu() @ wb.T).numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,M", [(4096, 4096, 1), (1024, 4096, 1), (14336, 4096, 1),
                                   (4096, 14336, 1), (4096, 4096, 3), (6144, 4096, 2),
                                   (1024, 4096, 7)])
def test_bf16_matmul_against_oracle(N, K, M):
    """matmul_w4a16_bf16 on the C1/C2 shapes (and 2, 3 and 7 rows); y is bf16.

    Against the fp32-accumulated oracle at rtol = atol = 1e-2. Against the
    bf16 oracle (weights rounded to bf16 first, as the reference's dequant
    path does for bf16 inputs, pare/layers/linear.py:129,138) at the same
    rtol/atol plus that oracle's own rounding bound, sum_k |x_k| |w_k| 2^-9:
    the kernel applies the weights at fp32 precision, so on long rows (K =
    14336) the two differ by up to ~0.02 from the oracle's rounding alone."""
    gs = 128
    g = torch.Generator().manual_seed(N + K + M)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    packed, s, z = O.rtn_quantize(w, gs)
    wk = P.repack_int4_for_kernel(torch.from_numpy(packed).to(DEV), gs)
    x = torch.randn(M, K, generator=g).bfloat16()
    y = P.matmul_w4a16_bf16(x.to(DEV), wk, torch.from_numpy(s).to(DEV),
                            P.zeros_to_u8(torch.from_numpy(z).to(DEV)), gs)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (M, N)
    w_hat = O.dequantize_packed(packed, s, z)
    got = y.float().cpu().numpy()
    xf = x.float().numpy()
    round_bound = (np.abs(xf) @ np.abs(w_hat).T) * 2.0 ** -9
    for ref, extra, what in ((O.linear_fp32(xf, w_hat), 0.0, "fp32"),
                             (_bf16_ref(x, w_hat), round_bound, "bf16 oracle")):
        err = np.abs(got - ref)
        print(f"[parity] bf16 M={M} N={N} K={K} vs {what}: max_abs={err.max():.3e}", flush=True)
        assert (err <= 1e-2 + 1e-2 * np.abs(ref) + extra).all(), f"{what}: max_abs={err.max():.4e}"


@pytest.mark.gpu
def test_bf16_one_hot_rows_give_the_dequantised_weight():
    """With one-hot activation rows each output is one weight: s (q - z) formed
    in fp32 and rounded to bf16, i.e. the reference's dequantisation
    (pare/core/functional.py:91) cast to bf16, bit for bit."""
    N, K, gs = 256, 1024, 128
    g = torch.Generator().manual_seed(5)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    packed, s, z = O.rtn_quantize(w, gs)
    wk = P.repack_int4_for_kernel(torch.from_numpy(packed).to(DEV), gs)
    cols = [0, 1, 63, 64, 65, 127, 128, 511, 777, 1023]
    x = torch.zeros(len(cols), K, dtype=torch.bfloat16)
    x[torch.arange(len(cols)), torch.tensor(cols)] = 1.0
    y = P.matmul_w4a16_bf16(x.to(DEV), wk, torch.from_numpy(s).to(DEV),
                            P.zeros_to_u8(torch.from_numpy(z).to(DEV)), gs)
    ref = torch.from_numpy(O.dequantize_packed(packed, s, z)[:, cols].T.copy()).bfloat16()
    assert torch.equal(y.cpu().view(torch.int16), ref.view(torch.int16))


@pytest.mark.gpu
def test_bf16_act_order_and_module_flag():
    """act_order rows (X[:, perm] gathered into the workspace first) and the
    module: default casts bf16 to fp16 as the reference does; native_bf16
    keeps bf16; both within the bar of the oracle."""
    N, K, gs = 2048, 4096, 128
    g0 = torch.Generator().manual_seed(17)
    w = (torch.randn(N, K, generator=g0) * 0.02).numpy().astype(np.float32)
    packed, s, z, g_idx = O.rtn_quantize_act_order(w, np.random.default_rng(3).permutation(K), gs)
    perm = P.perm_from_g_idx(torch.from_numpy(g_idx).to(DEV), gs)
    wk = P.repack_int4_for_kernel(torch.from_numpy(packed).to(DEV), gs, perm=perm)
    x = torch.randn(2, K, generator=g0).bfloat16()
    y = P.matmul_w4a16_bf16(x.to(DEV), wk, torch.from_numpy(s).to(DEV),
                            P.zeros_to_u8(torch.from_numpy(z).to(DEV)), gs, perm=perm)
    w_hat = O.dequantize_gidx(O.unpack_int4(packed), s, z, g_idx)
    ref = O.linear_fp32(x.float().numpy(), w_hat)
    err = np.abs(y.float().cpu().numpy() - ref)
    assert (err <= 1e-2 + 1e-2 * np.abs(ref)).all(), f"act_order bf16 max_abs={err.max():.4e}"

    lin = torch.nn.Linear(1024, 512, bias=True).to(torch.bfloat16)
    ql = P.QuantizedLinear.from_linear(lin.to(DEV), P.QuantConfig(bits=4, group_size=gs))
    ql.use_kernel = True
    xb = torch.randn(3, 5, 1024, generator=g0).bfloat16().to(DEV)
    assert ql.native_bf16 is False
    y16 = ql(xb)
    ql.native_bf16 = True
    ynat = ql(xb)
    assert y16.dtype == ynat.dtype == torch.bfloat16 and ynat.shape == (3, 5, 512)
    ref = xb.float() @ ql.dequantize(torch.float32).T + ql.bias.float()
    for yy in (y16, ynat):
        assert torch.allclose(yy.float(), ref, rtol=2e-2, atol=2e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,M", [(4096, 4096, 2), (4096, 4096, 16), (14336, 4096, 4),
                                   (14336, 4096, 16), (1024, 4096, 8), (4096, 14336, 16),
                                   (1024, 4096, 64), (6144, 4096, 5)])
def test_bf16_tiled_gemm_against_oracle(N, K, M):
    """The tiled GEMM's bf16 variant (16-row blocks, one K range; forced), with
    the same bar as the GEMV's: the fp32-accumulated oracle at rtol = atol =
    1e-2, and the bf16 oracle plus its own weight-rounding bound. Two launches
    are bit-identical, and the automatic dispatch picks the same kernel where
    an fp16 call would run on the tiled GEMM."""
    gs = 128
    g = torch.Generator().manual_seed(N + 3 * K + M)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    packed, s, z = O.rtn_quantize(w, gs)
    wk = P.repack_int4_for_kernel(torch.from_numpy(packed).to(DEV), gs)
    sd, zd = torch.from_numpy(s).to(DEV), P.zeros_to_u8(torch.from_numpy(z).to(DEV))
    sz = P.sz_group_major(sd, zd)
    wt = P.tile_w4a16(wk, gs)
    x = torch.randn(M, K, generator=g).bfloat16()
    xd = x.to(DEV)
    with force_kernel("tgemm"):
        y = P.matmul_w4a16_bf16(xd, wk, sd, zd, gs, sz_gm=sz, w_tiled=wt)
        y2 = P.matmul_w4a16_bf16(xd, wk, sd, zd, gs, sz_gm=sz, w_tiled=wt)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (M, N)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    w_hat = O.dequantize_packed(packed, s, z)
    got = y.float().cpu().numpy()
    xf = x.float().numpy()
    round_bound = (np.abs(xf) @ np.abs(w_hat).T) * 2.0 ** -9
    for ref, extra, what in ((O.linear_fp32(xf, w_hat), 0.0, "fp32"),
                             (_bf16_ref(x, w_hat), round_bound, "bf16 oracle")):
        err = np.abs(got - ref)
        print(f"[parity] bf16 tiled M={M} N={N} K={K} vs {what}: max_abs={err.max():.3e}", flush=True)
        assert (err <= 1e-2 + 1e-2 * np.abs(ref) + extra).all(), f"{what}: max_abs={err.max():.4e}"
    if P.kernel_choice(M, N, K, gs, tiled=True) == "tgemm":
        ya = P.matmul_w4a16_bf16(xd, wk, sd, zd, gs, sz_gm=sz, w_tiled=wt)
        assert torch.equal(ya.view(torch.int16), y.view(torch.int16))


@pytest.mark.gpu
def test_bf16_tiled_gemm_one_hot_rows_and_unsupported_forcing():
    """One-hot rows through the tiled bf16 variant give the reference
    dequantisation cast to bf16, bit for bit (the -(128 + z) correction MFMA
    is exact); forcing it with a permutation raises."""
    N, K, gs = 256, 2048, 128
    g = torch.Generator().manual_seed(9)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    packed, s, z = O.rtn_quantize(w, gs)
    wk = P.repack_int4_for_kernel(torch.from_numpy(packed).to(DEV), gs)
    sd, zd = torch.from_numpy(s).to(DEV), P.zeros_to_u8(torch.from_numpy(z).to(DEV))
    sz = P.sz_group_major(sd, zd)
    wt = P.tile_w4a16(wk, gs)
    cols = [0, 1, 31, 32, 63, 64, 127, 128, 1000, 2047]
    x = torch.zeros(len(cols), K, dtype=torch.bfloat16)
    x[torch.arange(len(cols)), torch.tensor(cols)] = 1.0
    with force_kernel("tgemm"):
        y = P.matmul_w4a16_bf16(x.to(DEV), wk, sd, zd, gs, sz_gm=sz, w_tiled=wt)
    ref = torch.from_numpy(O.dequantize_packed(packed, s, z)[:, cols].T.copy()).bfloat16()
    assert torch.equal(y.cpu().view(torch.int16), ref.view(torch.int16))
    perm = torch.arange(K, dtype=torch.int32, device=DEV)
    with force_kernel("tgemm"), pytest.raises(RuntimeError, match="bf16 variant"):
        P.matmul_w4a16_bf16(x.to(DEV), wk, sd, zd, gs, perm=perm, sz_gm=sz, w_tiled=wt)


@pytest.mark.gpu
def test_bf16_module_builds_the_tiled_copy():
    """A native-bf16 module at 8 rows builds its tiled copy and runs the bf16
    variant; the result equals the functional call with the same buffers."""
    lin = torch.nn.Linear(4096, 4096, bias=False)
    ql = P.QuantizedLinear.from_linear(lin.to(DEV), P.QuantConfig(bits=4, group_size=128))
    ql.use_kernel = True
    ql.native_bf16 = True
    x = torch.randn(8, 4096, generator=torch.Generator().manual_seed(2)).bfloat16().to(DEV)
    y = ql(x)
    assert ql._packed_weight_tiled is not None
    w_k, zero_u8, perm, sz_gm = ql._kernel_buffers()
    ref = P.matmul_w4a16_bf16(x, w_k, ql.scale, zero_u8, 128, sz_gm=sz_gm,
                              w_tiled=ql._packed_weight_tiled)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
