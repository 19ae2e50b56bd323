"""Device-side INT4 layout operators (HIP): repack, zero-point conversion,
dequantisation and the act_order permutation helper.

Mirrors pare/core/pack.py:88-132 (``repack_int4_for_kernel``) and
pare/layers/linear.py:101-118 / pare/core/functional.py:78-91 (dequantise),
running on the HIP device only.
"""

from __future__ import annotations

import torch

from . import _lib
from .kernels import _DeviceGuard, _stream_handle, _to_2d, _validated_zero_tensor


def _require_cuda(t: torch.Tensor, fn: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{fn} runs on the HIP device; got a tensor on {t.device}")


def repack_int4_for_kernel(packed: torch.Tensor, group_size: int = 128, *,
                           perm: torch.Tensor | None = None) -> torch.Tensor:
    """Storage-layout INT4 weights [N, K//2] -> kernel layout, same shape and bytes
    (pare/core/pack.py:88-132), computed in one HIP pass.

    ``perm`` (int32 [K]) first reorders the columns as q[:, perm] (act_order).
    """
    L = _lib.lib()
    _require_cuda(packed, "repack_int4_for_kernel")
    assert packed.dtype == torch.uint8 and packed.dim() == 2, "packed must be uint8 [N, K//2]"
    N, K_half = packed.shape
    K = K_half * 2
    assert K % group_size == 0, f"K={K} must be divisible by group_size={group_size}"
    src = packed.contiguous()
    out = torch.empty_like(src)
    if perm is not None:
        assert perm.dtype == torch.int32 and perm.numel() == K and perm.device == packed.device
        perm = perm.contiguous()
    with _DeviceGuard(packed.device):
        _lib.check(L.pmi_repack_int4_for_kernel(
            src.data_ptr(), out.data_ptr(), perm.data_ptr() if perm is not None else None,
            N, K, group_size, _stream_handle(packed.device)), "pmi_repack_int4_for_kernel")
    return out


def zeros_to_u8(zeros: torch.Tensor) -> torch.Tensor:
    """fp32 zero points [N, G(, 1)] -> uint8 [N, G]; raises ValueError unless
    every value is an integer in [0, 15]."""
    L = _lib.lib()
    _require_cuda(zeros, "zeros_to_u8")
    z = _to_2d(zeros).float().contiguous()
    out = torch.empty(z.shape, dtype=torch.uint8, device=z.device)
    bad = torch.zeros(1, dtype=torch.int32, device=z.device)
    with _DeviceGuard(z.device):
        _lib.check(L.pmi_zeros_to_u8(z.data_ptr(), out.data_ptr(), bad.data_ptr(), z.numel(),
                                     _stream_handle(z.device)), "pmi_zeros_to_u8")
    if int(bad.item()) != 0:
        raise ValueError(f"{int(bad.item())} zero points are not integers in [0, 15]")
    return out


def sz_group_major(scales: torch.Tensor, zeros: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Group-major copies of a layer's scales and zero points, fp32 [G, N] and
    uint8 [G, N], for the MFMA GEMM (``matmul_w4a16(..., sz_gm=...)``): one
    group's scales and zeros of consecutive rows are contiguous. Built once per
    layer, like the kernel-layout weight. Raises ValueError unless every zero
    point is an integer in [0, 15]."""
    L = _lib.lib()
    _require_cuda(scales, "sz_group_major")
    s = _to_2d(scales).float().contiguous()
    z = _to_2d(zeros)
    z = z.contiguous() if z.dtype == torch.uint8 else z.float().contiguous()
    assert s.shape == z.shape and s.device == z.device, "scales and zeros must be [N, G] on one device"
    N, G = s.shape
    s_gm = torch.empty(G, N, dtype=torch.float32, device=s.device)
    z_gm = torch.empty(G, N, dtype=torch.uint8, device=s.device)
    bad = torch.zeros(1, dtype=torch.int32, device=s.device)
    zdt = _lib.PMI_U8 if z.dtype == torch.uint8 else _lib.PMI_F32
    with _DeviceGuard(s.device):
        _lib.check(L.pmi_sz_group_major(s.data_ptr(), z.data_ptr(), zdt, s_gm.data_ptr(),
                                        z_gm.data_ptr(), bad.data_ptr(), N, G,
                                        _stream_handle(s.device)), "pmi_sz_group_major")
    if int(bad.item()) != 0:
        raise ValueError(f"{int(bad.item())} zero points are not integers in [0, 15]")
    return s_gm, z_gm


def tile_w4a16(w_kernel: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """Tiled copy (uint8, ``pmi_tiled_bytes(N, K)`` bytes) of a kernel-layout
    INT4 weight [N, K//2] for the tiled-weight GEMM (``matmul_w4a16(...,
    w_tiled=...)``): 64-row panels x 128-column units, each a 4 KiB block that
    a wave reads as four contiguous 1 KiB runs. Built once per layer, like the
    kernel-layout weight; with act_order, tile the permuted kernel layout."""
    L = _lib.lib()
    _require_cuda(w_kernel, "tile_w4a16")
    assert w_kernel.dtype == torch.uint8 and w_kernel.dim() == 2, "w_kernel must be uint8 [N, K//2]"
    N, K_half = w_kernel.shape
    K = K_half * 2
    w = w_kernel.contiguous()
    if w.data_ptr() % 16:
        w = w.clone()
    out = torch.empty(L.pmi_tiled_bytes(N, K), dtype=torch.uint8, device=w.device)
    with _DeviceGuard(w.device):
        _lib.check(L.pmi_tile_w4a16(w.data_ptr(), out.data_ptr(), N, K, group_size,
                                    _stream_handle(w.device)), "pmi_tile_w4a16")
    return out


def tiled_supported(N: int, K: int, group_size: int) -> bool:
    """Whether the tiled-weight GEMM can run an [N, K] layer of this group size."""
    return (N % 4 == 0 and K % 512 == 0 and K >= 1536 and K % group_size == 0
            and (group_size in (32, 64) or group_size % 128 == 0))


_OUT_DTYPES = {torch.float16: _lib.PMI_F16, torch.bfloat16: _lib.PMI_BF16,
               torch.float32: _lib.PMI_F32}


def dequantize_int4(packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor,
                    group_size: int, *, dtype: torch.dtype = torch.float32,
                    layout: str = "storage", g_idx: torch.Tensor | None = None,
                    perm: torch.Tensor | None = None) -> torch.Tensor:
    """Dequantised weights [N, K] in the original column order.

    w = (float(q) - zero) * scale in fp32 (pare/core/functional.py:90-91), then
    one round-to-nearest-even cast to ``dtype``: bit-exact with the reference's
    ``QuantizedLinear.dequantize().to(dtype)`` (pare/layers/linear.py:101-118,129).
    layout="storage" reads pack_int4 order (optional g_idx, int32 [K]);
    layout="kernel" reads repack_int4_for_kernel order (optional perm).
    """
    L = _lib.lib()
    _require_cuda(packed, "dequantize_int4")
    if dtype not in _OUT_DTYPES:
        raise ValueError(f"unsupported output dtype {dtype}")
    N, K_half = packed.shape
    K = K_half * 2
    G = K // group_size
    s2 = _to_2d(scale).float().contiguous()
    z2, zdt = (_to_2d(zero).contiguous(), _lib.PMI_U8) if zero.dtype == torch.uint8 else \
        (_to_2d(zero).float().contiguous(), _lib.PMI_F32)
    assert tuple(s2.shape) == (N, G) and tuple(z2.shape) == (N, G), \
        f"scale/zero must be [N, G]=[{N}, {G}]"
    if layout == "storage":
        lay, idx = _lib.PMI_LAYOUT_STORAGE, g_idx
        assert perm is None, "perm applies to the kernel layout"
    elif layout == "kernel":
        lay, idx = _lib.PMI_LAYOUT_KERNEL, perm
        assert g_idx is None, "g_idx applies to the storage layout"
    else:
        raise ValueError(f"unknown layout {layout!r}")
    if idx is not None:
        assert idx.dtype == torch.int32 and idx.numel() == K and idx.device == packed.device
        idx = idx.contiguous()
    out = torch.empty(N, K, dtype=dtype, device=packed.device)
    with _DeviceGuard(packed.device):
        _lib.check(L.pmi_dequant_w4a16(
            packed.contiguous().data_ptr(), lay, s2.data_ptr(), z2.data_ptr(), zdt,
            idx.data_ptr() if idx is not None else None, out.data_ptr(), _OUT_DTYPES[dtype],
            N, K, group_size, _stream_handle(packed.device)), "pmi_dequant_w4a16")
    return out


def perm_u16(perm: torch.Tensor) -> torch.Tensor | None:
    """The 16-bit copy of an act_order permutation (int16 [K] holding the
    uint16 values) for ``matmul_w4a16(..., perm16=...)``, built once per layer;
    None when K > 65536 (no 16-bit copy exists). Raises ValueError unless every
    entry lies in [0, K)."""
    L = _lib.lib()
    _require_cuda(perm, "perm_u16")
    assert perm.dtype == torch.int32 and perm.dim() == 1, "perm must be an int32 [K] tensor"
    K = perm.numel()
    if K > 65536:
        return None
    p = perm.contiguous()
    out = torch.empty(K, dtype=torch.int16, device=p.device)
    bad = torch.zeros(1, dtype=torch.int32, device=p.device)
    with _DeviceGuard(p.device):
        _lib.check(L.pmi_perm_u16(p.data_ptr(), out.data_ptr(), bad.data_ptr(), K,
                                  _stream_handle(p.device)), "pmi_perm_u16")
    if int(bad.item()) != 0:
        raise ValueError(f"{int(bad.item())} permutation entries lie outside [0, {K})")
    return out


def perm_from_g_idx(g_idx: torch.Tensor, group_size: int) -> torch.Tensor:
    """Column order that makes act_order groups contiguous: perm with
    g_idx[perm[j]] == j // group_size. Requires exactly group_size columns per
    group (the GPTQ act_order layout); raises ValueError otherwise."""
    g = g_idx.to(torch.int64)
    K = g.numel()
    G = K // group_size
    if K % group_size != 0 or G == 0:
        raise ValueError(f"g_idx length {K} is not a multiple of group_size={group_size}")
    if bool(((g < 0) | (g >= G)).any()):
        raise ValueError("g_idx holds group indices outside [0, K/group_size)")
    counts = torch.bincount(g, minlength=G)
    if bool((counts != group_size).any()):
        raise ValueError("every act_order group must hold exactly group_size columns")
    return torch.sort(g, stable=True).indices.to(torch.int32)
