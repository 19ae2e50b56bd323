"""Fused INT4 W4A16 matmul on MI355X — the operator API of the kernel path.

Mirrors pare/kernels/matmul_int4.py:183-248 (``matmul_w4a16``,
``triton_available``) with the Triton kernel replaced by hand-written HIP
kernels for gfx950 behind libpare_amd.so:
  - M <= 2, or M <= 4 with N < 8192 and K <= 8192: split-K GEMV
    (w4a16_gemv.hip), HBM-bandwidth bound;
  - M <= 16 with the activations within 64 KiB of LDS and group size % 128 == 0:
    the skinny MFMA kernel (w4a16_skinny.hip);
  - otherwise: MFMA GEMM (w4a16_gemm.hip) for group sizes that are multiples
    of 128 and K % 256 == 0, or the GEMV four activation rows at a time.
There is no CPU or PyTorch fallback: every call runs the HIP library or raises.
"""

from __future__ import annotations

import torch

from . import _lib


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class _DeviceGuard:
    """Makes `device` the current HIP device for the duration of a launch."""

    def __init__(self, device: torch.device):
        self.device = device
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if self.device.index is not None and self.device.index != cur:
            self.prev = cur
            torch.cuda.set_device(self.device)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def kernel_available() -> bool:
    """True if libpare_amd.so is built and the current device is a gfx950 GPU
    (the probe the reference calls ``triton_available``, matmul_int4.py:246-248)."""
    try:
        L = _lib.lib()
    except (RuntimeError, OSError):
        return False
    if not torch.cuda.is_available():
        return False
    return L.pmi_device_supported(torch.cuda.current_device()) == 1


# The reference's tests and callers probe the kernel with this name.
triton_available = kernel_available


def _to_2d(t: torch.Tensor) -> torch.Tensor:
    """[N] -> [N,1], [N,G,1] -> [N,G] (matmul_int4.py:219-225)."""
    if t.dim() == 1:
        return t.unsqueeze(1)
    if t.dim() == 3:
        return t.squeeze(2)
    if t.dim() == 0:
        return t.reshape(1, 1)
    return t


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _validated_zero_tensor(zeros: torch.Tensor) -> tuple[torch.Tensor, int]:
    """Zero points as the kernels read them: u8 as-is, anything else as fp32
    after a one-time check (cached per tensor version) that every value is an
    integer in [0, 15], the INT4 contract of pare/core/scale.py:89-90."""
    if zeros.dtype == torch.uint8:
        return zeros, _lib.PMI_U8
    z = zeros.float()
    stamp = (zeros.data_ptr(), zeros._version)
    if getattr(zeros, "_pmi_checked", None) != stamp:
        bad = ((z < 0) | (z > 15) | (z != torch.round(z))).any().item()
        if bad:
            raise ValueError("zeros must hold integers in [0, 15] for INT4 (asymmetric RTN/GPTQ/AWQ "
                             "zero points); got values outside that set")
        try:
            zeros._pmi_checked = stamp
        except (AttributeError, RuntimeError):
            pass
    return z, _lib.PMI_F32


_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def _workspace(dev: torch.device, stream: int, nbytes: int) -> torch.Tensor | None:
    """Zero-filled scratch for the GEMM's split-K counters/partials and the
    act_order gather, one per (device, stream): launches on one stream are
    ordered, so they can share it (each call leaves it zero-filled again)."""
    if nbytes == 0:
        return None
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _WORKSPACES[key] = ws
    return ws


def matmul_w4a16(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    group_size: int,
    *,
    perm: torch.Tensor | None = None,
    perm16: torch.Tensor | None = None,
    sz_gm: tuple[torch.Tensor, torch.Tensor] | None = None,
    w_tiled: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Y[M,N] = X[M,K] @ dequant(W)^T with the dequantisation fused (fp16 in, fp16 out).

    Same arguments and errors as the reference (matmul_int4.py:183-217):
      x:             [M, K] float16, contiguous, on a HIP device.
      packed_weight: [N, K//2] uint8 in *kernel layout* (``repack_int4_for_kernel``).
      scales:        [N], [N, G] or [N, G, 1], any float dtype (read as fp32).
      zeros:         same shape as scales; fp32 integer values or uint8.
      group_size:    quantisation group size; the K-tile of the kernel layout.
    Extensions: ``perm`` (int32 [K]) for act_order layers whose weights were
    repacked with the same permutation, and ``perm16``, its ``pack.perm_u16``
    copy, which the GEMV's act_order gather reads instead (same results);
    ``sz_gm``, the group-major copies of
    scales and zeros from ``pack.sz_group_major`` (fp32 and uint8 [G, N]), which
    the MFMA GEMM reads as contiguous runs; ``w_tiled``, the ``pack.tile_w4a16``
    copy of the weights, which (with ``sz_gm``) lets 3..32 activation rows run
    on the tiled-weight GEMM; ``out`` to write into a preallocated [M, N] fp16
    tensor.
    Raises RuntimeError when x is not on a HIP device or the library is
    missing; AssertionError on layout violations, like the reference.
    """
    if not x.is_cuda:
        raise RuntimeError("matmul_w4a16 requires HIP (cuda) tensors.")
    assert x.is_contiguous(), "x must be contiguous"
    assert x.dtype == torch.float16, f"x must be float16, got {x.dtype}"
    return _matmul(x, packed_weight, scales, zeros, group_size, perm, perm16, sz_gm, w_tiled, out)


def matmul_w4a16_bf16(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    group_size: int,
    *,
    perm: torch.Tensor | None = None,
    perm16: torch.Tensor | None = None,
    sz_gm: tuple[torch.Tensor, torch.Tensor] | None = None,
    w_tiled: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Y[M,N] = X[M,K] @ dequant(W)^T with bf16 X and Y (native bf16 activations).

    An extension without a reference counterpart: the reference casts bf16
    activations to fp16 before its kernel (pare/layers/linear.py:154-156),
    which ``matmul_w4a16`` keeps. Here the bf16 values are used as they are
    (fp32 accumulation, y rounded to bf16): with ``w_tiled`` and ``sz_gm`` and
    no ``perm``, the row counts an fp16 call runs on the tiled GEMM's 16-row
    blocks take its bf16 variant; the rest run on the GEMV, four activation
    rows per launch. Other arguments as for ``matmul_w4a16``."""
    if not x.is_cuda:
        raise RuntimeError("matmul_w4a16_bf16 requires HIP (cuda) tensors.")
    assert x.is_contiguous(), "x must be contiguous"
    assert x.dtype == torch.bfloat16, f"x must be bfloat16, got {x.dtype}"
    return _matmul(x, packed_weight, scales, zeros, group_size, perm, perm16, sz_gm, w_tiled, out)


def _matmul(x, packed_weight, scales, zeros, group_size, perm, perm16, sz_gm, w_tiled, out):
    """The shared argument checks and the pmi_matmul_w4a16 call (x fp16 or
    bf16, y of the same dtype)."""
    L = _lib.lib()
    assert x.dim() == 2, f"x must be 2-D [M, K], got shape {tuple(x.shape)}"
    M, K = x.shape
    N, K_half = packed_weight.shape
    assert K == K_half * 2, f"packed_weight has {K_half} columns, expected K//2={K // 2}"
    assert packed_weight.dtype == torch.uint8, "packed_weight must be uint8"
    assert K % group_size == 0, f"K={K} must be divisible by group_size={group_size}"
    dev = x.device
    for name, t in (("packed_weight", packed_weight), ("scales", scales), ("zeros", zeros)):
        if t.device != dev:
            raise RuntimeError(f"{name} is on {t.device}, x is on {dev}")
    G = K // group_size
    s2 = _to_2d(scales).float().contiguous()
    z2, zdt = _validated_zero_tensor(_to_2d(zeros))
    z2 = z2.contiguous()
    assert tuple(s2.shape) == (N, G), f"scales must be [N, G]=[{N}, {G}], got {tuple(scales.shape)}"
    assert tuple(z2.shape) == (N, G), f"zeros must be [N, G]=[{N}, {G}], got {tuple(zeros.shape)}"
    w = _aligned16(packed_weight.contiguous())
    xa = _aligned16(x)
    if perm is not None:
        assert perm.dtype == torch.int32 and perm.numel() == K and perm.device == dev, \
            "perm must be an int32 [K] tensor on x's device"
        perm = perm.contiguous()
    if perm16 is not None:
        assert perm is not None, "perm16 is given with perm"
        assert perm16.dtype == torch.int16 and perm16.numel() == K and perm16.device == dev \
            and perm16.is_contiguous(), "perm16 must be a contiguous int16 [K] tensor on x's device"
        perm16 = _aligned16(perm16)
    s_gm = z_gm = None
    if sz_gm is not None:
        s_gm, z_gm = sz_gm
        assert s_gm.dtype == torch.float32 and tuple(s_gm.shape) == (G, N) and s_gm.is_contiguous(), \
            "sz_gm[0] must be a contiguous float32 [G, N] tensor"
        assert z_gm.dtype == torch.uint8 and tuple(z_gm.shape) == (G, N) and z_gm.is_contiguous(), \
            "sz_gm[1] must be a contiguous uint8 [G, N] tensor"
        assert s_gm.device == dev and z_gm.device == dev, "sz_gm must be on x's device"
    if w_tiled is not None:
        assert w_tiled.dtype == torch.uint8 and w_tiled.device == dev and w_tiled.is_contiguous(), \
            "w_tiled must be a contiguous uint8 tensor on x's device"
        assert w_tiled.numel() == L.pmi_tiled_bytes(N, K), \
            f"w_tiled must hold pmi_tiled_bytes(N, K)={L.pmi_tiled_bytes(N, K)} bytes"
        w_tiled = _aligned16(w_tiled)
    code = _lib.PMI_BF16 if x.dtype == torch.bfloat16 else _lib.PMI_F16
    if out is None:
        out = torch.empty(M, N, device=dev, dtype=x.dtype)
    else:
        assert out.dtype == x.dtype and tuple(out.shape) == (M, N) and out.is_contiguous(), \
            f"out must be a contiguous [M, N] {x.dtype} tensor"
    with _DeviceGuard(dev):
        stream = _stream_handle(dev)
        nbytes = L.pmi_matmul_workspace_bytes(M, N, K, group_size, int(perm is not None))
        ws = _workspace(dev, stream, nbytes)
        _lib.check(L.pmi_matmul_w4a16(
            xa.data_ptr(), code, w.data_ptr(), s2.data_ptr(), z2.data_ptr(), zdt,
            perm.data_ptr() if perm is not None else None,
            perm16.data_ptr() if perm16 is not None else None,
            s_gm.data_ptr() if s_gm is not None else None,
            z_gm.data_ptr() if z_gm is not None else None,
            w_tiled.data_ptr() if w_tiled is not None else None, out.data_ptr(), code,
            M, N, K, group_size, ws.data_ptr() if ws is not None else None,
            ws.numel() if ws is not None else 0, stream), "pmi_matmul_w4a16")
    return out


def matmul_w4a16_glu(gate_up: torch.Tensor, packed_weight: torch.Tensor, scales: torch.Tensor,
                     zeros_u8: torch.Tensor, group_size: int) -> torch.Tensor:
    """Y = (silu(gate) * up) @ dequant(W)^T for M <= 4: the down projection of
    a gated MLP fused with its activation. ``gate_up`` is the fused gate/up
    output [M, 2K] fp16; the result equals ``silu_mul`` followed by
    ``matmul_w4a16`` bit for bit. ``zeros_u8``: uint8 [N, G] zero points."""
    L = _lib.lib()
    if not gate_up.is_cuda:
        raise RuntimeError("matmul_w4a16_glu requires HIP (cuda) tensors.")
    assert gate_up.dtype == torch.float16 and gate_up.dim() == 2 and gate_up.is_contiguous(), \
        "gate_up must be a contiguous float16 [M, 2K] tensor"
    M, K2 = gate_up.shape
    K = K2 // 2
    N, K_half = packed_weight.shape
    assert K2 == 2 * K and K == 2 * K_half, f"gate_up has {K2} columns, expected 2*K={4 * K_half}"
    assert M <= 4, f"the gated GEMV takes M <= 4, got {M}"
    z2 = _to_2d(zeros_u8)
    assert z2.dtype == torch.uint8, "zeros must be uint8 [N, G]"
    s2 = _to_2d(scales).float().contiguous()
    dev = gate_up.device
    out = torch.empty(M, N, device=dev, dtype=torch.float16)
    with _DeviceGuard(dev):
        _lib.check(L.pmi_matmul_w4a16_glu(
            _aligned16(gate_up).data_ptr(), _aligned16(packed_weight.contiguous()).data_ptr(),
            s2.data_ptr(), z2.contiguous().data_ptr(), _lib.PMI_U8, out.data_ptr(), M, N, K,
            group_size, _stream_handle(dev)), "pmi_matmul_w4a16_glu")
    return out


def glu_row_order(F: int, device=None) -> torch.Tensor:
    """Row order of a fused [gate (F rows); up (F rows)] weight that
    ``matmul_w4a16_gate_up_silu`` reads: row 64p + 4n + j of the reordered
    weight is gate row 32p + 2n + j for j < 2 and up row 32p + 2n + j - 2 for
    j >= 2, so that each 64-row panel holds 32 gate rows and their up rows.
    F % 32 == 0."""
    assert F % 32 == 0, "the interleave needs F % 32 == 0"
    r = torch.arange(2 * F, device=device)
    p, t = r // 64, r % 64
    n, j = t // 4, t % 4
    return torch.where(j < 2, 32 * p + 2 * n + j, F + 32 * p + 2 * n + j - 2)


def gate_up_silu_supported(M: int, N: int, K: int, group_size: int) -> bool:
    """Whether ``matmul_w4a16_gate_up_silu`` runs this shape (N: rows of the
    fused gate/up weight)."""
    return bool(_lib.lib().pmi_gate_up_silu_supported(M, N, K, group_size))


def matmul_w4a16_gate_up_silu(x: torch.Tensor, w_tiled: torch.Tensor,
                              sz_gm: tuple[torch.Tensor, torch.Tensor], group_size: int,
                              N: int) -> torch.Tensor:
    """silu(x @ Wg^T) * (x @ Wu^T) in one launch: the tiled GEMM over the fused
    gate/up weight with its rows in ``glu_row_order`` (``w_tiled``, ``sz_gm``:
    the tiled and group-major copies of the reordered weight), the activation
    formed in its epilogue. x fp16 [M, K]; returns fp16 [M, N / 2], equal to
    the fused matmul followed by ``silu_mul`` bit for bit."""
    L = _lib.lib()
    if not x.is_cuda:
        raise RuntimeError("matmul_w4a16_gate_up_silu requires HIP (cuda) tensors.")
    assert x.dtype == torch.float16 and x.dim() == 2 and x.is_contiguous(), \
        "x must be a contiguous float16 [M, K] tensor"
    M, K = x.shape
    s_gm, z_gm = sz_gm
    dev = x.device
    out = torch.empty(M, N // 2, device=dev, dtype=torch.float16)
    with _DeviceGuard(dev):
        _lib.check(L.pmi_matmul_w4a16_gate_up_silu(
            _aligned16(x).data_ptr(), _aligned16(w_tiled).data_ptr(), _aligned16(s_gm).data_ptr(),
            z_gm.data_ptr(), out.data_ptr(), M, N, K, group_size, _stream_handle(dev)),
            "pmi_matmul_w4a16_gate_up_silu")
    return out


def matmul_w4a16_rmsnorm(x: torch.Tensor, residual: torch.Tensor | None, norm_weight: torch.Tensor,
                         eps: float, packed_weight: torch.Tensor, scales: torch.Tensor,
                         zeros_u8: torch.Tensor, group_size: int):
    """(Y, h) with h = x + residual (x when residual is None) and
    Y = (RMSNorm(h) * norm_weight) @ dequant(W)^T, for M <= 4: a decoder's
    residual add and pre-norm fused into the GEMV. x, residual: fp16 [M, K];
    norm_weight fp16 [K]; zeros_u8 uint8 [N, G]."""
    L = _lib.lib()
    if not x.is_cuda:
        raise RuntimeError("matmul_w4a16_rmsnorm requires HIP (cuda) tensors.")
    assert x.dtype == torch.float16 and x.dim() == 2 and x.is_contiguous(), \
        "x must be a contiguous float16 [M, K] tensor"
    M, K = x.shape
    N, K_half = packed_weight.shape
    assert K == 2 * K_half, f"x has {K} columns, expected K={2 * K_half}"
    assert M <= 4, f"the fused GEMV takes M <= 4, got {M}"
    assert norm_weight.dtype == torch.float16 and norm_weight.numel() == K
    z2 = _to_2d(zeros_u8)
    assert z2.dtype == torch.uint8, "zeros must be uint8 [N, G]"
    s2 = _to_2d(scales).float().contiguous()
    dev = x.device
    xa = _aligned16(x)
    r = None
    h = x
    if residual is not None:
        assert residual.shape == x.shape and residual.dtype == torch.float16
        r = _aligned16(residual.contiguous())
        h = torch.empty_like(x)   # never aliases x or residual: other workgroups still read them
    out = torch.empty(M, N, device=dev, dtype=torch.float16)
    with _DeviceGuard(dev):
        _lib.check(L.pmi_matmul_w4a16_rmsnorm(
            xa.data_ptr(), r.data_ptr() if r is not None else None,
            _aligned16(norm_weight.contiguous()).data_ptr(), eps,
            h.data_ptr() if r is not None else None,
            _aligned16(packed_weight.contiguous()).data_ptr(), s2.data_ptr(),
            z2.contiguous().data_ptr(), _lib.PMI_U8, out.data_ptr(), M, N, K, group_size,
            _stream_handle(dev)), "pmi_matmul_w4a16_rmsnorm")
    return out, h


def residual_stats_count(N: int, K: int, glu: bool = False) -> int:
    """Partials of sum(h^2) that ``matmul_w4a16_residual`` writes for this
    shape (0 when it does not run it)."""
    return int(_lib.lib().pmi_residual_stats_count(N, K, int(glu)))


def matmul_w4a16_residual(x: torch.Tensor, residual: torch.Tensor, stats: torch.Tensor,
                          packed_weight: torch.Tensor, scales: torch.Tensor,
                          zeros_u8: torch.Tensor, group_size: int, glu: bool = False,
                          out: torch.Tensor | None = None) -> int:
    """One activation row: ``out`` = residual + x @ dequant(W)^T (each output
    rounded to fp16, then added as ``add_rmsnorm`` adds), with x the fused
    gate/up output consumed as SiLU(gate) * up when ``glu``. Writes the
    per-workgroup partial sums of out^2 to ``stats`` (fp32) and returns how
    many, for ``matmul_w4a16_prenormed``. ``out`` may be ``residual``."""
    L = _lib.lib()
    N, K_half = packed_weight.shape
    K = 2 * K_half
    assert x.dtype == torch.float16 and x.is_contiguous() and x.numel() == (2 * K if glu else K)
    assert residual.dtype == torch.float16 and residual.is_contiguous() and residual.numel() == N
    assert stats.dtype == torch.float32 and stats.is_contiguous()
    n = residual_stats_count(N, K, glu)
    if n == 0 or stats.numel() < n:
        raise RuntimeError(f"matmul_w4a16_residual: shape N={N} K={K} glu={glu} not supported "
                           f"(or stats holds fewer than {n} floats)")
    out = residual if out is None else out
    dev = x.device
    with _DeviceGuard(dev):
        _lib.check(L.pmi_matmul_w4a16_residual(
            _aligned16(x).data_ptr(), int(glu), residual.data_ptr(), stats.data_ptr(),
            _aligned16(packed_weight.contiguous()).data_ptr(), _to_2d(scales).float().contiguous().data_ptr(),
            _to_2d(zeros_u8).contiguous().data_ptr(), out.data_ptr(), N, K, group_size,
            _stream_handle(dev)), "pmi_matmul_w4a16_residual")
    return n


def matmul_w4a16_prenormed(x: torch.Tensor, stats: torch.Tensor, n_stats: int,
                           norm_weight: torch.Tensor, eps: float, packed_weight: torch.Tensor,
                           scales: torch.Tensor, zeros_u8: torch.Tensor,
                           group_size: int) -> torch.Tensor:
    """(RMSNorm(x) * norm_weight) @ dequant(W)^T for one row x [1, K] formed
    by ``matmul_w4a16_residual``, whose ``n_stats`` partial sums of x^2 give
    the norm; returns fp16 [1, N]."""
    L = _lib.lib()
    N, K_half = packed_weight.shape
    K = 2 * K_half
    assert x.dtype == torch.float16 and x.is_contiguous() and x.numel() == K
    assert norm_weight.dtype == torch.float16 and norm_weight.numel() == K
    assert stats.dtype == torch.float32 and stats.numel() >= n_stats
    dev = x.device
    out = torch.empty(1, N, device=dev, dtype=torch.float16)
    with _DeviceGuard(dev):
        _lib.check(L.pmi_matmul_w4a16_prenormed(
            _aligned16(x).data_ptr(), stats.data_ptr(), n_stats,
            _aligned16(norm_weight.contiguous()).data_ptr(), eps,
            _aligned16(packed_weight.contiguous()).data_ptr(), _to_2d(scales).float().contiguous().data_ptr(),
            _to_2d(zeros_u8).contiguous().data_ptr(), out.data_ptr(), N, K, group_size,
            _stream_handle(dev)), "pmi_matmul_w4a16_prenormed")
    return out


def tiled_rmsnorm_supported(M: int, N: int, K: int, group_size: int, glu: bool = False) -> bool:
    """True when ``matmul_w4a16_tiled_rmsnorm`` runs this shape (2..4 rows in
    practice, K <= 4096, group_size % 128 == 0)."""
    return bool(_lib.lib().pmi_tiled_rmsnorm_supported(M, N, K, group_size, int(glu)))


def matmul_w4a16_tiled_rmsnorm(x: torch.Tensor, residual: torch.Tensor | None,
                               norm_weight: torch.Tensor, eps: float, w_tiled: torch.Tensor,
                               sz_gm: tuple[torch.Tensor, torch.Tensor], group_size: int, N: int,
                               glu: bool = False):
    """(Y, h) with h = x + residual (x when residual is None) and
    Y = (RMSNorm(h) * norm_weight) @ dequant(W)^T on the tiled GEMM, one
    launch; with ``glu`` the weight is the gate/up layout of
    ``matmul_w4a16_gate_up_silu`` and Y = silu(gate) * up, [M, N / 2]. Equal
    bit for bit to ``add_rmsnorm`` followed by the matmul (or the gate/up
    launch). x, residual fp16 [M, K]; norm_weight fp16 [K]; ``w_tiled``,
    ``sz_gm`` the tiled and group-major copies."""
    L = _lib.lib()
    if not x.is_cuda:
        raise RuntimeError("matmul_w4a16_tiled_rmsnorm requires HIP (cuda) tensors.")
    assert x.dtype == torch.float16 and x.dim() == 2 and x.is_contiguous(), \
        "x must be a contiguous float16 [M, K] tensor"
    M, K = x.shape
    assert norm_weight.dtype == torch.float16 and norm_weight.numel() == K
    s_gm, z_gm = sz_gm
    dev = x.device
    r = None
    h = x
    if residual is not None:
        assert residual.shape == x.shape and residual.dtype == torch.float16
        r = _aligned16(residual.contiguous())
        h = torch.empty_like(x)   # never aliases x or residual: other workgroups still read them
    out = torch.empty(M, N // 2 if glu else N, device=dev, dtype=torch.float16)
    with _DeviceGuard(dev):
        _lib.check(L.pmi_matmul_w4a16_tiled_rmsnorm(
            _aligned16(x).data_ptr(), r.data_ptr() if r is not None else None,
            _aligned16(norm_weight.contiguous()).data_ptr(), eps,
            h.data_ptr() if r is not None else None, _aligned16(w_tiled).data_ptr(),
            _aligned16(s_gm).data_ptr(), z_gm.data_ptr(), out.data_ptr(), M, N, K, group_size,
            int(glu), _stream_handle(dev)), "pmi_matmul_w4a16_tiled_rmsnorm")
    return out, h


_KERNEL_IDS = {"auto": 0, "gemv": 1, "gemm": 2, "skinny": 3, "gemm64": 4, "tgemm": 5, "bgemm": 6}


class force_kernel:
    """Context manager pinning matmul_w4a16 to one kernel ('gemv', 'gemm',
    'skinny'; 'auto' for the automatic choice) — for tests and benchmarks."""

    def __init__(self, name: str):
        self.id = _KERNEL_IDS[name]
        self.prev = 0

    def __enter__(self):
        self.prev = _lib.lib().pmi_set_kernel_override(self.id)
        return self

    def __exit__(self, *exc):
        _lib.lib().pmi_set_kernel_override(self.prev)
        return False


def kernel_choice(M: int, N: int, K: int, group_size: int, tiled: bool = False,
                  perm: bool = False) -> str:
    """'gemv', 'gemm', 'skinny', 'gemm64', 'tgemm' or 'bgemm' (the tiled GEMM's
    big-tile variant): the kernel matmul_w4a16 runs for this shape (``tiled``: the
    caller passes the tiled weight copy; ``perm``: an act_order permutation)."""
    flags = (_lib.PMI_CHOICE_TILED if tiled else 0) | (_lib.PMI_CHOICE_PERM if perm else 0)
    c = _lib.lib().pmi_matmul_kernel_choice(M, N, K, group_size, flags)
    return {1: "gemv", 2: "gemm", 3: "skinny", 4: "gemm64", 5: "tgemm", 6: "bgemm"}[c]


def tgemm_splits(M: int, N: int, K: int, group_size: int, perm: bool = False) -> int:
    """K ranges the tiled GEMM splits this shape into when matmul_w4a16 runs it
    (1: unsplit)."""
    return _lib.lib().pmi_tgemm_splits(M, N, K, group_size, int(perm))
