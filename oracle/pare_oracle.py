"""CPU oracle for the INT4 W4A16 dequant-matmul path — TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU, the reference's algorithm for the
``QuantizedLinear.use_kernel=True`` path and its dequantize-on-the-fly oracle.
It is the checker, never the product: only ``tests/``, ``__graft_entry__.smoke``
and the ``cpu_baseline`` leg of ``bench.py`` may import it. The shipped path
(``pare_amd``) never calls into it and has no CPU fallback.

Integer/byte work and the fp32 elementwise formulas are numpy (float32
arithmetic, IEEE round-to-nearest-even, ``np.rint`` = round-half-to-even like
``torch.round``). The fp16 matmul of the reference's dequant path is restated
with torch on the CPU (``F.linear`` on fp16, as the reference runs it), which
is also the CPU baseline timed by ``bench.py``.

Each function cites the reference file:line it follows (paths relative to the
reference repository root). Pinning of every function — by the reference's
own known-answer tests, closed forms, invariants and brute force — lives in
``tests/test_oracle.py`` (the AWQ-GEMM functions: ``tests/test_awq.py``); no
function here is "parity unpinned".
"""

from __future__ import annotations

import numpy as np

QMIN = 0   # INT4 is unsigned: pare/core/dtype.py:15-25,46
QMAX = 15


# ---------------------------------------------------------------------------
# Packing (pare/core/pack.py)
# ---------------------------------------------------------------------------

def pack_int4(q: np.ndarray) -> np.ndarray:
    """Even column -> low nibble, odd column -> high nibble (pack.py:29-48)."""
    q = np.asarray(q)
    if q.shape[-1] % 2 != 0:
        raise ValueError(f"Last dimension must be even for INT4 packing, got {q.shape[-1]}")
    q = q.astype(np.int32)
    low = q[..., 0::2] & 0xF
    high = (q[..., 1::2] & 0xF) << 4
    return (low | high).astype(np.uint8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """Inverse of pack_int4, int32 values in [0,15] (pack.py:51-67)."""
    p = np.asarray(packed).astype(np.int32)
    out = np.stack([p & 0xF, (p >> 4) & 0xF], axis=-1)
    return out.reshape(*p.shape[:-1], -1)


def repack_int4_for_kernel(packed: np.ndarray, group_size: int = 128) -> np.ndarray:
    """Storage layout -> kernel layout (pack.py:88-132).

    Inside each group_size-wide tile starting at column k0, byte j holds
    q[k0 + j] (low nibble) and q[k0 + j + group_size/2] (high nibble).
    """
    N, K_half = packed.shape
    K = 2 * K_half
    assert K % group_size == 0, f"K={K} must be divisible by group_size={group_size}"
    half = group_size // 2
    q = unpack_int4(packed).reshape(N, K // group_size, group_size)
    lo = q[:, :, :half]
    hi = q[:, :, half:]
    return (lo | (hi << 4)).astype(np.uint8).reshape(N, K_half)


def permute_columns_packed(packed: np.ndarray, perm: np.ndarray) -> np.ndarray:
    """Storage-layout weights with columns reordered as q[:, perm] (act_order
    extension; the reference has no g_idx, see pare/schemes/gptq.py:196-201)."""
    return pack_int4(unpack_int4(packed)[:, np.asarray(perm)])


# ---------------------------------------------------------------------------
# AWQ-GEMM int32 layout (pare/model/export_awq.py)
# ---------------------------------------------------------------------------

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)   # export_awq.py:37-39


def pack_awq(x: np.ndarray) -> np.ndarray:
    """[..., N] codes in [0,15] -> [..., N//8] int32: element 8c + AWQ_ORDER[i]
    goes to bits 4i..4i+3 of word c (export_awq.py:42-49)."""
    x = np.asarray(x).astype(np.int64)
    x = x.reshape(*x.shape[:-1], x.shape[-1] // 8, 8)
    out = np.zeros(x.shape[:-1], dtype=np.int64)
    for i, o in enumerate(AWQ_ORDER):
        out |= x[..., o] << (4 * i)
    return out.astype(np.uint32).view(np.int32)


def unpack_awq(w: np.ndarray) -> np.ndarray:
    """Inverse of pack_awq for codes in [0,15]: [..., C] int32 -> [..., 8C]."""
    u = np.asarray(w).view(np.uint32).astype(np.int64)
    out = np.empty((*u.shape, 8), dtype=np.int32)
    for i, o in enumerate(AWQ_ORDER):
        out[..., o] = (u >> (4 * i)) & 0xF
    return out.reshape(*u.shape[:-1], -1)


def to_awq_gemm(packed: np.ndarray, scale: np.ndarray, zero: np.ndarray):
    """Storage-layout packed [N, K/2] + scale, zero [N, G] -> (qweight int32
    [K, N/8], qzeros int32 [G, N/8], scales fp16 [G, N]) (export_awq.py:75-94:
    zeros rounded half-to-even, scales cast to fp16)."""
    N = packed.shape[0]
    q = unpack_int4(packed).reshape(N, -1)
    z = np.rint(np.asarray(zero, dtype=np.float32).reshape(N, -1)).astype(np.int64)
    s = np.asarray(scale, dtype=np.float32).reshape(N, -1)
    with np.errstate(over="ignore"):   # |s| >= 65520 becomes +-inf, as torch's .half()
        s16 = s.T.astype(np.float16)
    return pack_awq(q.T), pack_awq(z.T), s16


def from_awq_gemm(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray):
    """AWQ-GEMM tensors -> (packed storage layout [N, K/2], scale fp32 [N, G],
    zero fp32 [N, G]); inverts to_awq_gemm up to the fp16 scales."""
    q = unpack_awq(qweight).T              # [N, K]
    z = unpack_awq(qzeros).T.astype(np.float32)
    s = np.asarray(scales, dtype=np.float16).T.astype(np.float32)
    return pack_int4(q), np.ascontiguousarray(s), np.ascontiguousarray(z)


# ---------------------------------------------------------------------------
# Scale / zero and quantize / dequantize (pare/core/scale.py, functional.py)
# ---------------------------------------------------------------------------

def _minmax_to_scale_zero(x_min, x_max, sym: bool):
    """scale.py:65-91 with qmin=0, qmax=15, all in float32."""
    f32 = np.float32
    if sym:
        abs_max = np.maximum(np.abs(x_min), np.abs(x_max))
        abs_max = np.maximum(abs_max, f32(1e-8))
        half = f32(max(abs(QMIN), abs(QMAX)))
        scale = (abs_max / half).astype(f32)
        zero = np.zeros_like(scale)
    else:
        x_min = np.minimum(x_min, f32(0.0))
        x_max = np.maximum(x_max, f32(0.0))
        scale = ((x_max - x_min) / f32(QMAX - QMIN)).astype(f32)
        scale = np.maximum(scale, f32(1e-8))
        zero = np.rint(-x_min / scale + f32(QMIN)).astype(f32)
        zero = np.clip(zero, f32(QMIN), f32(QMAX))
    return scale.astype(f32), zero.astype(f32)


def compute_scale(w: np.ndarray, granularity: str = "per_group", group_size: int = 128,
                  sym: bool = False):
    """compute_scale for INT4 (scale.py:24-137). Shapes: per_group [N,G,1],
    per_channel [N,1], per_tensor scalar."""
    w = np.asarray(w, dtype=np.float32)
    if granularity == "per_group":
        if w.ndim != 2:
            raise ValueError(f"per_group expects a 2-D weight matrix, got shape {w.shape}")
        N, K = w.shape
        if K % group_size != 0:
            raise ValueError(f"in_features={K} is not divisible by group_size={group_size}")
        g = w.reshape(N, K // group_size, group_size)
        return _minmax_to_scale_zero(g.min(-1, keepdims=True), g.max(-1, keepdims=True), sym)
    if granularity == "per_channel":
        red = tuple(range(1, w.ndim))
        return _minmax_to_scale_zero(w.min(red, keepdims=True), w.max(red, keepdims=True), sym)
    if granularity == "per_tensor":
        s, z = _minmax_to_scale_zero(w.min().reshape(1), w.max().reshape(1), sym)
        return s.reshape(()), z.reshape(())
    raise ValueError(f"Unknown granularity: {granularity!r}")


def _align(x: np.ndarray, scale: np.ndarray):
    """_align_shapes (functional.py:193-214): per_group reshapes x to [N,G,gs]."""
    if scale.ndim == 3:
        out, n_groups, _ = scale.shape
        return x.reshape(out, n_groups, x.shape[-1] // n_groups)
    return x


def quantize_tensor(w: np.ndarray, scale: np.ndarray, zero: np.ndarray) -> np.ndarray:
    """q = clamp(round(x / scale + zero), 0, 15) in float32 (functional.py:46-75)."""
    x = _align(np.asarray(w, dtype=np.float32), scale)
    q = np.clip(np.rint(x / scale + zero), QMIN, QMAX)
    return q.astype(np.int32)


def dequantize_tensor(q: np.ndarray, scale: np.ndarray, zero: np.ndarray) -> np.ndarray:
    """(q.float() - zero) * scale in float32 (functional.py:78-91)."""
    x = _align(np.asarray(q).astype(np.float32), scale)
    return ((x - zero) * scale).astype(np.float32)


def dequantize_packed(packed: np.ndarray, scale: np.ndarray, zero: np.ndarray) -> np.ndarray:
    """QuantizedLinear.dequantize for INT4 (linear.py:101-118): fp32 [N, K]."""
    N = packed.shape[0]
    return dequantize_tensor(unpack_int4(packed), scale, zero).reshape(N, -1)


def dequantize_gidx(q: np.ndarray, scale: np.ndarray, zero: np.ndarray,
                    g_idx: np.ndarray) -> np.ndarray:
    """act_order extension: w[n,k] = (q[n,k] - zero[n, g_idx[k]]) * scale[n, g_idx[k]].
    With g_idx = k // group_size it is dequantize_tensor (functional.py:78-91)."""
    s = scale.reshape(scale.shape[0], -1)[:, np.asarray(g_idx)]
    z = zero.reshape(zero.shape[0], -1)[:, np.asarray(g_idx)]
    return ((np.asarray(q).astype(np.float32) - z) * s).astype(np.float32)


def rtn_quantize(w: np.ndarray, group_size: int = 128, sym: bool = False,
                 granularity: str = "per_group"):
    """RTN producer (pare/schemes/rtn.py:46-65 + QuantizedLinear.__init__
    linear.py:74-89): returns (packed u8 [N,K/2], scale f32, zero f32)."""
    w = np.asarray(w, dtype=np.float32)
    if sym == "offset8":   # symmetric with zero 8 (offset8_scale_zero), per group
        N, K = w.shape
        gs = group_size if granularity == "per_group" else K
        scale, zero = offset8_scale_zero(w.reshape(N, K // gs, gs))
        scale, zero = scale[..., None], zero[..., None]
        if granularity != "per_group":
            scale, zero = scale.reshape(N, 1), zero.reshape(N, 1)
    else:
        scale, zero = compute_scale(w, granularity, group_size, sym)
    q = quantize_tensor(w, scale, zero).reshape(w.shape)
    return pack_int4(q), scale, zero


def gidx_from_perm(perm: np.ndarray, group_size: int) -> np.ndarray:
    """g_idx of a layer quantised in permuted column order P with contiguous
    groups: column P[j] belongs to group j // group_size."""
    perm = np.asarray(perm)
    g = np.empty(perm.shape[0], dtype=np.int32)
    g[perm] = np.arange(perm.shape[0], dtype=np.int32) // group_size
    return g


def rtn_quantize_act_order(w: np.ndarray, perm: np.ndarray, group_size: int = 128):
    """Quantise W[:, P] with contiguous groups, return q in the original column
    order plus g_idx (the act_order layout): (packed, scale, zero, g_idx)."""
    w = np.asarray(w, dtype=np.float32)
    perm = np.asarray(perm)
    wp = w[:, perm]
    scale, zero = compute_scale(wp, "per_group", group_size, False)
    qp = quantize_tensor(wp, scale, zero).reshape(w.shape)
    q = np.empty_like(qp)
    q[:, perm] = qp
    return pack_int4(q), scale, zero, gidx_from_perm(perm, group_size)


# ---------------------------------------------------------------------------
# GPTQ (pare/schemes/gptq.py, pare/calibration/hessian.py)
# ---------------------------------------------------------------------------

GPTQ_BLOCK = 128   # gptq.py:42


def hessian(x: np.ndarray) -> np.ndarray:
    """H = 2/n * X^T X over n token rows (hessian.py:34-67), float64."""
    x = np.asarray(x, dtype=np.float64).reshape(-1, np.shape(x)[-1])
    return (2.0 / x.shape[0]) * (x.T @ x)


def offset8_scale_zero(w_group: np.ndarray):
    """Symmetric INT4 on the unsigned grid with zero point 8 (AutoGPTQ's sym
    rule): scale = 2 max|w| / 15 over the group (last axis), zero = 8. The
    reference's own sym rule (scale.py:73-82) puts zero at 0 and so clamps
    every negative weight to 0."""
    f32 = np.float32
    amax = np.maximum(np.max(np.abs(np.asarray(w_group, dtype=f32)), axis=-1), f32(1e-8))
    scale = (f32(2.0) * amax / f32(15.0)).astype(f32)
    return scale, np.full_like(scale, f32(8.0))


def group_scale_zero(w_group: np.ndarray, sym):
    """(scale, zero) of each row of w_group [N, gs]: sym False = asymmetric,
    True = the reference's rule (scale.py:65-91), "offset8" = offset8_scale_zero."""
    w_group = np.asarray(w_group, dtype=np.float32)
    if sym == "offset8":
        return offset8_scale_zero(w_group)
    s, z = _minmax_to_scale_zero(w_group.min(-1), w_group.max(-1), bool(sym))
    return s, z


def gptq_prepare(H: np.ndarray, damp_percent: float = 0.01, act_order: bool = False):
    """gptq.py:184-200 in float32: dead columns (diag 0) get diag 1, damping
    damp_percent * mean(diag) on the diagonal, and with act_order the stable
    descending order of the damped diagonal. Returns (H damped and permuted,
    perm, dead mask)."""
    H = np.array(H, dtype=np.float32)
    dead = np.diag(H) == 0.0
    H[dead, dead] = 1.0
    damp = np.float32(damp_percent) * np.mean(np.diag(H), dtype=np.float32)
    H[np.diag_indices_from(H)] += np.float32(damp)
    K = H.shape[0]
    perm = np.argsort(-np.diag(H), kind="stable") if act_order else np.arange(K)
    if act_order:
        H = H[np.ix_(perm, perm)]
    return H, perm, dead


def gptq_cholesky(H: np.ndarray) -> np.ndarray:
    """Upper Cholesky factor C of H^-1 for a damped H (gptq.py:203-206:
    cholesky, cholesky_inverse, cholesky upper), computed in float64 and
    returned as float32."""
    L = np.linalg.cholesky(np.asarray(H, dtype=np.float64))
    Linv = np.linalg.inv(L)
    Hinv = Linv.T @ Linv                       # cholesky_inverse
    return np.ascontiguousarray(np.linalg.cholesky(Hinv).T, dtype=np.float32)


def gptq_columns(Wp: np.ndarray, C: np.ndarray, colg: np.ndarray, scale: np.ndarray,
                 zero: np.ndarray, group_starts=None, sym=False, group_size: int = 128):
    """The column loop of gptq.py:215-256 on the permuted float32 W [N, K]:
    per column j, q = clamp(rint(w / s + z)) with the (scale, zero) of group
    colg[j]; e = (w - (q - z) s) / C[j, j]; the block's later columns get
    w -= e * C[j, later] one column at a time (a rounded product, then the
    subtraction), and the columns right of the block the lazy update
    E @ C[block, right]. Returns the codes in processed order [N, K].

    group_starts (dynamic groups): scale and zero [N, G] are filled as the loop
    reaches each group's first column, from W at the start of that column's
    block (AutoGPTQ's desc_act rule); otherwise they are fixed inputs."""
    f32 = np.float32
    W = np.array(Wp, dtype=f32)
    N, K = W.shape
    Q = np.zeros((N, K), dtype=np.int32)
    for b0 in range(0, K, GPTQ_BLOCK):
        b1 = min(b0 + GPTQ_BLOCK, K)
        if group_starts is not None:
            for g0 in range(b0, b1):
                if g0 % group_size == 0:
                    g = g0 // group_size
                    scale[:, g], zero[:, g] = group_scale_zero(W[:, g0:g0 + group_size], sym)
        Wb = W[:, b0:b1].copy()
        E = np.zeros_like(Wb)
        for k in range(b1 - b0):
            j = b0 + k
            s, z = scale[:, colg[j]], zero[:, colg[j]]
            q = np.clip(np.rint(Wb[:, k] / s + z), f32(QMIN), f32(QMAX))
            Q[:, j] = q.astype(np.int32)
            e = (Wb[:, k] - (q - z) * s) / C[j, j]
            E[:, k] = e
            if k + 1 < b1 - b0:
                Wb[:, k + 1:] -= (e[:, None] * C[j, j + 1:b1][None, :]).astype(f32)
        if b1 < K:
            W[:, b1:] -= (E @ C[b0:b1, b1:]).astype(f32)
    return Q


def gptq_quantize(W: np.ndarray, H: np.ndarray, group_size: int = 128, sym=False,
                  act_order: bool = False, damp_percent: float = 0.01,
                  groups: str = "dynamic"):
    """One GPTQ layer: (packed [N, K/2] storage layout in the original column
    order, scale [N, G, 1], zero [N, G, 1], g_idx int32 [K] or None).

    groups "reference": the reference's quantize_layer (gptq.py:108-149,
    156-263): scale/zero from the original W (compute_scale, the reference's
    sym rule), each column rounded with its original group; no g_idx.
    groups "dynamic": AutoGPTQ desc_act: groups are runs of group_size columns
    in processing order, their scale/zero taken from the updated W when the
    loop reaches them; sym=True means offset-8; with act_order the output
    carries g_idx[k] = (position of column k in the order) // group_size.
    act_order sorts columns by descending diag(H) (stable)."""
    W = np.array(W, dtype=np.float32)
    N, K = W.shape
    G = K // group_size
    W0 = W.copy()
    Hp, perm, dead = gptq_prepare(H, damp_percent, act_order)
    W[:, dead] = 0.0
    C = gptq_cholesky(Hp)
    Wp = W[:, perm]
    if groups == "reference":
        scale, zero = compute_scale(W0, "per_group", group_size, bool(sym))
        scale, zero = scale[..., 0].copy(), zero[..., 0].copy()
        colg = (perm // group_size).astype(np.int64)
        Qp = gptq_columns(Wp, C, colg, scale, zero)
        g_idx = None
    elif groups == "dynamic":
        scale = np.zeros((N, G), dtype=np.float32)
        zero = np.zeros((N, G), dtype=np.float32)
        colg = np.arange(K) // group_size
        sym_rule = "offset8" if sym else False
        Qp = gptq_columns(Wp, C, colg, scale, zero, group_starts=True, sym=sym_rule,
                          group_size=group_size)
        g_idx = gidx_from_perm(perm, group_size) if act_order else None
    else:
        raise ValueError(f"groups must be 'reference' or 'dynamic', got {groups!r}")
    Q = np.empty_like(Qp)
    Q[:, perm] = Qp
    return pack_int4(Q), scale[..., None], zero[..., None], g_idx


def gptq_objective(W: np.ndarray, W_hat: np.ndarray, H: np.ndarray) -> float:
    """Layer-output error tr((W - W_hat) H (W - W_hat)^T), the quantity GPTQ
    minimises (gptq.py:8-10)."""
    D = np.asarray(W, dtype=np.float64) - np.asarray(W_hat, dtype=np.float64)
    return float(np.einsum("nk,kl,nl->", D, np.asarray(H, dtype=np.float64), D))


# ---------------------------------------------------------------------------
# Layer outputs
# ---------------------------------------------------------------------------

def linear_fp32(x: np.ndarray, w_hat: np.ndarray) -> np.ndarray:
    """fp32-accumulated reference output x @ W^T, with the weights first
    rounded to fp16 as the reference path does (linear.py:129)."""
    w16 = np.asarray(w_hat, dtype=np.float32).astype(np.float16).astype(np.float32)
    return np.asarray(x, dtype=np.float32) @ w16.T


def dequant_path_forward_torch(x, packed, scale, zero, bias=None):
    """The reference's dequantize-on-the-fly forward on the CPU, op for op
    (linear.py:112-118,129,138 with pack.py:60-67 and functional.py:90-91):
    unpack -> float -> (q - z) * s -> .to(x.dtype) -> F.linear.

    Arguments are torch CPU tensors; used as the CPU baseline of bench.py."""
    import torch
    import torch.nn.functional as F

    p = packed.to(torch.int32)
    q = torch.stack([p & 0xF, (p >> 4) & 0xF], dim=-1).reshape(packed.shape[0], -1)
    qf = q.float()
    if scale.dim() == 3:
        qf = qf.reshape(scale.shape[0], scale.shape[1], -1)
    w = ((qf - zero) * scale).reshape(packed.shape[0], -1)
    return F.linear(x, w.to(x.dtype), bias)
