"""GPTQ producer on the HIP device, with act_order layers that carry g_idx.

Two variants of one algorithm (pare/schemes/gptq.py:156-263, the column loop
of Frantar et al. with lazy block updates):

``groups="reference"``: the reference's ``GPTQQuantizer.quantize_layer``
(gptq.py:108-149).
  - Scale and zero come from the original weight, with the reference's
    ``compute_scale`` rule (including its sym quirk).
  - act_order rounds each permuted column with its original group. The layout
    is the RTN layout, with no g_idx.

``groups="dynamic"``: AutoGPTQ's desc_act rule.
  - Groups are runs of ``group_size`` columns in processing order.
  - Each group's scale and zero come from the partly updated weight when the
    loop reaches its first column.
  - With act_order the layer carries ``g_idx[k] = (position of column k in
    the order) // group_size``, which the matmul consumes through its
    permutation path.
  - ``sym=True`` is offset-8 symmetric: zero 8, scale 2·max|w|/15. The
    reference's rule puts the zero at 0, so every negative weight clamps to
    code 0.

Device work per layer:
  - the Cholesky chain, in float64 through torch.linalg (rocSOLVER);
  - per 128-column block, the sequential column loop as one HIP launch
    (``pmi_gptq_block``: rows on lanes, the block's C and W in LDS);
  - the lazy update of the columns right of the block, as a rocBLAS GEMM;
  - a final pack (``pmi_gptq_pack``).
The loop's rounding steps are those of gptq.py:230-249: one rounded product,
then one subtraction.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib
from .config import QuantConfig
from .kernels import _DeviceGuard, _stream_handle
from .linear import QuantizedLinear
from .quant import rtn_quantize

BLOCK = 128   # pare/schemes/gptq.py:42


class HessianAccumulator:
    """GPTQ's per-layer input statistic H = (2/n) XᵀX, gathered batch by batch
    without keeping the batches (the role of pare/calibration/hessian.py:19-73,
    with the same ``H`` / ``n_tokens`` attributes and ``accumulate`` /
    ``finalize`` / ``reset`` calls).

    ``H`` is the un-normalised Gram sum in fp32 on the device of the first
    batch: the first batch's Gram matrix becomes it, later ones are added to
    it. Token rows are the input flattened over its leading dims; a batch is
    [tokens, features] or [batch, seq, features].
    """

    def __init__(self) -> None:
        self.reset()

    def reset(self) -> None:
        self.H: torch.Tensor | None = None
        self.n_tokens = 0

    def accumulate(self, x: torch.Tensor) -> None:
        if x.dim() not in (2, 3):
            raise ValueError("HessianAccumulator.accumulate takes [tokens, features] or "
                             f"[batch, seq, features] activations, not shape {tuple(x.shape)}")
        rows = x.detach().reshape(-1, x.shape[-1]).to(torch.float32)
        gram = rows.mT @ rows
        self.H = gram if self.H is None else self.H.add_(gram)
        self.n_tokens += rows.shape[0]

    def finalize(self) -> torch.Tensor:
        """(2 / n_tokens) · H as a new tensor; RuntimeError before any batch."""
        if not self.n_tokens:
            raise RuntimeError("HessianAccumulator.finalize: no samples accumulated yet "
                               "(call accumulate with calibration activations first)")
        return self.H.mul(2.0 / self.n_tokens)


def _cholesky_chain(H: torch.Tensor, damp: float) -> torch.Tensor:
    """Upper Cholesky factor of H⁻¹ (gptq.py:203-213), float64, with the
    reference's retry at ten times the damping."""
    H64 = H.double()
    try:
        L = torch.linalg.cholesky(H64)
    except torch.linalg.LinAlgError:
        H64.diagonal().add_(damp * 10.0)
        L = torch.linalg.cholesky(H64)
    Hinv = torch.cholesky_inverse(L)
    return torch.linalg.cholesky(Hinv, upper=True).float().contiguous()


def gptq_columns(W: torch.Tensor, C: torch.Tensor, colg: torch.Tensor, scale: torch.Tensor,
                 zero: torch.Tensor, group_size: int, dynamic_sym: int | None = None) -> torch.Tensor:
    """The column loop over the (permuted) fp32 W [N, K] with the factor C
    [K, K]: returns the codes u8 [K, N] in processed order. ``W`` receives the
    lazy updates in place. With ``dynamic_sym`` (0 or 2) the scale/zero [N, G]
    of each group are written when the loop reaches its first column, from W
    at the start of that column's block."""
    L = _lib.lib()
    N, K = W.shape
    G = scale.shape[1]
    dev = W.device
    if not (W.is_contiguous() and scale.is_contiguous() and zero.is_contiguous()):
        raise ValueError("W, scale and zero must be contiguous (W is updated in place)")
    if tuple(C.shape) != (K, K) or C.dtype != torch.float32 or colg.dtype != torch.int32:
        raise ValueError("C must be fp32 [K, K] and colg int32 [K]")
    C = C.contiguous()
    colg = colg.contiguous()
    codes = torch.empty(K, N, dtype=torch.uint8, device=dev)
    errors = torch.empty(BLOCK, N, dtype=torch.float32, device=dev)
    stream = _stream_handle(dev)
    with _DeviceGuard(dev):
        for b0 in range(0, K, BLOCK):
            b1 = min(b0 + BLOCK, K)
            if dynamic_sym is not None:
                for g in range(-(-b0 // group_size), -(-b1 // group_size)):
                    _lib.check(L.pmi_gptq_group_params(
                        W.data_ptr(), K, N, g * group_size, group_size, dynamic_sym,
                        scale.data_ptr(), zero.data_ptr(), G, g, stream), "pmi_gptq_group_params")
            _lib.check(L.pmi_gptq_block(W.data_ptr(), C.data_ptr(), colg.data_ptr(), scale.data_ptr(),
                                        zero.data_ptr(), codes.data_ptr(), errors.data_ptr(), N, K, G,
                                        b0, b1 - b0, stream), "pmi_gptq_block")
            if b1 < K:
                W[:, b1:].addmm_(errors[: b1 - b0].t(), C[b0:b1, b1:], alpha=-1.0)
    return codes


def gptq_quantize(weight: torch.Tensor, hessian: torch.Tensor, group_size: int = 128, *,
                  sym: bool = False, act_order: bool = False, damp_percent: float = 0.01,
                  groups: str = "dynamic"):
    """GPTQ-quantise W [N, K] with Hessian H [K, K] on the HIP device.

    Returns (packed u8 [N, K/2] storage layout in the original column order,
    scale fp32 [N, G, 1], zero fp32 [N, G, 1], g_idx int32 [K] or None)."""
    if groups not in ("reference", "dynamic"):
        raise ValueError(f"groups must be 'reference' or 'dynamic', got {groups!r}")
    if not weight.is_cuda:
        raise RuntimeError("gptq_quantize runs on the HIP device; move the weight to cuda first")
    if weight.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(weight.shape)}")
    N, K = weight.shape
    if K % group_size != 0 or group_size % 2 != 0:
        raise ValueError(f"in_features={K} is not divisible by group_size={group_size}")
    if K % 16 != 0:
        raise ValueError(f"in_features={K} must be a multiple of 16")
    if tuple(hessian.shape) != (K, K):
        raise ValueError(f"hessian must be [{K}, {K}], got {tuple(hessian.shape)}")
    dev = weight.device
    G = K // group_size
    W0 = weight.detach().float()
    W = W0.clone()
    H = hessian.detach().to(dev, torch.float32).clone()

    dead = H.diagonal() == 0.0                                   # gptq.py:184-187
    H[dead, dead] = 1.0
    W[:, dead] = 0.0
    damp = damp_percent * H.diagonal().mean().item()           # gptq.py:189-191
    H.diagonal().add_(damp)
    if act_order:                                              # gptq.py:194-200
        perm = torch.argsort(H.diagonal(), descending=True, stable=True)
        W = W[:, perm]
        H = H[perm][:, perm]
    else:
        perm = torch.arange(K, device=dev)
    W = W.contiguous()
    C = _cholesky_chain(H, damp)

    if groups == "reference":
        _, scale, zero = rtn_quantize(W0, group_size, sym)     # gptq.py:121-127
        scale = scale.reshape(N, G).contiguous()
        zero = zero.reshape(N, G).contiguous()
        colg = (perm // group_size).to(torch.int32).contiguous()
        codes = gptq_columns(W, C, colg, scale, zero, group_size)
        g_idx = None
    else:
        scale = torch.zeros(N, G, dtype=torch.float32, device=dev)
        zero = torch.zeros(N, G, dtype=torch.float32, device=dev)
        colg = (torch.arange(K, device=dev) // group_size).to(torch.int32)
        codes = gptq_columns(W, C, colg, scale, zero, group_size, dynamic_sym=2 if sym else 0)
        g_idx = None
        if act_order:
            g_idx = (torch.argsort(perm) // group_size).to(torch.int32)

    inv_perm = torch.argsort(perm).to(torch.int32).contiguous() if act_order else None
    packed = torch.empty(N, K // 2, dtype=torch.uint8, device=dev)
    with _DeviceGuard(dev):
        _lib.check(_lib.lib().pmi_gptq_pack(codes.data_ptr(),
                                            inv_perm.data_ptr() if inv_perm is not None else None,
                                            packed.data_ptr(), N, K, _stream_handle(dev)),
                   "pmi_gptq_pack")
    return packed, scale.unsqueeze(-1), zero.unsqueeze(-1), g_idx


def quantize_linear_gptq(linear: nn.Linear, hessian: torch.Tensor, config: QuantConfig | None = None,
                         groups: str = "dynamic") -> QuantizedLinear:
    """One ``nn.Linear`` -> ``QuantizedLinear`` with GPTQ (gptq.py:108-149).
    A CPU layer is quantised on the current HIP device and its buffers are
    returned on the layer's device."""
    config = config or QuantConfig(bits=4, scheme="gptq")
    gs = config.group_size if config.granularity == "per_group" else linear.in_features
    home = linear.weight.device
    w = linear.weight.detach()
    if not w.is_cuda:
        w = w.to("cuda")
    packed, scale, zero, g_idx = gptq_quantize(
        w, hessian.to(w.device), gs, sym=config.sym, act_order=config.act_order,
        damp_percent=getattr(config, "damp_percent", 0.01), groups=groups)
    return QuantizedLinear(packed.to(home), scale.to(home), zero.to(home), config, linear.bias,
                           linear.in_features, linear.out_features,
                           g_idx=g_idx.to(home) if g_idx is not None else None)
