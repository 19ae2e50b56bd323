"""RTN INT4 producer on the HIP device.

Produces exactly the buffers of the reference's RTN scheme
(pare/schemes/rtn.py:46-65 -> pare/core/scale.py:24-137 ->
pare/core/functional.py:46-75 -> pare/core/pack.py:29-48 via
pare/layers/linear.py:74-89): packed storage-layout uint8 [N, K//2], fp32
scale and zero of shape [N, G, 1] (per_group) or [N, 1] (per_channel).
"""

from __future__ import annotations

import torch

from . import _lib
from .kernels import _DeviceGuard, _stream_handle

_W_DTYPES = {torch.float32: _lib.PMI_F32, torch.float16: _lib.PMI_F16,
             torch.bfloat16: _lib.PMI_BF16}


def rtn_quantize(weight: torch.Tensor, group_size: int = 128, sym: bool = False,
                 granularity: str = "per_group"):
    """RTN-quantise W [N, K] on the HIP device: (packed, scale, zero).

    sym: False (asymmetric), True (the reference's symmetric rule, zero 0) or
    "offset8" (symmetric with zero 8 and scale 2·max|w|/15).
    granularity "per_group" uses ``group_size``; "per_channel" one group per
    row; "per_tensor" is not produced by this path (the reference's kernel
    path cannot consume it, pare/kernels/matmul_int4.py:219-225).
    """
    L = _lib.lib()
    if not weight.is_cuda:
        raise RuntimeError("rtn_quantize runs on the HIP device; move the weight to cuda first")
    if weight.dim() != 2:
        raise ValueError(f"per_group expects a 2-D weight matrix, got shape {tuple(weight.shape)}")
    if weight.dtype not in _W_DTYPES:
        weight = weight.float()
    N, K = weight.shape
    if granularity == "per_channel":
        gs = K
    elif granularity == "per_group":
        gs = group_size
    else:
        raise ValueError(f"rtn_quantize supports per_group and per_channel, not {granularity!r}")
    if K % gs != 0:
        raise ValueError(f"in_features={K} is not divisible by group_size={gs}")
    if K % 2 != 0 or gs % 2 != 0:
        raise ValueError(f"Last dimension must be even for INT4 packing, got {K}")
    w = weight.contiguous()
    G = K // gs
    packed = torch.empty(N, K // 2, dtype=torch.uint8, device=w.device)
    scale = torch.empty(N, G, dtype=torch.float32, device=w.device)
    zero = torch.empty(N, G, dtype=torch.float32, device=w.device)
    with _DeviceGuard(w.device):
        _lib.check(L.pmi_rtn_quantize(
            w.data_ptr(), _W_DTYPES[w.dtype], packed.data_ptr(), scale.data_ptr(),
            zero.data_ptr(), N, K, gs, 2 if sym == "offset8" else int(bool(sym)),
            _stream_handle(w.device)),
            "pmi_rtn_quantize")
    if granularity == "per_group":
        return packed, scale.unsqueeze(-1), zero.unsqueeze(-1)
    return packed, scale, zero
