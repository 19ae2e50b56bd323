"""QuantizedLinear for the INT4 W4A16 path on MI355X.

Drop-in for pare/layers/linear.py:40-202 on its kernel path: the same buffers
(``packed_weight`` uint8 [out, in//2] in pack_int4 order, ``scale`` and
``zero`` fp32 [out, G, 1], optional ``bias``), the same ``use_kernel`` flag,
``dequantize()`` and ``forward(x)``. Differences, all deliberate:
  - Everything runs on the HIP device. A CPU input raises RuntimeError instead
    of silently taking the reference's CPU dequant path (linear.py:121-127).
  - ``use_kernel`` is read with getattr(..., False), so layers built by
    ``from_tensors`` work (the reference never sets it there, linear.py:166-202).
  - The kernel-layout cache is refreshed when the packed weight changes device
    or contents (the reference caches forever, linear.py:148-151).
  - Optional ``g_idx`` (int32 [in]) for act_order layers.
  - ``quantize_inputs`` (SmoothQuant W8A8 fake-quant) is not part of this path.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .config import QuantConfig, is_int4, kernel_group_size
from .kernels import kernel_choice, matmul_w4a16, matmul_w4a16_bf16
from .pack import (dequantize_int4, perm_from_g_idx, perm_u16, repack_int4_for_kernel,
                   sz_group_major, tile_w4a16, tiled_supported, zeros_to_u8)


class QuantizedLinear(nn.Module):
    def __init__(self, packed_weight: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor,
                 config, bias: torch.Tensor | None, in_features: int, out_features: int,
                 use_kernel: bool = False, g_idx: torch.Tensor | None = None) -> None:
        super().__init__()
        if not is_int4(config):
            raise ValueError("pare_amd.QuantizedLinear implements the INT4 path only")
        if packed_weight.dtype != torch.uint8 or tuple(packed_weight.shape) != (out_features, in_features // 2):
            raise ValueError(f"packed_weight must be uint8 [{out_features}, {in_features // 2}]")
        self.config = config
        self.in_features = in_features
        self.out_features = out_features
        self.use_kernel = use_kernel
        # opt-in extension: bf16 inputs on the kernel path stay bf16 instead
        # of the reference's cast to fp16 (pare/layers/linear.py:154-156)
        self.native_bf16 = False
        self.quantize_inputs = False
        self.register_buffer("packed_weight", packed_weight)
        self.register_buffer("q_weight", None)
        self.register_buffer("scale", scale.float())
        self.register_buffer("zero", zero.float())
        self.register_buffer("g_idx", g_idx.to(torch.int32) if g_idx is not None else None)
        self.bias = nn.Parameter(bias.detach().clone()) if bias is not None else None

    # ------------------------------------------------------------------
    # Constructors
    # ------------------------------------------------------------------

    @classmethod
    def from_tensors(cls, packed_weight, q_weight, scale, zero, config, bias, in_features,
                     out_features, quantize_inputs: bool = False, g_idx=None) -> "QuantizedLinear":
        """Same signature as pare/layers/linear.py:166-177 (used by load paths)."""
        if quantize_inputs:
            raise NotImplementedError("quantize_inputs (SmoothQuant W8A8) is not part of the INT4 path")
        if packed_weight is None:
            raise ValueError("the INT4 path needs packed_weight (q_weight is for 8-bit layers)")
        return cls(packed_weight, scale, zero, config, bias, in_features, out_features,
                   g_idx=g_idx)

    @classmethod
    def from_reference(cls, ref: nn.Module, use_kernel: bool = True) -> "QuantizedLinear":
        """Takes over the buffers of a reference pare QuantizedLinear (INT4)."""
        return cls(ref.packed_weight, ref.scale, ref.zero, ref.config, ref.bias,
                   ref.in_features, ref.out_features, use_kernel=use_kernel,
                   g_idx=getattr(ref, "g_idx", None))

    @classmethod
    def from_linear(cls, linear: nn.Linear, config=None) -> "QuantizedLinear":
        """RTN-quantise an nn.Linear (pare/layers/linear.py:205-268, INT4 branch)
        with the HIP producer. A CPU layer is quantised on the current HIP device
        and the buffers are returned on the layer's device."""
        from .quant import rtn_quantize

        config = config or QuantConfig(bits=4, scheme="rtn")
        if not is_int4(config):
            raise ValueError("pare_amd.QuantizedLinear implements the INT4 path only")
        w = linear.weight.detach()
        home = w.device
        if not w.is_cuda:
            w = w.to("cuda")
        packed, scale, zero = rtn_quantize(w.float(), config.group_size, config.sym,
                                           config.granularity)
        return cls(packed.to(home), scale.to(home), zero.to(home), config, linear.bias,
                   linear.in_features, linear.out_features)

    # ------------------------------------------------------------------
    # Forward
    # ------------------------------------------------------------------

    def _group_size(self) -> int:
        return kernel_group_size(self.config, self.in_features)

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Full weight [out, in] = (q - zero) * scale (pare/layers/linear.py:101-118),
        cast once to ``dtype``."""
        return dequantize_int4(self.packed_weight, self.scale, self.zero, self._group_size(),
                               dtype=dtype, layout="storage", g_idx=self.g_idx)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("pare_amd.QuantizedLinear runs on the HIP device only "
                               "(no CPU fallback); move the module and input to cuda")
        if getattr(self, "use_kernel", False):
            return self._forward_kernel(x)
        weight = self.dequantize(dtype=x.dtype)
        return F.linear(x, weight, self.bias)

    def _stamp(self):
        return (self.packed_weight.device, self.packed_weight.data_ptr(),
                self.packed_weight._version, self.zero._version, self.scale._version)

    def _build_kernel_cache(self, w_kernel: torch.Tensor | None):
        gs = self._group_size()
        perm = None
        if self.g_idx is not None:
            perm = perm_from_g_idx(self.g_idx.to(self.packed_weight.device), gs)
        if w_kernel is None:
            w_kernel = repack_int4_for_kernel(self.packed_weight, gs, perm=perm)
        self._packed_weight_kernel = w_kernel
        self._packed_weight_tiled = None
        # the 16-bit copy the GEMV's act_order gather reads (None past K = 65536)
        self._perm16 = perm_u16(perm) if perm is not None else None
        zero_u8 = zeros_to_u8(self.zero)
        self._kernel_cache = (self._stamp(), zero_u8, perm, sz_group_major(self.scale, zero_u8))

    def _kernel_buffers(self):
        """Kernel-layout weight, u8 zeros, group-major scales/zeros and the
        act_order permutation, built once per (device, weight contents) like
        linear.py:148-151."""
        cache = getattr(self, "_kernel_cache", None)
        if cache is None or cache[0] != self._stamp():
            self._build_kernel_cache(None)
            cache = self._kernel_cache
        return self._packed_weight_kernel, cache[1], cache[2], cache[3]

    def _tiled_buffer(self, w_kernel: torch.Tensor, M: int, perm: torch.Tensor | None = None):
        """Tiled copy of the kernel-layout weight for the tiled-weight GEMM,
        built on the first forward whose row count runs on it (decode-only use
        at one row never pays for it) and kept with the kernel-layout weight
        (dropped with it when the weights change). Under graph capture a copy
        that does not exist yet is not built (it would only be recorded, and
        eager calls would read it unfilled): the call runs without it."""
        if getattr(self, "_packed_weight_tiled", None) is None:
            if not tiled_supported(self.out_features, self.in_features, self._group_size()):
                return None
            if kernel_choice(M, self.out_features, self.in_features, self._group_size(),
                             tiled=True, perm=perm is not None) not in ("tgemm", "bgemm"):
                return None
            if torch.cuda.is_current_stream_capturing():
                return None
            self._packed_weight_tiled = tile_w4a16(w_kernel, self._group_size())
        return self._packed_weight_tiled

    def adopt_kernel_layout(self, w_kernel: torch.Tensor) -> None:
        """Uses a stored kernel-layout weight of this layer (the output of
        ``repack_int4_for_kernel``, with the act_order permutation when the
        layer has g_idx) instead of repacking on the first forward."""
        if (w_kernel.dtype != torch.uint8 or w_kernel.shape != self.packed_weight.shape
                or w_kernel.device != self.packed_weight.device):
            raise ValueError("kernel-layout weight must be uint8 with the packed weight's shape "
                             "and device")
        self._build_kernel_cache(w_kernel.contiguous())

    def _forward_kernel(self, x: torch.Tensor) -> torch.Tensor:
        """pare/layers/linear.py:140-159 with the HIP kernels. bf16 inputs are
        cast to fp16 as the reference does (linear.py:154-156), unless
        ``native_bf16`` is set on the module: then they run as bf16
        (``matmul_w4a16_bf16``)."""
        w_k, zero_u8, perm, sz_gm = self._kernel_buffers()
        orig_shape = x.shape
        if x.dtype == torch.bfloat16 and getattr(self, "native_bf16", False):
            xb = x.reshape(-1, self.in_features).contiguous()
            w_t = None if perm is not None else self._tiled_buffer(w_k, xb.shape[0])
            y = matmul_w4a16_bf16(xb, w_k, self.scale, zero_u8, self._group_size(), perm=perm,
                                  perm16=self._perm16, sz_gm=sz_gm, w_tiled=w_t)
            if self.bias is not None:
                y = y + self.bias
            return y.reshape(*orig_shape[:-1], self.out_features)
        x_2d = x.reshape(-1, self.in_features).to(torch.float16).contiguous()
        w_t = self._tiled_buffer(w_k, x_2d.shape[0], perm)
        y = matmul_w4a16(x_2d, w_k, self.scale, zero_u8, self._group_size(), perm=perm,
                         perm16=self._perm16, sz_gm=sz_gm, w_tiled=w_t)
        y = y.to(x.dtype)
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(*orig_shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        return (f"in={self.in_features}, out={self.out_features}, dtype=INT4, "
                f"scheme={self.config.scheme}, granularity={self.config.granularity}, "
                f"use_kernel={getattr(self, 'use_kernel', False)}")


class FusedQuantizedLinear(nn.Module):
    """Several INT4 linears that read the same input (q/k/v, gate/up) run as one
    kernel launch over their buffers concatenated along out_features.

    Caller-side fusion: the reference launches one kernel per QuantizedLinear
    (pare/layers/linear.py:140-159). Every output element is the same
    dot product as in the separate layers; only the launch count changes, which
    at decode sizes removes a fixed per-launch cost (ramp-up to full memory
    bandwidth and drain) per merged layer. ``forward`` returns one tensor per
    fused layer, in order (views of one [..., sum(out_features)] result).
    """

    def __init__(self, layers, use_kernel: bool = True) -> None:
        super().__init__()
        layers = list(layers)
        if not layers:
            raise ValueError("FusedQuantizedLinear needs at least one layer")
        first = layers[0]
        for lay in layers[1:]:
            if lay.in_features != first.in_features:
                raise ValueError("fused layers must share in_features")
            if lay._group_size() != first._group_size() or lay.config.bits != first.config.bits:
                raise ValueError("fused layers must share the quantisation group size")
            same_gidx = (lay.g_idx is None and first.g_idx is None) or (
                lay.g_idx is not None and first.g_idx is not None and torch.equal(lay.g_idx, first.g_idx))
            if not same_gidx:
                raise ValueError("fused layers must share g_idx (act_order permutation)")
        bias = None
        if any(lay.bias is not None for lay in layers):
            dtype = next(lay.bias.dtype for lay in layers if lay.bias is not None)
            bias = torch.cat([lay.bias.detach() if lay.bias is not None else
                              torch.zeros(lay.out_features, dtype=dtype, device=lay.packed_weight.device)
                              for lay in layers])
        self.split_sizes = [lay.out_features for lay in layers]
        self.fused = QuantizedLinear(
            torch.cat([lay.packed_weight for lay in layers]),
            torch.cat([lay.scale for lay in layers]),
            torch.cat([lay.zero for lay in layers]),
            first.config, bias, first.in_features, sum(self.split_sizes), use_kernel=use_kernel,
            g_idx=first.g_idx)

    @property
    def in_features(self) -> int:
        return self.fused.in_features

    def forward(self, x: torch.Tensor):
        return tuple(torch.split(self.fused(x), self.split_sizes, dim=-1))
