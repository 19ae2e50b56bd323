"""pare_amd — MI355X (gfx950) INT4 W4A16 dequant-matmul, a drop-in for the
``QuantizedLinear.use_kernel=True`` path of Pare.

Operator API (mirrors pare.kernels.matmul_int4 and pare.core.pack):
  matmul_w4a16, repack_int4_for_kernel, kernel_available / triton_available
Module: QuantizedLinear (mirrors pare.layers.linear.QuantizedLinear)
Producers: rtn_quantize (pare.schemes.rtn on the device); gptq_quantize,
     quantize_linear_gptq, HessianAccumulator (pare.schemes.gptq, with g_idx)
I/O: save_quantized / load_quantized (pare.model.io's on-disk format);
     export_awq / load_awq (the AWQ-GEMM int32 checkpoint of pare.model.export_awq)
All compute runs in libpare_amd.so (hand-written HIP); there is no CPU fallback.
"""

from .awq import export_awq, load_awq
from .config import QuantConfig, QuantDtype
from .gptq import HessianAccumulator, gptq_quantize, quantize_linear_gptq
from .kernels import kernel_available, kernel_choice, matmul_w4a16, matmul_w4a16_bf16, triton_available
from .linear import FusedQuantizedLinear, QuantizedLinear
from .model_io import load_quantized, save_quantized
from .pack import (dequantize_int4, perm_from_g_idx, perm_u16, repack_int4_for_kernel, sz_group_major,
                   tile_w4a16, tiled_supported, zeros_to_u8)
from .quant import rtn_quantize

__all__ = [
    "FusedQuantizedLinear", "QuantConfig", "QuantDtype", "QuantizedLinear", "dequantize_int4",
    "export_awq", "gptq_quantize", "HessianAccumulator", "kernel_available", "load_awq",
    "quantize_linear_gptq",
    "kernel_choice", "matmul_w4a16", "matmul_w4a16_bf16", "perm_from_g_idx", "perm_u16",
    "repack_int4_for_kernel",
    "load_quantized", "rtn_quantize", "save_quantized", "sz_group_major", "tile_w4a16",
    "tiled_supported", "triton_available", "zeros_to_u8",
]
