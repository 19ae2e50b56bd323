"""ctypes binding of libpare_amd.so (declarations: include/pare_amd.h).

The library is loaded lazily from this package directory. A missing library is
an error, never a silent fallback: every operator of the package raises when
it cannot run on the HIP device.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libpare_amd.so"

# PMI_ABI_VERSION of include/pare_amd.h that these bindings follow.
ABI_VERSION = 16

PMI_OK = 0
PMI_ERR_INVALID = -1
PMI_ERR_UNSUPPORTED = -2
PMI_ERR_HIP = -3
PMI_ERR_NO_DEVICE = -4

PMI_F16, PMI_BF16, PMI_F32, PMI_U8 = 0, 1, 2, 3
PMI_CHOICE_TILED, PMI_CHOICE_PERM = 1, 2
PMI_LAYOUT_STORAGE, PMI_LAYOUT_KERNEL = 0, 1

_ERR_NAMES = {
    PMI_ERR_INVALID: "PMI_ERR_INVALID",
    PMI_ERR_UNSUPPORTED: "PMI_ERR_UNSUPPORTED",
    PMI_ERR_HIP: "PMI_ERR_HIP",
    PMI_ERR_NO_DEVICE: "PMI_ERR_NO_DEVICE",
}

_vp, _i, _i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64

# name -> (restype, argtypes); must match include/pare_amd.h
SIGNATURES = {
    "pmi_abi_version": (_i, []),
    "pmi_last_error": (ctypes.c_char_p, []),
    "pmi_device_supported": (_i, [_i]),
    "pmi_repack_int4_for_kernel": (_i, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "pmi_zeros_to_u8": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "pmi_perm_u16": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "pmi_sz_group_major": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i64, _i64, _vp]),
    "pmi_matmul_w4a16_glu": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i64, _i64, _i64, _i64, _vp]),
    "pmi_matmul_w4a16_rmsnorm": (_i, [_vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _i, _vp,
                                      _i64, _i64, _i64, _i64, _vp]),
    "pmi_gptq_group_params": (_i, [_vp, _i64, _i64, _i64, _i64, _i, _vp, _vp, _i64, _i64, _vp]),
    "pmi_gptq_block": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                            _vp]),
    "pmi_gptq_pack": (_i, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "pmi_awq_gemm_to_storage": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "pmi_storage_to_awq_gemm": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                     _vp]),
    "pmi_tiled_bytes": (ctypes.c_size_t, [_i64, _i64]),
    "pmi_tile_w4a16": (_i, [_vp, _vp, _i64, _i64, _i64, _vp]),
    "pmi_matmul_w4a16": (_i, [_vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i64, _i64,
                             _i64, _i64, _vp, ctypes.c_size_t, _vp]),
    "pmi_matmul_w4a16_noalloc": (_i, [_vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i64,
                                      _i64, _i64, _i64, _vp]),
    "pmi_matmul_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, _i]),
    "pmi_dequant_w4a16": (_i, [_vp, _i, _vp, _vp, _i, _vp, _vp, _i, _i64, _i64, _i64, _vp]),
    "pmi_rtn_quantize": (_i, [_vp, _i, _vp, _vp, _vp, _i64, _i64, _i64, _i, _vp]),
    "pmi_matmul_kernel_choice": (_i, [_i64, _i64, _i64, _i64, _i]),
    "pmi_tgemm_splits": (_i, [_i64, _i64, _i64, _i64, _i]),
    "pmi_matmul_w4a16_gate_up_silu": (_i, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "pmi_gate_up_silu_supported": (_i, [_i64, _i64, _i64, _i64]),
    "pmi_matmul_w4a16_tiled_rmsnorm": (_i, [_vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _vp,
                                            _i64, _i64, _i64, _i64, _i, _vp]),
    "pmi_tiled_rmsnorm_supported": (_i, [_i64, _i64, _i64, _i64, _i]),
    "pmi_matmul_w4a16_residual": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "pmi_residual_stats_count": (_i, [_i64, _i64, _i]),
    "pmi_matmul_w4a16_prenormed": (_i, [_vp, _vp, _i, _vp, ctypes.c_float, _vp, _vp, _vp, _vp,
                                        _i64, _i64, _i64, _vp]),
    "pmi_set_kernel_override": (_i, [_i]),
    "pmi_add_rmsnorm_f16": (_i, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp]),
    "pmi_rope_kv_f16": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                             _vp]),
    "pmi_decode_attention_f16": (_i, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                      ctypes.c_float, _vp, ctypes.c_size_t, _vp]),
    "pmi_decode_attention_rope_f16": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                           _i64, _i64, ctypes.c_float, _vp, ctypes.c_size_t,
                                           _vp]),
    "pmi_decode_attention_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64]),
    "pmi_argmax_f16": (_i, [_vp, _i64, _i64, _vp, _i64, _vp, ctypes.c_size_t, _vp]),
    "pmi_argmax_workspace_bytes": (ctypes.c_size_t, [_i64, _i64]),
    "pmi_read_probe": (_i, [_vp, _i64, _i64, _vp, _vp]),
    "pmi_silu_mul_f16": (_i, [_vp, _vp, _i64, _i64, _vp]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class PmiError(RuntimeError):
    """A libpare_amd entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, message: str):
        self.code = code
        super().__init__(f"{fn} failed ({_ERR_NAMES.get(code, code)}): {message}")


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            # torch first: its bundled HIP runtime carries the soname
            # libamdhip64.so.7, so the library binds to that same runtime
            # (torch's stream handles are then valid inside it).
            import torch  # noqa: F401

            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m pare_amd.build` "
                    "(pare_amd has no CPU fallback)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def last_error() -> str:
    return lib().pmi_last_error().decode("utf-8", "replace")


def check(rc: int, fn: str) -> None:
    if rc != PMI_OK:
        raise PmiError(fn, rc, last_error())


def call(fn: str, *args) -> None:
    """Calls entry point `fn` and raises PmiError on a non-zero status."""
    check(getattr(lib(), fn)(*args), fn)
