"""Host-side checks of the module layer that need no GPU: buffer validation and
fusion rules (pare/layers/linear.py:40-99 buffer contract)."""

from __future__ import annotations

import pytest
import torch

import pare_amd as P


def _ql(N, K, gs=128, g_idx=None):
    packed = torch.zeros(N, K // 2, dtype=torch.uint8)
    scale = torch.ones(N, K // gs, 1)
    zero = torch.full((N, K // gs, 1), 8.0)
    return P.QuantizedLinear(packed, scale, zero, P.QuantConfig(group_size=gs), None, K, N,
                             use_kernel=True, g_idx=g_idx)


def test_quantized_linear_rejects_bad_packed_shape():
    with pytest.raises(ValueError, match="packed_weight"):
        P.QuantizedLinear(torch.zeros(8, 10, dtype=torch.uint8), torch.ones(8, 1, 1),
                          torch.zeros(8, 1, 1), P.QuantConfig(group_size=128), None, 128, 8)


def test_quantized_linear_cpu_forward_raises():
    with pytest.raises(RuntimeError, match="HIP device"):
        _ql(8, 128)(torch.zeros(1, 128))


def test_fused_concatenates_buffers():
    f = P.FusedQuantizedLinear([_ql(64, 256), _ql(16, 256), _ql(16, 256)])
    assert f.split_sizes == [64, 16, 16]
    assert tuple(f.fused.packed_weight.shape) == (96, 128)
    assert tuple(f.fused.scale.shape) == (96, 2, 1)
    assert f.in_features == 256 and f.fused.use_kernel


def test_fused_rejects_mismatched_layers():
    with pytest.raises(ValueError, match="in_features"):
        P.FusedQuantizedLinear([_ql(64, 256), _ql(64, 512)])
    with pytest.raises(ValueError, match="group size"):
        P.FusedQuantizedLinear([_ql(64, 256, gs=128), _ql(64, 256, gs=64)])
    g = torch.arange(256, dtype=torch.int32) // 128
    with pytest.raises(ValueError, match="g_idx"):
        P.FusedQuantizedLinear([_ql(64, 256, g_idx=g), _ql(64, 256)])
    with pytest.raises(ValueError, match="at least one"):
        P.FusedQuantizedLinear([])
