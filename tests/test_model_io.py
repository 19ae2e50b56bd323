"""Save/load in the reference's on-disk format (pare/model/io.py:1-216)."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
import torch.nn as nn
from safetensors.torch import save_file

import pare_amd as P
from oracle import pare_oracle as O
from pare_amd.model_io import KERNEL_LAYOUT_VERSION, load_quantized, save_quantized


class Tiny(nn.Module):
    def __init__(self, K=256, N=64):
        super().__init__()
        self.embed = nn.Embedding(10, K)
        self.norm = nn.LayerNorm(K)
        self.proj = nn.Linear(K, N)
        self.head = nn.Linear(N, 10, bias=False)


def _quantized_tiny(seed=0, K=256, N=64, gs=128, bias=True):
    torch.manual_seed(seed)
    m = Tiny(K, N)
    w = (torch.randn(N, K) * 0.02).numpy()
    packed, s, z = O.rtn_quantize(w, gs)
    b = torch.randn(N) if bias else None
    ql = P.QuantizedLinear(torch.from_numpy(packed), torch.from_numpy(s), torch.from_numpy(z),
                           P.QuantConfig(bits=4, group_size=gs), b, K, N)
    m.proj = ql
    return m


def test_roundtrip_cpu(tmp_path):
    src = _quantized_tiny(1)
    save_quantized(src, tmp_path)
    meta = json.loads((tmp_path / "pare_config.json").read_text())
    lm = meta["quantized_layers"]["proj"]
    assert lm["in_features"] == 256 and lm["out_features"] == 64 and lm["has_bias"]
    assert lm["bits"] == 4 and lm["group_size"] == 128 and lm["granularity"] == "per_group"
    dst = load_quantized(Tiny(), tmp_path)
    assert isinstance(dst.proj, P.QuantizedLinear) and dst.proj.use_kernel
    for k in ("packed_weight", "scale", "zero"):
        assert torch.equal(getattr(dst.proj, k), getattr(src.proj, k))
    assert torch.equal(dst.proj.bias, src.proj.bias)
    assert torch.equal(dst.embed.weight, src.embed.weight)
    assert torch.equal(dst.head.weight, src.head.weight)


def test_loads_a_reference_format_directory(tmp_path):
    """A directory laid out exactly as the reference's save_quantized writes it
    (state_dict keys of its QuantizedLinear: packed_weight, scale [N,G,1],
    zero [N,G,1], bias; metadata fields of pare/model/io.py:71-82)."""
    N, K, gs = 64, 256, 128
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, (N, K))
    packed = O.pack_int4(q)
    scale = rng.uniform(0.001, 0.01, (N, K // gs, 1)).astype(np.float32)
    zero = rng.integers(0, 16, (N, K // gs, 1)).astype(np.float32)
    m = Tiny(K, N)
    tensors = {"proj.packed_weight": torch.from_numpy(packed), "proj.scale": torch.from_numpy(scale),
               "proj.zero": torch.from_numpy(zero), "proj.bias": torch.zeros(N),
               "embed.weight": m.embed.weight.detach(), "norm.weight": m.norm.weight.detach(),
               "norm.bias": m.norm.bias.detach(), "head.weight": m.head.weight.detach()}
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(tmp_path / "model.safetensors"))
    meta = {"pare_version": "0.1.3", "quantized_layers": {"proj": {
        "bits": 4, "scheme": "gptq", "granularity": "per_group", "group_size": gs, "sym": False,
        "smooth_alpha": 0.5, "in_features": K, "out_features": N, "quantize_inputs": False,
        "has_bias": True}}}
    (tmp_path / "pare_config.json").write_text(json.dumps(meta))
    out = load_quantized(Tiny(K, N), tmp_path)
    assert out.proj.use_kernel and out.proj.config.scheme == "gptq"
    assert np.array_equal(out.proj.packed_weight.numpy(), packed)
    assert np.array_equal(out.proj.zero.numpy(), zero) and np.array_equal(out.proj.scale.numpy(), scale)


def test_rejects_w8a8_layers(tmp_path):
    src = _quantized_tiny(2)
    save_quantized(src, tmp_path)
    meta = json.loads((tmp_path / "pare_config.json").read_text())
    meta["quantized_layers"]["proj"]["quantize_inputs"] = True
    (tmp_path / "pare_config.json").write_text(json.dumps(meta))
    with pytest.raises(NotImplementedError):
        load_quantized(Tiny(), tmp_path)


@pytest.mark.gpu
@pytest.mark.parametrize("kernel_layout", [False, True])
def test_roundtrip_gpu_forward(tmp_path, kernel_layout):
    dev = torch.device("cuda:0")
    src = _quantized_tiny(4).to(dev)
    src.proj.use_kernel = True
    x = torch.randn(3, 256, device=dev).half()
    y0 = src.proj(x)
    save_quantized(src, tmp_path, kernel_layout=kernel_layout)
    meta = json.loads((tmp_path / "pare_config.json").read_text())
    assert (meta.get("kernel_layout_version") == KERNEL_LAYOUT_VERSION) == kernel_layout
    dst = load_quantized(Tiny(), tmp_path, device=dev).to(dev)
    if kernel_layout:
        assert dst.proj._packed_weight_kernel is not None
    y1 = dst.proj(x)
    assert torch.equal(y0, y1)


@pytest.mark.gpu
@pytest.mark.parametrize("act_order", [False, True])
@pytest.mark.parametrize("kernel_layout", [False, True])
def test_reloaded_layer_matches_oracle(tmp_path, kernel_layout, act_order):
    """A layer written by save_quantized and read back by load_quantized (with
    and without the stored kernel layout, with and without g_idx) against the
    oracle: dequantized weights bit-exact, forward within rtol/atol 1e-2 of the
    fp32-accumulated reference."""
    import warnings

    dev = torch.device("cuda:0")
    N, K, gs = 192, 512, 128
    w = (torch.randn(N, K, generator=torch.Generator().manual_seed(11)) * 0.02).numpy()
    g_idx = None
    if act_order:
        perm = np.random.default_rng(5).permutation(K)
        packed, s, z, g_idx = O.rtn_quantize_act_order(w, perm, gs)
        w_hat = O.dequantize_gidx(O.unpack_int4(packed), s, z, g_idx)
    else:
        packed, s, z = O.rtn_quantize(w, gs)
        w_hat = O.dequantize_packed(packed, s, z)
    m = Tiny(K, N)
    m.proj = P.QuantizedLinear(torch.from_numpy(packed), torch.from_numpy(s), torch.from_numpy(z),
                               P.QuantConfig(bits=4, group_size=gs), None, K, N,
                               g_idx=torch.from_numpy(g_idx) if act_order else None)
    m = m.to(dev)
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        save_quantized(m, tmp_path, kernel_layout=kernel_layout)
    assert any("g_idx" in str(c.message) for c in caught) == act_order
    dst = load_quantized(Tiny(K, N), tmp_path, device=dev).to(dev)
    assert (dst.proj.g_idx is not None) == act_order
    dq = dst.proj.dequantize(torch.float16).cpu().numpy()
    assert (dq.view(np.uint16) == w_hat.astype(np.float16).view(np.uint16)).all()
    x = torch.randn(5, K, generator=torch.Generator().manual_seed(12)).half()
    y = dst.proj(x.to(dev)).float().cpu().numpy()
    ref = O.linear_fp32(x.float().numpy(), w_hat)
    err = np.abs(y - ref)
    print(f"[reload] kernel_layout={kernel_layout} act_order={act_order}: max_abs={err.max():.3e}",
          flush=True)
    assert (err <= 1e-2 + 1e-2 * np.abs(ref)).all()
