"""Save and load models whose linears are INT4 QuantizedLinear layers.

The on-disk format is the reference's (pare/model/io.py:1-216): a directory
with ``model.safetensors`` (every tensor of the state dict: the quantized
buffers ``<layer>.packed_weight`` / ``.scale`` / ``.zero`` / ``.bias`` and all
non-quantized parameters) and ``pare_config.json`` (``{"pare_version": ..,
"quantized_layers": {name: {bits, scheme, granularity, group_size, sym,
smooth_alpha, in_features, out_features, quantize_inputs, has_bias}}}``).
Directories written by the reference load here. The reverse holds for INT4
layers without g_idx only: the reference's loader ignores ``<layer>.g_idx``
and dequantizes act_order layers with contiguous groups, which gives wrong
weights without an error, so ``save_quantized`` warns when it writes such a
layer.

Differences from the reference, all additive:
  - ``load_quantized`` sets ``use_kernel`` on every loaded layer (the
    reference's ``from_tensors`` never sets it, pare/layers/linear.py:166-202,
    so its reloaded layers fail on their first forward) and can place the
    buffers on a device.
  - act_order layers keep their ``<layer>.g_idx`` tensor (int32 [in]); the
    metadata records ``has_g_idx``.
  - ``save_quantized(..., kernel_layout=True)`` also stores each layer's
    derived kernel-layout weight as ``<layer>.packed_weight_kernel`` and
    records ``kernel_layout_version``; a loader with the same version takes it
    instead of repacking. Unknown keys are ignored by the reference's loader.
Only safetensors and JSON are read: nothing in a checkpoint is executed.
"""

from __future__ import annotations

import json
import warnings
from pathlib import Path

import torch
import torch.nn as nn

from .config import QuantConfig
from .linear import QuantizedLinear

PARE_CONFIG_FILE = "pare_config.json"
TENSORS_FILE = "model.safetensors"
# Version of the stored kernel layout (pare/core/pack.py:88-132 byte order,
# optionally with the act_order column permutation applied first).
KERNEL_LAYOUT_VERSION = 1


def save_quantized(model: nn.Module, path, kernel_layout: bool = False) -> None:
    """Writes ``path/model.safetensors`` and ``path/pare_config.json``
    (pare/model/io.py:52-123)."""
    from safetensors.torch import save_file

    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    layers: dict[str, dict] = {}
    extra: dict[str, torch.Tensor] = {}
    for name, m in model.named_modules():
        if isinstance(m, QuantizedLinear):
            layers[name] = {
                "bits": m.config.bits,
                "scheme": m.config.scheme,
                "granularity": m.config.granularity,
                "group_size": m.config.group_size,
                "sym": m.config.sym,
                "smooth_alpha": getattr(m.config, "smooth_alpha", 0.5),
                "in_features": m.in_features,
                "out_features": m.out_features,
                "quantize_inputs": False,
                "has_bias": m.bias is not None,
                "has_g_idx": m.g_idx is not None,
            }
            if kernel_layout:
                w_k = m._kernel_buffers()[0]
                extra[name + ".packed_weight_kernel"] = w_k
    act_order = [n for n, meta in layers.items() if meta["has_g_idx"]]
    if act_order:
        warnings.warn(f"save_quantized: {len(act_order)} act_order layer(s) (first: {act_order[0]}) "
                      "carry g_idx; the reference's load_quantized ignores it and would "
                      "dequantize them with contiguous groups", stacklevel=2)
    if not layers:
        raise ValueError("save_quantized: the model holds no QuantizedLinear layer to save "
                         "(quantize it before saving)")
    # one copy per storage (tied weights, pare/model/io.py:92-107)
    seen: set[int] = set()
    tensors: dict[str, torch.Tensor] = {}
    for k, v in list(model.state_dict().items()) + list(extra.items()):
        v = v.detach().contiguous().cpu()
        ptr = v.untyped_storage().data_ptr()
        if ptr not in seen:
            seen.add(ptr)
            tensors[k] = v
    save_file(tensors, str(path / TENSORS_FILE))
    meta = {"pare_version": "pare_amd", "quantized_layers": layers}
    if kernel_layout:
        meta["kernel_layout_version"] = KERNEL_LAYOUT_VERSION
    (path / PARE_CONFIG_FILE).write_text(json.dumps(meta, indent=2))


def replace_module(root: nn.Module, dotted: str, new: nn.Module) -> None:
    """Puts `new` in place of the submodule at dotted path `dotted` of `root`."""
    parent_name, _, leaf = dotted.rpartition(".")
    setattr(root.get_submodule(parent_name), leaf, new)


def load_quantized(model: nn.Module, path, use_kernel: bool = True, device=None) -> nn.Module:
    """Rebuilds the QuantizedLinear layers of ``path`` in ``model`` and loads
    the other tensors (pare/model/io.py:130-196). INT4 layers only: this
    package implements the INT4 kernel path."""
    from safetensors.torch import load_file

    path = Path(path)
    meta = json.loads((path / PARE_CONFIG_FILE).read_text())
    layers: dict[str, dict] = meta["quantized_layers"]
    tensors = load_file(str(path / TENSORS_FILE), device=str(device) if device is not None else "cpu")
    stored_layout = meta.get("kernel_layout_version") == KERNEL_LAYOUT_VERSION
    for name, lm in layers.items():
        if lm.get("quantize_inputs", False):
            raise NotImplementedError(f"{name}: quantize_inputs (SmoothQuant W8A8) is not part of "
                                      "the INT4 path")
        config = QuantConfig(bits=lm["bits"], scheme=lm["scheme"], granularity=lm["granularity"],
                             group_size=lm["group_size"], sym=lm["sym"])
        pre = name + "."
        ql = QuantizedLinear.from_tensors(
            packed_weight=tensors.get(pre + "packed_weight"), q_weight=tensors.get(pre + "q_weight"),
            scale=tensors[pre + "scale"], zero=tensors[pre + "zero"], config=config,
            bias=tensors.get(pre + "bias"), in_features=lm["in_features"],
            out_features=lm["out_features"], g_idx=tensors.get(pre + "g_idx"))
        ql.use_kernel = use_kernel
        w_k = tensors.get(pre + "packed_weight_kernel")
        if stored_layout and w_k is not None and ql.packed_weight.is_cuda:
            ql.adopt_kernel_layout(w_k)
        replace_module(model, name, ql)
    prefixes = tuple(n + "." for n in layers)
    rest = {k: v for k, v in tensors.items() if not k.startswith(prefixes)}
    model.load_state_dict(rest, strict=False)
    return model
