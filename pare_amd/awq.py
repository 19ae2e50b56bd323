"""AWQ-GEMM int32 checkpoints on the INT4 path.

The format is the one pare/model/export_awq.py:37-136 writes (AutoAWQ's
``WQLinear_GEMM``, which vLLM loads). Each linear has these tensors:
  - ``qweight`` int32 [in, out/8];
  - ``qzeros`` int32 [G, out/8];
  - ``scales`` fp16 [G, out];
  - optional ``bias`` fp16 [out].
Eight 4-bit codes share an int32 along the output dimension. Output column
``8c + AWQ_ORDER[i]`` sits in bits ``4i..4i+3`` of word ``c``. The model's
``config.json`` carries ``quantization_config = {"quant_method": "awq", "bits": 4,
"group_size": gs, "version": "gemm", "zero_point": True}``.

Both directions run on the HIP device, one pass each:
  - ``awq_to_storage`` turns the AWQ tensors into this path's buffers:
    storage-layout packed weight, and fp32 scale and zero [N, G, 1].
  - ``storage_to_awq`` is the reverse, the repack of ``_to_awq_linear``.
The weights and zero points convert exactly both ways. Export rounds the
fp32 scales to fp16, as the reference does (export_awq.py:92).

An imported layer is an ordinary ``QuantizedLinear``. Its first kernel
forward builds the kernel layout, as for any other layer. Every token
afterwards reads that layout, so AWQ checkpoints run on the same tuned GEMV
and GEMM kernels as natively quantized layers.
"""

from __future__ import annotations

import json
from pathlib import Path

import torch
import torch.nn as nn

from . import _lib
from .config import QuantConfig, kernel_group_size
from .kernels import _DeviceGuard, _stream_handle, _to_2d
from .linear import QuantizedLinear
from .model_io import replace_module

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)   # pare/model/export_awq.py:37-39
CONFIG_FILE = "config.json"


def _cuda(t: torch.Tensor, fn: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{fn} runs on the HIP device; got a tensor on {t.device}")


def awq_to_storage(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                   group_size: int | None = None):
    """AWQ-GEMM tensors -> (packed uint8 [N, K/2] storage layout, scale fp32
    [N, G, 1], zero fp32 [N, G, 1]) with K = qweight rows and N = 8 x its
    columns. ``group_size`` defaults to K / G (G = scales rows)."""
    L = _lib.lib()
    _cuda(qweight, "awq_to_storage")
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32 or qweight.dim() != 2:
        raise ValueError("qweight and qzeros must be int32 matrices")
    if scales.dtype != torch.float16:
        raise ValueError(f"scales must be fp16 [G, N], got {scales.dtype}")
    K, NC = qweight.shape
    N = NC * 8
    G = scales.shape[0]
    gs = group_size if group_size not in (None, -1) else (K // G if G else 0)
    if G == 0 or K % gs != 0 or K // gs != G:
        raise ValueError(f"scales have {G} groups; K={K} with group_size={gs} needs {K // max(gs, 1)}")
    if tuple(scales.shape) != (G, N) or tuple(qzeros.shape) != (G, NC):
        raise ValueError(f"expected qzeros [{G}, {NC}] and scales [{G}, {N}], got "
                         f"{tuple(qzeros.shape)} and {tuple(scales.shape)}")
    dev = qweight.device
    qw, qz, sc = qweight.contiguous(), qzeros.to(dev).contiguous(), scales.to(dev).contiguous()
    packed = torch.empty(N, K // 2, dtype=torch.uint8, device=dev)
    scale = torch.empty(N, G, dtype=torch.float32, device=dev)
    zero = torch.empty(N, G, dtype=torch.float32, device=dev)
    with _DeviceGuard(dev):
        _lib.check(L.pmi_awq_gemm_to_storage(qw.data_ptr(), qz.data_ptr(), sc.data_ptr(),
                                             packed.data_ptr(), scale.data_ptr(), zero.data_ptr(),
                                             N, K, gs, _stream_handle(dev)),
                   "pmi_awq_gemm_to_storage")
    return packed, scale.unsqueeze(-1), zero.unsqueeze(-1)


def storage_to_awq(packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor,
                   group_size: int):
    """Storage-layout weight + scale/zero [N, G(, 1)] -> (qweight int32 [K, N/8],
    qzeros int32 [G, N/8], scales fp16 [G, N]) (pare/model/export_awq.py:75-94).
    Raises ValueError when a zero point rounds to a value outside [0, 15]."""
    L = _lib.lib()
    _cuda(packed, "storage_to_awq")
    if packed.dtype != torch.uint8 or packed.dim() != 2:
        raise ValueError("packed must be uint8 [N, K//2]")
    N, K = packed.shape[0], packed.shape[1] * 2
    dev = packed.device
    s = _to_2d(scale).to(dev).float().contiguous()
    z = _to_2d(zero).to(dev)
    z = z.contiguous() if z.dtype == torch.uint8 else z.float().contiguous()
    G = K // group_size
    if tuple(s.shape) != (N, G) or tuple(z.shape) != (N, G):
        raise ValueError(f"scale and zero must be [{N}, {G}], got {tuple(s.shape)}, {tuple(z.shape)}")
    src = packed.contiguous()
    qweight = torch.empty(K, N // 8, dtype=torch.int32, device=dev)
    qzeros = torch.empty(G, N // 8, dtype=torch.int32, device=dev)
    scales = torch.empty(G, N, dtype=torch.float16, device=dev)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    zdt = _lib.PMI_U8 if z.dtype == torch.uint8 else _lib.PMI_F32
    with _DeviceGuard(dev):
        _lib.check(L.pmi_storage_to_awq_gemm(src.data_ptr(), s.data_ptr(), z.data_ptr(), zdt,
                                             qweight.data_ptr(), qzeros.data_ptr(),
                                             scales.data_ptr(), bad.data_ptr(), N, K, group_size,
                                             _stream_handle(dev)),
                   "pmi_storage_to_awq_gemm")
    if int(bad.item()) != 0:
        raise ValueError(f"{int(bad.item())} zero points round to values outside [0, 15]")
    return qweight, qzeros, scales


class AwqGemmLinear(nn.Module):
    """Holder of one layer's AWQ-GEMM buffers, so a state dict serialises in
    the format (pare/model/export_awq.py:52-72). It has no forward: a serving
    stack replaces it at load time, and ``load_awq`` turns it back into a
    ``QuantizedLinear``."""

    def __init__(self, in_features: int, out_features: int, group_size: int, has_bias: bool):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.w_bit = 4
        self.group_size = group_size
        G = in_features // group_size
        self.register_buffer("qweight", torch.zeros(in_features, out_features // 8, dtype=torch.int32))
        self.register_buffer("qzeros", torch.zeros(G, out_features // 8, dtype=torch.int32))
        self.register_buffer("scales", torch.zeros(G, out_features, dtype=torch.float16))
        if has_bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=torch.float16))
        else:
            self.bias = None


def to_awq_linear(ql: QuantizedLinear, group_size: int | None = None) -> AwqGemmLinear:
    """Repacks one INT4 layer (pare/model/export_awq.py:75-94). The buffers come
    back on the layer's device; a CPU layer is repacked on the current HIP
    device."""
    gs = group_size or kernel_group_size(ql.config, ql.in_features)
    out_f, in_f = ql.out_features, ql.in_features
    if in_f % gs != 0 or out_f % 8 != 0:
        raise ValueError(f"AWQ-GEMM packs eight output columns per int32 word and whole groups "
                         f"per row: out_features={out_f} must be a multiple of 8 and "
                         f"in_features={in_f} a multiple of group_size={gs}")
    if ql.g_idx is not None:
        raise ValueError("AWQ-GEMM has no g_idx: act_order layers cannot be exported")
    home = ql.packed_weight.device
    dev = home if home.type == "cuda" else torch.device("cuda")
    qweight, qzeros, scales = storage_to_awq(ql.packed_weight.to(dev), ql.scale.to(dev),
                                             ql.zero.to(dev), gs)
    m = AwqGemmLinear(in_f, out_f, gs, ql.bias is not None)
    m.qweight, m.qzeros, m.scales = qweight.to(home), qzeros.to(home), scales.to(home)
    if ql.bias is not None:
        m.bias = ql.bias.data.half().to(home)
    return m


def awq_quantization_config(group_size: int) -> dict:
    """The ``quantization_config`` of an AWQ-GEMM checkpoint
    (pare/model/export_awq.py:126-132)."""
    return {"quant_method": "awq", "bits": 4, "group_size": group_size, "version": "gemm",
            "zero_point": True}


def export_awq(model: nn.Module, save_dir, tokenizer=None) -> str:
    """Replaces every QuantizedLinear of ``model`` in place with an
    ``AwqGemmLinear`` and writes the checkpoint (pare/model/export_awq.py:97-136).

    A HuggingFace model is written with ``save_pretrained`` as the reference
    does. Any other module gets ``model.safetensors`` (its state dict) and a
    ``config.json`` that holds ``quantization_config``."""
    qls = [(n, m) for n, m in model.named_modules() if isinstance(m, QuantizedLinear)]
    if not qls:
        raise ValueError("export_awq: the model holds no INT4 QuantizedLinear layer to export")
    sizes = {kernel_group_size(m.config, m.in_features) for _, m in qls}
    if len(sizes) != 1:
        raise ValueError(f"AWQ checkpoints have one group size; the layers use {sorted(sizes)}")
    gs = sizes.pop()
    for name, m in qls:
        replace_module(model, name, to_awq_linear(m, gs))
    qcfg = awq_quantization_config(gs)
    save_dir = str(save_dir)
    if hasattr(model, "save_pretrained") and hasattr(model, "config"):
        model.config.quantization_config = qcfg
        model.save_pretrained(save_dir)
    else:
        from safetensors.torch import save_file

        path = Path(save_dir)
        path.mkdir(parents=True, exist_ok=True)
        seen, tensors = set(), {}
        for k, v in model.state_dict().items():
            v = v.detach().contiguous().cpu()
            if v.untyped_storage().data_ptr() not in seen:
                seen.add(v.untyped_storage().data_ptr())
                tensors[k] = v
        save_file(tensors, str(path / "model.safetensors"))
        (path / CONFIG_FILE).write_text(json.dumps({"quantization_config": qcfg}, indent=2))
    if tokenizer is not None:
        tokenizer.save_pretrained(save_dir)
    return save_dir


def read_awq_config(path) -> dict:
    """``quantization_config`` of an AWQ-GEMM checkpoint directory, checked for
    what this path runs: 4-bit, GEMM packing, zero points."""
    path = Path(path)
    cfg = json.loads((path / CONFIG_FILE).read_text()) if (path / CONFIG_FILE).exists() else {}
    q = cfg.get("quantization_config")
    if q is None and (path / "quant_config.json").exists():   # older AutoAWQ directories
        q = json.loads((path / "quant_config.json").read_text())
    if q is None:
        raise ValueError(f"{path}: no quantization_config in {CONFIG_FILE}")
    method = q.get("quant_method", "awq")
    bits = q.get("bits", q.get("w_bit"))
    version = str(q.get("version", "gemm")).lower()
    if method != "awq" or bits != 4 or version != "gemm":
        raise ValueError(f"{path}: need an AWQ 4-bit GEMM checkpoint, got quant_method={method!r} "
                         f"bits={bits!r} version={version!r}")
    if not q.get("zero_point", True):
        raise ValueError(f"{path}: checkpoints without zero points are not AWQ-GEMM")
    return {"group_size": int(q.get("group_size", q.get("q_group_size", 128)))}


def from_awq_tensors(qweight, qzeros, scales, bias=None, group_size=None,
                     use_kernel: bool = True) -> QuantizedLinear:
    """One ``QuantizedLinear`` from a layer's AWQ-GEMM tensors (on the HIP
    device; the layer's buffers stay there)."""
    K = qweight.shape[0]
    gs = K if group_size in (None, -1) else int(group_size)
    packed, scale, zero = awq_to_storage(qweight, qzeros, scales, gs)
    config = QuantConfig(bits=4, scheme="awq", granularity="per_group", group_size=gs)
    ql = QuantizedLinear(packed, scale, zero, config, bias, K, packed.shape[0])
    ql.use_kernel = use_kernel
    return ql


def load_awq(model: nn.Module, path, use_kernel: bool = True, device="cuda") -> nn.Module:
    """Loads an AWQ-GEMM checkpoint directory into ``model``. Every
    ``<name>.qweight`` becomes a ``QuantizedLinear`` at ``<name>``, built on
    ``device``. The other tensors load into the model's own parameters, with
    ``strict=False``. Reads ``*.safetensors`` (sharded checkpoints included)
    and JSON only."""
    from safetensors.torch import load_file

    path = Path(path)
    gs = read_awq_config(path)["group_size"]
    files = sorted(path.glob("*.safetensors"))
    if not files:
        raise ValueError(f"{path}: no .safetensors files")
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("load_awq repacks on the HIP device; pass a cuda device")
    tensors: dict[str, torch.Tensor] = {}
    for f in files:
        tensors.update(load_file(str(f), device=str(dev)))
    layers = sorted(k[: -len(".qweight")] for k in tensors if k.endswith(".qweight"))
    if not layers:
        raise ValueError(f"{path}: no '<layer>.qweight' tensors")
    for name in layers:
        pre = name + "."
        ql = from_awq_tensors(tensors[pre + "qweight"], tensors[pre + "qzeros"],
                              tensors[pre + "scales"], tensors.get(pre + "bias"), gs, use_kernel)
        replace_module(model, name, ql)
    prefixes = tuple(n + "." for n in layers)
    rest = {k: v for k, v in tensors.items() if not k.startswith(prefixes)}
    model.load_state_dict(rest, strict=False)
    return model
