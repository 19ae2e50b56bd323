"""A random-init Llama-3.1-8B-shaped decoder with every linear on the INT4 HIP
path: the caller side of QuantizedLinear, used to measure end-to-end decode.

The reference measures decode with HuggingFace ``generate`` on a quantised
checkpoint (pare/eval/throughput.py:84-126: greedy, tok/s = batch * n_generate
/ elapsed, elapsed including the prefill). No checkpoint can be fetched here,
so the model is built from seeded random weights of the Llama-3.1-8B shape
(hidden 4096, 32 heads, 8 KV heads, FFN 14336, vocab 128256), quantised with
RTN INT4 g128 on the device. Every linear except lm_head is a QuantizedLinear
(lm_head stays fp16, as the reference's default excludes it, pare/config.py:52);
q/k/v and gate/up each run as one fused launch (FusedQuantizedLinear).
Activations, the KV cache and lm_head are fp16; RoPE is the plain form with
theta 500000 (Llama 3.1's long-context frequency scaling changes no cost at
these lengths); prefill attention is PyTorch's fp16 SDPA.

Decode steps run as one captured HIP graph per batch size: the step reads the
token and position from device tensors, writes its K/V at that position of a
fixed-length cache and attends over the cache up to that position, so every
replay has the same shapes. The greedy argmax runs outside the graph.

With ``fused_ops`` (the default) the ops around the linears are the library's
caller-side kernels: residual add + RMSNorm, RoPE + KV-cache write, grouped-
query decode attention and SiLU-gate multiply, one launch each. With
``fused_ops=False`` they are plain PyTorch ops (the check in the tests).
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .config import QuantConfig
from .kernels import (_stream_handle, gate_up_silu_supported, glu_row_order, kernel_choice,
                      matmul_w4a16_gate_up_silu, matmul_w4a16_glu, matmul_w4a16_prenormed,
                      matmul_w4a16_residual, matmul_w4a16_rmsnorm, matmul_w4a16_tiled_rmsnorm,
                      residual_stats_count, tiled_rmsnorm_supported)
from .pack import sz_group_major, tile_w4a16
from .linear import FusedQuantizedLinear, QuantizedLinear
from .quant import rtn_quantize


@dataclass
class DecoderConfig:
    hidden: int = 4096
    heads: int = 32
    kv_heads: int = 8
    ffn: int = 14336
    vocab: int = 128256
    layers: int = 32
    rope_theta: float = 500000.0
    rms_eps: float = 1e-5
    group_size: int = 128
    init_std: float = 0.02

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


def _int4_linear(n_out: int, n_in: int, gen: torch.Generator, cfg: DecoderConfig,
                 dev: torch.device) -> QuantizedLinear:
    w = torch.randn(n_out, n_in, generator=gen, device=dev) * cfg.init_std
    packed, scale, zero = rtn_quantize(w, cfg.group_size)
    del w
    qcfg = QuantConfig(bits=4, scheme="rtn", group_size=cfg.group_size)
    return QuantizedLinear(packed, scale, zero, qcfg, None, n_in, n_out, use_kernel=True)


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float, dev: torch.device):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=torch.float16, device=dev))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (xf * self.weight.float()).to(x.dtype)


def _rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """RoPE on the two halves of the head dimension (Llama's rotate_half)."""
    d = x.shape[-1] // 2
    x1, x2 = x[..., :d].float(), x[..., d:].float()
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(x.dtype)


def rope_tables(head_dim: int, theta: float, max_len: int, device):
    """cos, sin fp32 [max_len, head_dim/2] of the RoPE angles pos * theta^(-2i/d)."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim))
    ang = torch.arange(max_len, device=device).float()[:, None] * inv[None, :]
    return ang.cos(), ang.sin()


def _check(rc: int, fn: str) -> None:
    _lib.check(rc, fn)


def add_rmsnorm(x: torch.Tensor, r: torch.Tensor | None, w: torch.Tensor, eps: float):
    """(norm(x + r) * w, x + r) in one launch; r None: (norm(x) * w, x)."""
    dim = x.shape[-1]
    y = torch.empty_like(x)
    h = torch.empty_like(x) if r is not None else x
    _check(_lib.lib().pmi_add_rmsnorm_f16(
        x.data_ptr(), r.data_ptr() if r is not None else None, w.data_ptr(), y.data_ptr(),
        h.data_ptr() if r is not None else None, x.numel() // dim, dim, eps,
        _stream_handle(x.device)), "pmi_add_rmsnorm_f16")
    return y, h


def rope_kv(qkv, cos, sin, pos, cache_k, cache_v, B, T, H, KV, D):
    """Rotated q [B, H, T, D]; rotated k and v written into the caches at pos."""
    q = torch.empty(B, H, T, D, dtype=torch.float16, device=qkv.device)
    _check(_lib.lib().pmi_rope_kv_f16(
        qkv.data_ptr(), cos.data_ptr(), sin.data_ptr(), pos.data_ptr(), q.data_ptr(),
        cache_k.data_ptr(), cache_v.data_ptr(), B, T, H, KV, D, cache_k.shape[2],
        _stream_handle(qkv.device)), "pmi_rope_kv_f16")
    return q


_ATTN_WORKSPACES: dict = {}


def _attention_workspace(dev: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """Zero-filled scratch of the split attention, one per (device, stream):
    launches on one stream are ordered and each leaves its counters at zero.
    Allocated by the first (eager) call, so graph captures reuse it."""
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), stream)
    ws = _ATTN_WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=dev)
        _ATTN_WORKSPACES[key] = ws
    return ws


def decode_attention(q, cache_k, cache_v, pos, scale: float, split: bool = True):
    """q [B, H, 1, D] against cache positions 0..pos -> [B, H, D]. ``split``
    spreads the positions over workgroups (flash-decoding) through a cached
    workspace; False runs one workgroup per (sequence, KV head)."""
    B, H, _, D = q.shape
    KV, L = cache_k.shape[1], cache_k.shape[2]
    L_ = _lib.lib()
    out = torch.empty(B, H, D, dtype=torch.float16, device=q.device)
    stream = _stream_handle(q.device)
    ws, nbytes = None, 0
    if split:
        nbytes = L_.pmi_decode_attention_workspace_bytes(B, H, KV, L)
        ws = _attention_workspace(q.device, stream, nbytes)
    _check(L_.pmi_decode_attention_f16(
        q.data_ptr(), cache_k.data_ptr(), cache_v.data_ptr(), pos.data_ptr(), out.data_ptr(), B, H,
        KV, D, L, scale, ws.data_ptr() if ws is not None else None, nbytes, stream),
        "pmi_decode_attention_f16")
    return out


def decode_attention_rope(qkv, cos, sin, pos, cache_k, cache_v, scale: float):
    """RoPE + KV-cache write + attention of one new token in one launch:
    qkv [B, (H + 2*KV)*D] -> [B, H, D] (equal to rope_kv + decode_attention)."""
    B = qkv.shape[0]
    KV, L, D = cache_k.shape[1], cache_k.shape[2], cache_k.shape[3]
    H = qkv.shape[-1] // D - 2 * KV
    L_ = _lib.lib()
    out = torch.empty(B, H, D, dtype=torch.float16, device=qkv.device)
    stream = _stream_handle(qkv.device)
    nbytes = L_.pmi_decode_attention_workspace_bytes(B, H, KV, L)
    ws = _attention_workspace(qkv.device, stream, nbytes)
    _check(L_.pmi_decode_attention_rope_f16(
        qkv.data_ptr(), cos.data_ptr(), sin.data_ptr(), pos.data_ptr(), cache_k.data_ptr(),
        cache_v.data_ptr(), out.data_ptr(), B, H, KV, D, L, scale, ws.data_ptr(), nbytes, stream),
        "pmi_decode_attention_rope_f16")
    return out


_ARGMAX_WORKSPACES: dict = {}
_STATS_BUFFERS: dict = {}


def _stats_buffer(dev: torch.device) -> torch.Tensor:
    """The fp32 partials of sum(h^2) that a residual-forming GEMV leaves for
    the next pre-normed one, one buffer per (device, stream): launches on a
    stream are ordered, and every consumer runs before the next producer.
    Allocated by the first (eager) call, so graph captures reuse it."""
    key = (dev.index if dev.index is not None else torch.cuda.current_device(),
           _stream_handle(dev))
    buf = _STATS_BUFFERS.get(key)
    if buf is None:
        buf = torch.zeros(512, dtype=torch.float32, device=dev)
        _STATS_BUFFERS[key] = buf
    return buf


class _Summed:
    """The pending residual of a one-token layer that already added it: the
    residual stream h is complete, and ``stats[:n]`` are the partial sums of
    h^2 its last GEMV left for the next layer's pre-normed q/k/v."""
    __slots__ = ("stats", "n")

    def __init__(self, stats: torch.Tensor, n: int):
        self.stats, self.n = stats, n



def argmax_into(x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[r] = argmax of row r of x [rows, n] fp16 (the first index on ties),
    in one launch through a cached zero-filled workspace (allocated by the
    first, eager call so that graph captures reuse it). ``out``: int64 with one
    element per row at a constant stride (e.g. a [rows, 1] token buffer)."""
    rows, n = x.shape
    assert out.dtype == torch.int64 and out.numel() == rows
    L_ = _lib.lib()
    stream = _stream_handle(x.device)
    nbytes = L_.pmi_argmax_workspace_bytes(rows, n)
    key = (x.device.index if x.device.index is not None else torch.cuda.current_device(), stream)
    ws = _ARGMAX_WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 12), dtype=torch.uint8, device=x.device)
        _ARGMAX_WORKSPACES[key] = ws
    stride = out.stride(0) if out.dim() >= 1 and rows > 1 else 1
    _check(L_.pmi_argmax_f16(x.data_ptr(), rows, n, out.data_ptr(), stride, ws.data_ptr(),
                             nbytes, stream), "pmi_argmax_f16")
    return out


def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up of a fused [.., 2F] gate/up output."""
    F2 = gu.shape[-1]
    out = torch.empty(*gu.shape[:-1], F2 // 2, dtype=torch.float16, device=gu.device)
    _check(_lib.lib().pmi_silu_mul_f16(gu.data_ptr(), out.data_ptr(), gu.numel() // F2, F2 // 2,
                                       _stream_handle(gu.device)), "pmi_silu_mul_f16")
    return out


class DecoderLayer(nn.Module):
    def __init__(self, cfg: DecoderConfig, gen: torch.Generator, dev: torch.device):
        super().__init__()
        h, kvd = cfg.hidden, cfg.kv_heads * cfg.head_dim
        self.cfg = cfg
        self.attn_norm = RMSNorm(h, cfg.rms_eps, dev)
        self.mlp_norm = RMSNorm(h, cfg.rms_eps, dev)
        self.qkv = FusedQuantizedLinear([_int4_linear(h, h, gen, cfg, dev),
                                         _int4_linear(kvd, h, gen, cfg, dev),
                                         _int4_linear(kvd, h, gen, cfg, dev)])
        self.o = _int4_linear(h, h, gen, cfg, dev)
        self.gate_up = FusedQuantizedLinear([_int4_linear(cfg.ffn, h, gen, cfg, dev),
                                             _int4_linear(cfg.ffn, h, gen, cfg, dev)])
        self.down = _int4_linear(h, cfg.ffn, gen, cfg, dev)

    def forward(self, x, cos, sin, cache_k, cache_v, pos, mask, causal: bool):
        """x [B, T, hidden]; cos/sin [T, head_dim/2]; cache_k/v [B, kv_heads,
        L, head_dim]; pos int64 [T] cache positions of the T tokens; mask
        (bool [L], True = attend) for decode, or None with ``causal`` for a
        prefill that fills positions 0..T-1."""
        cfg = self.cfg
        B, T, _ = x.shape
        q, k, v = self.qkv(self.attn_norm(x))
        q = q.reshape(B, T, cfg.heads, cfg.head_dim).transpose(1, 2)
        k = k.reshape(B, T, cfg.kv_heads, cfg.head_dim).transpose(1, 2)
        v = v.reshape(B, T, cfg.kv_heads, cfg.head_dim).transpose(1, 2)
        q, k = _rotate(q, cos, sin), _rotate(k, cos, sin)
        cache_k.index_copy_(2, pos, k)
        cache_v.index_copy_(2, pos, v)
        if causal:
            a = F.scaled_dot_product_attention(q, k.contiguous(), v.contiguous(), is_causal=True,
                                               enable_gqa=True)
        else:
            a = F.scaled_dot_product_attention(q, cache_k, cache_v, attn_mask=mask, enable_gqa=True)
        a = a.transpose(1, 2).reshape(B, T, cfg.hidden)
        x = x + self.o(a)
        g, u = self.gate_up(self.mlp_norm(x))
        return x + self.down(F.silu(g) * u)

    def forward_fused(self, h, d, cos_t, sin_t, cache_k, cache_v, pos, causal: bool):
        """The same layer on the library's fused ops. The residual stream is
        carried as (h, d) with d the previous layer's pending output (None for
        the first layer): each residual add happens inside the next RMSNorm.
        One-token layers at batch 1 return d as a ``_Summed`` instead: h then
        already holds the residual, and d the partial sums of h^2 that the
        next layer's q/k/v GEMV takes its RMSNorm from.
        cos_t/sin_t are the full [L, head_dim/2] tables (indexed by pos on the
        device). Returns the new (h, d)."""
        cfg = self.cfg
        B, T, _ = h.shape
        if not causal and T == 1 and B == 1 and self._summed_ok():
            return self._forward_summed(h, d, cos_t, sin_t, cache_k, cache_v, pos)
        if isinstance(d, _Summed):
            d = None
        if not causal and T == 1:
            # one new token: each residual add + RMSNorm runs inside the GEMV that
            # consumes it where that is the GEMV, and RoPE, the cache write and
            # attention are one launch
            qkv, h = self._norm_linear(self.qkv.fused, h, d, self.attn_norm.weight)
            a = decode_attention_rope(qkv.reshape(B, -1), cos_t, sin_t, pos, cache_k, cache_v,
                                      1.0 / math.sqrt(cfg.head_dim))
            o = self.o(a.reshape(B, 1, cfg.hidden))
            if B > 1:
                # several sequences: the gate/up launch on the tiled GEMM forms
                # the norm and SiLU(gate) * up itself where it can
                return self._norm_mlp(h, o, B, T)
            gu, h = self._norm_linear(self.gate_up.fused, h, o, self.mlp_norm.weight)
            return h, self._down(gu, B, T)
        n1, h = add_rmsnorm(h, d, self.attn_norm.weight, cfg.rms_eps)
        qkv = self.qkv.fused(n1)
        q = rope_kv(qkv, cos_t, sin_t, pos, cache_k, cache_v, B, T, cfg.heads, cfg.kv_heads,
                    cfg.head_dim)
        if causal:
            a = F.scaled_dot_product_attention(q, cache_k[:, :, :T], cache_v[:, :, :T],
                                               is_causal=True, enable_gqa=True)
            a = a.transpose(1, 2).reshape(B, T, cfg.hidden)
        else:
            a = decode_attention(q, cache_k, cache_v, pos, 1.0 / math.sqrt(cfg.head_dim))
            a = a.reshape(B, 1, cfg.hidden)
        n2, h = add_rmsnorm(h, self.o(a), self.mlp_norm.weight, cfg.rms_eps)
        return h, self._mlp(n2, B, T)

    def _summed_ok(self) -> bool:
        """One-token layers can carry the residual stream as (h, partials): every
        linear on the GEMV with u8 zero points, no act_order, no bias on o and
        down, and the residual-forming launches supported."""
        lins = (self.qkv.fused, self.o, self.gate_up.fused, self.down)
        if not (all(getattr(l, "use_kernel", False) and l.g_idx is None for l in lins)
                and self.o.bias is None and self.down.bias is None):
            return False
        shapes_ok = getattr(self, "_summed_shapes", None)  # shape-only, so kept
        if shapes_ok is None:
            cfg = self.cfg
            shapes_ok = (
                all(kernel_choice(1, l.out_features, l.in_features, l._group_size()) == "gemv"
                    for l in lins)
                and 0 < residual_stats_count(cfg.hidden, self.o.in_features) <= 512
                and 0 < residual_stats_count(cfg.hidden, self.down.in_features, glu=True) <= 512)
            self._summed_shapes = shapes_ok
        return shapes_ok

    def _forward_summed(self, h, d, cos_t, sin_t, cache_k, cache_v, pos):
        """A one-token layer whose residual adds run in the epilogues of the o
        and down GEMVs, each leaving per-workgroup partials of sum(h^2) for the
        next GEMV's RMSNorm (q/k/v of the next layer, gate/up of this one): no
        launch reduces a whole row before its first weight batch. Returns (h,
        _Summed)."""
        cfg = self.cfg
        K = cfg.hidden
        stats = _stats_buffer(h.device)
        qf = self.qkv.fused
        if isinstance(d, _Summed):
            w_k, z_u8, _, _ = qf._kernel_buffers()
            qkv = matmul_w4a16_prenormed(h.reshape(1, K), d.stats, d.n, self.attn_norm.weight,
                                         cfg.rms_eps, w_k, qf.scale, z_u8, qf._group_size())
            if qf.bias is not None:
                qkv = qkv + qf.bias
        else:
            qkv, h = self._norm_linear(qf, h, d, self.attn_norm.weight)
            qkv = qkv.reshape(1, -1)
        a = decode_attention_rope(qkv, cos_t, sin_t, pos, cache_k, cache_v,
                                  1.0 / math.sqrt(cfg.head_dim))
        w_o, z_o, _, _ = self.o._kernel_buffers()
        h2 = torch.empty_like(h)
        n = matmul_w4a16_residual(a.reshape(1, -1), h.reshape(1, K), stats, w_o, self.o.scale, z_o,
                                  self.o._group_size(), out=h2.reshape(1, K))
        gl = self.gate_up.fused
        w_g, z_g, _, _ = gl._kernel_buffers()
        gu = matmul_w4a16_prenormed(h2.reshape(1, K), stats, n, self.mlp_norm.weight, cfg.rms_eps,
                                    w_g, gl.scale, z_g, gl._group_size())
        if gl.bias is not None:
            gu = gu + gl.bias
        w_d, z_d, _, _ = self.down._kernel_buffers()
        h3 = torch.empty_like(h)
        n = matmul_w4a16_residual(gu, h2.reshape(1, K), stats, w_d, self.down.scale, z_d,
                                  self.down._group_size(), glu=True, out=h3.reshape(1, K))
        return h3, _Summed(stats, n)

    def _norm_linear(self, lin: QuantizedLinear, h, d, norm_w):
        """(lin(RMSNorm(h + d) * norm_w), h + d) for one token per sequence: one
        GEMV launch when the layer runs on the GEMV, else add_rmsnorm + lin."""
        B, T, K = h.shape
        M = B * T
        # one activation row only: with more rows the per-row norm prologue of
        # every wave costs more than the launch it saves (measured on the
        # Llama q/k/v GEMV at 4 rows)
        if M == 1 and lin.g_idx is None and \
                kernel_choice(M, lin.out_features, K, lin._group_size()) == "gemv":
            w_k, z_u8, _, _ = lin._kernel_buffers()
            y, h2 = matmul_w4a16_rmsnorm(h.reshape(M, K), d.reshape(M, K) if d is not None else None,
                                         norm_w, self.cfg.rms_eps, w_k, lin.scale, z_u8,
                                         lin._group_size())
            if lin.bias is not None:
                y = y + lin.bias
            return y.reshape(B, T, -1), h2.reshape(B, T, K)
        # 2..4 rows on the tiled GEMM: the norm formed in its prologue
        if 2 <= M <= 4 and lin.g_idx is None and \
                tiled_rmsnorm_supported(M, lin.out_features, K, lin._group_size()) and \
                kernel_choice(M, lin.out_features, K, lin._group_size(), tiled=True) == "tgemm":
            w_k, _, _, sz_gm = lin._kernel_buffers()
            w_t = lin._tiled_buffer(w_k, M)
            if w_t is not None:
                y, h2 = matmul_w4a16_tiled_rmsnorm(
                    h.reshape(M, K), d.reshape(M, K) if d is not None else None, norm_w,
                    self.cfg.rms_eps, w_t, sz_gm, lin._group_size(), lin.out_features)
                if lin.bias is not None:
                    y = y + lin.bias
                return y.reshape(B, T, -1), h2.reshape(B, T, K)
        n, h = add_rmsnorm(h, d, norm_w, self.cfg.rms_eps)
        return lin(n), h

    def _norm_mlp(self, h, o, B: int, T: int):
        """(h + o, the MLP of RMSNorm(h + o)) for several one-token sequences:
        one gate/up launch with the norm in its prologue and SiLU(gate) * up in
        its epilogue where the tiled GEMM takes the shape, else add_rmsnorm and
        _mlp."""
        M, K = B * T, h.shape[-1]
        gu = self.gate_up.fused
        gs = gu._group_size()
        if 2 <= M <= 4 and gu.g_idx is None and gu.bias is None and \
                gate_up_silu_supported(M, gu.out_features, K, gs) and \
                tiled_rmsnorm_supported(M, gu.out_features, K, gs, glu=True):
            w_t, sz = self._glu_buffers()
            act, h2 = matmul_w4a16_tiled_rmsnorm(
                h.reshape(M, K).contiguous(), o.reshape(M, K).contiguous(), self.mlp_norm.weight,
                self.cfg.rms_eps, w_t, sz, gs, gu.out_features, glu=True)
            return h2.reshape(B, T, K), self.down(act.reshape(B, T, -1))
        n2, h = add_rmsnorm(h, o, self.mlp_norm.weight, self.cfg.rms_eps)
        return h, self._mlp(n2, B, T)

    def _mlp(self, n2, B: int, T: int):
        M = B * T
        gu = self.gate_up.fused
        if M >= 2 and gu.g_idx is None and gu.bias is None and \
                gate_up_silu_supported(M, gu.out_features, gu.in_features, gu._group_size()):
            # 2..16 tokens on the tiled GEMM: SiLU(gate) * up in its epilogue, one
            # launch less than the fused matmul + silu_mul
            w_t, sz = self._glu_buffers()
            act = matmul_w4a16_gate_up_silu(n2.reshape(M, -1).contiguous(), w_t, sz,
                                            gu._group_size(), gu.out_features)
            return self.down(act.reshape(B, T, -1))
        return self._down(gu(n2), B, T)

    def _glu_buffers(self):
        """Tiled and group-major copies of the fused gate/up weight with its rows
        in glu_row_order, built on first use and rebuilt when the weights change
        (keyed on the fused module's weight stamp). They are never built under
        graph capture: the copies would then only be recorded, not made."""
        gu = self.gate_up.fused
        stamp = gu._stamp()
        cache = getattr(self, "_glu", None)
        if cache is None or cache[0] != stamp:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("the gate/up SiLU copies are built on the first eager call; "
                                   "run one eager forward before capturing a graph")
            w_k, z_u8, _, _ = gu._kernel_buffers()
            idx = glu_row_order(gu.out_features // 2, w_k.device)
            gs = gu._group_size()
            s = gu.scale.reshape(gu.out_features, -1)
            self._glu = cache = (stamp, tile_w4a16(w_k[idx].contiguous(), gs),
                                 sz_group_major(s[idx].contiguous(),
                                                z_u8.reshape(gu.out_features, -1)[idx].contiguous()))
        return cache[1], cache[2]

    def _down(self, gu, B: int, T: int):
        if B * T == 1 and self.down.g_idx is None:
            # one-token decode: the down GEMV forms silu(gate) * up itself, one
            # launch less (9.6 us against 11.4 us for silu_mul + GEMV on the
            # Llama down shape; from two rows on, the per-wave SiLU costs more
            # than the launch it saves)
            w_k, z_u8, _, _ = self.down._kernel_buffers()
            y = matmul_w4a16_glu(gu.reshape(B * T, -1).contiguous(), w_k, self.down.scale, z_u8,
                                 self.down._group_size())
            if self.down.bias is not None:
                y = y + self.down.bias
            return y.reshape(B, T, -1)
        return self.down(silu_mul(gu))


class QuantizedDecoder(nn.Module):
    """Embedding -> ``layers`` x DecoderLayer -> RMSNorm -> fp16 lm_head."""

    def __init__(self, cfg: DecoderConfig, device, seed: int = 0, fused_ops: bool = True):
        super().__init__()
        dev = torch.device(device)
        gen = torch.Generator(device=dev).manual_seed(seed)
        self.cfg = cfg
        self.fused_ops = fused_ops
        self.embed = nn.Parameter(
            (torch.randn(cfg.vocab, cfg.hidden, generator=gen, device=dev) * cfg.init_std).half())
        self.layers = nn.ModuleList([DecoderLayer(cfg, gen, dev) for _ in range(cfg.layers)])
        self.norm = RMSNorm(cfg.hidden, cfg.rms_eps, dev)
        self.lm_head = nn.Parameter(
            (torch.randn(cfg.vocab, cfg.hidden, generator=gen, device=dev) * cfg.init_std).half())
        self._graphs: dict = {}

    def rope_tables(self, max_len: int):
        return rope_tables(self.cfg.head_dim, self.cfg.rope_theta, max_len, self.embed.device)

    def new_cache(self, batch: int, max_len: int):
        cfg = self.cfg
        shape = (batch, cfg.kv_heads, max_len, cfg.head_dim)
        return [(torch.zeros(shape, dtype=torch.float16, device=self.embed.device),
                 torch.zeros(shape, dtype=torch.float16, device=self.embed.device))
                for _ in range(cfg.layers)]

    def forward_tokens(self, tokens, cos, sin, cache, pos, mask, causal: bool,
                       last_only: bool = False):
        """Logits [B, T, vocab] of ``tokens`` [B, T] at cache positions ``pos``
        (a prefill, ``causal``, writes positions 0..T-1). With ``last_only`` the
        final norm and lm_head run on the last position only: [B, 1, vocab],
        all a greedy prefill needs."""
        x = F.embedding(tokens, self.embed)
        if self.fused_ops:
            d = None
            for layer, (ck, cv) in zip(self.layers, cache):
                x, d = layer.forward_fused(x, d, cos, sin, ck, cv, pos, causal)
            if isinstance(d, _Summed):
                d = None  # x already holds the residual stream
            if last_only:
                x = x[:, -1:].contiguous()
                d = d[:, -1:].contiguous() if d is not None else None
            n, _ = add_rmsnorm(x, d, self.norm.weight, self.cfg.rms_eps)
            return F.linear(n, self.lm_head)
        c, s = cos.index_select(0, pos), sin.index_select(0, pos)
        for layer, (ck, cv) in zip(self.layers, cache):
            x = layer(x, c, s, ck, cv, pos, mask, causal)
        if last_only:
            x = x[:, -1:]
        return F.linear(self.norm(x), self.lm_head)

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, n_generate: int, use_graph: bool = True):
        """Greedy decode: returns (tokens [B, n_generate], timings). The prompt
        [B, P] is prefilled in one pass; each decode step is one graph replay
        (or the same ops eagerly) plus an argmax."""
        B, P = prompt.shape
        L = P + n_generate
        cos, sin = self.rope_tables(L)
        cache = self.new_cache(B, L)
        dev = self.embed.device
        out = torch.empty(B, n_generate, dtype=torch.long, device=dev)
        tok = torch.empty(B, 1, dtype=torch.long, device=dev)
        pos = torch.zeros(1, dtype=torch.long, device=dev)
        ar = torch.arange(L, device=dev)
        mask = torch.zeros(L, dtype=torch.bool, device=dev)

        def step():
            # the step's greedy token replaces its input token (the fused path
            # runs the argmax in the graph, after the embedding has read tok)
            if not self.fused_ops:
                mask.copy_(ar <= pos)
                logits = self.forward_tokens(tok, cos, sin, cache, pos, mask, False)[:, -1]
                tok.copy_(logits.argmax(-1, keepdim=True))
                return logits
            logits = self.forward_tokens(tok, cos, sin, cache, pos, mask, False)[:, -1]
            argmax_into(logits.contiguous(), tok)
            return logits

        graph = None
        if use_graph:
            # capture on a side stream after one eager run of the same step
            # (lazy per-layer buffers must exist before capture)
            s = torch.cuda.Stream(dev)
            s.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(s):
                tok.zero_()
                pos.fill_(P)
                step()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=s):
                    step()
            torch.cuda.current_stream(dev).wait_stream(s)
            for ck, cv in cache:
                ck.zero_()
                cv.zero_()
        torch.cuda.synchronize(dev)

        t0 = time.perf_counter()
        logits = self.forward_tokens(prompt, cos, sin, cache, torch.arange(P, device=dev), None,
                                     True, last_only=True)[:, -1]
        tok.copy_(logits.argmax(-1, keepdim=True))
        out[:, 0] = tok[:, 0]
        torch.cuda.synchronize(dev)
        t1 = time.perf_counter()
        for i in range(1, n_generate):
            pos.fill_(P + i - 1)
            if graph is not None:
                graph.replay()
            else:
                step()
            out[:, i] = tok[:, 0]
        torch.cuda.synchronize(dev)
        t2 = time.perf_counter()
        return out, {"prefill_s": t1 - t0, "decode_s": t2 - t1, "elapsed_s": t2 - t0}

    def linear_bytes_per_token(self) -> int:
        """INT4 codes + fp32 scale + u8 zero of every QuantizedLinear, plus the
        fp16 lm_head: the bytes one decode step must stream."""
        total = 0
        for m in self.modules():
            if isinstance(m, QuantizedLinear):
                g = m.scale.numel()
                total += m.packed_weight.numel() + g * 5
        return total + self.lm_head.numel() * 2


def decoder_throughput(model: QuantizedDecoder, batch: int, prompt_len: int = 512,
                       n_generate: int = 128, seed: int = 1, warmup: int = 1) -> dict:
    """The reference's tok/s (pare/eval/throughput.py:106-116): batch *
    n_generate / elapsed with the prefill inside elapsed; also decode-only
    tok/s (n_generate - 1 steps after the prefill's first token)."""
    dev = model.embed.device
    g = torch.Generator(device=dev).manual_seed(seed)
    prompt = torch.randint(0, model.cfg.vocab, (1, prompt_len), generator=g, device=dev)
    prompt = prompt.repeat(batch, 1)
    for _ in range(warmup):
        model.generate(prompt, n_generate)
    toks, t = model.generate(prompt, n_generate)
    return {"batch": batch, "prompt_len": prompt_len, "n_generate": n_generate,
            "tokens_per_sec": round(batch * n_generate / t["elapsed_s"], 2),
            "ms_per_token": round(t["elapsed_s"] * 1e3 / n_generate, 3),
            "decode_tokens_per_sec": round(batch * (n_generate - 1) / t["decode_s"], 2),
            "decode_ms_per_step": round(t["decode_s"] * 1e3 / (n_generate - 1), 3),
            "prefill_ms": round(t["prefill_s"] * 1e3, 2),
            "first_tokens": toks[0, :8].tolist()}
