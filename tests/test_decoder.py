"""End-to-end decoder on a small Llama-shaped config: the
HIP path inside a model, graph-captured decode, and the reference's
dequantize-on-the-fly path as the check (pare/layers/linear.py:101-138)."""

from __future__ import annotations

import pytest
import torch

import pare_amd as P
from pare_amd import _lib
from pare_amd.decoder import (DecoderConfig, QuantizedDecoder, add_rmsnorm, decode_attention,
                              decoder_throughput, rope_kv, rope_tables, silu_mul)

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SMALL = DecoderConfig(hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=2000, layers=2)


def _set_kernel(model, on: bool):
    for m in model.modules():
        if isinstance(m, P.QuantizedLinear):
            m.use_kernel = on


@pytest.fixture(scope="module")
def model():
    assert P.kernel_available()
    return QuantizedDecoder(SMALL, DEV, seed=3)


def test_graph_decode_matches_eager(model):
    g = torch.Generator(device=DEV).manual_seed(5)
    prompt = torch.randint(0, SMALL.vocab, (2, 24), generator=g, device=DEV)
    eager, _ = model.generate(prompt, 12, use_graph=False)
    graph, _ = model.generate(prompt, 12, use_graph=True)
    again, _ = model.generate(prompt, 12, use_graph=True)
    print(f"[decoder] eager={eager[0].tolist()} graph={graph[0].tolist()}", flush=True)
    assert torch.equal(eager, graph)
    assert torch.equal(graph, again)


@pytest.mark.parametrize("batch,seq", [(1, 16), (3, 40)])
def test_prefill_last_only_logits(model, batch, seq):
    """A greedy prefill's logits of the last position only (final norm and
    lm_head on that row) against the last row of the full prefill."""
    g = torch.Generator(device=DEV).manual_seed(seq + 1)
    toks = torch.randint(0, SMALL.vocab, (batch, seq), generator=g, device=DEV)
    cos, sin = model.rope_tables(seq)
    pos = torch.arange(seq, device=DEV)
    with torch.no_grad():
        full = model.forward_tokens(toks, cos, sin, model.new_cache(batch, seq), pos, None, True)
        last = model.forward_tokens(toks, cos, sin, model.new_cache(batch, seq), pos, None, True,
                                    last_only=True)
    assert last.shape == (batch, 1, SMALL.vocab)
    err = (last[:, 0].float() - full[:, -1].float()).abs().max().item()
    assert err <= 2e-3 * full[:, -1].float().abs().max().item() + 1e-3, err
    assert torch.equal(last[:, 0].argmax(-1), full[:, -1].argmax(-1))


@pytest.mark.parametrize("batch,seq", [(1, 16), (3, 40)])
def test_prefill_logits_match_dequant_path(model, batch, seq):
    """Kernel path vs the reference's dequant path (fp16 F.linear on
    dequantize()), same model and inputs: logits within tolerance."""
    g = torch.Generator(device=DEV).manual_seed(seq)
    toks = torch.randint(0, SMALL.vocab, (batch, seq), generator=g, device=DEV)
    cos, sin = model.rope_tables(seq)
    pos = torch.arange(seq, device=DEV)
    with torch.no_grad():
        _set_kernel(model, True)
        a = model.forward_tokens(toks, cos, sin, model.new_cache(batch, seq), pos, None, True).float()
        _set_kernel(model, False)
        b = model.forward_tokens(toks, cos, sin, model.new_cache(batch, seq), pos, None, True).float()
        _set_kernel(model, True)
    err = (a - b).abs().max().item()
    scale = b.abs().max().item()
    agree = (a.argmax(-1) == b.argmax(-1)).float().mean().item()
    print(f"[decoder] B={batch} T={seq}: max_abs={err:.3e} (max |logit| {scale:.3e}), "
          f"argmax agreement {agree:.3f}", flush=True)
    assert err <= 1e-2 + 2e-2 * scale
    assert agree >= 0.9


def test_first_graph_step_matches_eager(model):
    """The first graph replay after a prefill picks the same token as the
    eager step (the graph's cache positions and mask start where the prefill
    ended)."""
    g = torch.Generator(device=DEV).manual_seed(9)
    prompt = torch.randint(0, SMALL.vocab, (2, 20), generator=g, device=DEV)
    toks, t = model.generate(prompt, 2, use_graph=True)
    toks_e, _ = model.generate(prompt, 2, use_graph=False)
    assert torch.equal(toks, toks_e)
    assert t["elapsed_s"] > 0


def test_throughput_report(model):
    r = decoder_throughput(model, batch=2, prompt_len=32, n_generate=8, warmup=0)
    print(f"[decoder] {r}", flush=True)
    assert r["tokens_per_sec"] > 0 and r["decode_tokens_per_sec"] >= r["tokens_per_sec"] * 0.5


def test_fused_ops_match_torch_ops(model):
    """The library's caller-side ops (fused_ops=True) against the same model
    on plain PyTorch ops: prefill logits and greedy tokens."""
    g = torch.Generator(device=DEV).manual_seed(21)
    toks = torch.randint(0, SMALL.vocab, (2, 30), generator=g, device=DEV)
    cos, sin = model.rope_tables(30)
    pos = torch.arange(30, device=DEV)
    with torch.no_grad():
        a = model.forward_tokens(toks, cos, sin, model.new_cache(2, 30), pos, None, True).float()
        model.fused_ops = False
        try:
            b = model.forward_tokens(toks, cos, sin, model.new_cache(2, 30), pos, None, True).float()
            ref_toks, _ = model.generate(toks[:, :12], 10, use_graph=False)
        finally:
            model.fused_ops = True
        got_toks, _ = model.generate(toks[:, :12], 10, use_graph=True)
    err = (a - b).abs().max().item()
    print(f"[decoder] fused vs torch ops: max_abs={err:.3e}; tokens {got_toks[0].tolist()} "
          f"vs {ref_toks[0].tolist()}", flush=True)
    assert err <= 1e-2 + 1e-2 * b.abs().max().item()
    assert (got_toks == ref_toks).float().mean().item() >= 0.9


# --- the caller-side ops against fp32 PyTorch ---------------------------------

@pytest.mark.parametrize("rows,dim,resid", [(1, 4096, False), (3, 4096, True), (7, 1024, True)])
def test_add_rmsnorm(rows, dim, resid):
    g = torch.Generator(device=DEV).manual_seed(rows * dim)
    x = torch.randn(rows, dim, generator=g, device=DEV).half()
    r = torch.randn(rows, dim, generator=g, device=DEV).half() if resid else None
    w = (1 + 0.1 * torch.randn(dim, generator=g, device=DEV)).half()
    y, h = add_rmsnorm(x, r, w, 1e-5)
    hh = (x + r) if resid else x
    hf = hh.float()
    ref = hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-5) * w.float()
    assert torch.equal(h, hh)
    assert (y.float() - ref).abs().max().item() <= 2e-3 * ref.abs().max().item() + 1e-3


@pytest.mark.parametrize("B,T", [(1, 1), (2, 5)])
def test_rope_kv(B, T):
    H, KV, D, L = 8, 2, 128, 16
    g = torch.Generator(device=DEV).manual_seed(B * 10 + T)
    qkv = torch.randn(B * T, (H + 2 * KV) * D, generator=g, device=DEV).half()
    cos_t, sin_t = rope_tables(D, 500000.0, L, DEV)
    pos = torch.arange(3, 3 + T, device=DEV)
    ck = torch.zeros(B, KV, L, D, dtype=torch.float16, device=DEV)
    cv = torch.zeros_like(ck)
    q = rope_kv(qkv, cos_t, sin_t, pos, ck, cv, B, T, H, KV, D)
    x = qkv.view(B, T, H + 2 * KV, D).float()
    c, s = cos_t[pos][None, :, None, :], sin_t[pos][None, :, None, :]
    rot = torch.cat([x[..., :64] * c - x[..., 64:] * s, x[..., 64:] * c + x[..., :64] * s], -1)
    assert (q.float() - rot[:, :, :H].transpose(1, 2)).abs().max().item() <= 2e-3
    assert (ck[:, :, 3:3 + T].float() - rot[:, :, H:H + KV].transpose(1, 2)).abs().max().item() <= 2e-3
    assert torch.equal(cv[:, :, 3:3 + T], qkv.view(B, T, H + 2 * KV, D)[:, :, H + KV:].transpose(1, 2))
    assert ck[:, :, :3].abs().max().item() == 0 and ck[:, :, 3 + T:].abs().max().item() == 0


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("B,H,KV,L,p", [(1, 32, 8, 640, 511), (4, 32, 8, 640, 639), (2, 8, 2, 100, 0),
                                        (3, 4, 4, 300, 77), (1, 32, 8, 640, 63), (1, 32, 8, 640, 64),
                                        (2, 16, 8, 130, 129), (1, 8, 8, 4096, 4000)])
def test_decode_attention(B, H, KV, L, p, split):
    D = 128
    g = torch.Generator(device=DEV).manual_seed(B * L + p)
    q = torch.randn(B, H, 1, D, generator=g, device=DEV).half()
    ck = torch.randn(B, KV, L, D, generator=g, device=DEV).half()
    cv = torch.randn(B, KV, L, D, generator=g, device=DEV).half()
    pos = torch.full((1,), p, dtype=torch.long, device=DEV)
    if not split and L > 3000:
        pytest.skip("one workgroup per KV head keeps the scores in 64 KB of LDS")
    out = decode_attention(q, ck, cv, pos, 1 / D ** 0.5, split=split)
    # fp32 reference over positions 0..p, each query head on its KV head
    grp = H // KV
    kf = ck[:, :, :p + 1].float().repeat_interleave(grp, dim=1)
    vf = cv[:, :, :p + 1].float().repeat_interleave(grp, dim=1)
    sc = (q.float() * (1 / D ** 0.5)) @ kf.transpose(-1, -2).contiguous()
    ref = (torch.softmax(sc, -1) @ vf)[:, :, 0]
    err = (out.float() - ref).abs().max().item()
    print(f"[attn] split={split} B={B} H={H} KV={KV} L={L} p={p}: max_abs={err:.3e}", flush=True)
    assert err <= 5e-3


@pytest.mark.parametrize("B,H,KV,L,p", [(1, 32, 8, 640, 511), (4, 32, 8, 640, 639), (2, 8, 2, 100, 0),
                                        (3, 4, 4, 300, 77), (1, 32, 8, 640, 64), (2, 16, 8, 130, 129),
                                        (1, 8, 8, 200, 500)])
def test_decode_attention_rope_equals_the_two_launches(B, H, KV, L, p):
    """RoPE + cache write + attention in one launch against rope_kv followed by
    decode_attention on copies of the same caches: equal outputs and caches."""
    from pare_amd.decoder import decode_attention_rope

    D = 128
    g = torch.Generator(device=DEV).manual_seed(B * L + p + 7)
    qkv = torch.randn(B, (H + 2 * KV) * D, generator=g, device=DEV).half()
    ck = torch.randn(B, KV, L, D, generator=g, device=DEV).half()
    cv = torch.randn(B, KV, L, D, generator=g, device=DEV).half()
    cos, sin = rope_tables(D, 500000.0, L, DEV)
    pos = torch.full((1,), p, dtype=torch.long, device=DEV)
    ck2, cv2 = ck.clone(), cv.clone()
    q = rope_kv(qkv.view(B, 1, -1), cos, sin, pos, ck2, cv2, B, 1, H, KV, D)
    ref = decode_attention(q, ck2, cv2, pos, 1 / D ** 0.5)
    got = decode_attention_rope(qkv, cos, sin, pos, ck, cv, 1 / D ** 0.5)
    assert torch.equal(ck, ck2) and torch.equal(cv, cv2)
    assert torch.equal(got, ref), (got.float() - ref.float()).abs().max().item()


@pytest.mark.parametrize("M,N,K", [(1, 6144, 4096), (2, 28672, 4096), (3, 6144, 4096),
                                   (4, 6144, 4096), (1, 136, 512), (2, 200, 8192)])
@pytest.mark.parametrize("with_residual", [True, False])
def test_rmsnorm_gemv_matches_norm_then_matmul(M, N, K, with_residual):
    """The GEMV with the residual add + RMSNorm inside against add_rmsnorm
    followed by the plain matmul: h bit for bit, y within the fp16 ulp the
    differently ordered mean can move an activation by."""
    from pare_amd.kernels import matmul_w4a16, matmul_w4a16_rmsnorm
    from pare_amd.pack import repack_int4_for_kernel, zeros_to_u8

    g = torch.Generator(device=DEV).manual_seed(M * N + K + int(with_residual))
    x = torch.randn(M, K, generator=g, device=DEV).half()
    r = torch.randn(M, K, generator=g, device=DEV).half() if with_residual else None
    nw = (1 + 0.1 * torch.randn(K, generator=g, device=DEV)).half()
    w = torch.randn(N, K, generator=g, device=DEV) * 0.02
    packed, s, z = P.rtn_quantize(w, 128)
    wk = repack_int4_for_kernel(packed, 128)
    zu = zeros_to_u8(z)
    y, h = matmul_w4a16_rmsnorm(x, r, nw, 1e-5, wk, s, zu, 128)
    n_ref, h_ref = add_rmsnorm(x, r, nw, 1e-5)
    y_ref = matmul_w4a16(n_ref, wk, s, zu, 128)
    assert torch.equal(h, h_ref)
    err = (y.float() - y_ref.float()).abs().max().item()
    scale = y_ref.float().abs().max().item()
    print(f"[rmsnorm-gemv] M={M} N={N} K={K} r={with_residual}: max_abs={err:.3e} (max {scale:.2f})",
          flush=True)
    assert err <= 2e-3 * scale + 1e-3


def _gemv_layer(N, K, seed):
    from pare_amd.pack import repack_int4_for_kernel, zeros_to_u8

    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(N, K, generator=g, device=DEV) * 0.02
    packed, s, z = P.rtn_quantize(w, 128)
    return repack_int4_for_kernel(packed, 128), s, zeros_to_u8(z)


@pytest.mark.parametrize("N,K,glu", [(4096, 4096, False), (4096, 14336, True), (3584, 18944, True),
                                     (1000, 4096, False), (4096, 2560, False)])
def test_residual_gemv_adds_as_add_rmsnorm_does(N, K, glu):
    """The GEMV that adds the residual in its epilogue: h equals the plain
    launch's fp16 output added to the residual and rounded as add_rmsnorm
    adds, bit for bit (also in place), and the partials add up to sum(h^2)."""
    from pare_amd.kernels import (matmul_w4a16, matmul_w4a16_glu, matmul_w4a16_residual,
                                  residual_stats_count)

    wk, s, zu = _gemv_layer(N, K, N + K)
    g = torch.Generator(device=DEV).manual_seed(K)
    x = (torch.randn(1, 2 * K if glu else K, generator=g, device=DEV) * (2 if glu else 1)).half()
    r = torch.randn(1, N, generator=g, device=DEV).half()
    n = residual_stats_count(N, K, glu)
    assert 0 < n <= 512
    stats = torch.full((512,), float("nan"), device=DEV)
    h = torch.empty_like(r)
    assert matmul_w4a16_residual(x, r, stats, wk, s, zu, 128, glu=glu, out=h) == n
    y = matmul_w4a16_glu(x, wk, s, zu, 128) if glu else matmul_w4a16(x, wk, s, zu, 128)
    ref = (y.float() + r.float()).half()
    assert torch.equal(h, ref), (h.float() - ref.float()).abs().max().item()
    tot = stats[:n].double().sum().item()
    assert abs(tot - (ref.double() ** 2).sum().item()) <= 1e-5 * tot
    r2 = r.clone()
    matmul_w4a16_residual(x, r2, stats, wk, s, zu, 128, glu=glu)  # in place
    assert torch.equal(r2, ref)


@pytest.mark.parametrize("N,K", [(6144, 4096), (28672, 4096), (1024, 4096), (37888, 3584)])
def test_prenormed_gemv_matches_norm_then_matmul(N, K):
    """The GEMV whose RMSNorm takes sum(h^2) from a residual launch's partials,
    against add_rmsnorm followed by the plain matmul: within the fp16 ulp the
    differently ordered mean can move an activation by."""
    from pare_amd.kernels import (matmul_w4a16, matmul_w4a16_prenormed, matmul_w4a16_residual)

    wk_o, s_o, z_o = _gemv_layer(K, K, K)   # forms h, [1, K]
    wk, s, zu = _gemv_layer(N, K, N + K)
    g = torch.Generator(device=DEV).manual_seed(N)
    a = torch.randn(1, K, generator=g, device=DEV).half()
    r = torch.randn(1, K, generator=g, device=DEV).half()
    nw = (1 + 0.1 * torch.randn(K, generator=g, device=DEV)).half()
    stats = torch.zeros(512, device=DEV)
    h = torch.empty_like(r)
    n = matmul_w4a16_residual(a, r, stats, wk_o, s_o, z_o, 128, out=h)
    y = matmul_w4a16_prenormed(h, stats, n, nw, 1e-5, wk, s, zu, 128)
    n_ref, _ = add_rmsnorm(h, None, nw, 1e-5)
    y_ref = matmul_w4a16(n_ref, wk, s, zu, 128)
    err = (y.float() - y_ref.float()).abs().max().item()
    scale = y_ref.float().abs().max().item()
    print(f"[prenormed-gemv] N={N} K={K}: max_abs={err:.3e} (max {scale:.2f})", flush=True)
    assert err <= 2e-3 * scale + 1e-3


def test_residual_and_prenormed_reject_what_they_do_not_run():
    L = _lib.lib()
    assert L.pmi_residual_stats_count(4096, 4096, 0) == 256
    assert L.pmi_residual_stats_count(1024, 1024, 0) == 0    # one GEMV slice per row
    assert L.pmi_matmul_w4a16_residual(None, 0, None, None, None, None, None, None, 1024, 1024,
                                       128, None) == _lib.PMI_ERR_UNSUPPORTED
    assert L.pmi_matmul_w4a16_prenormed(None, None, 0, None, 1e-5, None, None, None, None, 4096,
                                        4096, 128, None) == _lib.PMI_ERR_INVALID
    assert L.pmi_matmul_w4a16_prenormed(None, None, 513, None, 1e-5, None, None, None, None, 4096,
                                        4096, 128, None) == _lib.PMI_ERR_INVALID


def test_decoder_one_token_summed_path_matches_the_norm_launch_path():
    """A full-width two-layer decoder at batch 1: the one-token layers that add
    the residual in the o / down epilogues and take the norm from their partials
    against the same model with that path off (norm inside each consuming GEMV),
    over a prefill and greedy decode: equal tokens, logits within tolerance,
    and graph replay equal to eager."""
    from pare_amd.decoder import DecoderLayer

    cfg = DecoderConfig(layers=2, vocab=4000)
    model = QuantizedDecoder(cfg, DEV, seed=11)
    assert all(layer._summed_ok() for layer in model.layers)
    g = torch.Generator(device=DEV).manual_seed(3)
    prompt = torch.randint(0, cfg.vocab, (1, 24), generator=g, device=DEV)
    on_eager, _ = model.generate(prompt, 10, use_graph=False)
    on_graph, _ = model.generate(prompt, 10, use_graph=True)
    orig = DecoderLayer._summed_ok
    DecoderLayer._summed_ok = lambda self: False
    try:
        off_eager, _ = model.generate(prompt, 10, use_graph=False)
        cos, sin = model.rope_tables(32)
        pos = torch.tensor([24], device=DEV)
        tok = on_eager[:, :1]
        with torch.no_grad():
            cache = model.new_cache(1, 32)
            model.forward_tokens(prompt, cos, sin, cache, torch.arange(24, device=DEV), None, True)
            off = model.forward_tokens(tok, cos, sin, cache, pos, None, False).float()
    finally:
        DecoderLayer._summed_ok = orig
    with torch.no_grad():
        cache = model.new_cache(1, 32)
        model.forward_tokens(prompt, cos, sin, cache, torch.arange(24, device=DEV), None, True)
        on = model.forward_tokens(tok, cos, sin, cache, pos, None, False).float()
    err = (on - off).abs().max().item()
    print(f"[decoder] summed path: tokens {on_eager[0].tolist()} vs {off_eager[0].tolist()}, "
          f"logit max_abs {err:.3e}", flush=True)
    assert torch.equal(on_eager, on_graph)
    assert torch.equal(on_eager, off_eager)
    assert err <= 1e-2 + 1e-2 * off.abs().max().item()


@pytest.mark.parametrize("M,N,F", [(1, 4096, 14336), (2, 4096, 14336), (3, 1024, 4096),
                                   (4, 4096, 14336), (1, 136, 512), (4, 200, 1024)])
def test_glu_down_matches_silu_then_matmul(M, N, F):
    """The gated GEMV against silu_mul followed by the plain matmul on the GEMV:
    the same fp16 activations feed the same kernel, so the outputs are equal bit
    for bit. (Dispatch alone would send M = 4 at K = 14336 to the MFMA GEMM.)"""
    from pare_amd.kernels import force_kernel, matmul_w4a16, matmul_w4a16_glu
    from pare_amd.pack import repack_int4_for_kernel, zeros_to_u8

    g = torch.Generator(device=DEV).manual_seed(M * N + F)
    gu = (torch.randn(M, 2 * F, generator=g, device=DEV) * 2).half()
    w = torch.randn(N, F, generator=g, device=DEV) * 0.02
    packed, s, z = P.rtn_quantize(w, 128)
    wk = repack_int4_for_kernel(packed, 128)
    zu = zeros_to_u8(z)
    got = matmul_w4a16_glu(gu, wk, s, zu, 128)
    with force_kernel("gemv"):
        ref = matmul_w4a16(silu_mul(gu), wk, s, zu, 128)
    assert torch.equal(got, ref), (got.float() - ref.float()).abs().max().item()


def test_glu_down_rejects_what_it_does_not_run():
    from pare_amd.kernels import matmul_w4a16_glu
    from pare_amd.pack import repack_int4_for_kernel, zeros_to_u8

    w = torch.randn(256, 512, device=DEV) * 0.02
    packed, s, z = P.rtn_quantize(w, 128)
    wk = repack_int4_for_kernel(packed, 128)
    with pytest.raises(AssertionError, match="M <= 4"):
        matmul_w4a16_glu(torch.zeros(5, 1024, device=DEV).half(), wk, s, zeros_to_u8(z), 128)
    L = _lib.lib()
    assert L.pmi_matmul_w4a16_glu(None, None, None, None, _lib.PMI_F32, None, 1, 256, 512, 128,
                                  None) == _lib.PMI_ERR_UNSUPPORTED
    assert L.pmi_matmul_w4a16_glu(None, None, None, None, _lib.PMI_U8, None, 5, 256, 512, 128,
                                  None) == _lib.PMI_ERR_UNSUPPORTED


def _gate_up_layer(F, K, seed):
    """Fused gate/up weight RTN-quantised on the device: kernel layout [2F,
    K/2], fp32 scales and u8 zeros [2F, G], and the storage-layout codes and
    fp32 zeros the oracle dequantises."""
    from pare_amd.pack import repack_int4_for_kernel, zeros_to_u8

    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(2 * F, K, generator=g, device=DEV) * 0.02
    packed, s, z = P.rtn_quantize(w, 128)
    return (repack_int4_for_kernel(packed, 128), s.reshape(2 * F, -1).contiguous(),
            zeros_to_u8(z).reshape(2 * F, -1).contiguous(), packed, s, z)


@pytest.mark.parametrize("M,F,K", [(2, 14336, 4096), (4, 14336, 4096), (12, 7168, 1536),
                                   (16, 7168, 2048), (7, 6144, 3072)])
def test_gate_up_silu_matches_matmul_then_silu_mul(M, F, K):
    """The tiled GEMM with SiLU(gate) * up in its epilogue, over the fused weight
    with its rows in glu_row_order, against the fused matmul on the tiled GEMM
    (same configuration: four tiles per workgroup) followed by silu_mul: each
    output row's sum is formed the same way, so the result is equal bit for
    bit; and against the fp32 oracle within the usual tolerance."""
    from oracle import pare_oracle as O
    from pare_amd.kernels import (force_kernel, gate_up_silu_supported, glu_row_order,
                                  matmul_w4a16, matmul_w4a16_gate_up_silu)

    N = 2 * F
    assert gate_up_silu_supported(M, N, K, 128)
    wk, s, zu, packed, s_raw, z_raw = _gate_up_layer(F, K, M + F + K)
    x = (torch.randn(M, K, generator=torch.Generator(device=DEV).manual_seed(K), device=DEV)).half()
    with force_kernel("tgemm"):
        ref = silu_mul(matmul_w4a16(x, wk, s, zu, 128, sz_gm=P.sz_group_major(s, zu),
                                    w_tiled=P.tile_w4a16(wk, 128)))
    idx = glu_row_order(F, DEV)
    got = matmul_w4a16_gate_up_silu(x, P.tile_w4a16(wk[idx].contiguous(), 128),
                                    P.sz_group_major(s[idx].contiguous(), zu[idx].contiguous()),
                                    128, N)
    assert got.shape == (M, F)
    assert torch.equal(got, ref), (got.float() - ref.float()).abs().max().item()
    # the oracle: fp32-accumulated gate/up outputs rounded to fp16, then
    # SiLU(gate) * up in fp32
    w_ref = O.dequantize_packed(packed.cpu().numpy(), s_raw.cpu().numpy(), z_raw.cpu().numpy())
    gu = torch.from_numpy(O.linear_fp32(x.float().cpu().numpy(), w_ref)).half().float()
    act = torch.nn.functional.silu(gu[:, :F]) * gu[:, F:]
    err = (got.float().cpu() - act).abs()
    print(f"[parity] gate_up_silu M={M} F={F} K={K}: max_abs={err.max().item():.3e}", flush=True)
    assert torch.allclose(got.float().cpu(), act, rtol=1e-2, atol=1e-2)


def test_gate_up_silu_rejects_what_it_does_not_run():
    L = _lib.lib()
    assert L.pmi_gate_up_silu_supported(4, 28672, 4096, 128) == 1
    assert L.pmi_gate_up_silu_supported(4, 2048, 4096, 128) == 0    # one tile per workgroup there
    assert L.pmi_gate_up_silu_supported(4, 14336, 1024, 128) == 0   # K < 1536
    assert L.pmi_gate_up_silu_supported(32, 28672, 4096, 128) == 0  # past 16 rows
    assert L.pmi_matmul_w4a16_gate_up_silu(None, None, None, None, None, 4, 2048, 4096, 128,
                                           None) == _lib.PMI_ERR_UNSUPPORTED


def test_decoder_mlp_gate_up_silu_equals_two_launches():
    """A full-size decoder layer's MLP at 4 tokens (the batch-4 decode step) on
    the one-launch gate/up + SiLU path equals the fused matmul + silu_mul +
    down path bit for bit."""
    from pare_amd.decoder import DecoderLayer

    layer = DecoderLayer(DecoderConfig(), torch.Generator(device=DEV).manual_seed(9), DEV)
    n2 = (torch.randn(4, 1, 4096, generator=torch.Generator(device=DEV).manual_seed(2),
                      device=DEV)).half()
    got = layer._mlp(n2, 4, 1)
    ref = layer._down(layer.gate_up.fused(n2), 4, 1)
    assert layer._glu is not None, "the gate/up + SiLU path did not run"
    assert torch.equal(got, ref), (got.float() - ref.float()).abs().max().item()


def _norm_inputs(M, K, seed, residual=True):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=DEV).half()
    r = torch.randn(M, K, generator=g, device=DEV).half() if residual else None
    nw = (1.0 + 0.1 * torch.randn(K, generator=g, device=DEV)).half()
    return x, r, nw


@pytest.mark.parametrize("M,N,K,res", [(4, 6144, 4096, True), (2, 6144, 4096, False),
                                       (3, 4096, 4096, True), (4, 4608, 3584, True),
                                       (4, 4096, 2048, True), (1, 6144, 4096, True)])
def test_tiled_rmsnorm_matches_add_rmsnorm_then_matmul(M, N, K, res):
    """The residual add and RMSNorm formed in the tiled GEMM's prologue against
    add_rmsnorm followed by the matmul on the tiled GEMM (the same unsplit
    configuration): the normalised activations are formed with the same
    roundings and summation order, so y and h are equal bit for bit; and y
    against the fp32 oracle on those activations."""
    from oracle import pare_oracle as O
    from pare_amd.kernels import (force_kernel, matmul_w4a16, matmul_w4a16_tiled_rmsnorm,
                                  tiled_rmsnorm_supported)
    from pare_amd.pack import repack_int4_for_kernel, zeros_to_u8

    assert tiled_rmsnorm_supported(M, N, K, 128)
    g = torch.Generator(device=DEV).manual_seed(M * N + K)
    w = torch.randn(N, K, generator=g, device=DEV) * 0.02
    packed, s_raw, z_raw = P.rtn_quantize(w, 128)
    wk = repack_int4_for_kernel(packed, 128)
    s = s_raw.reshape(N, -1).contiguous()
    zu = zeros_to_u8(z_raw).reshape(N, -1).contiguous()
    sz, wt = P.sz_group_major(s, zu), P.tile_w4a16(wk, 128)
    x, r, nw = _norm_inputs(M, K, N + K, res)
    eps = 1e-5
    n_ref, h_ref = add_rmsnorm(x, r, nw, eps)
    with force_kernel("tgemm"):
        y_ref = matmul_w4a16(n_ref, wk, s, zu, 128, sz_gm=sz, w_tiled=wt)
    for _ in range(2):
        y, h = matmul_w4a16_tiled_rmsnorm(x, r, nw, eps, wt, sz, 128, N)
        assert torch.equal(h, h_ref)
        assert torch.equal(y, y_ref), (y.float() - y_ref.float()).abs().max().item()
    w_ref = O.dequantize_packed(packed.cpu().numpy(), s_raw.cpu().numpy(), z_raw.cpu().numpy())
    ref = torch.from_numpy(O.linear_fp32(n_ref.float().cpu().numpy(), w_ref))
    err = (y.float().cpu() - ref).abs()
    print(f"[parity] tiled_rmsnorm M={M} N={N} K={K}: max_abs={err.max().item():.3e}", flush=True)
    assert torch.allclose(y.float().cpu(), ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("M,F,K", [(4, 14336, 4096), (2, 14336, 4096), (3, 18944, 3584)])
def test_tiled_rmsnorm_glu_matches_norm_then_gate_up_silu(M, F, K):
    """Norm in the prologue and SiLU(gate) * up in the epilogue of one gate/up
    launch against add_rmsnorm followed by the gate/up + SiLU launch, bit for
    bit."""
    from pare_amd.kernels import (glu_row_order, matmul_w4a16_gate_up_silu,
                                  matmul_w4a16_tiled_rmsnorm, tiled_rmsnorm_supported)

    N = 2 * F
    assert tiled_rmsnorm_supported(M, N, K, 128, glu=True)
    wk, s, zu, _, _, _ = _gate_up_layer(F, K, M + F + K)
    idx = glu_row_order(F, DEV)
    wt = P.tile_w4a16(wk[idx].contiguous(), 128)
    sz = P.sz_group_major(s[idx].contiguous(), zu[idx].contiguous())
    x, r, nw = _norm_inputs(M, K, F + K)
    n_ref, h_ref = add_rmsnorm(x, r, nw, 1e-5)
    ref = matmul_w4a16_gate_up_silu(n_ref, wt, sz, 128, N)
    got, h = matmul_w4a16_tiled_rmsnorm(x, r, nw, 1e-5, wt, sz, 128, N, glu=True)
    assert got.shape == (M, F)
    assert torch.equal(h, h_ref)
    assert torch.equal(got, ref), (got.float() - ref.float()).abs().max().item()


def test_tiled_rmsnorm_rejects_what_it_does_not_run():
    L = _lib.lib()
    assert L.pmi_tiled_rmsnorm_supported(4, 6144, 4096, 128, 0) == 1
    assert L.pmi_tiled_rmsnorm_supported(4, 28672, 4096, 128, 1) == 1
    assert L.pmi_tiled_rmsnorm_supported(5, 6144, 4096, 128, 0) == 0   # past 4 rows
    assert L.pmi_tiled_rmsnorm_supported(4, 6144, 8192, 128, 0) == 0   # K > 4096
    assert L.pmi_tiled_rmsnorm_supported(4, 6144, 4096, 64, 0) == 0    # gs 64
    assert L.pmi_tiled_rmsnorm_supported(4, 6144, 4096, 128, 1) == 0   # glu needs four-tile workgroups
    assert L.pmi_tiled_rmsnorm_supported(4, 512, 4096, 128, 0) == 0    # the plain launch splits K
    assert L.pmi_matmul_w4a16_tiled_rmsnorm(None, None, None, 1e-5, None, None, None, None, None,
                                            5, 6144, 4096, 128, 0, None) == _lib.PMI_ERR_UNSUPPORTED


def test_decoder_norm_paths_equal_separate_launches():
    """A full-size decoder layer at 4 tokens (the batch-4 decode step): q/k/v
    and the gate/up + SiLU launch with the norm in their prologue equal
    add_rmsnorm followed by the layer's own launches, bit for bit, with and
    without the pending residual."""
    from pare_amd.decoder import DecoderLayer

    cfg = DecoderConfig()
    layer = DecoderLayer(cfg, torch.Generator(device=DEV).manual_seed(9), DEV)
    g = torch.Generator(device=DEV).manual_seed(4)
    h = torch.randn(4, 1, 4096, generator=g, device=DEV).half()
    d = torch.randn(4, 1, 4096, generator=g, device=DEV).half()
    for pending in (d, None):
        y, h2 = layer._norm_linear(layer.qkv.fused, h, pending, layer.attn_norm.weight)
        n, h_ref = add_rmsnorm(h, pending, layer.attn_norm.weight, cfg.rms_eps)
        assert torch.equal(h2, h_ref)
        assert torch.equal(y, layer.qkv.fused(n)), (y.float() - layer.qkv.fused(n).float()).abs().max()
    h3, out = layer._norm_mlp(h, d, 4, 1)
    n2, h_ref2 = add_rmsnorm(h, d, layer.mlp_norm.weight, cfg.rms_eps)
    assert layer._glu is not None, "the gate/up + SiLU path did not run"
    assert torch.equal(h3, h_ref2)
    assert torch.equal(out, layer._mlp(n2, 4, 1))


@pytest.mark.parametrize("rows,n", [(1, 128256), (4, 128256), (3, 2000), (2, 8), (1, 16392)])
def test_argmax_matches_torch(rows, n):
    from pare_amd.decoder import argmax_into

    g = torch.Generator(device=DEV).manual_seed(rows * n)
    x = torch.randn(rows, n, generator=g, device=DEV).half()
    # ties: the maximum twice in row 0, the first must win
    m = x[0].max()
    x[0, n // 3] = m + 1
    x[0, n // 2] = m + 1
    for _ in range(2):   # the workspace counters must be back at zero
        out = torch.full((rows, 1), -7, dtype=torch.long, device=DEV)
        argmax_into(x, out)
        assert torch.equal(out[:, 0], x.argmax(-1)), (out[:, 0], x.argmax(-1))
    assert out[0, 0].item() == n // 3
    # NaN counts as the largest value, the first one wins
    if n >= 16:
        x[0, 5] = float("nan")
        x[0, 9] = float("nan")
        out = torch.empty(rows, dtype=torch.long, device=DEV)
        argmax_into(x, out)
        assert out[0].item() == 5


@pytest.mark.parametrize("rows,F", [(1, 14336), (4, 1024)])
def test_silu_mul(rows, F):
    g = torch.Generator(device=DEV).manual_seed(rows + F)
    gu = torch.randn(rows, 2 * F, generator=g, device=DEV).half()
    got = silu_mul(gu)
    gf = gu.float()
    ref = torch.nn.functional.silu(gf[:, :F]) * gf[:, F:]
    err = (got.float() - ref).abs() / (ref.abs() + 1e-3)
    assert err.max().item() <= 2e-3, err.max().item()


def _attention_ref(q, ck, cv, p):
    """fp32 attention of q [B, H, 1, D] over cache positions 0..p."""
    B, H, _, D = q.shape
    grp = H // ck.shape[1]
    kf = ck[:, :, :p + 1].float().repeat_interleave(grp, dim=1)
    vf = cv[:, :, :p + 1].float().repeat_interleave(grp, dim=1)
    sc = (q.float() * (1 / D ** 0.5)) @ kf.transpose(-1, -2).contiguous()
    return (torch.softmax(sc, -1) @ vf)[:, :, 0]


def test_shared_workspaces_alternate_large_and_small_shapes():
    """One stream, one cached workspace per op, shapes alternating between many
    counters (B * KV = 128, 72 argmax rows) and few: each call's counters must
    start at zero whatever the previous shape's partials wrote. Checked against
    fp32 references for split attention, attention with fused RoPE and argmax."""
    from pare_amd.decoder import argmax_into, decode_attention_rope

    D, H, KV, L = 128, 32, 8, 200
    g = torch.Generator(device=DEV).manual_seed(99)
    cos, sin = rope_tables(D, 500000.0, L, DEV)
    for B in (16, 1, 16, 2, 16):
        p = 150 if B > 1 else 40
        pos = torch.full((1,), p, dtype=torch.long, device=DEV)
        q = torch.randn(B, H, 1, D, generator=g, device=DEV).half()
        ck = torch.randn(B, KV, L, D, generator=g, device=DEV).half()
        cv = torch.randn(B, KV, L, D, generator=g, device=DEV).half()
        err = (decode_attention(q, ck, cv, pos, 1 / D ** 0.5).float() - _attention_ref(q, ck, cv, p))
        assert err.abs().max().item() <= 5e-3, (B, err.abs().max().item())
        qkv = torch.randn(B, (H + 2 * KV) * D, generator=g, device=DEV).half()
        ck2, cv2 = ck.clone(), cv.clone()
        qr = rope_kv(qkv.view(B, 1, -1), cos, sin, pos, ck2, cv2, B, 1, H, KV, D)
        got = decode_attention_rope(qkv, cos, sin, pos, ck, cv, 1 / D ** 0.5)
        err = (got.float() - _attention_ref(qr, ck2, cv2, p)).abs().max().item()
        assert err <= 5e-3, ("rope", B, err)
        rows = 72 if B > 2 else B
        x = torch.randn(rows, 4000, generator=g, device=DEV).half()
        out = torch.full((rows,), -1, dtype=torch.long, device=DEV)
        argmax_into(x, out)
        assert torch.equal(out, x.argmax(-1)), ("argmax", rows)
        print(f"[workspace] B={B} argmax rows={rows} ok", flush=True)
