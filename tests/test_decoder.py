"""End-to-end decoder on a small Llama-shaped config: the
HIP path inside a model, graph-captured decode, and the reference's
dequantize-on-the-fly path as the check (pare/layers/linear.py:101-138)."""

from __future__ import annotations

import pytest
import torch

import pare_amd as P
from pare_amd.decoder import DecoderConfig, QuantizedDecoder, decoder_throughput

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SMALL = DecoderConfig(hidden=512, heads=8, kv_heads=2, ffn=1024, vocab=2000, layers=2)


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
