"""AWQ-GEMM int32 layout (pare/model/export_awq.py:37-136): the oracle's
restatement pinned by known answers, the device converters against it
bit for bit, and checkpoints written and read back."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
import torch.nn as nn

import pare_amd as P
from oracle import pare_oracle as O
from pare_amd import awq as A

# AutoAWQ and vLLM unpack with this "reverse order": the code of column o of
# a group of eight sits at bit 4 * AWQ_REVERSE_ORDER[o]. It is the published
# inverse of the packing order, written down independently of it.
AWQ_REVERSE_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)


# ---------------------------------------------------------------------------
# Oracle (CPU)
# ---------------------------------------------------------------------------

class TestOracleAwq:
    def test_known_answer_sequence(self):
        # columns 0..7 holding codes 0..7: nibbles, low to high, are 0,2,4,6,1,3,5,7
        assert O.pack_awq(np.arange(8)).view(np.uint32).tolist() == [0x75316420]
        assert O.pack_awq(np.arange(8, 16)).view(np.uint32).tolist() == [0xFDB9ECA8]

    def test_each_column_lands_at_the_published_slot(self):
        for o in range(8):
            x = np.zeros(8, dtype=np.int32)
            x[o] = 0xF
            assert O.pack_awq(x).view(np.uint32)[0] == 0xF << (4 * AWQ_REVERSE_ORDER[o])

    def test_pack_unpack_roundtrip(self):
        rng = np.random.default_rng(0)
        x = rng.integers(0, 16, size=(5, 3, 64))
        w = O.pack_awq(x)
        assert w.dtype == np.int32 and w.shape == (5, 3, 8)
        assert (O.unpack_awq(w) == x).all()

    def test_all_ones_is_minus_one(self):
        assert O.pack_awq(np.full(8, 15)).tolist() == [-1]

    def test_to_and_from_awq_gemm(self):
        rng = np.random.default_rng(1)
        N, K, gs = 24, 128, 32
        q = rng.integers(0, 16, size=(N, K))
        packed = O.pack_int4(q)
        z = rng.integers(0, 16, size=(N, K // gs)).astype(np.float32)
        s = (rng.standard_normal((N, K // gs)) * 0.01).astype(np.float32)
        qw, qz, sc = O.to_awq_gemm(packed, s, z)
        assert qw.shape == (K, N // 8) and qz.shape == (K // gs, N // 8) and sc.shape == (K // gs, N)
        assert sc.dtype == np.float16
        p2, s2, z2 = O.from_awq_gemm(qw, qz, sc)
        assert (p2 == packed).all() and (z2 == z).all()
        assert (s2 == s.astype(np.float16).astype(np.float32)).all()

    def test_dequant_brute_force(self):
        # element by element with the reverse order, against the storage-layout
        # dequantisation of the same layer
        rng = np.random.default_rng(2)
        N, K, gs = 16, 64, 32
        q = rng.integers(0, 16, size=(N, K))
        z = rng.integers(0, 16, size=(N, K // gs)).astype(np.float32)
        s = (rng.standard_normal((N, K // gs)) * 0.05).astype(np.float16).astype(np.float32)
        qw, qz, sc = O.to_awq_gemm(O.pack_int4(q), s, z)
        qwu, qzu = qw.view(np.uint32), qz.view(np.uint32)
        w = np.empty((N, K), dtype=np.float32)
        for k in range(K):
            for n in range(N):
                sh = 4 * AWQ_REVERSE_ORDER[n % 8]
                code = (int(qwu[k, n // 8]) >> sh) & 0xF
                zc = (int(qzu[k // gs, n // 8]) >> sh) & 0xF
                w[n, k] = np.float32(code - zc) * np.float32(sc[k // gs, n])
        ref = O.dequantize_packed(O.pack_int4(q), s[..., None], z[..., None])
        assert np.array_equal(w, ref.reshape(N, K))

    def test_zero_rounding_half_even(self):
        packed = np.zeros((8, 16), dtype=np.uint8)
        z = np.array([[2.5], [3.5], [0.4], [14.5], [15.4], [1.0], [0.0], [7.5]], dtype=np.float32)
        _, qz, _ = O.to_awq_gemm(packed, np.ones_like(z), z)
        assert O.unpack_awq(qz)[0].tolist() == [2, 4, 0, 14, 15, 1, 0, 8]


# ---------------------------------------------------------------------------
# Host logic (CPU)
# ---------------------------------------------------------------------------

def _write_config(path, qcfg):
    path.mkdir(parents=True, exist_ok=True)
    (path / "config.json").write_text(json.dumps({"quantization_config": qcfg}))


def test_read_awq_config(tmp_path):
    _write_config(tmp_path / "ok", A.awq_quantization_config(64))
    assert A.read_awq_config(tmp_path / "ok") == {"group_size": 64}
    legacy = tmp_path / "legacy"
    legacy.mkdir()
    (legacy / "quant_config.json").write_text(json.dumps(
        {"zero_point": True, "q_group_size": 128, "w_bit": 4, "version": "GEMM"}))
    assert A.read_awq_config(legacy) == {"group_size": 128}
    for bad in ({"quant_method": "gptq", "bits": 4},
                {"quant_method": "awq", "bits": 4, "version": "gemv"},
                {"quant_method": "awq", "bits": 8, "version": "gemm"},
                {"quant_method": "awq", "bits": 4, "version": "gemm", "zero_point": False}):
        _write_config(tmp_path / "bad", bad)
        with pytest.raises(ValueError):
            A.read_awq_config(tmp_path / "bad")
    (tmp_path / "none").mkdir()
    with pytest.raises(ValueError, match="quantization_config"):
        A.read_awq_config(tmp_path / "none")


def test_holder_shapes_match_the_reference():
    m = A.AwqGemmLinear(256, 64, 128, has_bias=True)
    assert m.qweight.shape == (256, 8) and m.qweight.dtype == torch.int32
    assert m.qzeros.shape == (2, 8) and m.qzeros.dtype == torch.int32
    assert m.scales.shape == (2, 64) and m.scales.dtype == torch.float16
    assert m.bias.shape == (64,) and m.bias.dtype == torch.float16


def test_no_cpu_fallback(tmp_path):
    with pytest.raises(RuntimeError, match="HIP device"):
        A.awq_to_storage(torch.zeros(32, 1, dtype=torch.int32), torch.zeros(1, 1, dtype=torch.int32),
                         torch.zeros(1, 8, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="HIP device"):
        A.storage_to_awq(torch.zeros(8, 16, dtype=torch.uint8), torch.ones(8, 1), torch.zeros(8, 1), 32)
    _write_config(tmp_path, A.awq_quantization_config(128))
    (tmp_path / "model.safetensors").write_bytes(b"")
    with pytest.raises(RuntimeError, match="cuda"):
        A.load_awq(nn.Module(), tmp_path, device="cpu")


# ---------------------------------------------------------------------------
# Device converters (GPU)
# ---------------------------------------------------------------------------

SHAPES = [  # (N, K, group_size)
    (8, 32, 32),
    (64, 256, 128),
    (136, 384, 128),
    (40, 192, 64),
    (512, 4096, 4096),      # one group per row
    (4096, 4096, 128),
    (11008, 4096, 128),
]


def _random_awq(N, K, gs, seed):
    g = torch.Generator().manual_seed(seed)
    G = K // gs
    qw = torch.randint(-2**31, 2**31 - 1, (K, N // 8), generator=g, dtype=torch.int64).to(torch.int32)
    qz = torch.randint(-2**31, 2**31 - 1, (G, N // 8), generator=g, dtype=torch.int64).to(torch.int32)
    sc = (torch.randn(G, N, generator=g) * 0.02).half()
    return qw, qz, sc


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,gs", SHAPES)
def test_import_matches_oracle(N, K, gs):
    print(f"awq import N={N} K={K} gs={gs}", flush=True)
    qw, qz, sc = _random_awq(N, K, gs, seed=N + K)
    packed, scale, zero = A.awq_to_storage(qw.cuda(), qz.cuda(), sc.cuda(), gs)
    torch.cuda.synchronize()
    p_ref, s_ref, z_ref = O.from_awq_gemm(qw.numpy(), qz.numpy(), sc.numpy())
    assert np.array_equal(packed.cpu().numpy(), p_ref)
    assert np.array_equal(scale.squeeze(-1).cpu().numpy(), s_ref)
    assert np.array_equal(zero.squeeze(-1).cpu().numpy(), z_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,gs", SHAPES)
@pytest.mark.parametrize("zero_dtype", ["f32", "u8"])
def test_export_matches_oracle(N, K, gs, zero_dtype):
    print(f"awq export N={N} K={K} gs={gs} zeros={zero_dtype}", flush=True)
    g = torch.Generator().manual_seed(7 * N + K)
    G = K // gs
    packed = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    scale = torch.randn(N, G, generator=g) * 0.02
    scale.view(-1)[:4] = torch.tensor([70000.0, -65520.0, 1e-7, 65504.0])[: scale.numel()]
    zero = torch.randint(0, 16, (N, G), generator=g).float()
    z_in = zero.to(torch.uint8) if zero_dtype == "u8" else zero
    qw, qz, sc = A.storage_to_awq(packed.cuda(), scale.cuda(), z_in.cuda(), gs)
    torch.cuda.synchronize()
    r_qw, r_qz, r_sc = O.to_awq_gemm(packed.numpy(), scale.numpy(), zero.numpy())
    assert np.array_equal(qw.cpu().numpy(), r_qw)
    assert np.array_equal(qz.cpu().numpy(), r_qz)
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), r_sc.view(np.uint16))


@pytest.mark.gpu
def test_export_rounds_zeros_half_even_and_rejects_out_of_range():
    packed = torch.zeros(8, 16, dtype=torch.uint8, device="cuda")
    z = torch.tensor([[2.5], [3.5], [0.4], [14.5], [15.4], [1.0], [-0.4], [7.5]], device="cuda")
    _, qz, _ = A.storage_to_awq(packed, torch.ones_like(z), z, 32)
    assert O.unpack_awq(qz.cpu().numpy())[0].tolist() == [2, 4, 0, 14, 15, 1, 0, 8]
    for bad in (15.6, -0.6, float("nan")):
        zb = z.clone()
        zb[3, 0] = bad
        with pytest.raises(ValueError, match="outside"):
            A.storage_to_awq(packed, torch.ones_like(z), zb, 32)


@pytest.mark.gpu
def test_roundtrip_at_the_gate_up_shape():
    # size-independent property at the decoder's largest layer: storage ->
    # AWQ -> storage is the identity on the codes and zeros; one column slab
    # is also checked against the oracle
    N, K, gs = 28672, 4096, 128
    print(f"awq roundtrip N={N} K={K}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(3)
    packed = torch.randint(0, 256, (N, K // 2), generator=g, device="cuda", dtype=torch.int32).to(torch.uint8)
    scale = (torch.randn(N, K // gs, generator=g, device="cuda") * 0.02).half().float()
    zero = torch.randint(0, 16, (N, K // gs), generator=g, device="cuda").float()
    qw, qz, sc = A.storage_to_awq(packed, scale, zero, gs)
    p2, s2, z2 = A.awq_to_storage(qw, qz, sc, gs)
    assert torch.equal(p2, packed) and torch.equal(s2.squeeze(-1), scale)
    assert torch.equal(z2.squeeze(-1), zero)
    r_qw, r_qz, r_sc = O.to_awq_gemm(packed[:256].cpu().numpy(), scale[:256].cpu().numpy(),
                                     zero[:256].cpu().numpy())
    assert np.array_equal(qw[:, :32].cpu().numpy(), r_qw)
    assert np.array_equal(qz[:, :32].cpu().numpy(), r_qz)


@pytest.mark.gpu
def test_converters_validate_shapes():
    with pytest.raises(RuntimeError, match="divisible by 8"):
        # N = 12 is not a multiple of 8: rejected by the library before any launch
        A.storage_to_awq(torch.zeros(12, 16, dtype=torch.uint8, device="cuda"),
                         torch.ones(12, 1, device="cuda"), torch.zeros(12, 1, device="cuda"), 32)
    with pytest.raises(ValueError, match="groups"):
        A.awq_to_storage(torch.zeros(64, 1, dtype=torch.int32, device="cuda"),
                         torch.zeros(3, 1, dtype=torch.int32, device="cuda"),
                         torch.zeros(3, 8, dtype=torch.float16, device="cuda"), 32)


# ---------------------------------------------------------------------------
# Layers and checkpoints (GPU)
# ---------------------------------------------------------------------------

def _rtn_awq_layer(N, K, gs, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    packed, s, z = O.rtn_quantize(w, gs)
    return O.to_awq_gemm(packed, s, z)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 5, 64])
@pytest.mark.parametrize("N,K,gs", [(256, 512, 128), (4096, 4096, 128), (1024, 4096, 64)])
def test_imported_layer_forward(M, N, K, gs):
    print(f"awq layer M={M} N={N} K={K} gs={gs}", flush=True)
    qw, qz, sc = _rtn_awq_layer(N, K, gs, seed=M)
    bias = (torch.randn(N) * 0.1).half().cuda()
    ql = A.from_awq_tensors(torch.from_numpy(qw).cuda(), torch.from_numpy(qz).cuda(),
                            torch.from_numpy(sc).cuda(), bias, gs)
    p_ref, s_ref, z_ref = O.from_awq_gemm(qw, qz, sc)
    ref = P.QuantizedLinear(torch.from_numpy(p_ref).cuda(), torch.from_numpy(s_ref)[..., None].cuda(),
                            torch.from_numpy(z_ref)[..., None].cuda(),
                            P.QuantConfig(bits=4, group_size=gs), bias, K, N, use_kernel=True)
    x = (torch.randn(M, K) * 0.5).half().cuda()
    with torch.no_grad():
        y = ql(x)
        assert torch.equal(y, ref(x))   # same buffers, same kernel
    w_hat = O.dequantize_packed(p_ref, s_ref[..., None], z_ref[..., None]).reshape(N, K)
    y32 = O.linear_fp32(x.float().cpu().numpy(), w_hat) + bias.float().cpu().numpy()
    # fp32 accumulation vs fp16 output: within half an fp16 ulp of the value
    # plus the accumulation-order difference
    tol = 2e-3 + 2e-3 * np.abs(y32)
    assert (np.abs(y.float().cpu().numpy() - y32) <= tol).all()


class Tiny(nn.Module):
    def __init__(self, K=512, N=256):
        super().__init__()
        self.embed = nn.Embedding(10, K)
        self.proj = nn.Linear(K, N)
        self.head = nn.Linear(N, 10, bias=False)


@pytest.mark.gpu
def test_export_then_load(tmp_path):
    torch.manual_seed(0)
    K, N, gs = 512, 256, 128
    src = Tiny(K, N).cuda()
    w = (torch.randn(N, K) * 0.02).numpy()
    packed, s, z = O.rtn_quantize(w, gs)
    bias = (torch.randn(N) * 0.1).half()
    src.proj = P.QuantizedLinear(torch.from_numpy(packed).cuda(), torch.from_numpy(s).cuda(),
                                 torch.from_numpy(z).cuda(), P.QuantConfig(bits=4, group_size=gs),
                                 bias.cuda(), K, N, use_kernel=True)
    x = (torch.randn(3, K) * 0.5).half().cuda()
    out_dir = tmp_path / "awq"
    P.export_awq(src, out_dir)
    assert isinstance(src.proj, A.AwqGemmLinear)
    cfg = json.loads((out_dir / "config.json").read_text())["quantization_config"]
    assert cfg == {"quant_method": "awq", "bits": 4, "group_size": gs, "version": "gemm",
                   "zero_point": True}
    from safetensors.torch import load_file
    t = load_file(str(out_dir / "model.safetensors"))
    r_qw, r_qz, r_sc = O.to_awq_gemm(packed, s, z)
    assert np.array_equal(t["proj.qweight"].numpy(), r_qw)
    assert np.array_equal(t["proj.qzeros"].numpy(), r_qz)
    assert np.array_equal(t["proj.scales"].numpy().view(np.uint16), r_sc.view(np.uint16))
    assert t["proj.bias"].dtype == torch.float16

    dst = Tiny(K, N).cuda()
    P.load_awq(dst, out_dir)
    assert isinstance(dst.proj, P.QuantizedLinear) and dst.proj.use_kernel
    assert torch.equal(dst.embed.weight, src.embed.weight)
    assert torch.equal(dst.proj.packed_weight.cpu(), torch.from_numpy(packed))
    s16 = torch.from_numpy(s).half().float()
    assert torch.equal(dst.proj.scale.cpu(), s16)
    assert torch.equal(dst.proj.zero.cpu(), torch.from_numpy(z))
    # the reloaded layer is the original with fp16-rounded scales
    want = P.QuantizedLinear(torch.from_numpy(packed).cuda(), s16.cuda(), torch.from_numpy(z).cuda(),
                             P.QuantConfig(bits=4, group_size=gs), bias.cuda(), K, N,
                             use_kernel=True)
    with torch.no_grad():
        assert torch.equal(dst.proj(x), want(x))
