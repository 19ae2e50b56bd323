"""GPTQ producer (pare/schemes/gptq.py:156-263, pare/calibration/hessian.py).

The oracle's GPTQ restatement is pinned by the reference's own numerical
tests (tests/test_gptq_numerical.py of the reference), by closed forms (a
diagonal Hessian reduces GPTQ to RTN exactly) and by an unblocked float64
formulation of the same algorithm. The device path is checked against the
oracle bit for bit where both start from the same factor C (one block). With
a block-diagonal Hessian the lazy updates are exact zeros, so the group
scales and g_idx must match exactly and the codes to 99.9 %; the factors
themselves come from rocSOLVER and LAPACK. Elsewhere the checks are code
agreement and the GPTQ objective.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import pare_amd as P
from oracle import pare_oracle as O
from pare_amd import _lib
from pare_amd import gptq as G


def _layer(N, K, n_tok=256, seed=0, scale=1.0):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    # activations with unequal column energy, so act_order has work to do
    X = (rng.standard_normal((n_tok, K)) * (scale * (0.2 + rng.random(K)))).astype(np.float32)
    return W, O.hessian(X).astype(np.float32), X


def _codes(packed):
    return O.unpack_int4(packed)


# ---------------------------------------------------------------------------
# Oracle pins (CPU)
# ---------------------------------------------------------------------------

class TestHessian:
    """The reference's HessianAccumulator tests (test_gptq_numerical.py:31-89)
    on this package's accumulator, and the oracle against numpy."""

    def test_single_batch(self):
        X = torch.randn(10, 8)
        acc = G.HessianAccumulator()
        acc.accumulate(X.unsqueeze(0))
        ref = torch.from_numpy(2.0 / 10 * (X.numpy().T @ X.numpy())).float()
        torch.testing.assert_close(acc.finalize(), ref, atol=1e-5, rtol=1e-5)
        np.testing.assert_allclose(O.hessian(X.numpy()), ref.numpy(), atol=1e-5, rtol=1e-5)

    def test_multi_batch_equals_concat(self):
        X1, X2 = torch.randn(6, 4), torch.randn(8, 4)
        a, b = G.HessianAccumulator(), G.HessianAccumulator()
        a.accumulate(X1)
        a.accumulate(X2)
        b.accumulate(torch.cat([X1, X2]))
        torch.testing.assert_close(a.finalize(), b.finalize(), atol=1e-5, rtol=1e-5)

    def test_3d_flattened_and_empty(self):
        X = torch.randn(2, 5, 4)
        a, b = G.HessianAccumulator(), G.HessianAccumulator()
        a.accumulate(X)
        b.accumulate(X.reshape(10, 4))
        torch.testing.assert_close(a.finalize(), b.finalize())
        with pytest.raises(RuntimeError, match="no samples"):
            G.HessianAccumulator().finalize()
        with pytest.raises(ValueError):
            G.HessianAccumulator().accumulate(torch.randn(3))


class TestCholeskyChain:
    def test_ct_c_is_hinv(self):
        """gptq_numerical.py:96-112: the chain satisfies C^T C = H^-1."""
        _, H, _ = _layer(4, 16, n_tok=100)
        Hp, _, _ = O.gptq_prepare(H, 0.01)
        C = O.gptq_cholesky(Hp)
        np.testing.assert_allclose(C.T.astype(np.float64) @ C, np.linalg.inv(Hp.astype(np.float64)),
                                   rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(np.diag(Hp), np.diag(H) + 0.01 * np.mean(np.diag(H)), rtol=1e-6)
        assert np.allclose(np.tril(C, -1), 0)

    def test_device_chain_matches(self):
        """The package's chain (torch.linalg in float64) on the CPU gives the
        oracle's factor."""
        _, H, _ = _layer(4, 32, n_tok=100)
        Hp, _, _ = O.gptq_prepare(H, 0.01)
        C = G._cholesky_chain(torch.from_numpy(Hp), 0.0).numpy()
        np.testing.assert_allclose(C, O.gptq_cholesky(Hp), rtol=1e-5, atol=1e-6)


def _unblocked_gptq(W, C, scale, zero, colg):
    """GPTQ without lazy batching, in float64: every column's error updates
    all later columns at once. Equal to the blocked loop in exact arithmetic."""
    W = W.astype(np.float64).copy()
    C = C.astype(np.float64)
    Q = np.zeros(W.shape, dtype=np.int32)
    for j in range(W.shape[1]):
        s, z = scale[:, colg[j]].astype(np.float64), zero[:, colg[j]].astype(np.float64)
        q = np.clip(np.rint(W[:, j] / s + z), 0, 15)
        Q[:, j] = q
        e = (W[:, j] - (q - z) * s) / C[j, j]
        W[:, j + 1:] -= np.outer(e, C[j, j + 1:])
    return Q


class TestOracleGptq:
    def test_diagonal_hessian_is_rtn(self):
        # C is diagonal, so every update is an exact zero: GPTQ = RTN
        rng = np.random.default_rng(1)
        W = (rng.standard_normal((16, 256)) * 0.05).astype(np.float32)
        H = np.diag(rng.random(256) + 0.5).astype(np.float32)
        p_rtn, s_rtn, z_rtn = O.rtn_quantize(W, 64)
        for groups in ("reference", "dynamic"):
            p, s, z, g_idx = O.gptq_quantize(W, H, 64, groups=groups)
            assert np.array_equal(p, p_rtn) and np.array_equal(s, s_rtn) and np.array_equal(z, z_rtn)
            assert g_idx is None
        # act_order with dynamic groups is RTN over the permuted columns
        p, s, z, g_idx = O.gptq_quantize(W, H, 64, act_order=True, groups="dynamic")
        _, perm, _ = O.gptq_prepare(H, 0.01, act_order=True)
        p2, s2, z2, g2 = O.rtn_quantize_act_order(W, perm, 64)
        assert np.array_equal(p, p2) and np.array_equal(s, s2) and np.array_equal(z, z2)
        assert np.array_equal(g_idx, g2)

    @pytest.mark.parametrize("groups", ["reference", "dynamic"])
    def test_blocked_equals_unblocked(self, groups):
        W, H, _ = _layer(24, 384, seed=2)
        C = O.gptq_cholesky(O.gptq_prepare(H, 0.01)[0])
        if groups == "reference":
            s, z = O.compute_scale(W, "per_group", 128, False)
            s, z = s[..., 0], z[..., 0]
            colg = np.arange(384) // 128
            Qb = O.gptq_columns(W, C, colg, s.copy(), z.copy())
            Qu = _unblocked_gptq(W, C, s, z, colg)
        else:
            # dynamic groups: freeze the group parameters the blocked loop found
            s = np.zeros((24, 3), np.float32)
            z = np.zeros((24, 3), np.float32)
            colg = np.arange(384) // 128
            Qb = O.gptq_columns(W, C, colg, s, z, group_starts=True, group_size=128)
            Qu = _unblocked_gptq(W, C, s, z, colg)
        agree = (Qb == Qu).mean()
        assert agree > 0.99, agree

    def test_output_error_below_rtn(self):
        """gptq_numerical.py:180-222 on the oracle: GPTQ's output error is at
        most RTN's (x 1.05)."""
        rng = np.random.default_rng(0)
        W = rng.standard_normal((16, 64)).astype(np.float32)
        X = rng.standard_normal((200, 64)).astype(np.float32)
        H = (2.0 / 200) * X.T @ X
        p_rtn, s, z = O.rtn_quantize(W, 16)
        rtn_err = (((W - O.dequantize_packed(p_rtn, s, z)) @ X.T) ** 2).mean()
        for groups in ("reference", "dynamic"):
            p, s2, z2, g_idx = O.gptq_quantize(W, H, 16, groups=groups)
            err = (((W - O.dequantize_packed(p, s2, z2)) @ X.T) ** 2).mean()
            assert err <= rtn_err * 1.05, (groups, err, rtn_err)

    def test_range_shape_and_order(self):
        """gptq_numerical.py:165-178,224-300: codes in [0, 15], shapes kept,
        act_order output in the original column order."""
        W, H, _ = _layer(8, 64, seed=3)
        for act_order in (False, True):
            for groups in ("reference", "dynamic"):
                p, s, z, g_idx = O.gptq_quantize(W, H, 16, act_order=act_order, groups=groups)
                q = _codes(p)
                assert q.shape == (8, 64) and q.min() >= 0 and q.max() <= 15
                assert s.shape == (8, 4, 1) and z.shape == (8, 4, 1)
                assert (g_idx is not None) == (act_order and groups == "dynamic")

    def test_g_idx_is_the_processing_order(self):
        # dequantising with g_idx equals dequantising the processed order with
        # contiguous groups, then undoing the permutation
        W, H, _ = _layer(8, 128, seed=4)
        p, s, z, g_idx = O.gptq_quantize(W, H, 32, act_order=True)
        _, perm, _ = O.gptq_prepare(H, 0.01, act_order=True)
        assert np.array_equal(g_idx, O.gidx_from_perm(perm, 32))
        q = _codes(p)
        w_g = O.dequantize_gidx(q, s, z, g_idx)
        w_p = O.dequantize_tensor(q[:, perm], s, z).reshape(8, 128)
        assert np.array_equal(w_g[:, perm], w_p)

    def test_act_order_helps_the_objective(self):
        W, H, _ = _layer(32, 256, seed=5, scale=3.0)
        objs = {}
        for act_order in (False, True):
            p, s, z, g_idx = O.gptq_quantize(W, H, 64, act_order=act_order)
            q = _codes(p)
            w_hat = O.dequantize_gidx(q, s, z, g_idx if g_idx is not None else np.arange(256) // 64)
            objs[act_order] = O.gptq_objective(W, w_hat, H)
        assert objs[True] <= objs[False] * 1.05, objs

    def test_offset8_known_answers(self):
        """Hand-derived offset-8 groups (zero 8, scale 2 max|w| / 15, codes
        clamp(rint(w / s + 8), 0, 15) with ties to even).
        Row 0: max|w| = 7.5, so the scale is exactly 1.0 and the codes are
        w + 8 rounded: -7.5 -> 0.5 -> 0; 7.5 -> 15.5 -> 16 -> clamped 15;
        -0.5 -> 7.5 -> 8; 0.5 -> 8.5 -> 8; 1.5 -> 9.5 -> 10; -3.2 -> 4.8 -> 5;
        2.49 -> 10.49 -> 10; -6.5 -> 1.5 -> 2; 6.5 -> 14.5 -> 14; 0 -> 8.
        Row 1: max|w| = 0.375, scale 0.05 -> fp32 0x3D4CCCCD (13421773 * 2^-28).
        0.375 / s rounds to 7.5 in fp32 -> 15.5 -> 16 -> 15; -0.375 -> 0;
        0.1 (fp32 13421773 * 2^-27) / s = 2 exactly -> 10; -0.125 / s rounds
        to -2.5 -> 5.5 -> 6."""
        w = np.zeros((2, 32), np.float32)
        w[0, :10] = [-7.5, 7.5, 0.0, -0.5, 0.5, 1.5, -3.2, 2.49, -6.5, 6.5]
        w[1, :4] = [0.375, -0.375, 0.1, -0.125]
        packed, s, z = O.rtn_quantize(w, 32, sym="offset8")
        assert s.reshape(2).view(np.uint32).tolist() == [0x3F800000, 0x3D4CCCCD]
        assert z.reshape(2).tolist() == [8.0, 8.0]
        q = O.unpack_int4(packed)
        assert q[0, :10].tolist() == [0, 15, 8, 8, 8, 10, 5, 10, 2, 14]
        assert (q[0, 10:] == 8).all()
        assert q[1, :4].tolist() == [15, 0, 10, 6]
        assert (q[1, 4:] == 8).all()

    def test_offset8_sym(self):
        W, H, _ = _layer(8, 128, seed=6)
        p, s, z, _ = O.gptq_quantize(W, H, 64, sym=True)
        assert (z == 8).all()
        # the reference's rule would clamp every negative weight to code 0
        q = _codes(p)
        assert (q[W < -0.05] < 8).all()
        p_ref, _, z_ref, _ = O.gptq_quantize(W, H, 64, sym=True, groups="reference")
        assert (z_ref == 0).all()

    def test_dead_columns(self):
        W, H, _ = _layer(8, 64, seed=7)
        H[:, 5] = 0
        H[5, :] = 0
        p, s, z, _ = O.gptq_quantize(W, H, 32)
        w_hat = O.dequantize_packed(p, s, z)
        # a dead column is quantised as zero weight: its code is the zero point
        assert np.array_equal(_codes(p)[:, 5].astype(np.float32), z[:, 0, 0])
        assert (w_hat[:, 5] == 0).all()


def test_entry_points_validate_before_launch():
    L = _lib.lib()
    assert L.pmi_gptq_block(None, None, None, None, None, None, None, 4, 20, 1, 0, 16, None) == \
        _lib.PMI_ERR_INVALID
    assert L.pmi_gptq_block(None, None, None, None, None, None, None, 4, 256, 2, 0, 144, None) == \
        _lib.PMI_ERR_INVALID
    assert L.pmi_gptq_block(None, None, None, None, None, None, None, 4, 256, 2, 200, 64, None) == \
        _lib.PMI_ERR_INVALID
    assert L.pmi_gptq_block(None, None, None, None, None, None, None, 4, 256, 2, 0, 128, None) == \
        _lib.PMI_ERR_INVALID   # null buffers
    assert L.pmi_gptq_pack(None, None, None, 4, 12, None) == _lib.PMI_ERR_INVALID
    assert L.pmi_gptq_group_params(None, 64, 4, 32, 64, 0, None, None, 2, 0, None) == \
        _lib.PMI_ERR_INVALID
    assert L.pmi_gptq_group_params(None, 64, 4, 0, 32, 3, None, None, 2, 0, None) == \
        _lib.PMI_ERR_INVALID
    assert L.pmi_rtn_quantize(None, _lib.PMI_F32, None, None, None, 4, 64, 32, 3, None) == \
        _lib.PMI_ERR_INVALID


def test_no_cpu_fallback():
    with pytest.raises(RuntimeError, match="HIP device"):
        G.gptq_quantize(torch.zeros(8, 64), torch.eye(64), 32)


# ---------------------------------------------------------------------------
# Device (GPU)
# ---------------------------------------------------------------------------

def _columns_on_device(W, C, colg, s, z, gs, dynamic_sym=None):
    Wt = torch.from_numpy(W).cuda().contiguous()
    st = torch.from_numpy(s).cuda().contiguous()
    zt = torch.from_numpy(z).cuda().contiguous()
    codes = G.gptq_columns(Wt, torch.from_numpy(C).cuda(), torch.from_numpy(colg).int().cuda(),
                           st, zt, gs, dynamic_sym=dynamic_sym)
    torch.cuda.synchronize()
    return codes.cpu().numpy().T.astype(np.int32), st.cpu().numpy(), zt.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,gs", [(1, 16, 16), (100, 64, 32), (128, 128, 128), (300, 128, 64),
                                    (129, 96, 32)])
@pytest.mark.parametrize("groups", ["reference", "dynamic"])
def test_block_kernel_bit_exact_one_block(N, K, gs, groups):
    print(f"gptq block N={N} K={K} gs={gs} {groups}", flush=True)
    W, H, _ = _layer(N, K, seed=N + K)
    C = O.gptq_cholesky(O.gptq_prepare(H, 0.01)[0])
    colg = (np.arange(K) // gs).astype(np.int64)
    if groups == "reference":
        s, z = O.compute_scale(W, "per_group", gs, False)
        s, z = s[..., 0].copy(), z[..., 0].copy()
        Q_ref = O.gptq_columns(W, C, colg, s.copy(), z.copy())
        Q, _, _ = _columns_on_device(W, C, colg, s, z, gs)
    else:
        s = np.zeros((N, K // gs), np.float32)
        z = np.zeros((N, K // gs), np.float32)
        Q_ref = O.gptq_columns(W, C, colg, s, z, group_starts=True, group_size=gs)
        Q, s_d, z_d = _columns_on_device(W, C, colg, np.zeros_like(s), np.zeros_like(z), gs,
                                         dynamic_sym=0)
        assert np.array_equal(s_d, s) and np.array_equal(z_d, z)
    assert np.array_equal(Q, Q_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("act_order", [False, True])
@pytest.mark.parametrize("sym", [False, True])
def test_block_diagonal_hessian(act_order, sym):
    # independent 128-column blocks: the lazy updates are exact zeros on both
    # sides, so every block, group start, permutation and pack step must match
    N, K, gs = 200, 512, 64
    print(f"gptq block-diagonal act_order={act_order} sym={sym}", flush=True)
    rng = np.random.default_rng(11)
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    H = np.zeros((K, K), np.float32)
    for b in range(0, K, 128):
        X = (rng.standard_normal((300, 128)) * (0.2 + rng.random(128))).astype(np.float32)
        H[b:b + 128, b:b + 128] = O.hessian(X)
    if act_order:
        # a permutation by diag(H) would mix the blocks; keep each block's
        # columns together by making the diagonal decrease block by block
        H[np.diag_indices(K)] += np.repeat(np.arange(K // 128, 0, -1) * 1000.0, 128).astype(np.float32)
    p_ref, s_ref, z_ref, g_ref = O.gptq_quantize(W, H, gs, sym=sym, act_order=act_order)
    p, s, z, g_idx = G.gptq_quantize(torch.from_numpy(W).cuda(), torch.from_numpy(H).cuda(), gs,
                                     sym=sym, act_order=act_order)
    assert np.array_equal(s.cpu().numpy(), s_ref) and np.array_equal(z.cpu().numpy(), z_ref)
    q, q_ref = _codes(p.cpu().numpy()), _codes(p_ref)
    # the device factor comes from rocSOLVER, the oracle's from LAPACK: allow
    # the rare code that sits on a rounding tie
    assert (q == q_ref).mean() > 0.999
    if act_order:
        assert np.array_equal(g_idx.cpu().numpy(), g_ref)
    else:
        assert g_idx is None


@pytest.mark.gpu
@pytest.mark.parametrize("act_order", [False, True])
@pytest.mark.parametrize("groups", ["reference", "dynamic"])
def test_against_oracle_dense_hessian(act_order, groups):
    N, K, gs = 256, 1024, 128
    print(f"gptq dense N={N} K={K} act_order={act_order} {groups}", flush=True)
    W, H, _ = _layer(N, K, seed=21, scale=2.0)
    p_ref, s_ref, z_ref, g_ref = O.gptq_quantize(W, H, gs, act_order=act_order, groups=groups)
    p, s, z, g_idx = G.gptq_quantize(torch.from_numpy(W).cuda(), torch.from_numpy(H).cuda(), gs,
                                     act_order=act_order, groups=groups)
    q, q_ref = _codes(p.cpu().numpy()), _codes(p_ref)
    agree = (q == q_ref).mean()
    assert agree > 0.99, agree
    gi = g_idx.cpu().numpy() if g_idx is not None else np.arange(K) // gs
    gi_ref = g_ref if g_ref is not None else np.arange(K) // gs
    assert np.array_equal(gi, gi_ref)
    obj = O.gptq_objective(W, O.dequantize_gidx(q, s.cpu().numpy(), z.cpu().numpy(), gi), H)
    obj_ref = O.gptq_objective(W, O.dequantize_gidx(q_ref, s_ref, z_ref, gi_ref), H)
    assert abs(obj - obj_ref) <= 0.02 * obj_ref, (obj, obj_ref)
    p_rtn, s_rtn, z_rtn = O.rtn_quantize(W, gs)
    obj_rtn = O.gptq_objective(W, O.dequantize_packed(p_rtn, s_rtn, z_rtn), H)
    assert obj < obj_rtn, (obj, obj_rtn)


@pytest.mark.gpu
def test_diagonal_hessian_equals_device_rtn():
    N, K, gs = 512, 1024, 128
    rng = np.random.default_rng(5)
    W = torch.from_numpy((rng.standard_normal((N, K)) * 0.05).astype(np.float32)).cuda()
    H = torch.diag(torch.from_numpy(rng.random(K).astype(np.float32) + 0.5)).cuda()
    p, s, z, g_idx = G.gptq_quantize(W, H, gs, groups="dynamic")
    p_rtn, s_rtn, z_rtn = P.rtn_quantize(W, gs)
    assert torch.equal(p, p_rtn) and torch.equal(s, s_rtn) and torch.equal(z, z_rtn)
    assert g_idx is None


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("gs", [32, 128, "per_channel"])
def test_rtn_offset8_matches_oracle(dtype, gs):
    N, K = 96, 512
    w = (torch.randn(N, K, generator=torch.Generator().manual_seed(3)) * 0.05).to(dtype)
    gran = "per_channel" if gs == "per_channel" else "per_group"
    g = K if gs == "per_channel" else gs
    p, s, z = P.rtn_quantize(w.cuda(), g, sym="offset8", granularity=gran)
    p_ref, s_ref, z_ref = O.rtn_quantize(w.float().numpy(), g, sym="offset8", granularity=gran)
    assert np.array_equal(p.cpu().numpy(), p_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref) and np.array_equal(z.cpu().numpy(), z_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 16, 64])
def test_gptq_layer_on_the_kernel_path(M):
    # an act_order layer with g_idx, produced on the device, run by the matmul
    torch.manual_seed(0)
    K, N = 1024, 512
    lin = nn.Linear(K, N, bias=True).cuda().half()
    acc = G.HessianAccumulator()
    acc.accumulate(torch.randn(4, 64, K, device="cuda") * (0.2 + torch.rand(K, device="cuda")))
    cfg = P.QuantConfig(bits=4, scheme="gptq", group_size=128, act_order=True)
    ql = G.quantize_linear_gptq(lin, acc.finalize(), cfg)
    assert ql.g_idx is not None and ql.g_idx.dtype == torch.int32
    x = torch.randn(M, K, device="cuda").half()
    with torch.no_grad():
        ql.use_kernel = True
        y = ql(x)
        ql.use_kernel = False
        y_ref = ql(x)
    torch.testing.assert_close(y, y_ref, rtol=1e-2, atol=1e-2)


@pytest.mark.gpu
def test_llama_layer_time_and_quality():
    # full-size q_proj-like layer: report the producer's time, check the objective
    import time
    N, K = 4096, 4096
    torch.manual_seed(1)
    W = torch.randn(N, K, device="cuda") * 0.02
    X = torch.randn(2048, K, device="cuda") * (0.2 + torch.rand(K, device="cuda"))
    H = (2.0 / X.shape[0]) * (X.T @ X)
    G.gptq_quantize(W[:256], H, 128, act_order=True)   # warm-up (library handles)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    p, s, z, g_idx = G.gptq_quantize(W, H, 128, act_order=True)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    print(f"gptq 4096x4096 act_order: {dt * 1e3:.1f} ms", flush=True)
    w_hat = P.dequantize_int4(p, s, z, 128, dtype=torch.float32, g_idx=g_idx)
    p_r, s_r, z_r = P.rtn_quantize(W, 128)
    w_rtn = P.dequantize_int4(p_r, s_r, z_r, 128, dtype=torch.float32)
    obj = ((W - w_hat) @ H * (W - w_hat)).sum().item()
    obj_rtn = ((W - w_rtn) @ H * (W - w_rtn)).sum().item()
    print(f"objective gptq {obj:.4g} rtn {obj_rtn:.4g}", flush=True)
    assert obj < 0.8 * obj_rtn
