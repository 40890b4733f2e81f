"""BlockLDLQ algebra: the float64 oracle pinned by closed forms, and the
backend's host-side pieces (block LDL, Hessian congruence, regularisation)
checked against it on CPU tensors."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ldlq as oldlq
from qsrt_amd import exl3_encoder_backend as be
from qsrt_amd.ldlq import make_shared_h


def _spd(n, seed, rho=0.8):
    rng = np.random.default_rng(seed)
    x = np.empty((4 * n, n))
    x[:, 0] = rng.standard_normal(4 * n)
    for j in range(1, n):
        x[:, j] = rho * x[:, j - 1] + np.sqrt(1 - rho * rho) * rng.standard_normal(4 * n)
    h = x.T @ x / x.shape[0]
    return h + 0.01 * np.mean(np.diag(h)) * np.eye(n)


def test_oracle_block_ldl_reconstructs_h():
    H = _spd(128, 1)
    L, D = oldlq.block_ldl(H, 16)
    Dfull = np.zeros_like(H)
    for i, blk in enumerate(D):
        Dfull[16 * i:16 * i + 16, 16 * i:16 * i + 16] = blk
    assert np.allclose(L @ Dfull @ L.T, H, atol=1e-12)
    for i in range(8):
        assert np.array_equal(L[16 * i:16 * i + 16, 16 * i:16 * i + 16], np.eye(16))
    assert np.all(np.triu(L, 1)[np.triu(np.ones_like(L), 16).astype(bool)] == 0)


def test_oracle_feedback_targets_identity_for_any_quantizer():
    rng = np.random.default_rng(2)
    H = _spd(64, 2)
    L, _ = oldlq.block_ldl(H, 16)
    L0 = oldlq.strictly_block_lower(L)
    W = rng.standard_normal((64, 32))
    Q, T = oldlq.ldlq(W, L0, lambda t, _b: np.round(t * 2.0) / 2.0)
    assert np.allclose(T - Q, (np.eye(64) + L0.T) @ (W - Q), atol=1e-12)
    assert np.allclose(T, oldlq.feedback_targets(W, L0, Q), atol=1e-12)
    # a planted sign error in the feedback is visible
    assert not np.allclose(T, W - L0.T @ (W - Q), atol=1e-6)


def test_backend_block_ldl_matches_oracle_on_cpu():
    H = torch.from_numpy(_spd(256, 3)).float()
    L, H_cpu = be.block_ldl(H.clone(), 16, {"sigma_reg": 0.025}, False)
    L_ref, _ = oldlq.block_ldl(H.double().numpy(), 16)
    assert np.allclose(L.double().numpy(), L_ref, rtol=1e-4, atol=1e-4)
    assert torch.equal(H_cpu, H)


def test_backend_block_ldl_retries_indefinite_hessian():
    # reference failure handling (exl3_encoder_backend.py:331-351)
    h = _spd(64, 4)
    h -= (np.linalg.eigvalsh(h)[0] + 0.01) * np.eye(64)  # smallest eigenvalue -0.01
    H = torch.from_numpy(h).float()
    L, H_used = be.block_ldl(H.clone(), 16, {"sigma_reg": 0.025}, False)
    assert torch.isfinite(L).all()
    assert float(H_used[0, 0]) > float(H[0, 0])  # damping was added


def test_backend_block_ldl_factors_in_float64_without_the_fp32_retry():
    """The factorisation runs in float64: a Hessian whose FP32 Cholesky fails
    but whose float64 one succeeds (rank 16 of 64 plus 2e-7 relative
    damping) is factored as given, with no extra damping.  The reference's
    FP32 factorisation would have retried with 2 sigma_reg mean(diag)
    (qsrt/exl3_encoder_backend.py:331-351); the retry here fires only for a
    matrix that is indefinite in float64 (previous test)."""

    g = torch.Generator().manual_seed(5)
    A = torch.randn(64, 16, generator=g, dtype=torch.float64)
    H64 = A @ A.T
    H = (H64 + 2e-7 * H64.diagonal().mean() * torch.eye(64, dtype=torch.float64)).float()
    assert int(torch.linalg.cholesky_ex(H)[1]) > 0  # FP32 Cholesky fails ...
    assert int(torch.linalg.cholesky_ex(H.double())[1]) == 0  # ... float64 succeeds
    L, H_used = be.block_ldl(H.clone(), 16, {"sigma_reg": 0.025}, False)
    assert torch.equal(H_used, H)  # no damping was added
    L_ref, _ = oldlq.block_ldl(H.double().numpy(), 16)
    assert np.allclose(L.double().numpy(), L_ref, rtol=1e-3, atol=1e-3)


def test_backend_hessian_finalisation_matches_oracle_congruence():
    k = 256
    H = torch.from_numpy(_spd(k, 5)).float()
    shared = make_shared_h(k, torch.device("cpu"), H)
    qa = {"seed": 1_000_002, "sigma_reg": 0.01}
    q_fallback, Hf, L, su, diag = be.finalize_capture_H(shared, qa, False)
    assert not q_fallback
    damped = H.double().numpy() + 0.01 * np.mean(np.diag(H.double().numpy())) * np.eye(k)
    want = oldlq.congruence(damped, su.numpy())
    assert np.allclose(Hf.double().numpy(), want, rtol=1e-4, atol=1e-5)
    L_ref, _ = oldlq.block_ldl(want, 16)
    L0 = oldlq.strictly_block_lower(L_ref)
    np.fill_diagonal(L0, 0.0)
    assert np.allclose(L.double().numpy(), L0, atol=2e-3)
    # seeds: CPU seeded_normal == manual_seed + randn (reference tests/test_qsrt_encoder.py:32-46)
    ref = torch.randn(k, generator=torch.Generator().manual_seed(1_000_002))
    assert torch.equal(su.flatten(), (ref.sign() + 1e-5).sign())


def test_backend_regularize_matches_oracle_with_fixed_scale():
    rng = np.random.default_rng(6)
    W = (rng.standard_t(5, size=(256, 512)) * 0.02).astype(np.float32)
    su = torch.from_numpy(np.sign(rng.standard_normal((256, 1))).astype(np.float32))
    sv = torch.from_numpy(np.sign(rng.standard_normal((1, 512))).astype(np.float32))
    qa = {"apply_out_scales": False, "g_scale_override": 0.8}
    w = torch.from_numpy(W.copy())
    _, w_r, g, su_r, sv_r = be.regularize(w, su.clone(), sv.clone(), qa, False, None, None)
    W_ref, su_ref, sv_ref = oldlq.regularize(W, su.numpy(), sv.numpy(), 0.8)
    assert g == 0.8
    assert w_r.dtype == torch.float64 and su_r.dtype == torch.float64
    # float64 on both sides: the two differ only in the order of the rotations' sums
    assert np.allclose(w_r.numpy(), W_ref, rtol=1e-12, atol=1e-13 * np.abs(W_ref).max())
    assert np.allclose(su_r.numpy(), su_ref, rtol=1e-12)
    assert np.array_equal(sv_r.numpy(), sv_ref)
    # the caller's FP32 weight ends as the FP32 rounding of the regularised weight
    assert torch.equal(w, w_r.float())
    assert qa["zeros"] is False


def test_fallback_hessian_marks_q_fallback():
    shared = make_shared_h(128, torch.device("cpu"), torch.zeros(128, 128))
    shared["count"] = 0
    q_fallback, *_ = be.finalize_capture_H(shared, {"seed": 3}, False)
    assert q_fallback and shared["L"] is None


def _block_had_signs(k, signs):
    """Dense T = (I_{k/128} (x) H_128 / sqrt(128)) D_signs, built with scipy's Sylvester Hadamard."""

    import scipy.linalg

    h = scipy.linalg.hadamard(128) / np.sqrt(128.0)
    return np.kron(np.eye(k // 128), h) @ np.diag(np.asarray(signs, dtype=np.float64).reshape(-1))


def test_oracle_congruence_pinned_by_dense_construction_and_invariants():
    # congruence is an orthogonal similarity T H T^T: a one-sided sign, a transposed or unnormalised
    # Hadamard, or a row-only transform fails the dense product, the spectrum or the round trip
    k = 256
    rng = np.random.default_rng(11)
    H = _spd(k, 12)
    s = np.sign(rng.standard_normal(k))
    T = _block_had_signs(k, s)
    got = oldlq.congruence(H, s)
    assert np.allclose(got, T @ H @ T.T, atol=1e-12)
    assert np.allclose(got, got.T, atol=1e-12)
    assert np.allclose(np.linalg.eigvalsh(got), np.linalg.eigvalsh(H), atol=1e-10)
    assert np.allclose(oldlq.congruence(np.eye(k), s), np.eye(k), atol=1e-12)
    ones = np.ones(k)
    assert np.allclose(oldlq.congruence(oldlq.congruence(H, ones), ones), H, atol=1e-12)  # H_128 is an involution


def test_oracle_regularize_pinned_by_inverse_and_closed_forms():
    # W' = g H_L diag(1/su') (W diag(1/sv) H_R) with su' = su rms / -c; the decoder's inverse
    # W = diag(sv)-scaled ((su_out * (H_L^T W')) H_R^T) must return W, each 128-row block of W' has RMS g c
    # (H_L is orthogonal within the block), and su_out = -su rms_rows(W) / (c g) with rms_rows unchanged by
    # the orthogonal H_R
    k, n, g = 256, 384, 0.8
    rng = np.random.default_rng(13)
    W = rng.standard_t(5, size=(k, n)) * 0.02
    W[7] = 0.0  # a zero row takes the reference's rms = 0.1 substitute
    su = np.sign(rng.standard_normal(k))
    sv = np.sign(rng.standard_normal(n))
    Wr, su_out, sv_out = oldlq.regularize(W, su, sv, g)
    c = oldlq.CODEBOOK_SCALE
    TL = _block_had_signs(k, np.ones(k))
    TR = _block_had_signs(n, np.ones(n))
    back = ((su_out.reshape(k, 1) * (TL.T @ Wr)) @ TR.T) * sv_out.reshape(1, n)
    assert np.allclose(back, W, atol=1e-12)
    rms = np.sqrt((W * W).mean(axis=1))
    rms[7] = 0.1
    assert np.allclose(su_out.reshape(-1), (-su * rms / c + 1e-10) / g, rtol=1e-12)
    nonzero = np.ones(k, dtype=bool)
    nonzero[7] = False
    for b in range(k // 128):
        rows = slice(128 * b, 128 * b + 128)
        if nonzero[rows].all():
            assert np.isclose(np.sqrt(np.mean(Wr[rows] ** 2)), g * c, rtol=1e-8)
    assert np.array_equal(sv_out.reshape(-1), sv)


def test_oracle_out_scale_policy_closed_form_share():
    # n // 50 = 10 entries of a, 490 of b: the top-2% share of the root diagonal is
    # 10 sqrt(a) / (10 sqrt(a) + 490 sqrt(b)); scaling the diagonal leaves it unchanged, the order of the
    # entries must not matter (a planted ascending sort reads the smallest 2% and flips both cases), and a
    # forced value or a fallback encode overrides the rule
    n, b = 500, 1.0
    for share, expect in ((0.149, True), (0.151, False)):
        ratio = share * 490.0 / (10.0 * (1.0 - share))  # sqrt(a) / sqrt(b)
        diag = np.full(n, b)
        diag[:10] = ratio ** 2 * b
        rng = np.random.default_rng(3)
        for d in (diag, rng.permutation(diag), 7.5 * diag):
            assert oldlq.out_scale_policy(d, None) is expect
            assert oldlq.out_scale_policy(d, not expect) is (not expect)
    assert oldlq.out_scale_policy(None, None) is True
    assert oldlq.out_scale_policy(None, False) is False
    assert oldlq.out_scale_policy(np.ones(n), None, q_fallback=True) is None


def test_oracle_regularize_output_scales_pinned_by_equal_column_rms():
    # with output scales, sv = sign * colRMS / mean(colRMS) + 1e-10, so every live column of W / sv has the
    # same RMS, mean(colRMS) -- not 1 (a missing mean normalisation fails) and not row-derived (a row RMS
    # fails); an all-zero column gets sv = 0 and stays zero; the decoder's inverse returns W
    k, n, g = 256, 384, 0.7
    rng = np.random.default_rng(17)
    W = rng.standard_t(5, size=(k, n)) * 0.02 * np.linspace(0.3, 3.0, n)[None, :]
    W[:, 11] = 0.0
    su = np.sign(rng.standard_normal(k))
    sv = np.sign(rng.standard_normal(n))
    Wr, su_out, sv_out = oldlq.regularize(W, su, sv, g, apply_out_scales=True)
    cols = np.sqrt((W * W).mean(axis=0))
    live = cols > 0
    assert sv_out.reshape(-1)[11] == 0.0
    assert np.array_equal(np.sign(sv_out.reshape(-1)[live]), sv[live])
    scaled = W[:, live] / sv_out.reshape(-1)[live]
    assert np.allclose(np.sqrt((scaled * scaled).mean(axis=0)), cols.mean(), rtol=1e-8)
    assert not np.isclose(cols.mean(), 1.0)
    TL = _block_had_signs(k, np.ones(k))
    TR = _block_had_signs(n, np.ones(n))
    back = ((su_out.reshape(k, 1) * (TL.T @ Wr)) @ TR.T) * sv_out.reshape(1, n)
    assert np.allclose(back, W, atol=1e-12)
    # without output scales the signs pass through, but the dead column's sv is still zeroed
    _, _, sv_plain = oldlq.regularize(W, su, sv, g)
    expect = sv.copy()
    expect[11] = 0.0
    assert np.array_equal(sv_plain.reshape(-1), expect)


def test_backend_out_scale_policy_matches_oracle():
    n = 500
    for share in (0.149, 0.151):
        ratio = share * 490.0 / (10.0 * (1.0 - share))
        diag = np.ones(n)
        diag[:10] = ratio ** 2
        d = torch.from_numpy(diag).float()
        for forced in (None, True, False):
            assert be._out_scale_policy(d, forced, False, False) == oldlq.out_scale_policy(diag, forced)
    assert be._out_scale_policy(None, None, False, False) is True
    assert be._out_scale_policy(torch.ones(n), None, True, False) is None


def test_backend_regularize_output_scales_matches_oracle_on_cpu():
    rng = np.random.default_rng(19)
    W = (rng.standard_t(5, size=(256, 384)) * 0.02).astype(np.float32)
    W[:, 5] = 0.0
    W[9, :] = 0.0
    su = torch.from_numpy(np.sign(rng.standard_normal((256, 1))).astype(np.float32))
    sv = torch.from_numpy(np.sign(rng.standard_normal((1, 384))).astype(np.float32))
    for apply in (True, False):
        qa = {"apply_out_scales": apply, "g_scale_override": 0.6}
        applied, w_r, _, su_r, sv_r = be.regularize(torch.from_numpy(W.copy()), su.clone(), sv.clone(), qa, False,
                                                    None, None)
        W_ref, su_ref, sv_ref = oldlq.regularize(W, su.numpy(), sv.numpy(), 0.6, apply_out_scales=apply)
        assert applied is apply
        assert np.allclose(w_r.numpy(), W_ref, rtol=1e-12, atol=1e-13 * np.abs(W_ref).max())
        assert np.allclose(su_r.numpy(), su_ref, rtol=1e-12)
        assert np.allclose(sv_r.numpy(), sv_ref, rtol=1e-14, atol=0)
