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
    assert np.allclose(w_r.double().numpy(), W_ref, rtol=1e-5, atol=1e-6 * np.abs(W_ref).max())
    assert np.allclose(su_r.double().numpy(), su_ref, rtol=1e-5)
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
