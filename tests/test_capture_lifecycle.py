"""Life cycle of a captured Hessian record (reference
``qsrt/exl3_encoder_backend.py:2163-2243``) on the CPU path: one-shot
finalisation, the two-stage conditioned preparation, the record captured
without a dense matrix, and the refusals of every out-of-order call.  The
finalised metric is checked against the congruence built from an explicit
Sylvester-Hadamard matrix (``scipy.linalg.hadamard``) and the float64 factor
against ``L D L^T`` of that metric."""

from __future__ import annotations

import pytest
import scipy.linalg
import torch

from qsrt_amd import exl3_encoder_backend as be

K = 256


def _record(count: int = 512, seed: int = 0) -> dict:
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(count, K, generator=g) * torch.linspace(0.2, 3.0, K)
    return {"H": (X.T @ X).float(), "count": count, "finalized": False, "device": "cpu"}


def _metric(H_sum: torch.Tensor, count: int, su: torch.Tensor, sigma_reg: float = 0.025) -> torch.Tensor:
    H = H_sum.double() / count
    H = H + sigma_reg * H.diagonal().mean() * torch.eye(K, dtype=torch.float64)
    had = torch.tensor(scipy.linalg.hadamard(128), dtype=torch.float64) / 128 ** 0.5
    R = torch.block_diag(had, had) @ torch.diag(su.double().flatten())
    return R @ H @ R.T


def _check_factor(L: torch.Tensor, H: torch.Tensor):
    # unit block-lower with its scalar diagonal zeroed: restore it, then L D L^T must give back the metric
    assert L.dtype == torch.float64 and torch.equal(L.diagonal(), torch.zeros(K, dtype=torch.float64))
    assert torch.equal(torch.triu(L, 1), torch.zeros_like(L))
    U = L + torch.eye(K, dtype=torch.float64)
    D = torch.linalg.solve(U, torch.linalg.solve(U, H.double()).T).T
    blocks = torch.block_diag(*[D[i:i + 16, i:i + 16] for i in range(0, K, 16)])
    assert (D - blocks).abs().max().item() <= 1e-9 * H.abs().max().item()


def test_one_shot_finalization_and_cached_result():
    rec = _record()
    H_sum = rec["H"].clone()
    q_fallback, H, L, su, diag = be.finalize_capture_H(rec, {"seed": 7}, False)
    assert q_fallback is False and rec["finalized"] and "_H64" not in rec
    assert su.shape == (K, 1) and torch.equal(su.abs(), torch.ones_like(su))
    ref = _metric(H_sum, 512, su)
    assert H.dtype == torch.float32
    assert (H.double() - ref).abs().max().item() <= 1e-6 * ref.abs().max().item()
    _check_factor(L, ref)
    again = be.finalize_capture_H(rec, {"seed": 7}, False)
    assert all(a is b for a, b in zip(again, (q_fallback, H, L, su, diag)))
    with pytest.raises(ValueError, match="already finalized"):
        be.prepare_capture_H_for_conditioning(rec, {}, False)


def test_two_stage_conditioned_preparation():
    rec = _record(seed=1)
    H_sum = rec["H"].clone()
    q_fallback, H, su, diag = be.prepare_capture_H_for_conditioning(rec, {"seed": 3}, False)
    assert q_fallback is False and rec["_conditioning_pending"] and not rec["finalized"]
    assert torch.equal(diag, H.diagonal())
    with pytest.raises(ValueError, match="already pending"):
        be.prepare_capture_H_for_conditioning(rec, {}, False)
    with pytest.raises(ValueError, match="ordinary finalization"):
        be.finalize_capture_H(rec, {}, False)
    flip = torch.ones((K, 1))
    flip[::3] = -1.0
    su2 = su * flip  # the caller's final conditioning replaces the drawn signs
    out = be.finalize_capture_H_with_conditioning(rec, su2, {}, False)
    assert "_conditioning_pending" not in rec and rec["finalized"]
    ref = _metric(H_sum, 512, su2)
    assert (out[1].double() - ref).abs().max().item() <= 1e-6 * ref.abs().max().item()
    _check_factor(out[2], ref)
    assert out[3] is su2
    with pytest.raises(ValueError, match="was not started"):
        be.finalize_capture_H_with_conditioning(rec, su2, {}, False)
    assert be.finalize_capture_H(rec, {}, False)[2] is out[2]


def test_record_without_a_dense_matrix():
    rec = {"H": torch.empty((K, K), device="meta"), "count": 0, "finalized": False, "device": "cpu"}
    with pytest.raises(ValueError, match="materialized dense"):
        be.prepare_capture_H_for_conditioning(rec, {}, False)
    q_fallback, H, L, su, diag = be.finalize_capture_H(rec, {"seed": 5}, False)
    assert (q_fallback, H, L, diag) == (True, None, None, None)
    assert rec["finalized"] and rec["q_fallback"] and rec["L"] is None and rec["su"] is su
    assert su.shape == (K, 1) and torch.equal(su.abs(), torch.ones_like(su))
    assert torch.equal(su, be._input_signs(K, torch.device("cpu"), 5))


def test_empty_capture_is_a_fallback_without_factor():
    rec = {"H": torch.zeros((K, K)), "count": 0, "finalized": False, "device": "cpu"}
    q_fallback, H, L, su, _ = be.finalize_capture_H(rec, {}, False)
    assert q_fallback is True and L is None and torch.equal(H, torch.zeros((K, K)))


def test_parked_matrix_is_brought_home_once():
    rec = _record(seed=2)
    rec["H_swap_device"] = "cpu"
    be.finalize_capture_H(rec, {}, False)
    assert "H_swap_device" not in rec
