"""Covariance producers of the expert encode: the weighted covariance that
feeds H13 and H2 (reference ``qsrt/candidate_hessian.py:70-112``), identity
shrinkage of a low-support covariance by the Oracle Approximating Shrinkage
estimator, and the post-activation H2 of a decoded gate/up pair (reference
``qsrt/blockldlq_proof.py:89-99, 275-303``).

``weighted_covariance`` runs on the HIP FP32 matrix-core GEMM for device
tensors (exact FP32 products, FP32 accumulation).  Candidate-selection
policy (document splits, request masks, per-rate H2 ladders) belongs to the
callers, outside the encoder.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import gemm


def weighted_covariance(rows: torch.Tensor, weights: torch.Tensor, *, device: torch.device, chunk_rows: int = 256,
                        return_cpu: bool = True) -> tuple[torch.Tensor, float]:
    """``sum(w x x^T) / sum(w)`` as symmetric FP32 (reference
    candidate_hessian.py:70-112).  On a GPU device the sum runs on the FP32
    matrix cores in row chunks of at least 16384."""

    if rows.ndim != 2 or weights.ndim != 1 or rows.shape[0] != weights.shape[0]:
        raise ValueError("invalid covariance sample shapes")
    if not rows.shape[0] or not rows.shape[1]:
        raise ValueError("covariance samples must be nonempty")
    if chunk_rows <= 0:
        raise ValueError("chunk_rows must be positive")
    if not bool(torch.all(torch.isfinite(rows))) or not bool(torch.all(torch.isfinite(weights))):
        raise ValueError("covariance samples must be finite")
    if bool(torch.any(weights < 0)):
        raise ValueError("covariance weights must be nonnegative")
    device = torch.device(device)
    d = int(rows.shape[1])
    denominator = float(weights.double().sum())
    if not math.isfinite(denominator) or denominator <= 0:
        raise ValueError("covariance weights must have a positive finite sum")
    acc = torch.zeros((d, d), dtype=torch.float32, device=device)
    step = max(chunk_rows, 16384) if device.type == "cuda" else chunk_rows
    for begin in range(0, int(rows.shape[0]), step):
        x = rows[begin:begin + step].to(device=device, dtype=torch.float32)
        w = weights[begin:begin + step].to(device=device, dtype=torch.float32)
        gemm.addmm_tn_(acc, x.contiguous(), (x * w[:, None]).contiguous())
    cov = acc.div_(denominator)
    cov = ((cov + cov.T) * 0.5).contiguous()
    if return_cpu:
        cov = cov.cpu()
    if not bool(torch.all(torch.isfinite(cov))):
        raise ValueError("weighted covariance is non-finite")
    return cov, denominator


def oas_identity_shrinkage(local_covariance: torch.Tensor, weights: torch.Tensor, *,
                           max_local_alpha: float = 0.75) -> tuple[torch.Tensor, dict[str, float]]:
    """Shrink ``S`` (a weighted covariance of the rows behind ``weights``)
    toward its scaled identity ``F = tr(S)/p I``:  ``(1 - a) F + a S``.

    ``a = min(max_local_alpha, 1 - rho)`` with ``rho`` the Oracle
    Approximating Shrinkage intensity of Chen, Wiesel, Eldar and Hero
    (IEEE TSP 58(10), 2010) in the form scikit-learn implements,
    ``rho = min(1, (tr(S^2) + tr(S)^2) / ((n + 1) (tr(S^2) - tr(S)^2 / p)))``,
    with ``n`` the Kish effective sample size ``(sum w)^2 / sum w^2`` of the
    weights (reference ``qsrt/candidate_hessian.py:156-216``).  A spherical
    ``S`` (zero denominator) takes the identity target entirely."""

    cap = float(max_local_alpha)
    if not math.isfinite(cap) or not 0.0 <= cap <= 1.0:
        raise ValueError("max_local_alpha must be finite and in [0, 1]")
    if local_covariance.ndim != 2 or local_covariance.shape[0] != local_covariance.shape[1]:
        raise ValueError("local covariance must be square")
    if not bool(torch.all(torch.isfinite(local_covariance))):
        raise ValueError("local covariance must be finite")
    if weights.ndim != 1 or not weights.numel():
        raise ValueError("weights must be a nonempty vector")
    w = weights.double()
    if not bool(torch.all(torch.isfinite(w))) or bool(torch.any(w < 0)) or float(w.square().sum()) <= 0:
        raise ValueError("weights must be finite, nonnegative and not all zero")
    n_eff = float(w.sum().square() / w.square().sum())
    S = local_covariance.double()
    p = S.shape[0]
    tr = float(torch.trace(S))
    if tr <= 0:
        raise ValueError("local covariance trace must be positive")
    tr_s2 = float((S * S).sum())  # tr(S^2) of a symmetric S
    den = (n_eff + 1.0) * (tr_s2 - tr * tr / p)
    rho = 1.0 if den <= 0 else min(1.0, max(0.0, (tr_s2 + tr * tr) / den))
    alpha = min(cap, 1.0 - rho)
    target = torch.eye(p, dtype=torch.float64, device=S.device) * (tr / p)
    shrunk = (1.0 - alpha) * target + alpha * S
    shrunk = ((shrunk + shrunk.T) * 0.5).float().contiguous()
    return shrunk, {"effective_sample_size": n_eff, "oas_shrinkage": rho, "local_alpha": alpha,
                    "max_local_alpha": cap, "identity_scale": tr / p}


def situ_middle(inputs: torch.Tensor, gate_weight: torch.Tensor, up_weight: torch.Tensor) -> torch.Tensor:
    """Post-SiTU rows ``silu(x W_g^T) * (x W_u^T)`` of a decoded gate/up pair
    (reference blockldlq_proof.py:275-289)."""

    for t, name in ((inputs, "inputs"), (gate_weight, "gate_weight"), (up_weight, "up_weight")):
        if t.ndim != 2 or not bool(torch.all(torch.isfinite(t))):
            raise ValueError(f"{name} must be a finite matrix")
    if gate_weight.shape != up_weight.shape or gate_weight.shape[1] != inputs.shape[1]:
        raise ValueError("gate/up shapes do not align with inputs")
    return (F.silu(F.linear(inputs, gate_weight)) * F.linear(inputs, up_weight)).contiguous()


def weighted_gram(rows: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """``sum w x x^T / sum w`` in FP64, symmetrised (reference
    blockldlq_proof.py:89-99; the proof-grade counterpart of
    :func:`weighted_covariance`)."""

    if rows.ndim != 2 or not bool(torch.all(torch.isfinite(rows))):
        raise ValueError("rows must be a finite matrix")
    if weights.ndim != 1 or weights.shape[0] != rows.shape[0]:
        raise ValueError("weights must align with rows")
    if not bool(torch.all(torch.isfinite(weights))) or bool(torch.any(weights < 0)):
        raise ValueError("weights must be finite and nonnegative")
    w = weights.to(torch.float64)
    den = w.sum()
    if den <= 0:
        raise ValueError("weights must have positive mass")
    r = rows.to(torch.float64)
    out = r.T @ (r * w[:, None]) / den
    return ((out + out.T) * 0.5).contiguous()


def conditional_h2(inputs: torch.Tensor, gates: torch.Tensor, gate_weight: torch.Tensor, up_weight: torch.Tensor):
    """Decoded upstream rows and their gate-square covariance (reference
    blockldlq_proof.py:292-303)."""

    if gates.ndim != 1 or gates.shape[0] != inputs.shape[0]:
        raise ValueError("gates must align with inputs")
    middle = situ_middle(inputs, gate_weight, up_weight)
    return middle, weighted_gram(middle, gates.square())
