"""Covariance producers of the expert encode and the support-aware expert
Hessian policy.

* ``weighted_covariance`` -- the weighted covariance that feeds H13 and H2
  (reference ``qsrt/candidate_hessian.py:70-112``), on the HIP FP32
  matrix-core GEMM for device tensors;
* ``shrink_covariance``, ``weighted_effective_sample_size`` and the OAS
  identity shrinkage ``oas_identity_shrinkage`` (the reference's
  ``adaptive_identity_shrinkage``, both names exported)
  (``candidate_hessian.py:115-216``);
* ``build_expert_hessians`` -- H13 as a gate-square weighted local covariance
  shrunk toward the layer's global H13, H2 as the OAS-shrunk local
  covariance of the expert's post-activation rows
  (``qsrt/qsrt_candidates.py:534-620``), and ``conditional_h2_by_rate`` -- one
  such H2 per upstream rate candidate, from the rows its decoded gate/up
  reconstructions produce (``qsrt/pack/qsrt_candidates.py:407-461``);
* ``situ_middle``/``weighted_gram``/``conditional_h2`` -- the post-activation
  H2 of a decoded gate/up pair (``qsrt/blockldlq_proof.py:89-99, 275-303``).

The policy constants (``PHASE1_H13_EXPERT_LOCAL_ALPHA`` etc.) live with the
mode ladder in ``qsrt_amd.qsrt``.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import gemm
from .qsrt import PHASE1_H13_EXPERT_LOCAL_ALPHA, PHASE1_H2_EXPERT_LOCAL_ALPHA, PHASE1_H2_SHRINKAGE_POLICY


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


def shrink_covariance(global_covariance: torch.Tensor, local_covariance: torch.Tensor, alpha: float) -> torch.Tensor:
    """``(1 - alpha) global + alpha local``, symmetrised, FP32 (reference
    candidate_hessian.py:115-138): a low-support local covariance pulled
    toward a prior."""

    alpha = float(alpha)
    if not math.isfinite(alpha) or not 0.0 <= alpha <= 1.0:
        raise ValueError("alpha must be finite and in [0, 1]")
    if (global_covariance.ndim != 2 or global_covariance.shape[0] != global_covariance.shape[1]
            or local_covariance.shape != global_covariance.shape):
        raise ValueError("global and local covariances must be equal-size squares")
    if not bool(torch.all(torch.isfinite(global_covariance))) or not bool(torch.all(torch.isfinite(local_covariance))):
        raise ValueError("covariances must be finite")
    blended = torch.lerp(global_covariance.float(), local_covariance.to(global_covariance.device).float(), alpha)
    return ((blended + blended.T) * 0.5).contiguous()


def weighted_effective_sample_size(weights: torch.Tensor) -> float:
    """Kish effective sample size ``(sum w)^2 / sum w^2`` of nonnegative row
    weights (reference candidate_hessian.py:141-153)."""

    if weights.ndim != 1 or not weights.numel():
        raise ValueError("weights must be a nonempty vector")
    if not bool(torch.all(torch.isfinite(weights))) or bool(torch.any(weights < 0)):
        raise ValueError("weights must be finite and nonnegative")
    w = weights.double()
    total, square = w.sum(), w.square().sum()
    if total <= 0 or square <= 0:
        raise ValueError("weights must have positive effective support")
    return float(total.square() / square)


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
    n_eff = weighted_effective_sample_size(weights)
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


adaptive_identity_shrinkage = oas_identity_shrinkage  # the reference's name (candidate_hessian.py:156)


def build_expert_hessians(inputs: torch.Tensor, gates: torch.Tensor, source_middle: torch.Tensor, *,
                          global_h13: torch.Tensor, global_h2: torch.Tensor, device,
                          h13_alpha: float = PHASE1_H13_EXPERT_LOCAL_ALPHA, h2_alpha: float | None = None,
                          chunk_rows: int = 256) -> tuple[torch.Tensor, torch.Tensor, dict]:
    """H13 and a support-aware post-activation H2 of one expert (reference
    qsrt/qsrt_candidates.py:534-620).  Rows are weighted by their gate
    squared.  H13: the local weighted input covariance shrunk toward
    ``global_h13`` with ``h13_alpha`` (at 0, the production default, the
    global H13 itself).  H2: the local weighted covariance of
    ``source_middle`` shrunk toward its own trace-scaled identity, with the
    OAS weight capped at ``PHASE1_H2_EXPERT_LOCAL_ALPHA`` (or a fixed
    ``h2_alpha``); ``global_h2`` only fixes the dimension -- post-activation
    coordinates have no meaning shared across experts.  Covariances run on
    the FP32 matrix cores.  Returns ``(h13, h2, evidence)``."""

    if inputs.ndim != 2 or gates.ndim != 1 or inputs.shape[0] != gates.shape[0]:
        raise ValueError("invalid expert input covariance samples")
    if source_middle.ndim != 2 or source_middle.shape[0] != inputs.shape[0]:
        raise ValueError("source middle rows do not match expert inputs")
    device = torch.device(device)
    global_h13 = global_h13.to(device=device, dtype=torch.float32)
    if tuple(global_h2.shape) != (source_middle.shape[1], source_middle.shape[1]):
        raise ValueError("global H2 dimension does not match source middle rows")
    weights = gates.float().square()
    if float(h13_alpha) == 0.0:
        h13 = global_h13
        h13_weight = float(weights.double().sum())
    else:
        local_h13, h13_weight = weighted_covariance(inputs, weights, device=device, chunk_rows=chunk_rows,
                                                    return_cpu=False)
        h13 = shrink_covariance(global_h13, local_h13, h13_alpha)
    local_h2, h2_weight = weighted_covariance(source_middle, weights, device=device, chunk_rows=chunk_rows,
                                              return_cpu=False)
    if not math.isclose(h13_weight, h2_weight, rel_tol=1e-9, abs_tol=1e-12):
        raise ValueError("H13 and H2 expert covariance weights differ")
    if h2_alpha is None:
        h2, shrink = oas_identity_shrinkage(local_h2, weights, max_local_alpha=PHASE1_H2_EXPERT_LOCAL_ALPHA)
        h2_evidence = {"h2_shrinkage_policy": PHASE1_H2_SHRINKAGE_POLICY, "h2_local_alpha": shrink["local_alpha"],
                       "h2_local_alpha_cap": shrink["max_local_alpha"],
                       "h2_effective_sample_size": shrink["effective_sample_size"],
                       "h2_oas_shrinkage": shrink["oas_shrinkage"], "h2_identity_scale": shrink["identity_scale"]}
    else:
        scale = float(torch.trace(local_h2) / local_h2.shape[0])
        prior = torch.eye(local_h2.shape[0], dtype=torch.float32, device=device) * scale
        h2 = shrink_covariance(prior, local_h2, h2_alpha)
        h2_evidence = {"h2_shrinkage_policy": "fixed_alpha_scaled_identity", "h2_local_alpha": float(h2_alpha),
                       "h2_local_alpha_cap": float(h2_alpha), "h2_identity_scale": scale}
    return h13, h2, {"gate_square_sum": h13_weight, "h13_local_alpha": float(h13_alpha), **h2_evidence}


def conditional_h2_by_rate(inputs: torch.Tensor, gates: torch.Tensor, fit_mask: torch.Tensor,
                           reconstructions: dict, *, global_h13: torch.Tensor, global_h2: torch.Tensor, device,
                           hessian_policy: str = "support_aware", have_local_support: bool = True,
                           activation=None) -> tuple[dict, dict]:
    """One down-projection H2 per upstream rate candidate (reference
    qsrt/pack/qsrt_candidates.py:407-461): for each rate key, the candidate's
    decoded gate and up reconstructions (``reconstructions[key] = (w1, w3)``,
    ``[intermediate, hidden]``) turn the fit rows into post-activation rows,
    and :func:`build_expert_hessians` turns those into that rate's H2.  Under
    the ``identity`` policy, or without local support, every rate gets the
    identity.  All candidates' forward products run as one batched product.
    Returns ``(h2 by rate, evidence by "R<key>")``."""

    from .qsrt_coupled import situ

    act = situ if activation is None else activation
    device = torch.device(device)
    width = int(global_h2.shape[0])
    h2_by_rate, evidence = {}, {}
    if hessian_policy == "identity" or not have_local_support:
        identity = torch.eye(width, dtype=torch.float32, device=device)
        for key in reconstructions:
            h2_by_rate[int(key)] = identity
            evidence[f"R{int(key)}"] = {"h2_shrinkage_policy": "identity_fallback", "h2_local_alpha": 0.0,
                                        "h2_effective_sample_size": 0.0, "h2_identity_scale": 1.0}
        return h2_by_rate, evidence
    if hessian_policy != "support_aware":
        raise ValueError("hessian_policy must be 'support_aware' or 'identity'")
    mask = fit_mask.to(device=device, dtype=torch.bool)
    x = inputs.to(device=device, dtype=torch.float32)[mask]
    g = gates.to(device=device)[mask]
    keys = [int(k) for k in reconstructions]
    # [rates, 2 * intermediate, hidden]: gate rows then up rows of each candidate, one batched product
    stacked = torch.stack([torch.cat((reconstructions[k][0], reconstructions[k][1])).to(device=device,
                                                                                     dtype=torch.float32)
                           for k in keys])
    pre = torch.matmul(x.unsqueeze(0), stacked.transpose(1, 2).contiguous())
    for i, key in enumerate(keys):
        middle = act(pre[i, :, :width], pre[i, :, width:]).contiguous()
        _, h2, ev = build_expert_hessians(x, g, middle, global_h13=global_h13, global_h2=global_h2, device=device)
        h2_by_rate[key] = h2
        evidence[f"R{key}"] = ev
    return h2_by_rate, evidence


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
