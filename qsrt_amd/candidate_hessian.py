"""Covariance producers of the expert encode (mirrors
``qsrt/candidate_hessian.py``, ``qsrt/qsrt_candidates.py:534-618`` and the
post-SiTU helpers of ``qsrt/blockldlq_proof.py:86-99, 275-303``).

The weighted covariance ``sum_i w_i x_i x_i^T / sum_i w_i`` that feeds H13
and H2 runs on the HIP FP32 matrix-core GEMM for device tensors (exact FP32
products, FP32 accumulation); the shrinkage and diagnostics are small host
or torch reductions.
"""

from __future__ import annotations

import hashlib
import math
from collections.abc import Mapping, Sequence

import torch
import torch.nn.functional as F

from . import gemm
from .qsrt_coupled import situ

# Phase-1 policy constants (reference qsrt/qsrt.py:228-233)
PHASE1_H13_EXPERT_LOCAL_ALPHA = 0.0
PHASE1_H2_EXPERT_LOCAL_ALPHA = 0.75
PHASE1_H2_SHRINKAGE_POLICY = "weighted_oas_scaled_identity"
# Candidate-encode Hessian policies (reference qsrt/pack/qsrt_candidates.py:67-68)
HESSIAN_POLICIES = ("captured_blend", "identity")


def partition_documents(documents: Sequence[str], *, modulus: int, confirmation_index: int):
    """Deterministic fit / confirmation split by an 8-byte BLAKE2b hash of
    each document (reference candidate_hessian.py:12-31)."""

    if modulus < 2:
        raise ValueError("document partition modulus must be at least 2")
    if not 0 <= confirmation_index < modulus:
        raise ValueError("confirmation index must be in the partition modulus")
    if not documents or len(set(documents)) != len(documents):
        raise ValueError("documents must be a nonempty unique sequence")
    fit, confirmation = [], []
    for doc in documents:
        bucket = int.from_bytes(hashlib.blake2b(doc.encode(), digest_size=8).digest(), "little") % modulus
        (confirmation if bucket == confirmation_index else fit).append(doc)
    if not fit or not confirmation:
        raise ValueError("document partition produced an empty side")
    return fit, confirmation


def subset_request_documents(request_documents: Mapping[int, str], documents: Sequence[str]) -> dict[int, str]:
    selected = set(documents)
    if not selected:
        raise ValueError("document subset must be nonempty")
    out = {int(r): d for r, d in request_documents.items() if d in selected}
    missing = selected - set(out.values())
    if missing:
        raise ValueError(f"documents lack request epochs: {sorted(missing)[:8]}")
    return out


def request_mask(observations: torch.Tensor, request_documents: Mapping[int, str]) -> torch.Tensor:
    """Capture rows whose request epoch (bits 32..63) is in the subset."""

    if observations.ndim != 1:
        raise ValueError("observations must be one-dimensional")
    if not request_documents:
        raise ValueError("request document mapping must be nonempty")
    steps = torch.bitwise_right_shift(observations, 32)
    return torch.isin(steps, torch.tensor(sorted(request_documents), dtype=steps.dtype, device=steps.device))


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
    """Convex shrinkage of a low-support local covariance toward a global one."""

    alpha = float(alpha)
    if not math.isfinite(alpha) or not 0.0 <= alpha <= 1.0:
        raise ValueError("alpha must be finite and in [0, 1]")
    if (global_covariance.ndim != 2 or global_covariance.shape[0] != global_covariance.shape[1]
            or local_covariance.shape != global_covariance.shape):
        raise ValueError("global and local covariances must be equal-size squares")
    if not bool(torch.all(torch.isfinite(global_covariance))) or not bool(torch.all(torch.isfinite(local_covariance))):
        raise ValueError("covariances must be finite")
    blended = torch.lerp(global_covariance.float(), local_covariance.float(), alpha)
    return ((blended + blended.T) * 0.5).contiguous()


def weighted_effective_sample_size(weights: torch.Tensor) -> float:
    """Kish effective sample size ``(sum w)^2 / sum w^2``."""

    if weights.ndim != 1 or not weights.numel():
        raise ValueError("weights must be a nonempty vector")
    if not bool(torch.all(torch.isfinite(weights))) or bool(torch.any(weights < 0)):
        raise ValueError("weights must be finite and nonnegative")
    w = weights.double()
    total, squares = w.sum(), w.square().sum()
    if total <= 0 or squares <= 0:
        raise ValueError("weights must have positive effective support")
    return float(total.square() / squares)


def adaptive_identity_shrinkage(local_covariance: torch.Tensor, weights: torch.Tensor, *,
                                max_local_alpha: float = 0.75) -> tuple[torch.Tensor, dict[str, float]]:
    """Oracle Approximating Shrinkage toward ``trace/d * I`` with the Kish
    effective sample size in place of the row count, the local weight capped
    at ``max_local_alpha`` (reference candidate_hessian.py:156-216)."""

    max_local_alpha = float(max_local_alpha)
    if not math.isfinite(max_local_alpha) or not 0.0 <= max_local_alpha <= 1.0:
        raise ValueError("max_local_alpha must be finite and in [0, 1]")
    if local_covariance.ndim != 2 or local_covariance.shape[0] != local_covariance.shape[1]:
        raise ValueError("local covariance must be square")
    if not bool(torch.all(torch.isfinite(local_covariance))):
        raise ValueError("local covariance must be finite")
    n_eff = weighted_effective_sample_size(weights)
    d = int(local_covariance.shape[0])
    local64 = local_covariance.double()
    trace = torch.trace(local64)
    if trace <= 0:
        raise ValueError("local covariance trace must be positive")
    mu = trace / d
    mean_square = local64.square().mean()
    denominator = (n_eff + 1.0) * (mean_square - mu.square() / d)
    oas = 1.0 if denominator <= 0 else min(1.0, max(0.0, float((mean_square + mu.square()) / denominator)))
    local_alpha = min(max_local_alpha, 1.0 - oas)
    scale = float(mu)
    target = torch.eye(d, dtype=torch.float32, device=local_covariance.device).mul_(scale)
    return shrink_covariance(target, local_covariance, local_alpha), {
        "effective_sample_size": n_eff, "oas_shrinkage": oas, "local_alpha": local_alpha,
        "max_local_alpha": max_local_alpha, "identity_scale": scale}


def covariance_comparison(reference: torch.Tensor, candidate: torch.Tensor) -> dict[str, float]:
    """Scale and shape diagnostics of two covariances."""

    if reference.ndim != 2 or reference.shape[0] != reference.shape[1]:
        raise ValueError("reference covariance must be square")
    if candidate.shape != reference.shape:
        raise ValueError("candidate covariance shape differs")
    reference, candidate = reference.float(), candidate.float()
    if not bool(torch.all(torch.isfinite(reference))) or not bool(torch.all(torch.isfinite(candidate))):
        raise ValueError("covariances must be finite")
    ref_norm = torch.linalg.vector_norm(reference.double())
    rd, cd = torch.diagonal(reference).double(), torch.diagonal(candidate).double()
    diag_den = torch.linalg.vector_norm(rd) * torch.linalg.vector_norm(cd)
    trace = torch.trace(reference.double())
    return {
        "relative_frobenius_difference": float(torch.linalg.vector_norm((candidate - reference).double()) / ref_norm)
        if ref_norm > 0 else math.inf,
        "trace_ratio": float(torch.trace(candidate.double()) / trace) if trace != 0 else math.inf,
        "diagonal_cosine_similarity": float(torch.dot(rd, cd) / diag_den) if diag_den > 0 else 0.0,
        "candidate_symmetry_max_abs": float((candidate - candidate.T).abs().max()),
    }


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


def build_expert_hessians(inputs: torch.Tensor, gates: torch.Tensor, source_middle: torch.Tensor, *,
                          global_h13: torch.Tensor, global_h2: torch.Tensor, device: torch.device,
                          h13_alpha: float = PHASE1_H13_EXPERT_LOCAL_ALPHA, h2_alpha: float | None = None,
                          chunk_rows: int = 256):
    """H13 and a support-aware post-SiTU H2 of one expert (reference
    qsrt_candidates.py:534-618): gate-square weights, H13 shrunk toward the
    layer-global H13 by ``h13_alpha``, H2 the expert-local covariance under
    weighted OAS shrinkage toward its scaled identity (``global_h2`` only
    fixes the dimension)."""

    if inputs.ndim != 2 or inputs.shape[0] != gates.shape[0]:
        raise ValueError("invalid expert input covariance samples")
    if source_middle.ndim != 2 or source_middle.shape[0] != inputs.shape[0]:
        raise ValueError("source middle rows do not match expert inputs")
    global_h13 = global_h13.to(device=device, dtype=torch.float32)
    if global_h2.shape != (source_middle.shape[1], source_middle.shape[1]):
        raise ValueError("global H2 dimension does not match source middle rows")
    weights = gates.float().square()
    if h13_alpha == 0.0:
        h13, h13_weight = global_h13, float(weights.double().sum())
    else:
        local_h13, h13_weight = weighted_covariance(inputs, weights, device=device, chunk_rows=chunk_rows,
                                                    return_cpu=False)
        h13 = shrink_covariance(global_h13, local_h13, h13_alpha)
    local_h2, h2_weight = weighted_covariance(source_middle, weights, device=device, chunk_rows=chunk_rows,
                                              return_cpu=False)
    if not math.isclose(h13_weight, h2_weight, rel_tol=1e-9, abs_tol=1e-12):
        raise ValueError("H13 and H2 expert covariance weights differ")
    if h2_alpha is None:
        h2, s = adaptive_identity_shrinkage(local_h2, weights, max_local_alpha=PHASE1_H2_EXPERT_LOCAL_ALPHA)
        evidence = {"h2_shrinkage_policy": PHASE1_H2_SHRINKAGE_POLICY, "h2_local_alpha": s["local_alpha"],
                    "h2_local_alpha_cap": s["max_local_alpha"], "h2_effective_sample_size": s["effective_sample_size"],
                    "h2_oas_shrinkage": s["oas_shrinkage"], "h2_identity_scale": s["identity_scale"]}
    else:
        scale = float(torch.trace(local_h2) / local_h2.shape[0])
        h2 = shrink_covariance(torch.eye(local_h2.shape[0], dtype=torch.float32, device=device).mul_(scale), local_h2,
                               h2_alpha)
        evidence = {"h2_shrinkage_policy": "fixed_alpha_scaled_identity", "h2_local_alpha": float(h2_alpha),
                    "h2_local_alpha_cap": float(h2_alpha), "h2_identity_scale": scale}
    return h13, h2, {"gate_square_sum": h13_weight, "h13_local_alpha": float(h13_alpha), **evidence}


def _candidate_middle_by_r13(inputs: torch.Tensor, upstream, evaluated_modes) -> dict[int, torch.Tensor]:
    """Post-SiTU rows of each upstream rate's decoded gate/up reconstruction
    (``upstream["w1"][r13].reconstruction`` and ``["w3"]``, reference
    qsrt/pack/qsrt_candidates.py:406-419)."""

    return {int(r13): situ(F.linear(inputs, upstream["w1"][int(r13)].reconstruction),
                           F.linear(inputs, upstream["w3"][int(r13)].reconstruction)) for r13 in evaluated_modes}


def _conditional_h2_by_r13(inputs: torch.Tensor, gates: torch.Tensor, fit_mask_device: torch.Tensor,
                           middle_by_r13: dict[int, torch.Tensor], *, global_h13: torch.Tensor,
                           global_h2: torch.Tensor, device: torch.device, hessian_policy: str,
                           have_local_support: bool):
    """One down-projection H2 per upstream rate from that rate's decoded rows
    over the fit rows, or the identity under the ``"identity"`` policy or
    without local support (reference qsrt/pack/qsrt_candidates.py:422-461)."""

    h2_by_r13: dict[int, torch.Tensor] = {}
    evidence: dict[str, object] = {}
    identity = torch.eye(global_h2.shape[0], dtype=torch.float32, device=device)
    for r13, middle in middle_by_r13.items():
        if hessian_policy == "identity" or not have_local_support:
            h2_by_r13[r13] = identity
            evidence[f"R{r13}"] = {"h2_shrinkage_policy": "identity_fallback", "h2_local_alpha": 0.0,
                                   "h2_effective_sample_size": 0.0, "h2_identity_scale": 1.0}
            continue
        _, h2, ev = build_expert_hessians(inputs[fit_mask_device], gates[fit_mask_device], middle[fit_mask_device],
                                          global_h13=global_h13, global_h2=global_h2, device=device)
        h2_by_r13[r13] = h2
        evidence[f"R{r13}"] = ev
    return h2_by_r13, evidence
