"""Linear objective guidance for fixed-format trellis quantization (mirrors
``qsrt/gradient_guided_viterbi.py``).

A gradient measured at an anchor changes only the offline quantization
target: completing the square turns ``quadratic + strength <g, q - anchor>``
into a shifted quadratic target, so the same tile Viterbi optimises it.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


def _finite(*tensors: torch.Tensor) -> bool:
    return all(bool(torch.all(torch.isfinite(t))) for t in tensors)


def _check_identity_and_strength(anchor_id: str, objective_id: str, strength: float) -> None:
    if not anchor_id or not objective_id:
        raise ValueError("gradient guidance requires anchor and objective identities")
    if not math.isfinite(strength) or strength < 0.0:
        raise ValueError("gradient strength must be finite and nonnegative")


@dataclass(frozen=True)
class ViterbiGradientGuidance:
    """A dense objective gradient and the anchor it was measured at
    (reference gradient_guided_viterbi.py:17-40)."""

    gradient: torch.Tensor
    anchor: torch.Tensor
    anchor_id: str
    objective_id: str
    strength: float = 1.0

    def validate(self, shape) -> None:
        expected = tuple(shape)
        if tuple(self.gradient.shape) != expected or tuple(self.anchor.shape) != expected:
            raise ValueError("gradient guidance tensors do not match the encoded matrix")
        if not self.gradient.is_floating_point() or not self.anchor.is_floating_point():
            raise TypeError("gradient guidance tensors must be floating point")
        if not _finite(self.gradient):
            raise ValueError("objective gradient must be finite")
        if not _finite(self.anchor):
            raise ValueError("gradient anchor must be finite")
        _check_identity_and_strength(self.anchor_id, self.objective_id, self.strength)


@dataclass(frozen=True)
class LowRankViterbiGradientGuidance:
    """A gradient kept as ``left @ right`` (rank r) with its full anchor
    (reference gradient_guided_viterbi.py:43-120)."""

    left: torch.Tensor
    right: torch.Tensor
    anchor: torch.Tensor
    anchor_id: str
    objective_id: str
    strength: float = 1.0

    def validate(self, shape) -> None:
        expected = tuple(shape)
        if len(expected) != 2:
            raise ValueError("low-rank gradient guidance requires a matrix")
        rows, columns = expected
        if self.left.ndim != 2 or self.right.ndim != 2:
            raise ValueError("low-rank gradient factors must be matrices")
        rank = self.left.shape[1]
        if self.left.shape[0] != rows or self.right.shape != (rank, columns) or self.anchor.shape != expected:
            raise ValueError("low-rank gradient guidance has incompatible geometry")
        if rank <= 0:
            raise ValueError("low-rank gradient guidance must have positive rank")
        if not all(t.is_floating_point() for t in (self.left, self.right, self.anchor)):
            raise TypeError("gradient guidance tensors must be floating point")
        if not _finite(self.left, self.right, self.anchor):
            raise ValueError("gradient guidance tensors must be finite")
        _check_identity_and_strength(self.anchor_id, self.objective_id, self.strength)

    def rows(self, row_slice: slice, *, device, dtype) -> torch.Tensor:
        """Only the requested rows of ``left @ right``."""

        return self.left[row_slice].to(device=device, dtype=dtype) @ self.right.to(device=device, dtype=dtype)

    def linear_term(self, candidate: torch.Tensor, *, dtype) -> float:
        """``strength <left @ right, candidate - anchor>`` as ``sum((left^T D) * right)``,
        never forming the full gradient."""

        delta = candidate.to(dtype=dtype) - self.anchor.to(device=candidate.device, dtype=dtype)
        left = self.left.to(device=candidate.device, dtype=dtype)
        right = self.right.to(device=candidate.device, dtype=dtype)
        return float(float(self.strength) * torch.sum((left.T @ delta) * right).item())


def shift_elementwise_target(target: torch.Tensor, gradient: torch.Tensor, *, strength: float,
                             quadratic_weight: torch.Tensor | float = 1.0) -> torch.Tensor:
    """Target with the minimiser of ``a (q - t)^2 + strength g q``: ``t - strength g / (2 a)``."""

    if target.shape != gradient.shape:
        raise ValueError("target and gradient must have matching shapes")
    if not target.is_floating_point() or not gradient.is_floating_point():
        raise TypeError("target and gradient must be floating point")
    if not math.isfinite(strength) or strength < 0.0:
        raise ValueError("gradient strength must be finite and nonnegative")
    weight = torch.as_tensor(quadratic_weight, device=target.device, dtype=torch.float32)
    if weight.ndim and weight.shape != target.shape:
        raise ValueError("quadratic weights must be scalar or match the target")
    if not _finite(weight) or not bool(torch.all(weight > 0)):
        raise ValueError("quadratic weights must be finite and positive")
    return target.float() - 0.5 * float(strength) * gradient.float() / weight


def shift_two_sided_target(target: torch.Tensor, gradient: torch.Tensor, row_hessian: torch.Tensor,
                           column_hessian: torch.Tensor, *, strength: float) -> torch.Tensor:
    """Target under ``tr(E^T H_row E H_col) + strength <G, Q>``:
    ``T - strength/2 H_row^-1 G H_col^-1`` (two linear solves)."""

    if target.ndim != 2 or gradient.shape != target.shape:
        raise ValueError("two-sided target and gradient must be matching matrices")
    rows, columns = target.shape
    if tuple(row_hessian.shape) != (rows, rows):
        raise ValueError("row Hessian has incompatible geometry")
    if tuple(column_hessian.shape) != (columns, columns):
        raise ValueError("column Hessian has incompatible geometry")
    if not math.isfinite(strength) or strength < 0.0:
        raise ValueError("gradient strength must be finite and nonnegative")
    dtype = torch.float64 if target.dtype == torch.float64 else torch.float32
    device = target.device
    left = torch.linalg.solve(row_hessian.to(device=device, dtype=dtype), gradient.to(device=device, dtype=dtype))
    correction = torch.linalg.solve(column_hessian.to(device=device, dtype=dtype).T, left.T).T
    if not _finite(correction):
        raise FloatingPointError("two-sided gradient target shift is non-finite")
    return target.to(dtype=dtype) - 0.5 * float(strength) * correction


def two_sided_guided_objective(target, candidate, anchor, gradient, row_hessian, column_hessian, *, strength: float):
    """(quadratic, linear, quadratic + linear) of a candidate."""

    if not (target.shape == candidate.shape == anchor.shape == gradient.shape):
        raise ValueError("guided objective matrices must have matching shapes")
    error = candidate - target
    quadratic = torch.sum(error * (row_hessian @ error @ column_hessian))
    linear = float(strength) * torch.sum(gradient * (candidate - anchor))
    return quadratic, linear, quadratic + linear


__all__ = [
    "LowRankViterbiGradientGuidance",
    "ViterbiGradientGuidance",
    "shift_elementwise_target",
    "shift_two_sided_target",
    "two_sided_guided_objective",
]
