"""Linear objective guidance for fixed-format trellis quantization
(reference ``qsrt/gradient_guided_viterbi.py``).

A gradient ``g`` of some downstream objective, measured at an identified
anchor reconstruction, adds the linear term ``strength <g, Q - anchor>`` to
the quadratic proxy.  The payload format and the decoder do not change: the
term only moves the target the tile Viterbi is asked to approach, by
completing the square.  For a quadratic ``(q - t)^T A (q - t)`` the minimiser
of the guided objective is the one of ``(q - t')^T A (q - t')`` with
``t' = t - strength/2 A^-1 g``; the elementwise, dense-block and two-sided
forms below are that identity for a diagonal ``A``, a block of the dense H,
and ``tr(E^T H_row E H_col)``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


def _check_strength(strength: float) -> None:
    if not math.isfinite(float(strength)) or float(strength) < 0.0:
        raise ValueError("gradient strength must be finite and nonnegative")


def _check_identities(anchor_id: str, objective_id: str) -> None:
    if not anchor_id or not objective_id:
        raise ValueError("gradient guidance requires anchor and objective identities")


@dataclass(frozen=True)
class ViterbiGradientGuidance:
    """A dense objective gradient and the anchor reconstruction it was
    measured at (reference :17-41)."""

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
        if not bool(torch.all(torch.isfinite(self.gradient))):
            raise ValueError("objective gradient must be finite")
        if not bool(torch.all(torch.isfinite(self.anchor))):
            raise ValueError("gradient anchor must be finite")
        _check_identities(self.anchor_id, self.objective_id)
        _check_strength(self.strength)

    def rows(self, row_slice: slice, *, device, dtype) -> torch.Tensor:
        return self.gradient[row_slice].to(device=device, dtype=dtype)

    def linear_term(self, candidate: torch.Tensor, *, dtype) -> float:
        """``strength <gradient, candidate - anchor>``."""

        g = self.gradient.to(device=candidate.device, dtype=dtype)
        delta = candidate.to(dtype) - self.anchor.to(device=candidate.device, dtype=dtype)
        return float(self.strength) * float(torch.sum(g * delta))


@dataclass(frozen=True)
class LowRankViterbiGradientGuidance:
    """A gradient held as rank factors ``left @ right`` plus the full anchor
    (reference :44-128): a routed expert's W1/W3 gradient is a sum over its
    rows of outer products, so it is never materialised whole; only the rows
    a 16-row block needs are."""

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
        rows, cols = expected
        if self.left.ndim != 2 or self.right.ndim != 2:
            raise ValueError("low-rank gradient factors must be matrices")
        rank = self.left.shape[1]
        if rank <= 0:
            raise ValueError("low-rank gradient guidance must have positive rank")
        if self.left.shape[0] != rows or tuple(self.right.shape) != (rank, cols) or tuple(self.anchor.shape) != expected:
            raise ValueError("low-rank gradient guidance has incompatible geometry")
        if not all(t.is_floating_point() for t in (self.left, self.right, self.anchor)):
            raise TypeError("gradient guidance tensors must be floating point")
        if not all(bool(torch.all(torch.isfinite(t))) for t in (self.left, self.right, self.anchor)):
            raise ValueError("gradient guidance tensors must be finite")
        _check_identities(self.anchor_id, self.objective_id)
        _check_strength(self.strength)

    def rows(self, row_slice: slice, *, device, dtype) -> torch.Tensor:
        """The gradient's rows ``row_slice`` (one small product)."""

        return self.left[row_slice].to(device=device, dtype=dtype) @ self.right.to(device=device, dtype=dtype)

    def linear_term(self, candidate: torch.Tensor, *, dtype) -> float:
        """``strength <left @ right, candidate - anchor>`` as
        ``sum((left^T D) * right)``: the rank dimension is contracted last,
        so the full gradient never exists."""

        delta = candidate.to(dtype) - self.anchor.to(device=candidate.device, dtype=dtype)
        left = self.left.to(device=candidate.device, dtype=dtype)
        right = self.right.to(device=candidate.device, dtype=dtype)
        return float(self.strength) * float(torch.sum((left.T @ delta) * right))


def shift_elementwise_target(target: torch.Tensor, gradient: torch.Tensor, *, strength: float,
                             quadratic_weight=1.0) -> torch.Tensor:
    """Target with the same minimiser under ``a (q - target')^2`` as
    ``a (q - target)^2 + strength g q`` has: ``target - strength g / (2 a)``
    (reference :131-152), FP32."""

    if target.shape != gradient.shape:
        raise ValueError("target and gradient must have matching shapes")
    if not target.is_floating_point() or not gradient.is_floating_point():
        raise TypeError("target and gradient must be floating point")
    _check_strength(strength)
    a = torch.as_tensor(quadratic_weight, device=target.device, dtype=torch.float32)
    if a.ndim and a.shape != target.shape:
        raise ValueError("quadratic weights must be scalar or match the target")
    if not bool(torch.all(torch.isfinite(a))) or not bool(torch.all(a > 0)):
        raise ValueError("quadratic weights must be finite and positive")
    return target.float() - 0.5 * float(strength) * gradient.float() / a


def shift_two_sided_target(target: torch.Tensor, gradient: torch.Tensor, row_hessian: torch.Tensor,
                           column_hessian: torch.Tensor, *, strength: float) -> torch.Tensor:
    """Complete the square under ``tr(E^T H_row E H_col)`` (reference
    :155-187): ``target - strength/2 H_row^-1 g H_col^-1``, by two solves
    (no inverse is formed)."""

    if target.ndim != 2 or gradient.shape != target.shape:
        raise ValueError("two-sided target and gradient must be matching matrices")
    rows, cols = target.shape
    if tuple(row_hessian.shape) != (rows, rows):
        raise ValueError("row Hessian has incompatible geometry")
    if tuple(column_hessian.shape) != (cols, cols):
        raise ValueError("column Hessian has incompatible geometry")
    _check_strength(strength)
    dtype = torch.float64 if target.dtype == torch.float64 else torch.float32
    dev = target.device
    g = gradient.to(device=dev, dtype=dtype)
    left = torch.linalg.solve(row_hessian.to(device=dev, dtype=dtype), g)
    correction = torch.linalg.solve(column_hessian.to(device=dev, dtype=dtype).T, left.T).T
    if not bool(torch.all(torch.isfinite(correction))):
        raise FloatingPointError("two-sided gradient target shift is non-finite")
    return target.to(dtype) - 0.5 * float(strength) * correction


def two_sided_guided_objective(target: torch.Tensor, candidate: torch.Tensor, anchor: torch.Tensor,
                               gradient: torch.Tensor, row_hessian: torch.Tensor, column_hessian: torch.Tensor, *,
                               strength: float):
    """``(quadratic, linear, quadratic + linear)`` of a candidate under
    ``tr(E^T H_row E H_col) + strength <g, candidate - anchor>``,
    ``E = candidate - target`` (reference :190-207)."""

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
