"""Exact coupled gate/up/down coordinates of one SwiGLU-family expert
(mirrors ``qsrt/qsrt_coupled.py``).

Gate and up rows are interleaved and rotated by a signed block Hadamard
along the hidden axis (``residual_block_size``, 512) and along the
interleaved intermediate axis (``preactivation_block_size``, 128); the
down projection by ``postactivation_block_size`` (128) along the
intermediate axis and 512 along hidden.  Every rotation of a device tensor
runs the HIP butterfly kernel (``qsrt_amd.hadamard.rotate_``) with the sign
vector fused as its pre- (forward) or post-multiplier (inverse).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .hadamard import BLOCKS, rotate_

Tensor = torch.Tensor
WeightTriplet = tuple[Tensor, Tensor, Tensor]


def situ(gate: Tensor, up: Tensor, *, beta: float = 4.0, linear_beta: float = 25.0) -> Tensor:
    """``beta tanh(g / beta) sigmoid(g) * linear_beta tanh(u / linear_beta)``
    (reference ``qsrt/tp_simulator.py:83-94``)."""

    gate_value = beta * torch.tanh(gate.float() / beta) * torch.sigmoid(gate.float())
    up_value = linear_beta * torch.tanh(up.float() / linear_beta)
    return (gate_value * up_value).to(gate.dtype)


def situ_derivatives(gate: Tensor, up: Tensor, *, beta: float = 4.0, linear_beta: float = 25.0) -> tuple[Tensor, Tensor]:
    """Partial derivatives of :func:`situ` with respect to gate and up, each
    carrying the other factor (reference ``qsrt/coupled_expert_study.py:162-179``).

    With ``f(g) = beta tanh(g / beta) s(g)`` (``s`` the logistic) and
    ``h(u) = linear_beta tanh(u / linear_beta)``: ``d/dg = h f'`` where
    ``f' = (1 - tanh^2) s + beta tanh s (1 - s)``, and ``d/du = f (1 - tanh^2(u / linear_beta))``.
    """

    g, u = gate.float(), up.float()
    t_g = torch.tanh(g / beta)
    s = torch.sigmoid(g)
    t_u = torch.tanh(u / linear_beta)
    f = beta * t_g * s
    df = (1.0 - t_g.square()) * s + beta * t_g * s * (1.0 - s)
    return linear_beta * t_u * df, f * (1.0 - t_u.square())


@dataclass(frozen=True)
class CoupledHadamardSpec:
    """Transform parameters of a coupled profile (reference :26-46)."""

    residual_block_size: int = 512
    preactivation_block_size: int = 128
    postactivation_block_size: int = 128
    residual_draw: int = 0
    intermediate_draw: int = 0

    def __post_init__(self) -> None:
        for name, value in (
            ("residual_block_size", self.residual_block_size),
            ("preactivation_block_size", self.preactivation_block_size),
            ("postactivation_block_size", self.postactivation_block_size),
        ):
            if value <= 0 or value & (value - 1):
                raise ValueError(f"{name} must be a positive power of two")
        if self.residual_draw != 0:
            raise ValueError("the coupled profile fixes residual draw zero")
        if not 0 <= self.intermediate_draw < 8:
            raise ValueError("intermediate_draw must lie in 0..7")


def _butterfly_cpu(x2d: Tensor, block_size: int) -> None:
    """In-place normalised Sylvester transform of each ``block_size`` group of
    the last axis (any power of two; CPU tensors)."""

    m, n = x2d.shape
    view = x2d.view(m, n // block_size, block_size)
    width = 1
    while width < block_size:
        paired = view.view(m, n // block_size, block_size // (2 * width), 2, width)
        left = paired[..., 0, :].clone()
        right = paired[..., 1, :]
        paired[..., 0, :] += right
        paired[..., 1, :].neg_().add_(left)
        width *= 2
    x2d.div_(math.sqrt(block_size))


def _rotate_axis(values: Tensor, *, block_size: int, axis: int, pre=None, post=None) -> Tensor:
    out = values.float().contiguous().clone()
    if out.numel() == 0:
        return out
    ndim = out.ndim
    ext = out.shape[axis]
    before = math.prod(out.shape[:axis])
    after = math.prod(out.shape[axis + 1:])
    if out.is_cuda:
        if block_size not in BLOCKS:
            raise NotImplementedError(f"device Hadamard blocks are {BLOCKS}")
        if after == 1:
            rotate_(out.view(before, ext), block_size, side="right", pre_mul=pre, post_mul=post)
            return out
        if before == 1 and after % 4 == 0:
            rotate_(out.view(ext, after), block_size, side="left", pre_mul=pre, post_mul=post)
            return out
        moved = out.movedim(axis, -1).contiguous()
        rotate_(moved.view(-1, ext), block_size, side="right", pre_mul=pre, post_mul=post)
        return moved.movedim(-1, axis).contiguous()
    shape = [1] * ndim
    shape[axis] = ext
    if pre is not None:
        out.mul_(pre.to(out.device, torch.float32).reshape(shape))
    moved = out.movedim(axis, -1).contiguous()
    _butterfly_cpu(moved.view(-1, ext), block_size)
    out = moved.movedim(-1, axis).contiguous()
    if post is not None:
        out.mul_(post.to(out.device, torch.float32).reshape(shape))
    return out


def block_hadamard(values: Tensor, *, block_size: int, dim: int = -1) -> Tensor:
    """Normalised self-inverse block Walsh-Hadamard transform (reference
    :49-83); returns a new float32 tensor."""

    if values.ndim == 0 or not torch.is_floating_point(values):
        raise TypeError("block Hadamard input must be floating point")
    if block_size <= 0 or block_size & (block_size - 1):
        raise ValueError("block_size must be a positive power of two")
    axis = dim % values.ndim
    if values.shape[axis] % block_size:
        raise ValueError("Hadamard axis must be divisible by block_size")
    if values.numel() == 0:
        return values.float().contiguous().clone()
    return _rotate_axis(values, block_size=block_size, axis=axis)


def rotation_signs(length: int, *, draw: int, axis: int, device) -> Tensor:
    """Deterministic Rademacher vector of the frozen draw family (reference
    :86-105): all ones for draw 0, else ``randint(0, 2) * 2 - 1`` from a CPU
    generator seeded with ``(0x6A09E667F3BCC909 draw + 0xBB67AE8584CAA73B
    axis) mod 2^63``."""

    if length <= 0 or draw < 0:
        raise ValueError("length must be positive and draw nonnegative")
    if draw == 0:
        return torch.ones(length, dtype=torch.float32, device=device)
    generator = torch.Generator(device="cpu")
    generator.manual_seed((0x6A09E667F3BCC909 * draw + 0xBB67AE8584CAA73B * axis) & ((1 << 63) - 1))
    return torch.randint(0, 2, (length,), generator=generator).mul_(2).sub_(1).float().to(device=device)


def signed_block_hadamard(values: Tensor, *, block_size: int, signs: Tensor, dim: int = -1, inverse: bool = False) -> Tensor:
    """``H (values * signs)`` along ``dim``, or the inverse ``H(values) *
    signs`` (reference :108-126)."""

    axis = dim % values.ndim
    if signs.ndim != 1 or signs.numel() != values.shape[axis]:
        raise ValueError("rotation signs do not align with the transformed axis")
    if values.ndim == 0 or not torch.is_floating_point(values):
        raise TypeError("block Hadamard input must be floating point")
    if block_size <= 0 or block_size & (block_size - 1):
        raise ValueError("block_size must be a positive power of two")
    if values.shape[axis] % block_size:
        raise ValueError("Hadamard axis must be divisible by block_size")
    s = signs.to(device=values.device, dtype=torch.float32)
    if values.numel() == 0:
        return values.float().contiguous().clone()
    if inverse:
        return _rotate_axis(values, block_size=block_size, axis=axis, post=s)
    return _rotate_axis(values, block_size=block_size, axis=axis, pre=s)


def _validate_triplet(weights: WeightTriplet) -> tuple[int, int]:
    w1, w3, w2 = weights
    if w1.ndim != 2 or w3.ndim != 2 or w2.ndim != 2 or w1.shape != w3.shape:
        raise ValueError("coupled weights require matching two-dimensional w1/w3")
    intermediate, hidden = w1.shape
    if tuple(w2.shape) != (hidden, intermediate):
        raise ValueError("w2 must have shape [hidden, intermediate]")
    if not all(torch.is_floating_point(value) for value in weights):
        raise TypeError("coupled weights must be floating point")
    if len({value.device for value in weights}) != 1:
        raise ValueError("coupled weights must share one device")
    return intermediate, hidden


def _check_upstream(spec: CoupledHadamardSpec, intermediate: int, hidden: int) -> None:
    if hidden % spec.residual_block_size:
        raise ValueError("hidden size does not close residual Hadamard blocks")
    if 2 * intermediate % spec.preactivation_block_size:
        raise ValueError("interleaved size does not close preactivation blocks")


def _check_down(spec: CoupledHadamardSpec, intermediate: int, hidden: int) -> None:
    if hidden % spec.residual_block_size:
        raise ValueError("hidden size does not close residual Hadamard blocks")
    if intermediate % spec.postactivation_block_size:
        raise ValueError("intermediate size does not close postactivation blocks")


def _signs(spec: CoupledHadamardSpec, hidden: int, intermediate: int, axis: int, device) -> Tensor:
    lengths = (hidden, 2 * intermediate, intermediate, hidden)
    draw = spec.residual_draw if axis in (0, 3) else spec.intermediate_draw
    return rotation_signs(lengths[axis], draw=draw, axis=axis, device=device)


def _upstream(w1: Tensor, w3: Tensor, spec: CoupledHadamardSpec) -> tuple[Tensor, Tensor]:
    intermediate, hidden = map(int, w1.shape)
    dev = w1.device
    interleaved = torch.stack((w1.float(), w3.float()), dim=1).reshape(2 * intermediate, hidden)
    x = signed_block_hadamard(interleaved, block_size=spec.residual_block_size,
                              signs=_signs(spec, hidden, intermediate, 0, dev), dim=1)
    x = signed_block_hadamard(x, block_size=spec.preactivation_block_size,
                              signs=_signs(spec, hidden, intermediate, 1, dev), dim=0)
    return x[:intermediate].contiguous(), x[intermediate:].contiguous()


def _down(w2: Tensor, spec: CoupledHadamardSpec) -> Tensor:
    hidden, intermediate = map(int, w2.shape)
    dev = w2.device
    x = signed_block_hadamard(w2, block_size=spec.postactivation_block_size,
                              signs=_signs(spec, hidden, intermediate, 2, dev), dim=1)
    return signed_block_hadamard(x, block_size=spec.residual_block_size,
                                 signs=_signs(spec, hidden, intermediate, 3, dev), dim=0).contiguous()


def encode_coupled_weights(weights: WeightTriplet, spec: CoupledHadamardSpec) -> WeightTriplet:
    """Source expert -> coupled coordinates (reference :145-196)."""

    w1, w3, w2 = weights
    intermediate, hidden = _validate_triplet(weights)
    _check_upstream(spec, intermediate, hidden)
    _check_down(spec, intermediate, hidden)
    gate, up = _upstream(w1, w3, spec)
    return gate, up, _down(w2, spec)


def encode_coupled_upstream_weights(w1: Tensor, w3: Tensor, spec: CoupledHadamardSpec) -> tuple[Tensor, Tensor]:
    """Gate/up only (reference :199-243)."""

    if w1.ndim != 2 or w3.ndim != 2 or w1.shape != w3.shape:
        raise ValueError("coupled upstream weights must be matching matrices")
    if not torch.is_floating_point(w1) or not torch.is_floating_point(w3):
        raise TypeError("coupled upstream weights must be floating point")
    if w1.device != w3.device:
        raise ValueError("coupled upstream weights must share one device")
    intermediate, hidden = map(int, w1.shape)
    _check_upstream(spec, intermediate, hidden)
    return _upstream(w1, w3, spec)


def encode_coupled_down_weight(w2: Tensor, spec: CoupledHadamardSpec) -> Tensor:
    """Down only (reference :246-279)."""

    if w2.ndim != 2 or not torch.is_floating_point(w2):
        raise TypeError("coupled down weight must be a floating-point matrix")
    hidden, intermediate = map(int, w2.shape)
    _check_down(spec, intermediate, hidden)
    return _down(w2, spec)


def decode_coupled_weights(weights: WeightTriplet, spec: CoupledHadamardSpec) -> WeightTriplet:
    """Coupled coordinates -> source expert (reference :282-336)."""

    w1, w3, w2 = weights
    intermediate, hidden = _validate_triplet(weights)
    _check_upstream(spec, intermediate, hidden)
    _check_down(spec, intermediate, hidden)
    dev = w1.device
    upstream = torch.cat((w1, w3), dim=0)
    x = signed_block_hadamard(upstream, block_size=spec.preactivation_block_size,
                              signs=_signs(spec, hidden, intermediate, 1, dev), dim=0, inverse=True)
    interleaved = signed_block_hadamard(x, block_size=spec.residual_block_size,
                                        signs=_signs(spec, hidden, intermediate, 0, dev), dim=1, inverse=True)
    y = signed_block_hadamard(w2, block_size=spec.residual_block_size,
                              signs=_signs(spec, hidden, intermediate, 3, dev), dim=0, inverse=True)
    down = signed_block_hadamard(y, block_size=spec.postactivation_block_size,
                                 signs=_signs(spec, hidden, intermediate, 2, dev), dim=1, inverse=True)
    paired = interleaved.reshape(intermediate, 2, hidden)
    return paired[:, 0, :].contiguous(), paired[:, 1, :].contiguous(), down.contiguous()


@dataclass(frozen=True)
class CoupledHadamardExecution:
    """Calibration and scoring operations in one coupled basis (reference
    :339-530)."""

    hidden: int
    intermediate: int
    spec: CoupledHadamardSpec

    def _signs(self, axis: int, *, device) -> Tensor:
        return _signs(self.spec, self.hidden, self.intermediate, axis, device)

    def transform_inputs(self, rows: Tensor) -> Tensor:
        if rows.ndim != 2 or rows.shape[1] != self.hidden:
            raise ValueError("input rows do not match the hidden dimension")
        return signed_block_hadamard(rows, block_size=self.spec.residual_block_size,
                                     signs=self._signs(0, device=rows.device), dim=1)

    def transform_preactivation_gradients(self, gradients: Tensor) -> Tensor:
        if gradients.ndim != 2 or gradients.shape[1] != 2 * self.intermediate:
            raise ValueError("gate/up gradients do not match the intermediate dimension")
        interleaved = torch.stack((gradients[:, : self.intermediate], gradients[:, self.intermediate:]), dim=2)
        interleaved = interleaved.reshape(gradients.shape[0], 2 * self.intermediate)
        return signed_block_hadamard(interleaved, block_size=self.spec.preactivation_block_size,
                                     signs=self._signs(1, device=gradients.device), dim=1)

    def transform_upstream_weight_gradients(self, w1_gradient: Tensor, w3_gradient: Tensor) -> tuple[Tensor, Tensor]:
        expected = (self.intermediate, self.hidden)
        if tuple(w1_gradient.shape) != expected or tuple(w3_gradient.shape) != expected:
            raise ValueError("upstream weight gradients have incompatible geometry")
        if w1_gradient.device != w3_gradient.device:
            raise ValueError("upstream weight gradients must share one device")
        return _upstream(w1_gradient, w3_gradient, self.spec)

    def transform_down_weight_gradient(self, gradient: Tensor) -> Tensor:
        if tuple(gradient.shape) != (self.hidden, self.intermediate):
            raise ValueError("down weight gradient has incompatible geometry")
        return _down(gradient, self.spec)

    def transform_postactivation_rows(self, rows: Tensor) -> Tensor:
        if rows.ndim != 2 or rows.shape[1] != self.intermediate:
            raise ValueError("postactivation rows do not match the intermediate dimension")
        return signed_block_hadamard(rows, block_size=self.spec.postactivation_block_size,
                                     signs=self._signs(2, device=rows.device), dim=1)

    def transform_expert_output_gradients(self, gradients: Tensor) -> Tensor:
        if gradients.ndim != 2 or gradients.shape[1] != self.hidden:
            raise ValueError("expert-output gradients do not match the hidden dimension")
        return signed_block_hadamard(gradients, block_size=self.spec.residual_block_size,
                                     signs=self._signs(3, device=gradients.device), dim=1)

    def _both_sides(self, hessian: Tensor, block: int, axis: int) -> Tensor:
        signs = self._signs(axis, device=hessian.device)
        x = signed_block_hadamard(hessian, block_size=block, signs=signs, dim=0)
        return signed_block_hadamard(x, block_size=block, signs=signs, dim=1)

    def transform_h13(self, hessian: Tensor) -> Tensor:
        if tuple(hessian.shape) != (self.hidden, self.hidden):
            raise ValueError("H13 does not match the hidden dimension")
        return self._both_sides(hessian, self.spec.residual_block_size, 0)

    def transform_h2(self, hessian: Tensor) -> Tensor:
        if tuple(hessian.shape) != (self.intermediate, self.intermediate):
            raise ValueError("H2 does not match the intermediate dimension")
        return self._both_sides(hessian, self.spec.postactivation_block_size, 2)

    def transform_output_hessian(self, hessian: Tensor) -> Tensor:
        if tuple(hessian.shape) != (self.hidden, self.hidden):
            raise ValueError("output Hessian does not match the hidden dimension")
        return self._both_sides(hessian, self.spec.residual_block_size, 3)

    def decode_middle(self, rows: Tensor, w1: Tensor, w3: Tensor, activation=situ) -> Tensor:
        transformed = torch.cat((F.linear(rows, w1), F.linear(rows, w3)), dim=1)
        recovered = signed_block_hadamard(transformed, block_size=self.spec.preactivation_block_size,
                                          signs=self._signs(1, device=rows.device), dim=1, inverse=True)
        middle = activation(recovered[:, 0::2], recovered[:, 1::2])
        return signed_block_hadamard(middle, block_size=self.spec.postactivation_block_size,
                                     signs=self._signs(2, device=rows.device), dim=1)

    def decode_output(self, transformed: Tensor) -> Tensor:
        if transformed.ndim != 2 or transformed.shape[1] != self.hidden:
            raise ValueError("output rows do not match the hidden dimension")
        return signed_block_hadamard(transformed, block_size=self.spec.residual_block_size,
                                     signs=self._signs(3, device=transformed.device), dim=1, inverse=True)

    def execute(self, rows: Tensor, weights: WeightTriplet, activation=situ) -> Tensor:
        _validate_triplet(weights)
        middle = self.decode_middle(self.transform_inputs(rows), weights[0], weights[1], activation)
        return self.decode_output(F.linear(middle, weights[2]))


def coupled_execution(weights: WeightTriplet, spec: CoupledHadamardSpec) -> CoupledHadamardExecution:
    intermediate, hidden = _validate_triplet(weights)
    return CoupledHadamardExecution(hidden, intermediate, spec)


__all__ = [
    "CoupledHadamardExecution",
    "CoupledHadamardSpec",
    "WeightTriplet",
    "block_hadamard",
    "coupled_execution",
    "decode_coupled_weights",
    "encode_coupled_down_weight",
    "encode_coupled_upstream_weights",
    "encode_coupled_weights",
    "rotation_signs",
    "signed_block_hadamard",
    "situ",
    "situ_derivatives",
]
