"""Deterministic sign-stream seeds of the encoder's transforms (mirrors
``qsrt/pack/qsrt_encoder.py:151-224``).

``input_sign`` seeds ``su`` and ``output_sign`` seeds ``sv``.  Draw zero is
the production stream ``layer * 1e6 + matrix index`` and ``+ 499,979``;
nonzero residual draws move the layer-shared side (w1/w3 input, w2 output)
by ``10,000,019`` per draw, nonzero intermediate draws move the opposite
side by ``100,000,007`` per draw plus ``1,000,003`` per expert.
"""

from __future__ import annotations

from dataclasses import dataclass

from .qsrt import EXPERTS_PER_LAYER

MATRICES = ("w1", "w3", "w2")


@dataclass(frozen=True)
class QSRTTransformSeeds:
    input_sign: int
    output_sign: int

    def __post_init__(self) -> None:
        if any(isinstance(v, bool) or not isinstance(v, int) or v < 0 for v in (self.input_sign, self.output_sign)):
            raise ValueError("QSRT transform seeds must be nonnegative integers")


def default_qsrt_transform_seeds(layer: int, matrix: str) -> QSRTTransformSeeds:
    if not 1 <= layer <= 92:
        raise ValueError("Kimi-K3 MoE layer must be in 1..92")
    if matrix not in MATRICES:
        raise ValueError(f"unknown expert matrix: {matrix}")
    base = layer * 1_000_000 + MATRICES.index(matrix)
    return QSRTTransformSeeds(base, base + 499_979)


def qsrt_transform_seed_draw(layer: int, matrix: str, *, residual_draw: int = 0, intermediate_draw: int = 0,
                             expert: int | None = None) -> QSRTTransformSeeds:
    if any(isinstance(d, bool) or not isinstance(d, int) or d < 0 for d in (residual_draw, intermediate_draw)):
        raise ValueError("rotation draw indices must be nonnegative integers")
    if intermediate_draw and (expert is None or isinstance(expert, bool) or not isinstance(expert, int)
                              or not 0 <= expert < EXPERTS_PER_LAYER):
        raise ValueError(f"a nonzero intermediate draw requires an expert in 0..{EXPERTS_PER_LAYER - 1}")
    base = default_qsrt_transform_seeds(layer, matrix)
    residual = residual_draw * 10_000_019
    private = intermediate_draw * 100_000_007 + expert * 1_000_003 if intermediate_draw else 0
    if matrix == "w2":
        return QSRTTransformSeeds(base.input_sign + private, base.output_sign + residual)
    return QSRTTransformSeeds(base.input_sign + residual, base.output_sign + private)
