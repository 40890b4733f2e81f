"""Validated transform-draw plans for QSRT candidate construction (mirrors
``qsrt/qsrt_rotations.py``): one layer-shared residual draw per layer and an
intermediate draw per expert (default plus sorted overrides), JSON
round-trippable."""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

from .qsrt import EXPERTS_PER_LAYER, MOE_LAYERS

ROTATION_PLAN_KIND = "qsrt_rotation_plan"
ROTATION_PLAN_SCHEMA_VERSION = 1


def _draw(value: object, *, field: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise ValueError(f"{field} must be a nonnegative integer")
    return value


def _expert(value: object, message: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or not 0 <= value < EXPERTS_PER_LAYER:
        raise ValueError(message)
    return value


@dataclass(frozen=True)
class QSRTLayerRotationPlan:
    """One layer-shared residual draw and optional private expert draws."""

    residual_draw: int = 0
    intermediate_default: int = 0
    intermediate_overrides: tuple[tuple[int, int], ...] = ()

    def __post_init__(self) -> None:
        _draw(self.residual_draw, field="residual_draw")
        _draw(self.intermediate_default, field="intermediate_default")
        experts = tuple(e for e, _ in self.intermediate_overrides)
        if experts != tuple(sorted(set(experts))):
            raise ValueError("intermediate overrides must have sorted unique experts")
        for expert, draw_id in self.intermediate_overrides:
            _expert(expert, f"rotation-plan experts must lie in 0..{EXPERTS_PER_LAYER - 1}")
            _draw(draw_id, field=f"intermediate override for expert {expert}")

    def intermediate_draw(self, expert: int) -> int:
        _expert(expert, f"expert must lie in 0..{EXPERTS_PER_LAYER - 1}")
        return dict(self.intermediate_overrides).get(expert, self.intermediate_default)

    def to_json(self) -> dict:
        return {
            "residual_draw": self.residual_draw,
            "intermediate_default": self.intermediate_default,
            "intermediate_overrides": {str(e): d for e, d in self.intermediate_overrides},
        }

    @classmethod
    def from_json(cls, value: object) -> "QSRTLayerRotationPlan":
        if not isinstance(value, dict):
            raise ValueError("each rotation-plan layer must be an object")
        unknown = set(value) - {"residual_draw", "intermediate_default", "intermediate_overrides"}
        if unknown:
            raise ValueError(f"unknown layer rotation-plan fields: {sorted(unknown)}")
        raw = value.get("intermediate_overrides", {})
        if not isinstance(raw, dict):
            raise ValueError("intermediate_overrides must be an object")
        overrides = []
        for key, draw_id in raw.items():
            if not isinstance(key, str) or not key.isdecimal():
                raise ValueError("rotation-plan expert keys must be decimal strings")
            overrides.append((int(key), _draw(draw_id, field=f"intermediate override for expert {int(key)}")))
        return cls(
            residual_draw=_draw(value.get("residual_draw", 0), field="residual_draw"),
            intermediate_default=_draw(value.get("intermediate_default", 0), field="intermediate_default"),
            intermediate_overrides=tuple(sorted(overrides)),
        )


@dataclass(frozen=True)
class QSRTRotationPlan:
    """Sparse model-wide plan; omitted layers use the production draw zero."""

    layers: tuple[tuple[int, QSRTLayerRotationPlan], ...] = ()

    def __post_init__(self) -> None:
        ids = tuple(layer for layer, _ in self.layers)
        if ids != tuple(sorted(set(ids))):
            raise ValueError("rotation-plan layers must be sorted and unique")
        if any(layer not in MOE_LAYERS for layer in ids):
            raise ValueError("rotation-plan layers must lie in 1..92")

    def for_layer(self, layer: int) -> QSRTLayerRotationPlan:
        if layer not in MOE_LAYERS:
            raise ValueError("Kimi-K3 MoE layer must lie in 1..92")
        return dict(self.layers).get(layer, QSRTLayerRotationPlan())

    def to_json(self) -> dict:
        return {
            "kind": ROTATION_PLAN_KIND,
            "schema_version": ROTATION_PLAN_SCHEMA_VERSION,
            "layers": {str(layer): plan.to_json() for layer, plan in self.layers},
        }

    @classmethod
    def from_json(cls, value: object) -> "QSRTRotationPlan":
        if not isinstance(value, dict):
            raise ValueError("rotation plan must be an object")
        if value.get("kind") != ROTATION_PLAN_KIND:
            raise ValueError(f"rotation plan kind must be {ROTATION_PLAN_KIND!r}")
        if value.get("schema_version") != ROTATION_PLAN_SCHEMA_VERSION:
            raise ValueError("unsupported QSRT rotation-plan schema version")
        unknown = set(value) - {"kind", "schema_version", "layers"}
        if unknown:
            raise ValueError(f"unknown rotation-plan fields: {sorted(unknown)}")
        raw = value.get("layers")
        if not isinstance(raw, dict):
            raise ValueError("rotation-plan layers must be an object")
        layers = []
        for key, plan in raw.items():
            if not isinstance(key, str) or not key.isdecimal():
                raise ValueError("rotation-plan layer keys must be decimal strings")
            layers.append((int(key), QSRTLayerRotationPlan.from_json(plan)))
        return cls(tuple(sorted(layers)))


def load_qsrt_rotation_plan(path: Path) -> QSRTRotationPlan:
    """Load, validate and canonicalise a rotation plan."""

    return QSRTRotationPlan.from_json(json.loads(Path(path).read_text()))
