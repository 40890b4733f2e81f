"""Rotation-draw plans and transform seed streams (reference behaviour of
tests/test_qsrt_rotations.py and tests/test_qsrt_encoder.py:150-280)."""

from __future__ import annotations

import json

import pytest

from qsrt_amd.qsrt_rotations import QSRTLayerRotationPlan, QSRTRotationPlan, load_qsrt_rotation_plan
from qsrt_amd.transform_seeds import MATRICES, default_qsrt_transform_seeds, qsrt_transform_seed_draw


def test_rotation_plan_defaults_to_draw_zero():
    plan = QSRTRotationPlan()
    assert plan.for_layer(24) == QSRTLayerRotationPlan()
    assert plan.for_layer(24).intermediate_draw(127) == 0


def test_rotation_plan_round_trips(tmp_path):
    expected = QSRTRotationPlan(((12, QSRTLayerRotationPlan(residual_draw=6, intermediate_overrides=((102, 7), (326, 5)))),))
    path = tmp_path / "rotations.json"
    path.write_text(json.dumps(expected.to_json()))
    actual = load_qsrt_rotation_plan(path)
    assert actual == expected
    assert actual.for_layer(12).intermediate_draw(102) == 7
    assert actual.for_layer(12).intermediate_draw(160) == 0
    assert actual.for_layer(24) == QSRTLayerRotationPlan()


@pytest.mark.parametrize("value, match", (
    ({"kind": "wrong", "schema_version": 1, "layers": {}}, "kind"),
    ({"kind": "qsrt_rotation_plan", "schema_version": 1, "layers": {"0": {}}}, "1..92"),
    ({"kind": "qsrt_rotation_plan", "schema_version": 1, "layers": {"12": {"intermediate_overrides": {"896": 1}}}}, "0..895"),
))
def test_rotation_plan_rejects_malformed_values(value, match):
    with pytest.raises(ValueError, match=match):
        QSRTRotationPlan.from_json(value)


def test_default_seeds_are_the_production_streams():
    assert default_qsrt_transform_seeds(1, "w1").input_sign == 1_000_000
    assert default_qsrt_transform_seeds(24, "w2").input_sign == 24_000_002
    assert default_qsrt_transform_seeds(24, "w3").output_sign == 24_000_001 + 499_979
    with pytest.raises(ValueError):
        default_qsrt_transform_seeds(93, "w1")


def test_seed_draws_move_only_the_intended_side():
    for matrix in MATRICES:
        base = default_qsrt_transform_seeds(24, matrix)
        assert qsrt_transform_seed_draw(24, matrix) == base
        residual = qsrt_transform_seed_draw(24, matrix, residual_draw=2)
        private = qsrt_transform_seed_draw(24, matrix, intermediate_draw=3, expert=17)
        if matrix == "w2":
            assert residual.input_sign == base.input_sign and residual.output_sign != base.output_sign
            assert private.input_sign != base.input_sign and private.output_sign == base.output_sign
        else:
            assert residual.input_sign != base.input_sign and residual.output_sign == base.output_sign
            assert private.input_sign == base.input_sign and private.output_sign != base.output_sign
    with pytest.raises(ValueError, match="expert"):
        qsrt_transform_seed_draw(24, "w1", intermediate_draw=1)
