"""Host logic of ``qsrt_amd.h2_viterbi_refine`` on the CPU: with a toy
scalar quantizer standing in for the tile Viterbi (round to a 1/4 grid,
state = grid index), the product's sweeps equal the oracle's
(``oracle/refine.py``) tile for tile, with and without dithers, column
weights and guidance, and the receipts follow the reference's fields."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import refine as oref
from qsrt_amd import h2_viterbi_refine as hr
from qsrt_amd.gradient_guided_viterbi import ViterbiGradientGuidance


def _spd(k, rng, rho=0.9, rows=300):
    x = np.empty((rows, k))
    x[:, 0] = rng.standard_normal(rows)
    for j in range(1, k):
        x[:, j] = rho * x[:, j - 1] + np.sqrt(1 - rho * rho) * rng.standard_normal(rows)
    H = x.T @ x / rows
    return H + 0.01 * np.mean(np.diag(H)) * np.eye(k)


def _grid_np(tiles):
    idx = np.clip(np.round(np.asarray(tiles, np.float64) * 4.0), -64, 63)
    return (idx / 4.0).astype(np.float32), idx.astype(np.int16).view(np.uint16)


def _grid_torch(tiles):
    idx = torch.clamp(torch.round(tiles.double() * 4.0), -64, 63)
    return (idx / 4.0).float(), idx.to(torch.int16)


def _rows_to_grid_states(Q):
    from oracle.encode import rows_to_tiles

    k, n = Q.shape
    return np.stack([_grid_np(rows_to_tiles(Q[16 * b:16 * b + 16]))[1] for b in range(k // 16)])


@pytest.mark.parametrize("dither,weights,guided", [(False, False, False), (True, False, False),
                                                   (True, True, False), (False, True, True)])
def test_product_sweeps_equal_oracle_sweeps(dither, weights, guided):
    rng = np.random.default_rng(17)
    k, n = 64, 48
    H = _spd(k, rng)
    W = rng.standard_normal((k, n))
    Q0 = (np.round(W * 4.0) / 4.0).astype(np.float32)  # the unfed (H = I) encode of the toy quantizer
    S0 = _rows_to_grid_states(Q0.astype(np.float64))
    a = rng.uniform(0.5, 2.0, n) if weights else None
    grad = rng.standard_normal((k, n)) * 0.05 if guided else None
    kw = dict(sweeps=3, dither_scales=(0.3, 0.6) if dither else (), patterns=2 if dither else 0)
    cpu = oref.refine(W, H, Q0, S0, _grid_np, stop_on_no_change=False, a=a, grad=grad,
                      anchor=Q0.astype(np.float64) if guided else None, strength=0.8 if guided else 0.0, **kw)
    guidance = (ViterbiGradientGuidance(torch.from_numpy(grad), torch.from_numpy(Q0.astype(np.float64)), "a", "o",
                                        strength=0.8) if guided else None)
    cfg = hr.H2ViterbiRefineConfig(sweeps=3, dither_scales=kw["dither_scales"], num_dither_patterns=kw["patterns"],
                                   stop_on_no_change=False, max_quantizer_batch=7)
    res = hr.refine_h2_viterbi_paths(torch.from_numpy(W), torch.from_numpy(H), torch.from_numpy(Q0),
                                     torch.from_numpy(S0.view(np.int16)), _grid_torch, cfg,
                                     column_weights=None if a is None else torch.from_numpy(a), guidance=guidance)
    assert [s.accepted_tiles for s in res.sweep_stats] == [s["accepted"] for s in cpu["sweeps"]]
    assert res.sweep_stats[0].accepted_tiles > 0
    assert np.array_equal(res.encoded.numpy().view(np.uint16), cpu["states"])
    assert np.array_equal(res.weight_q.numpy(), cpu["Q"])
    for s, c in zip(res.sweep_stats, cpu["sweeps"]):
        assert abs(s.objective_after - c["after"]) <= 1e-10 * abs(c["after"])
        assert s.objective_after <= s.objective_before
        assert s.proposed_tiles == (k // 16) * (n // 16)
    stats = res.stats_dict()["sweeps"][0]
    assert set(stats) == {"sweep", "objective_before", "objective_after", "quadratic_before", "quadratic_after",
                          "linear_before", "linear_after", "relative_improvement", "accepted_tiles",
                          "proposed_tiles", "unique_candidate_paths"}


def test_objectives_and_config_keys():
    rng = np.random.default_rng(2)
    H = torch.from_numpy(_spd(32, rng))
    W = torch.from_numpy(rng.standard_normal((32, 16)))
    Q = W + 0.1
    E = (W - Q).numpy()
    assert abs(hr.dense_h_objective(W, Q, H, chunk_columns=5) - float(np.sum(E * (H.numpy() @ E)))) <= 1e-9
    a = torch.from_numpy(rng.uniform(0.1, 1.0, 16))
    want = float(np.sum(E * (H.numpy() @ E) * a.numpy()[None, :]))
    assert abs(hr.dense_h_objective(W, Q, H, column_weights=a) - want) <= 1e-9
    g = ViterbiGradientGuidance(torch.ones(32, 16), W.clone(), "a", "o", strength=2.0)
    q, lin, tot = hr.dense_h_guided_objective(W, Q, H, g)
    assert abs(lin - 2.0 * 0.1 * 32 * 16) <= 1e-9 and abs(tot - q - lin) <= 1e-12
    with pytest.raises(ValueError, match="nonnegative"):
        hr.dense_h_objective(W, Q, H, column_weights=-a)
    cfg = hr.config_from_quant_args({"h2_viterbi_refine_sweeps": 3, "h2_viterbi_refine_dither_scales": [0.5],
                                     "h2_viterbi_refine_patterns": 4, "h2_viterbi_refine_fp64_score": True,
                                     "h2_viterbi_refine_alternate_order": False, "h2_viterbi_refine_seed": 9,
                                     "h2_viterbi_refine_max_batch": 64})
    assert (cfg.sweeps, cfg.dither_scales, cfg.num_dither_patterns, cfg.score_dtype, cfg.alternate_sweep_order,
            cfg.seed, cfg.max_quantizer_batch) == (3, (0.5,), 4, torch.float64, False, 9, 64)
    assert hr.config_from_quant_args({}) == hr.H2ViterbiRefineConfig()


def test_uniform_candidate_entry_rate_and_refusals(monkeypatch):
    """``refine_uniform_h2_candidate`` (reference ``qsrt/exl3_encoder_backend.py:840-895``): no sweeps returns
    the candidate with the disabled receipt; a uniform rate map refines at that rate through a plain-``K``
    quantizer; every contract one callback cannot honour is refused before any work."""

    from qsrt_amd import exl3_encoder_backend as be

    calls = []

    class _Result:
        weight_q, encoded = "Q1", "S1"

        @staticmethod
        def stats_dict():
            return {"sweeps": ["s"]}

    def fake_refine(weight, hessian, weight_q, encoded, quantizer, config, guidance=None):
        quantizer("tiles")
        calls.append((config, guidance))
        return _Result

    def fake_quantize(tiles, args):
        calls.append(dict(args))

    monkeypatch.setattr(be.h2_viterbi_refine, "refine_h2_viterbi_paths", fake_refine)
    monkeypatch.setattr(be, "quantize_tiles_multigpu", fake_quantize)
    W, H = torch.zeros(32, 48), torch.eye(32)
    base = {"K": 2, "devices": [0]}
    assert be.refine_uniform_h2_candidate(W, H, "Q0", "S0", dict(base)) == ("Q0", "S0", {"enabled": False,
                                                                                    "sweeps": []})
    assert calls == []
    mixed = dict(base, h2_viterbi_refine_sweeps=2, h2_viterbi_refine_patterns=3, mixed_rate_axis="n",
                 mixed_tile_bits=(3, 3, 3))
    q, s, receipt = be.refine_uniform_h2_candidate(W, H, "Q0", "S0", mixed, guidance="g")
    assert (q, s, receipt) == ("Q1", "S1", {"enabled": True, "rate_bits": 3, "sweeps": ["s"]})
    args, (config, guidance) = calls
    assert args["K"] == 3 and "mixed_rate_axis" not in args and "mixed_tile_bits" not in args
    assert (config.sweeps, config.num_dither_patterns, guidance) == (2, 3, "g")
    assert mixed["K"] == 2 and mixed["mixed_tile_bits"] == (3, 3, 3)  # the caller's arguments are untouched
    on = dict(base, h2_viterbi_refine_sweeps=1)
    refusals = [
        (dict(on, periodic_rate_schedules=[(2, 3)]), "one fixed tile rate"),
        (dict(on, devices=[0, 1]), "one quantizer device"),
        (dict(on, mixed_rate_axis="k", mixed_tile_bits=(2, 3)), "uniform rate map"),
        (dict(on, mixed_tile_codebook_ids=[0]), "tile-local codebook selectors"),
    ]
    calls.clear()
    for args, message in refusals:
        with pytest.raises(ValueError, match=message):
            be.refine_uniform_h2_candidate(W, H, "Q0", "S0", args)
    assert calls == []
