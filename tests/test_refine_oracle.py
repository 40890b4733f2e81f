"""The CPU dense-H refinement oracle (``oracle/refine.py``) pinned by
mathematics: the conditional-target identity, brute force over each step's
candidate set, the block-diagonal special case, the dither whitening and
monotonicity."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import encode as oenc
from oracle import refine as oref
from oracle import tables as otables
from oracle import viterbi as oviterbi


def _spd(k: int, rng, rho: float = 0.8, rows: int = 400) -> np.ndarray:
    x = np.empty((rows, k))
    x[:, 0] = rng.standard_normal(rows)
    for j in range(1, k):
        x[:, j] = rho * x[:, j - 1] + np.sqrt(1 - rho * rho) * rng.standard_normal(rows)
    H = x.T @ x / rows
    return H + 0.01 * np.mean(np.diag(H)) * np.eye(k)


def _quantizer(bits: int):
    labels = otables.t12_values(bits)
    return lambda tiles: oviterbi.encode(tiles, labels, K=bits, boundary_lag=0)


def _blockldlq(W, H, bits):
    L, _ = oenc.oldlq.block_ldl(H, 16)
    L0 = oenc.oldlq.strictly_block_lower(L, 16)
    k, n = W.shape
    tile_bits = np.full((k // 16, n // 16), bits)
    out = oenc.blockldlq(W, L0, tile_bits, {bits: otables.t12_values(bits)}, {bits: 0})
    return out["Q"].astype(np.float32), out["states"]


@pytest.mark.parametrize("guided", [False, True])
def test_conditional_target_identity(guided):
    """Replacing block b by any candidate C changes the full (guided)
    objective by exactly the change of its block score."""

    rng = np.random.default_rng(7)
    k, n = 64, 48
    H = _spd(k, rng)
    W = rng.standard_normal((k, n))
    Q = W + 0.3 * rng.standard_normal((k, n))
    a = rng.uniform(0.5, 2.0, n)
    grad = rng.standard_normal((k, n)) if guided else None
    anchor = rng.standard_normal((k, n)) if guided else None
    s = 0.7 if guided else 0.0
    f0 = oref.objective(W, Q, H, a, grad, anchor, s)
    for b in range(k // 16):
        r = slice(16 * b, 16 * b + 16)
        t = oref.conditional_target(W, Q, H, b, a, grad, s)
        for _ in range(3):
            C = rng.standard_normal((16, n))
            Q2 = Q.copy()
            Q2[r] = C
            df = oref.objective(W, Q2, H, a, grad, anchor, s) - f0
            sc = oref.tile_scores(t, [Q[r], C], H[r, r], a).sum(axis=0)
            assert abs(df - (sc[1] - sc[0])) <= 1e-10 * abs(f0)


def test_each_choice_is_the_brute_force_minimiser():
    """At every step each tile keeps the candidate of least full objective
    (ties to the lowest index), and only a strict improvement beyond the
    tolerance replaces the current tile."""

    rng = np.random.default_rng(11)
    k, n = 48, 32
    H = _spd(k, rng, rho=0.9)
    W = rng.standard_normal((k, n)) * 0.8
    Q0, S0 = _blockldlq(W, H, 2)
    record = []
    snapshots = []

    def quantize(tiles):
        return _quantizer(2)(tiles)

    # the record holds each step's candidates; replay the steps to know Q before each one
    res = oref.refine(W, H, Q0, S0, quantize, sweeps=2, dither_scales=(0.05,), patterns=4, record=record)
    Q = Q0.astype(np.float64)
    Hs = 0.5 * (H + H.T)
    for b, t, cands, scores, choice in record:
        r = slice(16 * b, 16 * b + 16)
        for j in range(n // 16):
            cols = slice(16 * j, 16 * j + 16)
            full = []
            for c in cands:
                Q2 = Q.copy()
                Q2[r, cols] = c[:, cols]
                full.append(oref.objective(W, Q2, Hs))
            full = np.array(full)
            assert np.allclose(full - full[0], scores[j] - scores[j][0], rtol=0, atol=1e-9 * full[0])
            m = choice[j]
            if m:
                assert full[m] < full[0] and full[m] <= full.min() + 1e-9 * full[0]
            else:
                assert full.min() >= full[0] - 1e-8 * (1 + abs(full[0])) - 1e-9 * full[0]
            snapshots.append(m)
            Q[r, cols] = cands[m][:, cols]
    assert np.array_equal(Q.astype(np.float32), res["Q"])
    assert any(m >= 2 for m in snapshots), "no dithered proposal was ever kept"


def test_block_diagonal_metric_has_nothing_to_improve():
    """With block-diagonal H the conditional target is the source block
    itself, which is what BlockLDLQ encoded (its factor is zero): the
    undithered sweep proposes the stored paths and accepts none."""

    rng = np.random.default_rng(3)
    k, n = 48, 32
    H = np.zeros((k, k))
    for b in range(k // 16):
        H[16 * b:16 * b + 16, 16 * b:16 * b + 16] = _spd(16, rng)
    W = rng.standard_normal((k, n))
    Q0, S0 = _blockldlq(W, H, 2)
    for b in range(k // 16):
        assert np.allclose(oref.conditional_target(W, Q0, H, b), W[16 * b:16 * b + 16], atol=1e-12)
    res = oref.refine(W, H, Q0, S0, _quantizer(2), sweeps=2, stop_on_no_change=False)
    assert [s["accepted"] for s in res["sweeps"]] == [0, 0]
    assert np.array_equal(res["states"], S0)


def test_dither_patterns_are_whitened_signs():
    rng = np.random.default_rng(5)
    Hbb = _spd(16, rng)
    pats = oref.whitened_patterns(Hbb, 4, 1234)
    L = np.linalg.cholesky(Hbb)
    for p in pats:
        assert abs(np.sum(p * (Hbb @ p)) - 256.0) <= 1e-9
        signs = L.T @ p
        assert np.allclose(np.abs(signs), 1.0, atol=1e-9)
    assert not np.allclose(pats[0], pats[1])
    assert np.array_equal(pats, oref.whitened_patterns(Hbb, 4, 1234))


@pytest.mark.parametrize("guided", [False, True])
def test_sweeps_never_raise_the_objective(guided):
    rng = np.random.default_rng(13)
    k, n = 64, 32
    H = _spd(k, rng, rho=0.95)
    W = rng.standard_normal((k, n))
    Q0, S0 = _blockldlq(W, H, 2)
    grad = rng.standard_normal((k, n)) * 0.05 if guided else None
    anchor = Q0.astype(np.float64) if guided else None
    res = oref.refine(W, H, Q0, S0, _quantizer(2), sweeps=3, dither_scales=(0.25, 0.5), patterns=2,
                      grad=grad, anchor=anchor, strength=1.0 if guided else 0.0, stop_on_no_change=False)
    objs = [s["before"] for s in res["sweeps"]] + [res["sweeps"][-1]["after"]]
    assert all(b2 <= b1 + 1e-12 * abs(b1) for b1, b2 in zip(objs, objs[1:]))
    assert objs[-1] < objs[0]
    # the returned payload is the returned reconstruction
    labels = otables.t12_values(2)
    tiles = labels[res["states"].astype(np.int64) & 0xFFFF]
    rec = np.concatenate([oenc.tiles_to_rows(tiles[b]) for b in range(k // 16)])
    assert np.array_equal(rec.astype(np.float32), res["Q"])
