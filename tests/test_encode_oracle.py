"""Pinning the untethered CPU encode (``oracle/encode.py``) before it is
used as the end-to-end checker.

Its pieces are pinned in their own modules; what is checked here is the
composition, by facts that a wrong composition breaks:

* the row/tile reshapes agree with ``fmt.tiles_to_matrix`` (the decoder's
  layout) and invert each other;
* every 16-row block's Viterbi input is the float64 feedback target
  ``W + L0^T (W - Q)`` of the finished recursion rounded once to FP32, its
  states are what the oracle Viterbi returns for that input at the tile's own
  rate, and Q is those states' labels (closure);
* ``T - Q == (I + L0^T)(W - Q)`` over the whole matrix;
* ``compare_states`` classifies planted differences by column and recursion
  order, and a planted bottom-up/top-down swap in the classification fails;
* the ``conditioned`` preparation factors the congruence with ``su g`` (or
  ``su`` when g went into ``sv``), the plain one with the sign vector.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import encode as oenc
from oracle import fmt as ofmt
from oracle import ldlq as oldlq
from oracle import tables as otables

LABELS = {2: otables.t12_values(2), 3: otables.t12_values(3)}
LAGS = {2: 0, 3: 1}


def _spd(n, seed, rho=0.8):
    rng = np.random.default_rng(seed)
    x = np.empty((4 * n, n))
    x[:, 0] = rng.standard_normal(4 * n)
    for j in range(1, n):
        x[:, j] = rho * x[:, j - 1] + np.sqrt(1 - rho * rho) * rng.standard_normal(4 * n)
    return x.T @ x


def _signs(n, seed):
    return np.where(np.random.default_rng(seed).standard_normal(n) >= 0, 1.0, -1.0)


@pytest.fixture(scope="module")
def small_encode():
    k, n = 128, 128
    rng = np.random.default_rng(11)
    W = rng.standard_t(5, size=(k, n)) * 0.02
    H_sum = _spd(k, 12)
    bits = np.where(rng.random((k // 16, n // 16)) < 0.5, 2, 3)
    out = oenc.encode_matrix(W, H_sum, 4 * k, _signs(k, 1), _signs(n, 2), 1.0, bits, LABELS, LAGS,
                             sigma_reg=0.01, threads=1)
    return out, bits


def test_row_tile_reshapes_match_the_decoder_layout():
    rng = np.random.default_rng(3)
    tiles = rng.standard_normal((3, 5, 256))
    M = ofmt.tiles_to_matrix(tiles)
    for rb in range(3):
        rows = M[16 * rb:16 * rb + 16]
        assert np.array_equal(oenc.rows_to_tiles(rows), tiles[rb])
        assert np.array_equal(oenc.tiles_to_rows(tiles[rb]), rows)


def test_each_block_saw_its_feedback_target_and_holds_its_states_labels(small_encode):
    out, bits = small_encode
    W_r, L0, Q = out["W_r"], out["L0"], out["Q"]
    T = oldlq.feedback_targets(W_r, L0, Q)
    kt, nt = bits.shape
    for rb in range(kt):
        expect = oenc.rows_to_tiles(T[16 * rb:16 * rb + 16]).astype(np.float32)
        got = out["targets"][rb]
        assert np.allclose(got, expect, rtol=2e-6, atol=1e-7), f"block {rb}: targets are not W + L0^T (W - Q)"
        q_tiles = oenc.rows_to_tiles(Q[16 * rb:16 * rb + 16])
        for col in range(nt):
            b = int(bits[rb, col])
            assert np.array_equal(LABELS[b][out["states"][rb, col].astype(np.int64)].astype(np.float64),
                                  q_tiles[col])
        for b in (2, 3):
            where = np.flatnonzero(bits[rb] == b)
            if where.size:
                from oracle import viterbi as ov
                _, s = ov.encode(got[where], LABELS[b], K=b, context=128, boundary_lag=LAGS[b], threads=1)
                assert np.array_equal(s, out["states"][rb, where])


def test_recursion_identity_over_the_whole_matrix(small_encode):
    out, _ = small_encode
    W_r, L0, Q = out["W_r"], out["L0"], out["Q"]
    T = ofmt.tiles_to_matrix(out["targets"].astype(np.float64))
    lhs = T - Q
    rhs = (np.eye(W_r.shape[0]) + L0.T) @ (W_r - Q)
    assert np.max(np.abs(lhs - rhs)) <= 1e-6 * max(1.0, np.abs(T).max())


def test_compare_states_classifies_planted_differences(small_encode):
    out, bits = small_encode
    kt, nt = bits.shape
    g = out["states"].copy()
    assert oenc.compare_states(g, out, LABELS, bits, LAGS)["differ"] == 0
    # column 1: bottom block and one above it differ; column 4: only the top block
    g[kt - 1, 1, 7] ^= 1
    g[1, 1, 0] ^= 1
    g[0, 4, 3] ^= 1
    stats = oenc.compare_states(g, out, LABELS, bits, LAGS)
    assert stats["differ"] == 3
    assert sorted(stats["first"]) == sorted([(kt - 1, 1), (0, 4)])
    assert stats["propagated"] == 1
    assert stats["mismatch_rate"] == pytest.approx(3 / (kt * nt))
    assert len(stats["sse_rel_deltas"]) == 2 and all(d >= 0 for d in stats["sse_rel_deltas"])
    # a classification that walks the column top-down would name (1, 1) first
    assert (1, 1) not in stats["first"]
    assert stats["kinds"] == ["path", "path"] and stats["boundary_margins"] == [0.0, 0.0]


def test_compare_states_holds_a_planted_boundary_choice_to_its_margin(small_encode):
    """A tile re-encoded through another boundary state is a ``boundary``
    event: its path is the best one through that state (delta 0), but on
    these inputs the primer is nowhere near choosing it (margin far above
    any rounding); a path through that state that is not the best one shows
    a positive delta."""

    from oracle import viterbi as ov

    out, bits = small_encode
    kt, nt = bits.shape
    rb, col = kt - 1, 3
    b = int(bits[rb, col])
    t = out["targets"][rb, col]
    own = int(out["states"][rb, col, 0]) >> b
    other = (own + 12345) % (1 << (16 - b))
    _, via_other = ov.encode_from(t[None], LABELS[b], [other], K=b, threads=1)
    g = out["states"].copy()
    g[rb, col] = via_other[0]
    stats = oenc.compare_states(g, out, LABELS, bits, LAGS)
    assert stats["first"] == [(rb, col)] and stats["kinds"] == ["boundary"]
    assert stats["sse_rel_deltas"] == [0.0]
    assert stats["boundary_margins"][0] > 1e-3
    g[rb, col, 100] ^= 1  # no longer the best path through `other`
    stats = oenc.compare_states(g, out, LABELS, bits, LAGS)
    assert stats["kinds"] == ["boundary"] and stats["sse_rel_deltas"][0] > 0.0


@pytest.mark.parametrize("g_into_sv", (False, True))
def test_conditioned_preparation_factors_the_scaled_congruence(g_into_sv):
    k, n = 128, 128
    rng = np.random.default_rng(21)
    W = rng.standard_normal((k, n)) * 0.01
    H_sum = _spd(k, 22)
    su_signs, sv_signs = _signs(k, 5), _signs(n, 6)
    bits = np.full((k // 16, n // 16), 2)
    g = 0.7
    plain = oenc.encode_matrix(W, H_sum, 4 * k, su_signs, sv_signs, g, bits, LABELS, LAGS, sigma_reg=0.01,
                               threads=1)
    cond = oenc.encode_matrix(W, H_sum, 4 * k, su_signs, sv_signs, g, bits, LABELS, LAGS, sigma_reg=0.01,
                              conditioned=True, g_into_sv=g_into_sv, threads=1)
    H = oenc.prepare_hessian(H_sum, 4 * k, 0.01)
    assert np.allclose(plain["H_c"], oldlq.congruence(H, su_signs))
    s = cond["su"] if g_into_sv else cond["su"] * g
    assert np.allclose(cond["H_c"], oldlq.congruence(H, s))
    # the congruence with a scaled vector is not the sign congruence: the two modes are distinct
    assert not np.allclose(cond["H_c"], plain["H_c"])
    # and s carries the regularised input scales: |s| = rms / 1.24371088 (before g when g_into_sv is False)
    rms = oldlq.input_rms(W, sv_signs).reshape(-1)
    assert np.allclose(np.abs(s).reshape(-1), rms / oldlq.CODEBOOK_SCALE, rtol=1e-6)


def test_prepare_hessian_damps_the_mean_diagonal():
    H_sum = _spd(32, 30)
    H = oenc.prepare_hessian(H_sum, 7, 0.05)
    base = H_sum / 7
    assert np.allclose(H - base, 0.05 * np.mean(np.diag(base)) * np.eye(32))


def test_observed_boundary_ties_are_ties():
    """Tiles where an MI355X encode chose another boundary state than the
    oracle on the same target (``tests/golden/boundary_ties_k3.npz``, written
    by ``tests/golden/make_boundary_ties.py``): each is a ``boundary`` event
    whose GPU path is exactly the best closed path through its boundary
    state, and whose margin is within FP32 rounding of a tie -- while the
    read costs alone (the states whose own survivors trace to the GPU's
    boundary state) are percent-level away, so a margin that dropped the
    through-path term would reject these ties."""

    from pathlib import Path

    from oracle import viterbi as ov

    z = np.load(Path(__file__).parent / "golden" / "boundary_ties_k3.npz")
    t, g, c = z["targets"], z["gpu_states"], z["cpu_states"]
    n = len(t)
    assert n >= 3
    cpu = {"states": c[None], "targets": t[None]}
    bits = np.full((1, n), 3)
    stats = oenc.compare_states(g[None], cpu, {3: LABELS[3]}, bits, {3: 1})
    assert stats["kinds"] == ["boundary"] * n
    assert all(d == 0.0 for d in stats["sse_rel_deltas"])
    # 0 where the two costs are equal in FP32 on this target (the lowest-index rule chose the CPU's state)
    assert all(0.0 <= m <= 1e-6 for m in stats["boundary_margins"])
    for i in range(n):
        cost, _, end_of = ov.boundary_view(t[i], LABELS[3], K=3, boundary_lag=1)
        own = end_of == (int(g[i, 0]) >> 3)
        gap = (cost[own].min() - cost.min()) / cost.min() if own.any() else np.inf
        assert gap > 1e-4
