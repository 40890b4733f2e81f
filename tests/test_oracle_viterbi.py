"""Pinning the CPU Viterbi oracle (oracle/viterbi_ref.c) before trusting it.

* exhaustive search over closed paths on tiny trellises with exact integer
  arithmetic (every tie rule is exercised);
* closure and ``recon == LUT[state]`` at production size (reference
  tests/test_sqg_quantizer.py:178-231);
* degenerate table => scalar nearest neighbour (reference
  tests/test_synthetic_source_distortion.py:60-73): if a label depends only
  on the predecessor choice, every label sequence is a closed path, so the
  tail-biting search must return per-symbol nearest neighbours;
* a planted mistake in a copy of the oracle's tie rule is caught.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import tables as otables
from oracle import viterbi as ov
from qsrt_amd.exl3_reference import reconstruct_trellis_states

import torch

SMALL = [
    (6, 2, 8, 1), (6, 2, 8, 2), (6, 2, 8, 4), (6, 3, 6, 2), (6, 3, 6, 3),
    (4, 1, 8, 2), (4, 1, 8, 4), (8, 2, 6, 3), (8, 4, 4, 2), (8, 3, 4, 2),
    # 32 and 64 predecessors per state (the K5 / K6 trellis shape)
    (10, 5, 2, 1), (10, 5, 3, 1), (12, 6, 2, 1), (12, 6, 3, 1),
]


@pytest.mark.parametrize("lag", (0, 1))
@pytest.mark.parametrize(("L", "K", "T", "C"), SMALL)
def test_oracle_matches_exhaustive_search_with_ties(L, K, T, C, lag):
    rng = np.random.default_rng(1000 * L + 100 * K + 10 * T + C + lag)
    for _ in range(4):
        lab = rng.integers(-3, 4, size=1 << L).astype(np.float32)
        x = rng.integers(-4, 5, size=T).astype(np.float32)
        recon, states, boundary = ov.encode(x[None], lab, K=K, L=L, context=C, boundary_lag=lag, return_boundary=True)
        b_recon, b_states, b_end = ov.brute_force(x, lab, K=K, L=L, context=C, boundary_lag=lag)
        assert boundary[0] == b_end
        assert np.array_equal(states[0], b_states)
        assert np.array_equal(recon[0], b_recon)


def test_planted_tie_rule_mistake_is_detected():
    """Exhaustive search with the tie rules flipped (highest index) must
    disagree with the oracle on tie-rich inputs: the comparison above has
    teeth against a wrong tie rule."""

    rng = np.random.default_rng(7)
    L, K, T, C = 6, 2, 8, 2
    disagreements = 0
    for _ in range(10):
        lab = rng.integers(-2, 3, size=1 << L).astype(np.float32)
        x = rng.integers(-2, 3, size=T).astype(np.float32)
        _, states = ov.encode(x[None], lab, K=K, L=L, context=C)
        _, wrong, _ = ov.brute_force(x, lab, K=K, L=L, context=C, ties="highest")
        disagreements += int(not np.array_equal(states[0], wrong))
    assert disagreements > 0


@pytest.mark.parametrize("bits", (1, 2, 3, 4, 5, 6))
@pytest.mark.parametrize("context", (1, 32, 128))
def test_oracle_production_size_closure(bits, context):
    rng = np.random.default_rng(bits * 10 + context)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    x[1] *= 100.0
    x[2] = 1000.0
    lab = otables.t12_values(bits)
    recon, states = ov.encode(x, lab, K=bits, context=context)
    st = torch.from_numpy(states.astype(np.int64))
    assert torch.equal(reconstruct_trellis_states(st & ((1 << bits) - 1), bits).to(torch.int64) & 0xFFFF, st)
    assert np.array_equal(recon, lab[states])


def test_degenerate_table_reduces_to_scalar_nearest_neighbour():
    levels = np.array([-1.5104, -0.4528, 0.4528, 1.5104], dtype=np.float32)
    lab = levels[np.arange(1 << 16) >> 14]
    x = np.random.default_rng(3).standard_normal((4, 256)).astype(np.float32)
    recon, _ = ov.encode(x, lab, K=2)
    nn = levels[np.abs(x[..., None] - levels).argmin(-1)]
    assert np.array_equal(recon, nn)


def test_trellis_beats_scalar_at_k2():
    """Shaping gain of the frozen K2 law on N(0,1) at the reference's fitted
    scale 0.6624 (reference tests/test_synthetic_source_distortion.py:82-95):
    per-symbol MSE below 0.85x Lloyd-Max (0.1175) and near the published
    0.0664 (docs/qsrt-exl3-comparative-assessment.md:90-97)."""

    x = np.random.default_rng(5).standard_normal((16, 256)).astype(np.float32)
    scale = 0.6624
    recon, _ = ov.encode(x / scale, otables.t12_values(2), K=2)
    mse = float(((recon * scale - x) ** 2).mean())
    assert mse < 0.85 * 0.1175
    assert 0.060 < mse < 0.075


@pytest.mark.parametrize("K", (1, 2, 3, 4, 5, 6))
def test_vector_path_equals_scalar_path(K):
    """The oracle's AVX2 path against its scalar path, bit for bit, at
    production size (L = 16, C = 128) and on a tiny trellis, both boundary
    rules, with saturated and tied inputs mixed in."""

    rng = np.random.default_rng(40 + K)
    lab = otables.t12_values(K) if K in (1, 2, 3, 4, 5, 6) else None
    tiles = rng.standard_normal((6, 256)).astype(np.float32)
    tiles[1] = 0.0  # every label equally far from x: ties everywhere
    tiles[2] = 1e6  # saturated costs
    small_lab = rng.integers(-3, 4, size=1 << 8).astype(np.float32)
    small = rng.integers(-4, 5, size=(3, 12)).astype(np.float32)
    for lag in (0, 1):
        out = []
        for vector in (True, False):
            ov.set_vector(vector)
            try:
                out.append((ov.encode(tiles, lab, K=K, context=128, boundary_lag=lag, threads=2),
                            ov.encode(small, small_lab, K=min(K, 4), L=8, context=4, boundary_lag=lag, threads=1)
                            if 2 * min(K, 4) <= 8 else None))
            finally:
                ov.set_vector(True)
        (big_v, small_v), (big_s, small_s) = out
        assert np.array_equal(big_v[0].view(np.uint32), big_s[0].view(np.uint32))
        assert np.array_equal(big_v[1], big_s[1])
        if small_v is not None:
            assert np.array_equal(small_v[1], small_s[1])


# boundary views: tiny trellises where every state can be enumerated
BOUNDARY_SMALL = [(6, 2, 8, 2), (6, 2, 8, 4), (6, 3, 6, 3), (4, 1, 8, 4), (8, 2, 6, 3), (10, 5, 3, 1)]


@pytest.mark.parametrize("lag", (0, 1))
@pytest.mark.parametrize(("L", "K", "T", "C"), BOUNDARY_SMALL)
def test_boundary_view_matches_exhaustive_search(L, K, T, C, lag):
    """Read costs, final costs and each state's traced end_state against
    enumeration (ties exercised by the small integer alphabet); the encode's
    own boundary is end_of at the lowest minimum of the read costs."""

    rng = np.random.default_rng(7 * L + 3 * K + T + C + lag)
    for _ in range(3):
        lab = rng.integers(-3, 4, size=1 << L).astype(np.float32)
        x = rng.integers(-4, 5, size=T).astype(np.float32)
        cost, final, end_of = ov.boundary_view(x, lab, K=K, L=L, context=C, boundary_lag=lag)
        b_cost, b_final, b_end = ov.brute_force_boundary(x, lab, K=K, L=L, context=C, boundary_lag=lag)
        np.testing.assert_array_equal(cost, b_cost)
        np.testing.assert_array_equal(final, b_final)
        np.testing.assert_array_equal(end_of, b_end)
        _, _, boundary = ov.encode(x[None], lab, K=K, L=L, context=C, boundary_lag=lag, return_boundary=True)
        assert boundary[0] == end_of[int(np.argmin(cost))]


@pytest.mark.parametrize(("L", "K", "T", "C"), BOUNDARY_SMALL)
def test_primer_through_matches_exhaustive_search(L, K, T, C):
    """Costs through every boundary state against enumeration; the minimum
    over boundary states is the free primer's final cost, reached exactly at
    each state's own traced end_state."""

    rng = np.random.default_rng(11 * L + 5 * K + T + C)
    lab = rng.integers(-3, 4, size=1 << L).astype(np.float32)
    x = rng.integers(-4, 5, size=T).astype(np.float32)
    S = 1 << (L - K)
    _, final, end_of = ov.boundary_view(x, lab, K=K, L=L, context=C)
    through = np.stack([ov.primer_through(x, lab, e, K=K, L=L, context=C) for e in range(S)])
    for e in range(S):
        np.testing.assert_array_equal(through[e], ov.brute_force_through(x, lab, e, K=K, L=L, context=C))
    np.testing.assert_array_equal(through.min(axis=0), final)
    np.testing.assert_array_equal(through[end_of, np.arange(S)], final)


@pytest.mark.parametrize(("L", "K", "T", "C"), BOUNDARY_SMALL)
def test_encode_from_matches_exhaustive_search_and_encode(L, K, T, C):
    """The constrained pass from a given boundary state against enumeration;
    from the encode's own boundary state it reproduces the encode."""

    rng = np.random.default_rng(13 * L + 7 * K + T + C)
    S = 1 << (L - K)
    lab = rng.integers(-3, 4, size=1 << L).astype(np.float32)
    xs = rng.integers(-4, 5, size=(4, T)).astype(np.float32)
    ends = rng.integers(0, S, size=4)
    recon, states = ov.encode_from(xs, lab, ends, K=K, L=L)
    for i in range(4):
        b_recon, b_states = ov.brute_force_from(xs[i], lab, int(ends[i]), K=K, L=L)
        np.testing.assert_array_equal(states[i], b_states)
        np.testing.assert_array_equal(recon[i], b_recon)
    e_recon, e_states, boundary = ov.encode(xs, lab, K=K, L=L, context=C, return_boundary=True)
    f_recon, f_states = ov.encode_from(xs, lab, boundary, K=K, L=L)
    np.testing.assert_array_equal(f_states, e_states)
    np.testing.assert_array_equal(f_recon, e_recon)


def test_boundary_views_at_production_size():
    """L16 K3 with the frozen table: the traced end_state of the read-cost
    argmin is the encode's, and the cost through it equals the final cost of
    that state bit for bit (the primer's own operations)."""

    rng = np.random.default_rng(5)
    lab = otables.t12_values(3)
    x = rng.standard_normal(256).astype(np.float32)
    cost, final, end_of = ov.boundary_view(x, lab, K=3, boundary_lag=1)
    _, _, boundary = ov.encode(x[None], lab, K=3, boundary_lag=1, return_boundary=True)
    s = int(np.argmin(cost))
    assert end_of[s] == boundary[0]
    through = ov.primer_through(x, lab, int(boundary[0]), K=3)
    assert through[s] == final[s]
    assert np.all(through >= final)


def test_a_thread_count_applies_to_its_own_call_only():
    """``threads=1`` on one call must not shrink the team of later calls that
    pass 0 (the default): the count is a per-call clause, not a change of the
    process-wide OpenMP default."""

    lib = ov._load()
    before = lib.qsrt_oracle_default_threads()
    x = np.zeros((2, 8), dtype=np.float32)
    lab = np.zeros(1 << 6, dtype=np.float32)
    ov.encode(x, lab, K=2, L=6, context=2, threads=1)
    ov.encode_from(x, lab, [0, 1], K=2, L=6, threads=1)
    assert lib.qsrt_oracle_default_threads() == before
