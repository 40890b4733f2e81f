"""Pins of the BaKron band-update oracle (oracle/bakron.py) on the CPU:

* for block-lower factors the block-by-block update equals the dense masked
  product T + M2 (Lout (M1 (Q - T)) Lin^T) (a shortened source range planted
  in either helper fails it);
* identity factors leave T unchanged and put the band-masked error in I;
* composing the divide and conquer's band updates gives the same rounding
  path as the one-diagonal-at-a-time recurrence;
* the product's bounding-box update (the CPU path of
  qsrt_amd.two_sided_rounding) agrees with the oracle in float64.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.bakron as bk
from qsrt_amd.two_sided_rounding import apply_bakron_block_update

B = bk.BLOCK


def _block_lower(n, rng, unit=True):
    m = n // B
    f = rng.standard_normal((n, n)) / np.sqrt(n)
    mask = np.kron(np.tril(np.ones((m, m))), np.ones((B, B)))
    f *= mask
    if unit:
        for j in range(m):
            f[j * B:(j + 1) * B, j * B:(j + 1) * B] = np.eye(B)
    return f


def _case(n_out, n_in, seed):
    rng = np.random.default_rng(seed)
    T = rng.standard_normal((n_out, n_in))
    Q = np.round(T * 4) / 4 + 0.01 * rng.standard_normal((n_out, n_in))
    return T, Q, _block_lower(n_out, rng), _block_lower(n_in, rng)


def _dense(T, Q, Lout, Lin, first, middle, last):
    n_out, n_in = T.shape
    m1 = bk.band_mask(n_out, n_in, first, middle)
    m2 = bk.band_mask(n_out, n_in, middle, last)
    left = Lout @ np.where(m1, Q - T, 0.0)
    return T + np.where(m2, left @ Lin.T, 0.0), left


BANDS = [(64, 96, 0, 4, 9), (64, 96, 2, 3, 5), (96, 48, 0, 1, 8), (96, 48, 3, 6, 8), (48, 48, 0, 2, 5),
         (128, 32, 1, 5, 9)]


@pytest.mark.parametrize("n_out,n_in,first,middle,last", BANDS)
def test_band_update_equals_the_dense_masked_product(n_out, n_in, first, middle, last):
    T, Q, Lout, Lin = _case(n_out, n_in, 11 + first + 7 * last)
    got_t, got_i = bk.band_update(T, Q, Lout, Lin, first, middle, last)
    want_t, left = _dense(T, Q, Lout, Lin, first, middle, last)
    np.testing.assert_allclose(got_t, want_t, rtol=0, atol=1e-12)
    m = bk.band_mask(n_out, n_in, first, last)
    np.testing.assert_allclose(got_i[m], left[m], rtol=0, atol=1e-12)
    assert np.all(got_i[~m] == 0)
    outside = ~bk.band_mask(n_out, n_in, middle, last)
    assert np.array_equal(got_t[outside], T[outside])


@pytest.mark.parametrize("helper,shift", [("_left_sources", (0, -1)), ("_right_sources", (0, -1)),
                                          ("_left_sources", (1, 0)), ("_right_sources", (1, 0))])
def test_a_shortened_source_range_fails_the_dense_pin(monkeypatch, helper, shift):
    real = getattr(bk, helper)

    def short(*args):
        s0, s1 = real(*args)
        return s0 + shift[0], s1 + shift[1]

    monkeypatch.setattr(bk, helper, short)
    T, Q, Lout, Lin = _case(64, 96, 5)
    got_t, _ = bk.band_update(T, Q, Lout, Lin, 0, 4, 9)
    want_t, _ = _dense(T, Q, Lout, Lin, 0, 4, 9)
    assert np.abs(got_t - want_t).max() > 1e-3


def test_identity_factors_leave_the_targets_alone():
    T, Q, _, _ = _case(64, 64, 3)
    got_t, got_i = bk.band_update(T, Q, np.eye(64), np.eye(64), 1, 3, 7)
    assert np.array_equal(got_t, T)
    m1 = bk.band_mask(64, 64, 1, 3)
    np.testing.assert_array_equal(got_i, np.where(m1, Q - T, 0.0))


def _round_diagonal(T, Q, d):
    n_out, n_in = T.shape
    m = bk.band_mask(n_out, n_in, d, d + 1)
    Q[m] = np.round(T[m] * 4) / 4


def test_recursion_composes_to_the_diagonal_recurrence():
    n_out, n_in = 80, 48
    T0, _, Lout, Lin = _case(n_out, n_in, 21)
    D = n_out // B + n_in // B - 1
    # one diagonal at a time
    T, Q = T0.copy(), np.zeros_like(T0)
    for d in range(D):
        _round_diagonal(T, Q, d)
        if d + 1 < D:
            T, _ = bk.band_update(T, Q, Lout, Lin, d, d + 1, D)
    seq = Q.copy()
    # divide and conquer
    state = {"T": T0.copy()}
    Q = np.zeros_like(T0)

    def rec(first, last):
        if last == first + 1:
            _round_diagonal(state["T"], Q, first)
            return
        mid = (first + last) // 2
        rec(first, mid)
        state["T"], _ = bk.band_update(state["T"], Q, Lout, Lin, first, mid, last)
        rec(mid, last)

    rec(0, D)
    assert np.array_equal(Q, seq)


@pytest.mark.parametrize("n_out,n_in,first,middle,last", BANDS[:4])
def test_product_cpu_update_matches_the_oracle(n_out, n_in, first, middle, last):
    T, Q, Lout, Lin = _case(n_out, n_in, 31 + last)
    ws = torch.from_numpy(T.copy())
    apply_bakron_block_update(ws, torch.from_numpy(Q), torch.from_numpy(Lout), torch.from_numpy(Lin),
                              first_diagonal=first, middle_diagonal=middle, last_diagonal=last)
    want, _ = bk.band_update(T, Q, Lout, Lin, first, middle, last)
    np.testing.assert_allclose(ws.numpy(), want, rtol=0, atol=1e-12)


def test_batch_shares_a_rank_two_factor():
    T, Q, Lout, Lin = _case(48, 64, 41)
    Tb, Qb = np.stack([T, T * 0.5]), np.stack([Q, Q * 0.5])
    got, _ = bk.band_update_batch(Tb, Qb, Lout, np.stack([Lin, Lin]), 0, 3, 6)
    for j in range(2):
        want, _ = bk.band_update(Tb[j], Qb[j], Lout, Lin, 0, 3, 6)
        assert np.array_equal(got[j], want)
