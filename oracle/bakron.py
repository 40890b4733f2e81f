"""CPU oracle of the BaKron band propagation (float64, numpy).

TEST INFRASTRUCTURE: only ``tests/``, ``__graft_entry__.smoke()`` and the
bench's CPU baseline use this module, as the checker of the HIP kernel
``qsrt_bakron_band_update_f32``; nothing in ``qsrt_amd/`` imports it.

Restates the fused band update of the recursive BaKron two-sided rounding,
reference ``qsrt/csrc/sqg_quantize.cu:141-270`` (left and right band
kernels) and its launcher ``:991-1100``: with 16 x 16 blocks, block (o, i)
on anti-diagonal o + i, the finished band [first, middle) and the next band
[middle, last),

  left   I(o, i)  = sum_{s in [max(0, first - i), min(ob, middle - i))}  Lout(o, s) (Q - T)(s, i)
                    for first <= o + i < last                                   (:166-200)
  right  T(o, c) += sum_{s in [max(0, first - o), min(ib, middle, last - o))}  I(o, s) Lin(c, s)^T
                    for middle <= o + c < last                                  (:232-266)

Each block's source range is contiguous, so a target block is one product of
a 16-row strip by a 16-column strip.  Pinned (tests/test_bakron_oracle.py)
by the dense masked product ``T + M2 (Lout (M1 (Q - T)) Lin^T)`` for
block-lower factors (a shortened source range, planted in either helper,
fails it), by the composition of the recursion's band updates equalling the
one-diagonal-at-a-time recurrence, and by the identity factors reducing the
update to the band-masked error.
"""

from __future__ import annotations

import numpy as np

BLOCK = 16


def _left_sources(i: int, first: int, middle: int, ob: int) -> tuple[int, int]:
    """Source block rows of left target column i (reference :172-173)."""

    return max(0, first - i), min(ob, middle - i)


def _right_sources(o: int, first: int, middle: int, last: int, ib: int) -> tuple[int, int]:
    """Source block columns of right target row o (reference :227-230)."""

    return max(0, first - o), min(ib, middle, last - o)


def _diagonal_blocks(d: int, ob: int, ib: int):
    for o in range(max(0, d - ib + 1), min(ob, d + 1)):
        yield o, d - o


def band_update(T, Q, Lout, Lin, first: int, middle: int, last: int, intermediate=None, *, block: int = BLOCK):
    """Returns ``(T', I)`` for one band propagation of one matrix: ``T'`` is a
    float64 copy of ``T`` with the right product added on the next band,
    ``I`` the left product on diagonals ``[first, last)`` (other blocks
    are taken from ``intermediate``, zero when it is None)."""

    T = np.array(T, dtype=np.float64)
    Q = np.asarray(Q, dtype=np.float64)
    Lout = np.asarray(Lout, dtype=np.float64)
    Lin = np.asarray(Lin, dtype=np.float64)
    n_out, n_in = T.shape
    b = block
    ob, ib = n_out // b, n_in // b
    if not (0 <= first < middle < last <= ob + ib - 1):
        raise ValueError("diagonals must satisfy 0 <= first < middle < last <= ob + ib - 1")
    I = np.zeros_like(T) if intermediate is None else np.array(intermediate, dtype=np.float64)
    err = Q - T
    for d in range(first, last):
        for o, i in _diagonal_blocks(d, ob, ib):
            s0, s1 = _left_sources(i, first, middle, ob)
            acc = np.zeros((b, b))
            if s0 < s1:
                acc = Lout[o * b:(o + 1) * b, s0 * b:s1 * b] @ err[s0 * b:s1 * b, i * b:(i + 1) * b]
            I[o * b:(o + 1) * b, i * b:(i + 1) * b] = acc
    for d in range(middle, last):
        for o, c in _diagonal_blocks(d, ob, ib):
            s0, s1 = _right_sources(o, first, middle, last, ib)
            if s0 < s1:
                T[o * b:(o + 1) * b, c * b:(c + 1) * b] += (I[o * b:(o + 1) * b, s0 * b:s1 * b]
                                                           @ Lin[c * b:(c + 1) * b, s0 * b:s1 * b].T)
    return T, I


def band_update_batch(T, Q, Lout, Lin, first: int, middle: int, last: int, intermediate=None, *,
                      block: int = BLOCK):
    """``band_update`` over a leading batch axis; a factor of rank 2 is shared
    by every member."""

    T = np.asarray(T)
    outs, inters = [], []
    for j in range(T.shape[0]):
        lo = Lout if np.ndim(Lout) == 2 else Lout[j]
        li = Lin if np.ndim(Lin) == 2 else Lin[j]
        inter = None if intermediate is None else intermediate[j]
        t, i = band_update(T[j], Q[j], lo, li, first, middle, last, inter, block=block)
        outs.append(t)
        inters.append(i)
    return np.stack(outs), np.stack(inters)


def band_mask(n_out: int, n_in: int, first: int, last: int, *, block: int = BLOCK) -> np.ndarray:
    """Element mask of the blocks on anti-diagonals [first, last)."""

    o = np.arange(n_out // block)[:, None]
    i = np.arange(n_in // block)[None, :]
    m = ((o + i) >= first) & ((o + i) < last)
    return np.kron(m, np.ones((block, block), dtype=bool))


__all__ = ["BLOCK", "band_update", "band_update_batch", "band_mask"]
