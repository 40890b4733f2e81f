"""Oracle: SQG E4M3 alphabets in numpy -- test infrastructure only.

Independent restatement of the reference's table construction
(``qsrt/sqg_e4m3.py``).  Unlike the product module it uses scipy's
``ndtri`` and a hand-written E4M3 encoder, so a mistake shared by both
would have to be made twice.

Pinned by: the SHA-256 digests of the T12 table and of the K1..K6 label
maps held in the reference tests (``tests/test_sqg_e4m3.py:30-38``), the
151-distinct-values fact (``tests/test_synthetic_source_distortion.py:98-109``)
and the bijection/stratum invariants (``tests/test_sqg_e4m3.py:52-70``).
"""

from __future__ import annotations

from functools import lru_cache

import numpy as np
from scipy.special import ndtri

N = 1 << 16


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """Float -> E4M3 (fn variant) with round-to-nearest-even.

    For |x| with binary exponent e (clamped below at -6) the quantum is
    2^(e-3); the byte is ``((e + 7) << 3) - 8 + rint(|x| / quantum)``, which
    covers subnormals (e = -6 region) and mantissa carry (rint -> 16).
    Only finite inputs below the 448 saturation bound are supported.
    """

    x = np.asarray(x, dtype=np.float64)
    a = np.abs(x)
    if np.any(~np.isfinite(a)) or np.any(a >= 464.0):
        raise ValueError("e4m3_encode supports finite |x| < 464 only")
    _, ex = np.frexp(np.where(a > 0, a, 1.0))  # a = m * 2^ex, m in [0.5, 1)
    e = np.maximum(ex.astype(np.int64) - 1, -6)
    q = np.rint(a / np.ldexp(1.0, e - 3)).astype(np.int64)
    code = ((e + 7) << 3) - 8 + q
    code = np.where(a == 0, 0, code)
    code = code | np.where(np.signbit(x), 0x80, 0)
    return code.astype(np.uint8)


def e4m3_decode(code: np.ndarray) -> np.ndarray:
    """E4M3 byte -> float32 (0x7F/0xFF are NaN)."""

    c = np.asarray(code, dtype=np.int64)
    mag = c & 0x7F
    e = mag >> 3
    m = mag & 7
    val = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.ldexp(1.0, np.maximum(e, 1) - 10))
    val = np.where(mag == 0x7F, np.nan, val)
    return np.where(c & 0x80, -val, val).astype(np.float32)


def _bit_reverse(v: np.ndarray, width: int) -> np.ndarray:
    out = np.zeros_like(v)
    for b in range(width):
        out |= ((v >> b) & 1) << (width - 1 - b)
    return out


@lru_cache(maxsize=None)
def rank_permutation(bits: int) -> np.ndarray:
    """Carry-mixed SQG rank (reference qsrt/sqg_e4m3.py:259-284)."""

    w = np.arange(N, dtype=np.uint64)
    width = 16 - bits
    hmask = np.uint64((1 << width) - 1)
    h = w >> np.uint64(bits)
    br = w & np.uint64((1 << bits) - 1)
    x = h ^ (h >> np.uint64(11))
    x ^= (x << np.uint64(11)) & hmask
    p = (np.uint64(0x3FA7D929) * x + np.uint64(0xC928FD8E)) & np.uint64(0xFFFFFFFF)
    syn = p >> np.uint64(32 - bits)
    stratum = _bit_reverse(br, bits) ^ syn
    return ((stratum << np.uint64(width)) | (p & hmask)).astype(np.int64)


@lru_cache(maxsize=1)
def exact_normal_rank_bytes() -> np.ndarray:
    """E4M3(float32(1.5 * ndtri((r + 0.5) / 2^16))), zero canonicalised
    (reference qsrt/sqg_e4m3.py:196-229)."""

    r = np.arange(N, dtype=np.float64)
    v = (1.5 * ndtri((r + 0.5) / N)).astype(np.float32)
    b = e4m3_encode(v)
    b[(b & 0x7F) == 0] = 0
    return b


@lru_cache(maxsize=1)
def t12_bytes() -> np.ndarray:
    """Per-16-rank modal byte, lowest byte on ties
    (reference qsrt/sqg_e4m3.py:241-256)."""

    blocks = exact_normal_rank_bytes().reshape(4096, 16)
    out = np.empty(4096, dtype=np.uint8)
    for i, blk in enumerate(blocks):
        vals, counts = np.unique(blk, return_counts=True)
        out[i] = vals[counts == counts.max()].min()
    return out


@lru_cache(maxsize=None)
def t12_labels(bits: int) -> np.ndarray:
    """State-indexed labels ``T12[rank >> 4]`` (reference qsrt/sqg_e4m3.py:287-301)."""

    return t12_bytes()[rank_permutation(bits) >> 4]


def t12_values(bits: int) -> np.ndarray:
    return e4m3_decode(t12_labels(bits))
