"""Oracle: trellis payload format and reference decode in numpy -- test
infrastructure only.

Restates, from the reference:
* EXL word packing and its inverse (``qsrt/qsrt.py:861-907``) -- pinned by
  the known-answer word prefixes of ``tests/test_qsrt.py:242-258`` and by
  round trips;
* cyclic state reconstruction (``qsrt/exl3_reference.py:34-58``) -- pinned
  against the scalar recurrence (``tests/test_qsrt.py:281-295``);
* the tensor-core permutation (``qsrt/exl3_reference.py:86-105``) -- pinned
  as a bijection against the closed form below (rows 2(t%4)+{0,1,8,9},
  columns t//4 + {0,8});
* the normalised Sylvester Hadamard and the decode chain
  (``qsrt/exl3_reference.py:108-140``, ``:210-243``, ``:280-302``) -- pinned
  by H H^T = I, symmetry, and the H_2 Kronecker closed form.
"""

from __future__ import annotations

import numpy as np

TILE = 256


def pack_words(symbols: np.ndarray, bits: int) -> np.ndarray:
    """[..., 256] -> [..., 16 bits] uint16 (MSB-first stream, SWAP16)."""

    v = np.asarray(symbols, dtype=np.int64) & ((1 << bits) - 1)
    lead = v.shape[:-1]
    stream = np.zeros(lead + (TILE * bits,), dtype=np.int64)
    for b in range(bits):
        stream[..., b::bits] = (v >> (bits - 1 - b)) & 1
    words = np.zeros(lead + (16 * bits,), dtype=np.int64)
    for j in range(16):
        words |= stream[..., j::16] << (15 - j)
    idx = np.arange(16 * bits) ^ 1
    return words[..., idx].astype(np.uint16)


def unpack_symbols(words: np.ndarray, bits: int) -> np.ndarray:
    w = np.asarray(words, dtype=np.int64) & 0xFFFF
    w = w[..., np.arange(16 * bits) ^ 1]
    lead = w.shape[:-1]
    stream = np.zeros(lead + (TILE * bits,), dtype=np.int64)
    for j in range(16):
        stream[..., j::16] = (w >> (15 - j)) & 1
    sym = np.zeros(lead + (TILE,), dtype=np.int64)
    for b in range(bits):
        sym |= stream[..., b::bits] << (bits - 1 - b)
    return sym


def cyclic_states(edges: np.ndarray, bits: int) -> np.ndarray:
    """Scalar recurrence s_i = ((s_{i-1} << K) | e_i) & 0xFFFF around the
    cycle (warmed up by running the tile twice)."""

    e = np.asarray(edges, dtype=np.int64) & ((1 << bits) - 1)
    s = np.zeros(e.shape[:-1], dtype=np.int64)
    for i in range(TILE):
        s = ((s << bits) | e[..., i]) & 0xFFFF
    out = np.empty(e.shape, dtype=np.int64)
    for i in range(TILE):
        s = ((s << bits) | e[..., i]) & 0xFFFF
        out[..., i] = s
    return out.astype(np.uint16)


def tensor_core_perm() -> np.ndarray:
    perm = np.empty(TILE, dtype=np.int64)
    for t in range(32):
        rows = 2 * (t % 4) + np.array([0, 1, 8, 9])
        for h, col in enumerate((t // 4, t // 4 + 8)):
            perm[8 * t + 4 * h: 8 * t + 4 * h + 4] = rows * 16 + col
    return perm


def hadamard(n: int = 128) -> np.ndarray:
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h / np.sqrt(n)


def tiles_to_matrix(tile_values: np.ndarray) -> np.ndarray:
    """[K/16, N/16, 256] values in tensor-core order -> [K, N]."""

    kt, nt, _ = tile_values.shape
    rm = np.empty_like(tile_values)
    rm[..., tensor_core_perm()] = tile_values
    return rm.reshape(kt, nt, 16, 16).transpose(0, 2, 1, 3).reshape(16 * kt, 16 * nt)


def decode(states: np.ndarray, label_values: np.ndarray, suh: np.ndarray, svh: np.ndarray) -> np.ndarray:
    """float64 decode: labels -> [K, N] -> H_L -> *suh -> H_R -> *svh."""

    return decode_tile_values(label_values[np.asarray(states, dtype=np.int64) & 0xFFFF], suh, svh)


def decode_tile_values(tile_values: np.ndarray, suh: np.ndarray, svh: np.ndarray) -> np.ndarray:
    """float64 decode of per-tile label values ``[K/16, N/16, 256]`` (mixed
    rates: each tile's labels looked up in its own rate's table)."""

    x = tiles_to_matrix(np.asarray(tile_values, dtype=np.float64))
    k, n = x.shape
    h = hadamard(128)
    x = np.einsum("ij,bjn->bin", h, x.reshape(k // 128, 128, n)).reshape(k, n)
    x = x * np.asarray(suh, dtype=np.float64)[:, None]
    x = np.einsum("kbj,ji->kbi", x.reshape(k, n // 128, 128), h).reshape(k, n)
    return x * np.asarray(svh, dtype=np.float64)[None, :]
