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
* the record-major container (``qsrt/qsrt.py:1051-1172``): 128-channel
  records along the rate axis, each the EXL words of its tiles in row-major
  tile order -- pinned by round trips against ``pack_words`` on every record;
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


def unpack_records(payload: np.ndarray, record_bits, rate_axis: str, k_tiles: int, n_tiles: int):
    """Record-major payload -> ``(states uint16 [k_tiles, n_tiles, 256],
    tile_bits [k_tiles, n_tiles])``.  Record ``r`` holds the 8 rate-axis tiles
    ``8r .. 8r + 7`` across the whole other axis, tiles in row-major order of
    that ``[rows, cols]`` strip, each ``16 K`` words at the record's rate."""

    words = np.asarray(payload).reshape(-1).view(np.uint16) if np.asarray(payload).dtype == np.int16 else \
        np.asarray(payload, dtype=np.uint16).reshape(-1)
    states = np.zeros((k_tiles, n_tiles, TILE), dtype=np.uint16)
    tile_bits = np.zeros((k_tiles, n_tiles), dtype=np.int64)
    cursor = 0
    for r, bits in enumerate(record_bits):
        if rate_axis == "k":
            rows, cols = slice(8 * r, 8 * r + 8), slice(0, n_tiles)
            shape = (8, n_tiles)
        else:
            rows, cols = slice(0, k_tiles), slice(8 * r, 8 * r + 8)
            shape = (k_tiles, 8)
        count = shape[0] * shape[1] * 16 * bits
        chunk = words[cursor:cursor + count].reshape(shape[0], shape[1], 16 * bits)
        states[rows, cols] = cyclic_states(unpack_symbols(chunk, bits), bits)
        tile_bits[rows, cols] = bits
        cursor += count
    if cursor != words.size:
        raise ValueError("payload length does not match its records")
    return states, tile_bits


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
