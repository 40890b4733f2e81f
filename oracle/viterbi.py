"""Oracle: tail-biting tile Viterbi -- test infrastructure only.

``encode`` binds ``viterbi_ref.c`` (the FP32 C restatement of the
reference's pass structure; see its header).  ``brute_force`` is an
independent exhaustive search over closed paths for tiny trellises, used to
pin the C restatement:

* pinned by brute force (``tests/test_oracle_viterbi.py``) on small L/K/T
  with exact integer arithmetic, including the lowest-index tie rules;
  the diagnostic views of the same passes -- ``boundary_view`` (the primer
  costs and each state's traced boundary state), ``primer_through`` (the
  primer restricted to one boundary state) and ``encode_from`` (the
  constrained pass from a given boundary state) -- are pinned the same way,
  and against ``encode`` itself;
* pinned at production size (L=16, T=256) by closure
  (``tests/test_sqg_quantizer.py:178-231`` in the reference), by the
  degenerate-table => scalar nearest-neighbour identity
  (reference ``tests/test_synthetic_source_distortion.py:60-73``), and by
  the per-symbol MSE level of the frozen table
  (``docs/qsrt-exl3-comparative-assessment.md:78-100``).

Bit parity with the reference's FP16 CUDA kernel itself is *parity
unpinned*: that kernel cannot run here and differs by design (FP16 costs,
lane-order final reduction).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libqsrt_oracle.so"
_lib = None


def build() -> None:
    import subprocess

    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        lib.qsrt_oracle_viterbi.restype = ctypes.c_int
        lib.qsrt_oracle_viterbi.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
            ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
        ]
        lib.qsrt_oracle_viterbi_boundary.restype = ctypes.c_int
        lib.qsrt_oracle_viterbi_boundary.argtypes = [
            ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
            ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ]
        lib.qsrt_oracle_viterbi_primer_through.restype = ctypes.c_int
        lib.qsrt_oracle_viterbi_primer_through.argtypes = [
            ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
            ctypes.c_int, ctypes.c_void_p,
        ]
        lib.qsrt_oracle_viterbi_from.restype = ctypes.c_int
        lib.qsrt_oracle_viterbi_from.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
        ]
        lib.qsrt_oracle_default_threads.restype = ctypes.c_int
        lib.qsrt_oracle_default_threads.argtypes = []
        lib.qsrt_oracle_set_vector.restype = None
        lib.qsrt_oracle_set_vector.argtypes = [ctypes.c_int]
        _lib = lib
    return _lib


def set_vector(enable: bool) -> None:
    """Select the AVX2 path (default) or the scalar path of the C oracle;
    both compute the same values bit for bit."""

    _load().qsrt_oracle_set_vector(1 if enable else 0)


def encode(
    tiles: np.ndarray,
    labels: np.ndarray,
    *,
    K: int,
    L: int = 16,
    context: int = 128,
    boundary_lag: int = 0,
    threads: int = 0,
    return_boundary: bool = False,
):
    """Encode ``tiles [n, T]`` against state-indexed float ``labels [2^L]``.

    Returns ``(recon float32 [n, T], states uint16 [n, T])`` (and the
    boundary states when requested).
    """

    lib = _load()
    tiles = np.ascontiguousarray(tiles, dtype=np.float32)
    labels = np.ascontiguousarray(labels, dtype=np.float32)
    if tiles.ndim != 2 or labels.shape != (1 << L,):
        raise ValueError("tiles must be [n, T] and labels [2^L]")
    n, T = tiles.shape
    recon = np.empty_like(tiles)
    states = np.empty((n, T), dtype=np.uint16)
    boundary = np.empty(n, dtype=np.int32)
    rc = lib.qsrt_oracle_viterbi(
        tiles.ctypes.data, recon.ctypes.data, states.ctypes.data, n, L, K, T, context,
        labels.ctypes.data, boundary_lag, boundary.ctypes.data, int(threads),
    )
    if rc != 0:
        raise RuntimeError(f"oracle viterbi failed with code {rc}")
    if return_boundary:
        return recon, states, boundary
    return recon, states


def boundary_view(tile: np.ndarray, labels: np.ndarray, *, K: int, L: int = 16, context: int = 128,
                  boundary_lag: int = 0):
    """The boundary choice of one tile: ``(cost, final, end_of)`` over the
    ``2^(L-K)`` states -- the primer costs the boundary argmin reads, the
    final primer costs (the same array when ``boundary_lag = 0``) and the
    end_state each state's primer survivor traces back to.  ``encode``'s
    end_state is ``end_of[argmin(cost)]`` (lowest index on ties)."""

    lib = _load()
    tile = np.ascontiguousarray(tile, dtype=np.float32).reshape(-1)
    labels = np.ascontiguousarray(labels, dtype=np.float32)
    if labels.shape != (1 << L,):
        raise ValueError("labels must be [2^L]")
    S = 1 << (L - K)
    cost = np.empty(S, dtype=np.float32)
    final = np.empty(S, dtype=np.float32)
    end_of = np.empty(S, dtype=np.int32)
    rc = lib.qsrt_oracle_viterbi_boundary(tile.ctypes.data, L, K, len(tile), context, labels.ctypes.data,
                                          boundary_lag, cost.ctypes.data, final.ctypes.data, end_of.ctypes.data)
    if rc != 0:
        raise RuntimeError(f"oracle viterbi boundary failed with code {rc}")
    return cost, final, end_of


def primer_through(tile: np.ndarray, labels: np.ndarray, e: int, *, K: int, L: int = 16,
                   context: int = 128) -> np.ndarray:
    """Per final state, the cost of the best primer path whose state before
    position 0 is ``e`` (float32 ``[2^(L-K)]``, ``inf`` where none reaches),
    in the primer's own arithmetic: it equals ``boundary_view``'s ``final``
    wherever that state's survivor passes through ``e`` and exceeds it
    elsewhere."""

    lib = _load()
    tile = np.ascontiguousarray(tile, dtype=np.float32).reshape(-1)
    labels = np.ascontiguousarray(labels, dtype=np.float32)
    if labels.shape != (1 << L,):
        raise ValueError("labels must be [2^L]")
    through = np.empty(1 << (L - K), dtype=np.float32)
    rc = lib.qsrt_oracle_viterbi_primer_through(tile.ctypes.data, L, K, len(tile), context, labels.ctypes.data,
                                                int(e), through.ctypes.data)
    if rc != 0:
        raise RuntimeError(f"oracle viterbi primer_through failed with code {rc}")
    return through


def encode_from(tiles: np.ndarray, labels: np.ndarray, end_states, *, K: int, L: int = 16, threads: int = 0):
    """The constrained pass alone: the best closed path of each tile through
    the given boundary state (``end_states [n]``).  Returns ``(recon, states)``
    like ``encode``; with ``encode``'s own end_states it reproduces
    ``encode``."""

    lib = _load()
    tiles = np.ascontiguousarray(tiles, dtype=np.float32)
    labels = np.ascontiguousarray(labels, dtype=np.float32)
    ends = np.ascontiguousarray(end_states, dtype=np.int32).reshape(-1)
    if tiles.ndim != 2 or labels.shape != (1 << L,) or len(ends) != len(tiles):
        raise ValueError("tiles must be [n, T], labels [2^L], end_states [n]")
    n, T = tiles.shape
    recon = np.empty_like(tiles)
    states = np.empty((n, T), dtype=np.uint16)
    rc = lib.qsrt_oracle_viterbi_from(tiles.ctypes.data, recon.ctypes.data, states.ctypes.data, n, L, K, T,
                                      labels.ctypes.data, ends.ctypes.data, int(threads))
    if rc != 0:
        raise RuntimeError(f"oracle viterbi_from failed with code {rc}")
    return recon, states


def default_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


# ---------------------------------------------------------------------------
# Exhaustive search for tiny trellises (exact integer arithmetic)
# ---------------------------------------------------------------------------


def _enumerate(S: int, K: int, L: int, steps: int, start_states):
    """All paths from the given start states: (start, codewords [n, steps],
    choices k [n, steps]) as integer arrays."""

    P = 1 << K
    branches = np.array(np.meshgrid(*[np.arange(P)] * steps, indexing="ij")).reshape(steps, -1).T
    starts = np.repeat(np.asarray(list(start_states), dtype=np.int64), len(branches))
    branches = np.tile(branches, (len(start_states), 1))
    words = np.empty_like(branches)
    s = starts.copy()
    for i in range(steps):
        w = ((s << K) | branches[:, i]) & ((1 << L) - 1)
        words[:, i] = w
        s = w & (S - 1)
    return starts, words, words >> (L - K)


def _best_by_final_state(x, lab, K: int, L: int, start_states, positions, ties: str = "lowest") -> dict:
    """Per final state, the optimal path over ``positions`` from any of
    ``start_states`` under the Viterbi's survivor tie rule: ``{state: (cost,
    codewords)}`` (integer arithmetic)."""

    S, P = 1 << (L - K), 1 << K
    _, words, ks = _enumerate(S, K, L, len(positions), start_states)
    cost = ((lab[words] - x[np.asarray(positions)]) ** 2).sum(axis=1)
    digits = ks[:, ::-1] if ties == "lowest" else (P - 1 - ks[:, ::-1])
    order = np.zeros(len(words), dtype=np.int64)
    for col in range(digits.shape[1]):
        order = order * P + digits[:, col]
    key = cost * (P ** digits.shape[1]) + order
    fin = words[:, -1] & (S - 1)
    best = {}
    for f in np.unique(fin):
        idx = np.flatnonzero(fin == f)
        j = idx[np.argmin(key[idx])]
        best[int(f)] = (int(cost[j]), words[j])
    return best


def brute_force(x, labels, *, K: int, L: int, context: int, boundary_lag: int = 0, ties: str = "lowest"):
    """Reference result for one tile by enumeration.

    ``x`` and ``labels`` must be small integers so that every FP32 partial
    sum is exact; then the Viterbi's tie rules translate to:

    * per state, the survivor is the lexicographically smallest reversed
      choice sequence (k_last, k_last-1, ...) among optimal paths;
    * the boundary is the lowest state index among minimal final costs.

    ``ties="highest"`` flips both rules; it exists so a test can plant that
    mistake and show the comparison detects it.
    """

    x = np.asarray(x, dtype=np.int64)
    lab = np.asarray(labels, dtype=np.int64)
    T = len(x)
    S = 1 << (L - K)
    P = 1 << K
    C = context

    def best_by_final_state(start_states, positions):
        return _best_by_final_state(x, lab, K, L, start_states, positions, ties)

    def pick(table):
        fmin = min(v[0] for v in table.values())
        cands = [s for s, v in table.items() if v[0] == fmin]
        return min(cands) if ties == "lowest" else max(cands)

    window = [(T - C + i) % T for i in range(2 * C)]
    full = best_by_final_state(range(S), window)
    start = pick(full) if boundary_lag == 0 else pick(best_by_final_state(range(S), window[:-1]))
    survivor = full[start][1]
    # window index C is position 0; its codeword came from the state before it
    end_state = int(survivor[C] >> K)
    words = best_by_final_state([end_state], list(range(T)))[end_state][1]
    return lab[words].astype(np.float32), words.astype(np.uint16), end_state


def brute_force_boundary(x, labels, *, K: int, L: int, context: int, boundary_lag: int = 0):
    """``boundary_view`` by enumeration (small integer ``x`` and ``labels``):
    the optimal primer cost ending in each state over all but the window's
    last position (``boundary_lag = 1``) or over the whole window, the
    whole-window costs, and the end_state of each state's whole-window
    survivor."""

    x = np.asarray(x, dtype=np.int64)
    lab = np.asarray(labels, dtype=np.int64)
    T, C, S = len(x), context, 1 << (L - K)
    window = [(T - C + i) % T for i in range(2 * C)]
    full = _best_by_final_state(x, lab, K, L, range(S), window)
    read = full if boundary_lag == 0 else _best_by_final_state(x, lab, K, L, range(S), window[:-1])
    cost = np.array([read[s][0] for s in range(S)], dtype=np.float64)
    final = np.array([full[s][0] for s in range(S)], dtype=np.float64)
    end_of = np.array([int(full[s][1][C] >> K) for s in range(S)], dtype=np.int64)
    return cost, final, end_of


def brute_force_through(x, labels, e: int, *, K: int, L: int, context: int) -> np.ndarray:
    """``primer_through`` by enumeration: the best window path into state
    ``e`` at the position before 0, plus the best continuation from ``e`` to
    each final state (``inf`` where none)."""

    x = np.asarray(x, dtype=np.int64)
    lab = np.asarray(labels, dtype=np.int64)
    T, C, S = len(x), context, 1 << (L - K)
    window = [(T - C + i) % T for i in range(2 * C)]
    head = _best_by_final_state(x, lab, K, L, range(S), window[:C])
    out = np.full(S, np.inf)
    if e in head:
        for s, (cost, _) in _best_by_final_state(x, lab, K, L, [e], window[C:]).items():
            out[s] = head[e][0] + cost
    return out


def brute_force_from(x, labels, end_state: int, *, K: int, L: int):
    """``encode_from`` for one tile by enumeration: the optimal closed path
    through ``end_state`` (codewords, survivor tie rule)."""

    x = np.asarray(x, dtype=np.int64)
    lab = np.asarray(labels, dtype=np.int64)
    words = _best_by_final_state(x, lab, K, L, [end_state], list(range(len(x))))[end_state][1]
    return lab[words].astype(np.float32), words.astype(np.uint16)
