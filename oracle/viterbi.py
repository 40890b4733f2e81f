"""Oracle: tail-biting tile Viterbi -- test infrastructure only.

``encode`` binds ``viterbi_ref.c`` (the FP32 C restatement of the
reference's pass structure; see its header).  ``brute_force`` is an
independent exhaustive search over closed paths for tiny trellises, used to
pin the C restatement:

* pinned by brute force (``tests/test_oracle_viterbi.py``) on small L/K/T
  with exact integer arithmetic, including the lowest-index tie rules;
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
