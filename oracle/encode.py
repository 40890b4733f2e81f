"""Oracle: an untethered CPU encode of one matrix -- test infrastructure only.

Restates, on the CPU, the chain that ``quantize_qsrt`` runs for one
``[K = in, N = out]`` matrix (reference ``qsrt/exl3_encoder_backend.py:2754-3073``)
and the conditioned preparation of ``quantize_qsrt_batch`` (``:3076-3394``).
Everything is float64 except what the reference fixes as FP32 by contract:
the tile Viterbi's inputs and path metrics (``viterbi_ref.c``).

1. ``H <- H_sum / count + sigma_reg mean(diag) I``      (``_prepare_capture_H``, :2077-2122)
2. ``W_r, su, sv <- regularize(W, su_signs, sv_signs, g)`` at a given global
   scale ``g`` (``regularize``, :2580-2708; ``apply_g_scale``, :2727-2751)
3. ``H_c <- Had D_s H D_s Had`` with ``s`` the sign vector (``quantize_qsrt``)
   or the regularised ``su`` before ``g`` (``quantize_qsrt_batch``;
   ``_factor_capture_H``, :2125-2160)
4. ``L0`` = strictly block-lower part of ``block_ldl(H_c)`` (:323-393)
5. backward BlockLDLQ over 16-row blocks (``ldlq`` :420-539, ``ldlq_mixed``
   :898-1082): every block's ``N/16`` tiles go to ``viterbi_ref.c`` at their
   own rate, targets rounded once to FP32
6. states -> EXL words (``qsrt/qsrt.py:861-883``)

Nothing here is fed from the GPU: the test hands the same inputs (``W``,
``H_sum``, sign vectors) to both sides and, for step 2, the global scale the
GPU's search chose (the search is pinned separately).  Every piece is pinned
in its own module (``ldlq``, ``viterbi``, ``fmt``); the composition is what
the GPU encode is compared against, byte for byte.
"""

from __future__ import annotations

import numpy as np

from . import fmt
from . import ldlq as oldlq
from . import viterbi as ov


def prepare_hessian(H_sum: np.ndarray, count: int, sigma_reg: float) -> np.ndarray:
    """``H_sum / count`` damped by ``sigma_reg * mean(diag)`` on the diagonal."""

    H = np.asarray(H_sum, dtype=np.float64) / float(count)
    H = H + sigma_reg * np.mean(np.diag(H)) * np.eye(H.shape[0])
    return H


def factor(H: np.ndarray, s: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """``(H_c, L0)``: the congruence with ``s`` and the strictly block-lower
    part of its unit block LDL factor."""

    H_c = oldlq.congruence(H, s)
    L, _ = oldlq.block_ldl(H_c, 16)
    return H_c, oldlq.strictly_block_lower(L, 16)


def rows_to_tiles(rows: np.ndarray) -> np.ndarray:
    """``[16, N]`` -> ``[N/16, 256]`` in tensor-core order."""

    nt = rows.shape[1] // 16
    return rows.reshape(16, nt, 16).transpose(1, 0, 2).reshape(nt, 256)[:, fmt.tensor_core_perm()]


def tiles_to_rows(tiles: np.ndarray) -> np.ndarray:
    nt = tiles.shape[0]
    rm = np.empty_like(tiles)
    rm[:, fmt.tensor_core_perm()] = tiles
    return rm.reshape(nt, 16, 16).transpose(1, 0, 2).reshape(16, 16 * nt)


def blockldlq(W_r: np.ndarray, L0: np.ndarray, tile_bits: np.ndarray, labels: dict, lags: dict, *,
              context: int = 128, threads: int = 0) -> dict:
    """Backward BlockLDLQ with the oracle Viterbi.

    ``tile_bits [K/16, N/16]`` gives each tile's rate; ``labels[K]`` the
    state-indexed float table and ``lags[K]`` the boundary rule of that rate.
    Returns ``states uint16 [K/16, N/16, 256]``, ``targets float32
    [K/16, N/16, 256]`` (tensor-core order, what each Viterbi call saw) and
    ``Q float64 [K, N]``.
    """

    W_r = np.asarray(W_r, dtype=np.float64)
    k, n = W_r.shape
    kt, nt = k // 16, n // 16
    tile_bits = np.asarray(tile_bits)
    if tile_bits.shape != (kt, nt):
        raise ValueError("tile_bits must be [K/16, N/16]")
    states = np.zeros((kt, nt, 256), dtype=np.uint16)
    targets = np.zeros((kt, nt, 256), dtype=np.float32)

    def quantize_rows(t: np.ndarray, rb: int) -> np.ndarray:
        tiles = rows_to_tiles(t).astype(np.float32)
        targets[rb] = tiles
        recon = np.empty_like(tiles)
        for bits in sorted(set(tile_bits[rb].tolist())):
            where = np.flatnonzero(tile_bits[rb] == bits)
            r, s = ov.encode(tiles[where], labels[bits], K=int(bits), context=context, boundary_lag=lags[bits],
                             threads=threads)
            recon[where] = r
            states[rb, where] = s
        return tiles_to_rows(recon).astype(np.float64)

    Q, _ = oldlq.ldlq(W_r, L0, quantize_rows, 16)
    return {"states": states, "targets": targets, "Q": Q}


def encode_matrix(W: np.ndarray, H_sum: np.ndarray, count: int, su_signs: np.ndarray, sv_signs: np.ndarray,
                  g_scale: float, tile_bits: np.ndarray, labels: dict, lags: dict, *, sigma_reg: float,
                  conditioned: bool = False, g_into_sv: bool = False, input_scales: np.ndarray | None = None,
                  apply_out_scales: bool = False, context: int = 128, threads: int = 0) -> dict:
    """The whole chain for one matrix.  ``conditioned`` selects the batch
    preparation (congruence with the regularised ``su`` before ``g``)
    instead of the sign vector; ``g_into_sv``, ``input_scales`` and
    ``apply_out_scales`` are the options of ``regularize``.  Returns the
    ``blockldlq`` dict plus ``W_r``, ``su``, ``sv``, ``H_c`` and ``L0``."""

    H = prepare_hessian(H_sum, count, sigma_reg)
    W_r, su, sv = oldlq.regularize(W, su_signs, sv_signs, g_scale, g_into_sv=g_into_sv, input_scales=input_scales,
                                   apply_out_scales=apply_out_scales)
    if conditioned:
        s = su if g_into_sv else su * g_scale
    else:
        s = np.asarray(su_signs, dtype=np.float64).reshape(-1, 1)
    H_c, L0 = factor(H, s)
    out = blockldlq(W_r, L0, tile_bits, labels, lags, context=context, threads=threads)
    out.update({"W_r": W_r, "su": su, "sv": sv, "H_c": H_c, "L0": L0})
    return out


def proxy(W_r: np.ndarray, Q: np.ndarray, H_c: np.ndarray) -> float:
    """``tr(E^T H E) / tr(W^T H W)`` (reference ``block_trace``, :1951-1977)."""

    E = W_r - Q
    return float(np.sum(E * (H_c @ E)) / max(np.sum(W_r * (H_c @ W_r)), 1e-8))


def tile_sse(labels_tiles: np.ndarray, targets: np.ndarray) -> np.ndarray:
    """Squared error of each tile's reconstruction against its target,
    float64 ``[..., 256] -> [...]``."""

    d = np.asarray(labels_tiles, dtype=np.float64) - np.asarray(targets, dtype=np.float64)
    return np.sum(d * d, axis=-1)


def compare_states(gpu_states: np.ndarray, cpu: dict, labels: dict, tile_bits: np.ndarray, lags: dict, *,
                   context: int = 128) -> dict:
    """Tile-level agreement of a GPU encode with ``cpu`` (a ``blockldlq``
    result on the same inputs).

    Feedback flows only along K inside one tile column (target rows of block
    ``b`` depend on ``(W - Q)`` rows below it, same columns), so a tile that
    differs while every tile below it in its column agrees saw the same target
    up to rounding: that is a resolution of a near-tie (``first``).  Tiles
    above a differing tile in the same column saw different targets
    (``propagated``).

    A ``first`` tile is one of two kinds, told apart by the state before
    position 0 (``codeword[0] >> K``, the tile's end_state):

    * ``path``: both encodes chose the same end_state, so both paths are
      closed paths through it and the constrained pass resolved a tie; the
      delta is the relative SSE of the two paths on the CPU target;
    * ``boundary``: the end_states differ, i.e. the primer's choice resolved a
      tie (between two read costs, or between two primer paths into the
      chosen state that pass through different boundary states).  The delta
      is the GPU path's relative SSE against the best closed path through the
      GPU's own end_state, and the margin says how close the primer came to
      choosing that end_state: the least, over states ``s``, of the larger of
      ``s``'s read cost above the minimum and the cost of the best primer
      path into ``s`` through the GPU's end_state above ``s``'s final cost,
      both relative (0 for a ``path`` tile; ``inf`` if no primer path
      reaches it).  Both are on the CPU target."""

    g = np.asarray(gpu_states, dtype=np.uint16)
    c = cpu["states"]
    kt, nt, _ = c.shape
    differ = np.any(g != c, axis=2)
    first, kinds, propagated, deltas, margins = [], [], [], [], []
    for col in range(nt):
        seen = False
        for rb in range(kt - 1, -1, -1):  # the recursion's order: bottom block first
            if not differ[rb, col]:
                continue
            if seen:
                propagated.append((rb, col))
                continue
            seen = True
            first.append((rb, col))
            bits = int(tile_bits[rb, col])
            lab = labels[bits]
            t = cpu["targets"][rb, col]
            sse_g = tile_sse(lab[g[rb, col].astype(np.int64)], t)
            end_g, end_c = int(g[rb, col, 0]) >> bits, int(c[rb, col, 0]) >> bits
            if end_g == end_c:
                kinds.append("path")
                sse_c = tile_sse(lab[c[rb, col].astype(np.int64)], t)
                deltas.append(abs(sse_g - sse_c) / max(sse_c, 1e-30))
                margins.append(0.0)
                continue
            kinds.append("boundary")
            _, best = ov.encode_from(t[None], lab, [end_g], K=bits, threads=1)
            sse_b = tile_sse(lab[best[0].astype(np.int64)], t)
            deltas.append(abs(sse_g - sse_b) / max(sse_b, 1e-30))
            cost, final, _ = ov.boundary_view(t, lab, K=bits, context=context, boundary_lag=lags[bits])
            through = ov.primer_through(t, lab, end_g, K=bits, context=context).astype(np.float64)
            read_gap = (cost.astype(np.float64) - float(cost.min())) / max(float(cost.min()), 1e-30)
            with np.errstate(invalid="ignore"):
                path_gap = (through - final) / np.maximum(final.astype(np.float64), 1e-30)
            margin = np.maximum(read_gap, path_gap)
            margins.append(float(np.nanmin(margin)) if np.isfinite(margin).any() else float("inf"))
    return {
        "tiles": int(kt * nt),
        "differ": int(differ.sum()),
        "first": first,
        "kinds": kinds,
        "propagated": len(propagated),
        "sse_rel_deltas": deltas,
        "boundary_margins": margins,
        "mismatch_rate": float(differ.sum()) / float(kt * nt),
        "states_differing": int(np.sum(g != c)),
    }
