"""Oracle: dense-H block-coordinate path refinement -- test infrastructure only.

Restates, on the CPU in float64, the sweep of
``qsrt/h2_viterbi_refine.py:330-563`` (``refine_h2_viterbi_paths``), with
the conditional target in the reference's own form (``:225-248``)

    t_b = W_b + H_bb^-1 (sum_{j != b} H_bj E_j)    [- s/2 H_bb^-1 g_b / a]

recomputed from scratch at every block (no incremental product), the
H-whitened dithers of ``:187-222`` (probes from a seeded CPU torch
generator, the build's choice), the column-weighted scores of ``:251-265``
and the acceptance rule ``best + abs_tol + rel_tol |current| < current``
(``:489-493``), each tile keeping its lowest-index best candidate.
``viterbi_ref.c`` proposes the paths (targets rounded once to FP32).

Pinned in ``tests/test_refine_oracle.py`` by mathematics, not by restating
these lines: for any candidate block the change of the full dense objective
equals the change of the block score (the conditional-target identity, with
and without a linear term and column weights); each step's choice is the
brute-force minimiser of the full objective over its candidate set; under
``H = I`` the target is the source itself, so a BlockLDLQ encode has
nothing to improve; the dithers satisfy ``L^T p = +-1`` and ``p^T H_bb p =
256``; the objective never rises.
"""

from __future__ import annotations

import numpy as np
import torch

from .encode import rows_to_tiles, tiles_to_rows

B = 16


def objective(W, Q, H, a=None, grad=None, anchor=None, strength=0.0) -> float:
    """``sum_c a_c e_c^T H e_c + strength <g, Q - anchor>``, ``E = W - Q``."""

    E = np.asarray(W, np.float64) - np.asarray(Q, np.float64)
    a = np.ones(E.shape[1]) if a is None else np.asarray(a, np.float64)
    quad = float(np.sum(E * (np.asarray(H, np.float64) @ E) * a[None, :]))
    if grad is None or strength == 0.0:
        return quad
    return quad + float(strength) * float(np.sum(np.asarray(grad, np.float64) * (np.asarray(Q, np.float64) - anchor)))


def conditional_target(W, Q, H, b: int, a=None, grad=None, strength: float = 0.0) -> np.ndarray:
    """Block ``b``'s conditional target ``[16, N]``."""

    r = slice(B * b, B * b + B)
    E = np.asarray(W, np.float64) - np.asarray(Q, np.float64)
    Hbb = H[r, r]
    cross = H[r, :] @ E - Hbb @ E[r]
    t = W[r] + np.linalg.solve(Hbb, cross)
    if grad is not None and strength != 0.0:
        a = np.ones(E.shape[1]) if a is None else np.asarray(a, np.float64)
        t = t - 0.5 * float(strength) * np.linalg.solve(Hbb, grad[r] / a[None, :])
    return t


def tile_scores(target, cands, Hbb, a=None) -> np.ndarray:
    """``[tiles, M]``: per 16-column tile, ``sum_c a_c d_c^T H_bb d_c`` with
    ``d = target - cand`` over that tile's columns."""

    target = np.asarray(target, np.float64)
    n = target.shape[1]
    a = np.ones(n) if a is None else np.asarray(a, np.float64)
    out = np.empty((n // B, len(cands)))
    for m, c in enumerate(cands):
        d = target - np.asarray(c, np.float64)
        per_col = np.einsum("ic,ic->c", d, Hbb @ d) * a
        out[:, m] = per_col.reshape(n // B, B).sum(axis=1)
    return out


def whitened_patterns(Hbb, count: int, seed: int) -> np.ndarray:
    """``count`` patterns ``L^-T p`` (``L L^T = H_bb``, ``p`` in {-1, 1}^{16x16}
    from ``torch.Generator().manual_seed(seed)``) scaled to energy 256."""

    g = torch.Generator().manual_seed(int(seed))
    probes = (torch.randint(0, 2, (count, B, B), generator=g, dtype=torch.int64) * 2 - 1).numpy().astype(np.float64)
    L = np.linalg.cholesky(Hbb)
    pats = np.stack([np.linalg.solve(L.T, p) for p in probes])
    energy = np.array([np.sum(p * (Hbb @ p)) for p in pats])
    return pats * np.sqrt(B * B / np.maximum(energy, 1e-20))[:, None, None]


def refine(W, H, Q0, states0, quantize, *, sweeps: int = 1, alternate: bool = True, dither_scales=(),
           patterns: int = 0, seed: int = 0x48325643, abs_tol: float = 1e-8, rel_tol: float = 1e-8, a=None,
           grad=None, anchor=None, strength: float = 0.0, stop_on_no_change: bool = True, record=None) -> dict:
    """Sweeps of the refinement.  ``quantize(tiles f32 [T, 256]) -> (recon,
    states)`` in tensor-core order.  Returns ``Q`` (FP32 values), ``states
    [K/16, N/16, 256]`` and per-sweep ``accepted`` counts and objectives.
    ``record`` (a list) receives ``(b, target, cands, scores, choice)`` per
    step for the brute-force checks."""

    W = np.asarray(W, np.float64)
    H = np.asarray(H, np.float64)
    H = 0.5 * (H + H.T)
    Q = np.asarray(Q0, np.float32).astype(np.float64)
    states = np.array(states0, copy=True)
    k, n = W.shape
    nt = n // B
    a_vec = np.ones(n) if a is None else np.asarray(a, np.float64)
    obj = objective(W, Q, H, a_vec, grad, anchor, strength)
    hist = []
    for sweep in range(sweeps):
        before = obj
        accepted = 0
        order = range(k // B - 1, -1, -1) if (not alternate or sweep % 2 == 0) else range(k // B)
        for b in order:
            r = slice(B * b, B * b + B)
            t = conditional_target(W, Q, H, b, a_vec, grad, strength)
            variants = [t]
            if patterns > 0 and dither_scales:
                pats = whitened_patterns(H[r, r], patterns, seed + 1009 * sweep + 9176 * b)
                t_tiles = t.reshape(B, nt, B).transpose(1, 0, 2)
                rms = np.maximum(np.sqrt(np.mean(t_tiles ** 2, axis=(1, 2))), 1e-8)
                for s in dither_scales:
                    for p in pats:
                        shift = (float(s) * rms[:, None, None] * p[None]).transpose(1, 0, 2).reshape(B, n)
                        variants.extend((t + shift, t - shift))
            cands, cand_states = [Q[r].copy()], [states[b].copy()]
            for v in variants:
                recon, st = quantize(rows_to_tiles(v).astype(np.float32))
                cands.append(tiles_to_rows(np.asarray(recon, np.float32)).astype(np.float64))
                cand_states.append(np.asarray(st).astype(states.dtype))
            scores = tile_scores(t, cands, H[r, r], a_vec)
            best = scores.min(axis=1)
            choice = np.argmax(scores == best[:, None], axis=1)  # lowest index among exact ties
            accept = best + (abs_tol + rel_tol * np.abs(scores[:, 0])) < scores[:, 0]
            choice = np.where(accept, choice, 0)
            if record is not None:
                record.append((b, t, cands, scores, choice))
            accepted += int(accept.sum())
            for j in np.nonzero(accept)[0]:
                cols = slice(B * j, B * j + B)
                Q[r, cols] = cands[choice[j]][:, cols]
                states[b, j] = cand_states[choice[j]][j]
        obj = objective(W, Q, H, a_vec, grad, anchor, strength)
        hist.append({"sweep": sweep, "before": before, "after": obj, "accepted": accepted})
        if obj > before + max(1e-5, 1e-6 * abs(before)):
            raise RuntimeError("dense-H objective increased")
        if stop_on_no_change and accepted == 0:
            break
    return {"Q": Q.astype(np.float32), "states": states, "sweeps": hist}
