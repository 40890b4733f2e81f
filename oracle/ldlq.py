"""Oracle: BlockLDLQ algebra and regularisation in float64 -- test
infrastructure only.

Restates ``qsrt/exl3_encoder_backend.py``:
* ``block_ldl`` (:323-393): Cholesky C, L = C blockdiag(C_ii)^-1 -- pinned
  by L D L^T == H with D = blockdiag(C_ii C_ii^T) and unit diagonal blocks
  (the check of ``tests/test_blockldlq_proof.py:31-60``);
* the reverse feedback targets of ``ldlq`` (:420-539): block b is quantized
  against W_b + sum_{r > b} L_rb^T (W - Q)_r, i.e. T = W + L0^T (W - Q) with
  L0 the strictly block-lower part -- pinned by the identity
  T - Q == (I + L0^T)(W - Q) for an arbitrary quantizer
  (``tests/test_blockldlq_proof.py:62-95``) and by a direct per-block loop;
* ``regularize`` (:2580-2708) up to the global-scale search, its output-
  scale rule ``out_scale_policy`` (:2605-2628) and the Hessian congruence
  of ``_factor_capture_H`` (:2125-2160): no reference test or fixture holds
  values for them (the reference backend cannot be imported here).  They
  are pinned by the mathematics instead: the congruence equals T H T^T with
  T = (I (x) H_128) D_su built densely from scipy's Sylvester Hadamard,
  keeps H's spectrum and fixes I; the regularisation is inverted exactly by
  the decoder's formula, gives every 128-row block an RMS of
  g * 1.24371088, and returns su = -su rms_rows(W) / (1.24371088 g) in
  closed form; with output scales every live column of W / sv has the mean
  column RMS of W; the policy's share on a diagonal built from two values
  has a closed form.  The constants 1.24371088, 2% and 15% are the
  reference's (:2580-2708).
"""

from __future__ import annotations

import numpy as np

from .fmt import hadamard

CODEBOOK_SCALE = 1.24371088


def block_ldl(H: np.ndarray, b: int = 16):
    """Return (L unit block-lower, D block-diagonal blocks [m, b, b])."""

    H = np.asarray(H, dtype=np.float64)
    n = H.shape[0]
    m = n // b
    C = np.linalg.cholesky(H)
    blocks = np.stack([C[i * b:(i + 1) * b, i * b:(i + 1) * b] for i in range(m)])
    L = C.copy()
    for i in range(m):
        L[:, i * b:(i + 1) * b] = C[:, i * b:(i + 1) * b] @ np.linalg.inv(blocks[i])
    for i in range(m):
        L[i * b:(i + 1) * b, i * b:(i + 1) * b] = np.eye(b)
    D = np.einsum("mij,mkj->mik", blocks, blocks)
    return L, D


def strictly_block_lower(L: np.ndarray, b: int = 16) -> np.ndarray:
    L0 = np.array(L, dtype=np.float64, copy=True)
    for i in range(L0.shape[0] // b):
        L0[i * b:(i + 1) * b, i * b:(i + 1) * b] = 0.0
    return L0


def feedback_targets(W: np.ndarray, L0: np.ndarray, Q: np.ndarray) -> np.ndarray:
    """T = W + L0^T (W - Q) (float64)."""

    W = np.asarray(W, dtype=np.float64)
    return W + np.asarray(L0, dtype=np.float64).T @ (W - np.asarray(Q, dtype=np.float64))


def ldlq(W: np.ndarray, L0: np.ndarray, quantize_rows, b: int = 16):
    """Float64 backward recursion block by block with a caller-supplied
    quantizer ``quantize_rows(target_rows [16, N], row_block) -> Q rows``."""

    W = np.asarray(W, dtype=np.float64)
    Q = np.zeros_like(W)
    targets = np.zeros_like(W)
    k = W.shape[0]
    for blk_end in range(k, 0, -b):
        blk = blk_end - b
        t = W[blk:blk_end] + L0[blk_end:, blk:blk_end].T @ (W[blk_end:] - Q[blk_end:])
        targets[blk:blk_end] = t
        Q[blk:blk_end] = quantize_rows(t, blk // b)
    return Q, targets


def congruence(H: np.ndarray, su_signs: np.ndarray) -> np.ndarray:
    """Had D_su H D_su Had on 128-blocks (``_factor_capture_H``)."""

    H = np.asarray(H, dtype=np.float64)
    s = np.asarray(su_signs, dtype=np.float64).reshape(-1)
    k = H.shape[0]
    h = hadamard(128)
    M = (s[:, None] * H) * s[None, :]
    M = np.einsum("ij,bjn->bin", h, M.reshape(k // 128, 128, k)).reshape(k, k)
    return np.einsum("kbj,ji->kbi", M.reshape(k, k // 128, 128), h).reshape(k, k)


def out_scale_policy(H_diag, forced, q_fallback: bool = False):
    """Whether ``regularize`` applies output-channel scales (reference
    :2605-2628): with a Hessian diagonal, when the largest 2% (``n // 50``)
    of its square roots hold under 15% of their sum; ``forced`` (True or
    False) overrides the rule; without a diagonal the default is True; a
    fallback encode takes ``forced`` as it is."""

    if q_fallback:
        return forced
    if H_diag is None:
        return True if forced is None else forced
    root = np.sort(np.sqrt(np.asarray(H_diag, dtype=np.float64).reshape(-1)))[::-1]
    share = root[: root.shape[0] // 50].sum() / root.sum()
    return bool(share < 0.15) if forced is None else forced


def regularize(weight: np.ndarray, su_signs: np.ndarray, sv_signs: np.ndarray, g_scale: float, *,
               g_into_sv: bool = False, input_scales: np.ndarray | None = None, apply_out_scales: bool = False):
    """Regularisation at a fixed global scale: column RMS c of W normalised
    to mean 1 (dead columns at 0.1), sv = sv * c + 1e-10 when
    ``apply_out_scales``; W /= sv; sv of all-zero columns set to 0;
    W <- W Had; su = su * rms_rows(W) / -1.24371088 + 1e-10; W /= su;
    W <- Had W; W *= g; su /= g (sv /= g with ``g_into_sv``, as
    ``g_scale_into_sv`` does for w1/w3, :2727-2751).  ``input_scales``
    replaces rms_rows(W) by a layer-shared profile (the reference's
    ``shared_input_scales_key``, :2669-2672).  Returns (W, su, sv) in
    float64."""

    W = np.asarray(weight, dtype=np.float64).copy()
    k, n = W.shape
    sv = np.asarray(sv_signs, dtype=np.float64).reshape(1, n).copy()
    su = np.asarray(su_signs, dtype=np.float64).reshape(k, 1)
    h = hadamard(128)
    cols = np.sqrt((W * W).mean(axis=0, keepdims=True))
    mean = float(cols.mean())
    if mean > 1e-30:
        cols = cols / mean
    dead = np.abs(cols) < 1e-30
    if apply_out_scales:
        cols[dead] = 0.1
        sv = sv * cols + 1e-10
    W /= sv
    sv[dead] = 0.0
    W = np.einsum("kbj,ji->kbi", W.reshape(k, n // 128, 128), h).reshape(k, n)
    if input_scales is None:
        rms = np.sqrt((W * W).mean(axis=1, keepdims=True))
        rms[np.abs(rms) < 1e-30] = 0.1
    else:
        rms = np.asarray(input_scales, dtype=np.float64).reshape(k, 1)
    su = su * rms / (-CODEBOOK_SCALE) + 1e-10
    W /= su
    W = np.einsum("ij,bjn->bin", h, W.reshape(k // 128, 128, n)).reshape(k, n)
    W *= g_scale
    if g_into_sv:
        sv = sv / g_scale
    else:
        su = su / g_scale
    return W, su, sv


def input_rms(weight: np.ndarray, sv_signs: np.ndarray) -> np.ndarray:
    """rms_rows(W / sv @ Had): the input-channel profile ``regularize``
    derives (and a layer-shared key reuses)."""

    W = np.asarray(weight, dtype=np.float64)
    k, n = W.shape
    W = W / np.asarray(sv_signs, dtype=np.float64).reshape(1, n)
    W = np.einsum("kbj,ji->kbi", W.reshape(k, n // 128, 128), hadamard(128)).reshape(k, n)
    rms = np.sqrt((W * W).mean(axis=1, keepdims=True))
    rms[np.abs(rms) < 1e-30] = 0.1
    return rms
