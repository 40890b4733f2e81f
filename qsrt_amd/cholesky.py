"""Float64 Cholesky factorisation of the damped Hessian (the factorisation
inside ``block_ldl``, reference ``qsrt/exl3_encoder_backend.py:323-393``).

One matrix on the device: a right-looking blocked factorisation with
128-row blocks.  Each diagonal block is factored, and inverted, by one HIP
workgroup (``qsrt_chol_diag_block_f64``); the panel solve
``L21 = A21 L11^-T`` and the trailing update ``A22 -= L21 L21^T`` are DGEMMs.
A batch of matrices goes to rocsolver's batched Cholesky, which amortises
its own diagonal-block chain across the batch.  Either way the result is
``torch.linalg.cholesky_ex``'s contract: the lower factor with zeros above
the diagonal and a LAPACK-style ``info`` (0, or the order of the first
leading minor that is not positive definite).
"""

from __future__ import annotations

import torch

from . import _native

BLOCK = 128


def _blocked(A: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    n = A.shape[-1]
    C = A.contiguous().clone()
    info = torch.zeros(1, dtype=torch.int32, device=A.device)
    inv = torch.empty(BLOCK * BLOCK, dtype=torch.float64, device=A.device)
    lib = _native.lib()
    stream = _native.stream_handle(A.device)
    for j in range(0, n, BLOCK):
        e = min(j + BLOCK, n)
        w = e - j
        _native.check(lib.qsrt_chol_diag_block_f64(C.data_ptr(), n, 1, n * n, j, w, inv.data_ptr(),
                                                    info.data_ptr(), stream), "qsrt_chol_diag_block_f64")
        if e < n:
            x_t = inv[:w * w].view(w, w).t().contiguous()
            panel = torch.mm(C[e:, j:e], x_t)
            C[e:, j:e] = panel
            C[e:, e:].addmm_(panel, panel.t().contiguous(), alpha=-1.0)
    C.tril_()
    return C, info[0]


def cholesky_f64(A: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``(L, info)`` of a float64 ``[n, n]`` or ``[B, n, n]`` tensor, as
    ``torch.linalg.cholesky_ex`` returns them."""

    if A.dtype != torch.float64:
        raise TypeError("cholesky_f64 takes float64 matrices")
    if A.device.type != "cuda" or (A.ndim == 3 and A.shape[0] != 1):
        return torch.linalg.cholesky_ex(A)
    if A.ndim == 3:
        L, info = _blocked(A[0])
        return L.unsqueeze(0), info.unsqueeze(0)
    return _blocked(A)
