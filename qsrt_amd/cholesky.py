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


def block_unit_lower_f64_(C: torch.Tensor, inv_blocks: torch.Tensor) -> torch.Tensor:
    """In place, ``C [B, n, n]`` (lower Cholesky factors, zeros above the
    diagonal) becomes ``C blockdiag(C_jj)^-1`` with exact identity diagonal
    blocks, for 16 x 16 blocks whose inverses ``inv_blocks [B, n / 16, 16,
    16]`` the caller supplies (the column-block products of ``block_ldl``,
    reference ``qsrt/exl3_encoder_backend.py:375-390``).  Device tensors go
    through ``qsrt_block_unit_lower_f64``; CPU tensors take the same
    products in torch."""

    if C.dtype != torch.float64 or inv_blocks.dtype != torch.float64:
        raise TypeError("block_unit_lower_f64_ takes float64 tensors")
    if C.ndim != 3 or C.shape[1] != C.shape[2] or C.shape[1] % 16:
        raise ValueError("C must be [B, n, n] with n a multiple of 16")
    B, n, _ = C.shape
    m = n // 16
    if tuple(inv_blocks.shape) != (B, m, 16, 16):
        raise ValueError(f"inv_blocks must be [{B}, {m}, 16, 16], got {tuple(inv_blocks.shape)}")
    if C.device.type == "cuda":
        rs, cs = C.stride(1), C.stride(2)
        if 1 not in (rs, cs) or max(rs, cs) < n or (B > 1 and C.stride(0) < (n - 1) * max(rs, cs) + n):
            raise ValueError("C must hold row- or column-major n x n matrices that do not overlap")
        inv = inv_blocks.contiguous()
        lib = _native.lib()
        _native.check(lib.qsrt_block_unit_lower_f64(C.data_ptr(), inv.data_ptr(), B, n, rs, cs, C.stride(0),
                                                    _native.stream_handle(C.device)), "qsrt_block_unit_lower_f64")
        return C
    for i in range(B):
        cols = C[i].view(n, m, 16).transpose(0, 1)
        cols.copy_(torch.bmm(cols.contiguous(), inv_blocks[i]))
    blocks = C.view(B, m, 16, m, 16).permute(0, 1, 3, 2, 4)
    idx = torch.arange(m, device=C.device)
    blocks[:, idx, idx] = torch.eye(16, device=C.device, dtype=C.dtype).expand(B, m, 16, 16)
    return C
