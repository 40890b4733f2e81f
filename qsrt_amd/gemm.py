"""Dense products of the BlockLDLQ recursion and of Hessian capture.

Device tensors run the HIP matrix-core kernels behind ``qsrt_gemm_tn`` and
``qsrt_gemm_tn_f64`` (``include/qsrt_amd.h``): the BlockLDLQ feedback
``C += A^T (B - B2)`` (reference ``exl3_encoder_backend.py:496``, ``:534``,
batched ``:1170-1187``) with float64 factor, weight and product cache and an
FP32 reconstruction ``B2`` on the float64 matrix cores, or all-FP32 operands
on the FP32 ones; bf16 operands for ``H += X^T X``.  CPU tensors use torch.
"""

from __future__ import annotations

import torch

from . import _native


def _row_major(t: torch.Tensor) -> bool:
    return t.dim() == 2 and t.stride(1) == 1 and t.stride(0) >= t.shape[1]


def _launch(C, A, B, B2, alpha, dtype):
    K, M = A.shape
    N = B.shape[1]
    lib = _native.lib()
    args = (C.data_ptr(), A.data_ptr(), B.data_ptr())
    lds = (A.stride(0), B.stride(0), C.stride(0))
    # the split tiles' partial products (bf16 tile counts that leave the last round of CUs part-empty) go to a
    # workspace from torch's stream-ordered allocator
    nbytes = lib.qsrt_gemm_tn_workspace_bytes(*args, M, N, K, *lds, dtype)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=C.device) if nbytes else None
    _native.check(
        lib.qsrt_gemm_tn_ws(*args, None if B2 is None else B2.data_ptr(), M, N, K, *lds, float(alpha), dtype,
                            None if ws is None else ws.data_ptr(), nbytes, _native.stream_handle(C.device)),
        "qsrt_gemm_tn_ws",
    )


def _copy_padded(t: torch.Tensor, ld: int) -> torch.Tensor:
    rows, cols = t.shape
    view = torch.empty((rows, ld), dtype=t.dtype, device=t.device)[:, :cols]
    view.copy_(t)
    return view


def _aligned(t: torch.Tensor, multiple: int = 4) -> torch.Tensor:
    """``t`` as a row-major matrix with a 16-byte aligned base and a leading
    dimension that is a multiple of ``multiple`` elements (copied into a
    padded buffer when needed): the kernels read 16 bytes at a time."""

    if _row_major(t) and t.data_ptr() % 16 == 0 and t.stride(0) % multiple == 0:
        return t
    return _copy_padded(t, (t.shape[1] + multiple - 1) // multiple * multiple)


def addmm_sub_tn_(C: torch.Tensor, A: torch.Tensor, B: torch.Tensor, B2: torch.Tensor | None = None,
                  alpha: float = 1.0) -> torch.Tensor:
    """``C += alpha * A^T (B - B2)`` in place (``B2`` optional)."""

    K, M = A.shape
    if B.shape[0] != K or C.shape != (M, B.shape[1]) or (B2 is not None and B2.shape != B.shape):
        raise ValueError("addmm_sub_tn_: incompatible shapes")
    if C.is_cuda and C.dtype == torch.float64:
        return _addmm_sub_tn_f64_(C, A, B, B2, alpha)
    if C.is_cuda:
        if C.dtype != torch.float32 or A.dtype != torch.float32 or B.dtype != torch.float32:
            raise ValueError("addmm_sub_tn_: float32 operands expected")
        A, B = _aligned(A), _aligned(B)
        if B2 is not None:
            B2 = _aligned(B2)
            if B2.stride(0) != B.stride(0):  # one leading dimension serves both
                ld = (B.shape[1] + 3) // 4 * 4
                B, B2 = _copy_padded(B, ld), _copy_padded(B2, ld)
        if not _row_major(C):
            raise ValueError("addmm_sub_tn_: C must be row-major")
        _launch(C, A, B, B2, alpha, 0)
        return C
    rhs = B if B2 is None else B - B2.to(B.dtype)
    return C.addmm_(A.T, rhs.to(C.dtype), alpha=alpha)


def _addmm_sub_tn_f64_(C, A, B, B2, alpha):
    """Float64 ``C``, ``A``, ``B`` and an FP32 (or absent) ``B2`` on the
    float64 matrix cores."""

    if A.dtype != torch.float64 or B.dtype != torch.float64 or (B2 is not None and B2.dtype != torch.float32):
        raise ValueError("addmm_sub_tn_: a float64 C takes float64 A and B and a float32 B2")
    if not _row_major(C) or C.stride(0) % 2:
        raise ValueError("addmm_sub_tn_: C must be row-major with an even leading dimension")
    A, B = _aligned(A, 2), _aligned(B, 2)
    if B2 is not None and (not _row_major(B2) or B2.stride(0) % 2 or B2.data_ptr() % 8):
        B2 = _copy_padded(B2, (B2.shape[1] + 1) // 2 * 2)
    K, M = A.shape
    N = B.shape[1]
    _native.check(
        _native.lib().qsrt_gemm_tn_f64(C.data_ptr(), A.data_ptr(), B.data_ptr(), None if B2 is None else B2.data_ptr(),
                                       M, N, K, A.stride(0), B.stride(0), 0 if B2 is None else B2.stride(0),
                                       C.stride(0), float(alpha), _native.stream_handle(C.device)),
        "qsrt_gemm_tn_f64",
    )
    return C


def baddmm_sub_tn_f64_(C: torch.Tensor, A: torch.Tensor, B: torch.Tensor, B2: torch.Tensor | None = None,
                       alpha: float = 1.0) -> torch.Tensor:
    """Per member ``C[b] += alpha * A[b]^T (B[b] - B2[b])`` in one launch on
    the float64 matrix cores (the batched BlockLDLQ span product; the
    reference's ``_baddbmm_ldlq``, ``qsrt/exl3_encoder_backend.py:1170-1187``).
    ``C``, ``A``, ``B`` float64 and ``B2`` float32 (or None), each
    ``[batch, rows, cols]`` with row-major members at a uniform member
    stride.  Every element equals what ``addmm_sub_tn_`` computes for its
    member."""

    if C.dim() != 3 or A.dim() != 3 or B.dim() != 3 or (B2 is not None and B2.dim() != 3):
        raise ValueError("baddmm_sub_tn_f64_: [batch, rows, cols] operands expected")
    batch, K, M = A.shape
    if (B.shape[0] != batch or B.shape[1] != K or C.shape != (batch, M, B.shape[2])
            or (B2 is not None and B2.shape != B.shape)):
        raise ValueError("baddmm_sub_tn_f64_: incompatible shapes")
    if A.dtype != torch.float64 or B.dtype != torch.float64 or C.dtype != torch.float64 or (
            B2 is not None and B2.dtype != torch.float32):
        raise ValueError("baddmm_sub_tn_f64_: float64 C, A, B and a float32 B2 expected")
    if not C.is_cuda:
        rhs = B if B2 is None else B - B2.to(B.dtype)
        return C.baddbmm_(A.transpose(1, 2), rhs, alpha=alpha)
    N = B.shape[2]

    def members_ok(t, align):
        return (t.stride(2) == 1 and t.stride(1) % 2 == 0 and t.stride(0) % 2 == 0 and t.data_ptr() % align == 0
                and t.stride(1) >= t.shape[2])

    if batch <= 1 or not (members_ok(C, 8) and members_ok(A, 16) and members_ok(B, 16)
                          and (B2 is None or members_ok(B2, 8)) and C.stride(0) >= (M - 1) * C.stride(1) + N):
        for b in range(batch):
            addmm_sub_tn_(C[b], A[b], B[b], None if B2 is None else B2[b], alpha=alpha)
        return C
    _native.check(
        _native.lib().qsrt_gemm_tn_f64_batched(
            C.data_ptr(), A.data_ptr(), B.data_ptr(), None if B2 is None else B2.data_ptr(), batch, M, N, K,
            A.stride(1), B.stride(1), 0 if B2 is None else B2.stride(1), C.stride(1), C.stride(0), A.stride(0),
            B.stride(0), 0 if B2 is None else B2.stride(0), float(alpha), _native.stream_handle(C.device)),
        "qsrt_gemm_tn_f64_batched",
    )
    return C


def addmm_tn_(C: torch.Tensor, A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """``C += A^T @ B`` in FP32."""

    return addmm_sub_tn_(C, A, B)


def baddbmm_tn_(C: torch.Tensor, A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """Per batch member ``C[b] += A[b]^T @ B[b]``."""

    for b in range(C.shape[0]):
        addmm_sub_tn_(C[b], A[b], B[b])
    return C


def gram_(H: torch.Tensor, X: torch.Tensor, alpha: float = 1.0) -> torch.Tensor:
    """``H += alpha * X^T X`` (Hessian capture); bf16 ``X`` on the bf16 matrix
    cores, float32 ``X`` on the FP32 path."""

    n, k = X.shape
    if H.shape != (k, k) or H.dtype != torch.float32:
        raise ValueError("gram_: H must be float32 [k, k]")
    if H.is_cuda:
        if not _row_major(H):
            raise ValueError("gram_: H must be row-major")
        if X.dtype == torch.bfloat16:
            X = _aligned(X, 8)
            _launch(H, X, X, None, alpha, 1)
        elif X.dtype == torch.float32:
            X = _aligned(X)
            _launch(H, X, X, None, alpha, 0)
        else:
            raise ValueError("gram_: X must be bfloat16 or float32")
        return H
    Xf = X.float()
    return H.addmm_(Xf.T, Xf, alpha=alpha)
