"""Dense products of the BlockLDLQ recursion and of Hessian capture.

``addmm_tn_(C, A, B)``: ``C += A^T @ B`` in FP32 (the LDLQ feedback
products, reference ``exl3_encoder_backend.py:496``, ``:534``).
``baddbmm_tn_``: the same per batch member.
"""

from __future__ import annotations

import torch


def _fp32_matmul_policy():
    # IEEE FP32 products: TF32 would change the feedback targets.
    torch.backends.cuda.matmul.allow_tf32 = False


def addmm_tn_(C: torch.Tensor, A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    _fp32_matmul_policy()
    return C.addmm_(A.T, B)


def baddbmm_tn_(C: torch.Tensor, A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    _fp32_matmul_policy()
    return C.baddbmm_(A.transpose(1, 2), B)
