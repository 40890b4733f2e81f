"""The unit block-lower factor of ``block_ldl`` (reference
``qsrt/exl3_encoder_backend.py:323-393``) on the CPU path of
``qsrt_amd.cholesky.block_unit_lower_f64_`` and ``_block_ldl_f64``: the
factor is unit block-lower triangular and ``L D L^T`` reproduces the matrix
with ``D`` the blocks ``C_jj C_jj^T`` of its Cholesky factor (the block LDL
decomposition, unique for a positive definite matrix)."""

from __future__ import annotations

import pytest
import torch

from qsrt_amd.cholesky import block_unit_lower_f64_
from qsrt_amd.exl3_encoder_backend import _block_ldl_f64


def _spd(n: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(2 * n, n, generator=g, dtype=torch.float64)
    A = X.T @ X / X.shape[0]
    A.diagonal().add_(0.01 * A.diagonal().mean())
    return A


@pytest.mark.parametrize("n", [16, 64, 272])
def test_block_ldl_reproduces_the_matrix(n):
    A = _spd(n, n)
    L = _block_ldl_f64(A.clone(), 16, {})
    m = n // 16
    blocks = L.view(m, 16, m, 16).permute(0, 2, 1, 3)
    for i in range(m):
        assert torch.equal(blocks[i, i], torch.eye(16, dtype=torch.float64))
        for j in range(i + 1, m):
            assert torch.equal(blocks[i, j], torch.zeros(16, 16, dtype=torch.float64))
    C = torch.linalg.cholesky(A)
    D = torch.block_diag(*[C[16 * j:16 * j + 16, 16 * j:16 * j + 16] @ C[16 * j:16 * j + 16, 16 * j:16 * j + 16].T
                           for j in range(m)])
    assert (L @ D @ L.T - A).abs().max().item() <= 1e-12 * A.abs().max().item()


def test_block_unit_lower_checks_its_arguments():
    with pytest.raises(TypeError):
        block_unit_lower_f64_(torch.zeros(1, 16, 16), torch.zeros(1, 1, 16, 16, dtype=torch.float64))
    with pytest.raises(ValueError, match="multiple of 16"):
        block_unit_lower_f64_(torch.zeros(1, 24, 24, dtype=torch.float64), torch.zeros(1, 1, 16, 16,
                                                                                        dtype=torch.float64))
    with pytest.raises(ValueError, match="inv_blocks"):
        block_unit_lower_f64_(torch.zeros(2, 32, 32, dtype=torch.float64), torch.zeros(2, 1, 16, 16,
                                                                                        dtype=torch.float64))


@pytest.mark.parametrize("n,N,block", [(64, 24, 16), (272, 40, 128), (300, 7, 1024)])
def test_symmetric_trace_equals_the_full_trace(n, N, block):
    """``symmetric_trace_parts`` (the proxy errors' half-product trace)
    against ``trace(A^T H A)`` in float64 and against the reference-shaped
    ``block_trace``: equal to FP32 rounding for a symmetric ``H``, blocks
    that do not divide ``n`` included; it reads ``H``'s lower block triangle
    only (the blocks above the diagonal blocks may hold anything)."""

    from qsrt_amd.exl3_encoder_backend import block_trace, symmetric_trace_parts

    g = torch.Generator().manual_seed(n + N)
    H = _spd(n, n + 1).float()
    A = torch.randn(n, N, generator=g)
    exact = float(torch.trace(A.double().T @ H.double() @ A.double()))
    got = float(symmetric_trace_parts(A, H, block).double().sum())
    assert abs(got - exact) <= 1e-5 * exact
    assert abs(got - block_trace(A, H)) <= 1e-5 * exact
    rows = torch.arange(n) // block
    upper_blocks = rows.unsqueeze(1) < rows.unsqueeze(0)
    H2 = H.clone()
    H2[upper_blocks] += 1.0
    assert float(symmetric_trace_parts(A, H2, block).double().sum()) == got
