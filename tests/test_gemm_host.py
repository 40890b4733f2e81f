"""Host side of the BlockLDLQ span products: the batched float64 wrapper's
shape and dtype rules and its CPU path (torch), which the recursion runs on
CPU tensors."""

from __future__ import annotations

import pytest
import torch

from qsrt_amd import gemm


def test_batched_span_product_on_cpu_equals_the_member_loop():
    g = torch.Generator().manual_seed(3)
    batch, k, n, begin, end = 3, 64, 48, 32, 48
    L = torch.randn(batch, k, k, generator=g, dtype=torch.float64)
    W = torch.randn(batch, k, n, generator=g, dtype=torch.float64)
    Q = torch.randn(batch, k, n, generator=g)
    P = torch.randn(batch, k, n, generator=g, dtype=torch.float64)
    loop = P.clone()
    for b in range(batch):
        gemm.addmm_sub_tn_(loop[b, :begin], L[b, begin:end, :begin], W[b, begin:end], Q[b, begin:end], alpha=0.25)
    one = P.clone()
    gemm.baddmm_sub_tn_f64_(one[:, :begin], L[:, begin:end, :begin], W[:, begin:end], Q[:, begin:end], alpha=0.25)
    assert torch.allclose(one, loop, rtol=0, atol=1e-12)
    # closed form of one member
    want = P[1, :begin] + 0.25 * L[1, begin:end, :begin].T @ (W[1, begin:end] - Q[1, begin:end].double())
    assert torch.allclose(one[1, :begin], want, rtol=0, atol=1e-12)


def test_batched_span_product_rules():
    C = torch.zeros(2, 8, 8, dtype=torch.float64)
    A = torch.zeros(2, 4, 8, dtype=torch.float64)
    B = torch.zeros(2, 4, 8, dtype=torch.float64)
    with pytest.raises(ValueError, match="incompatible"):
        gemm.baddmm_sub_tn_f64_(C, A, B[:, :3])
    with pytest.raises(ValueError, match="float64"):
        gemm.baddmm_sub_tn_f64_(C, A.float(), B)
    with pytest.raises(ValueError, match="float32 B2"):
        gemm.baddmm_sub_tn_f64_(C, A, B, B.clone())
    with pytest.raises(ValueError, match="batch, rows, cols"):
        gemm.baddmm_sub_tn_f64_(C[0], A[0], B[0])
