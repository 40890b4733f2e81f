"""The weighted covariance on the GPU accumulates on the FP32 matrix cores
(qsrt_gemm_tn) and must agree with a float64 CPU evaluation of the same
definition."""

from __future__ import annotations

import sys

import pytest
import torch

from qsrt_amd import candidate_hessian as ch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _frob_rel(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.detach().cpu().double(), want.detach().cpu().double()
    return float((got - want).norm() / want.norm())


@pytest.mark.parametrize("n,d", [(20000, 1030), (300, 7168), (1, 64)])
def test_weighted_covariance_on_matrix_cores(n, d):
    print(f"[cov] weighted_covariance n{n} d{d}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(n + d)
    rows = torch.randn(n, d, generator=g) * torch.linspace(0.1, 3.0, d)
    weights = torch.rand(n, generator=g)
    got, den = ch.weighted_covariance(rows, weights, device=DEV)
    r64, w64 = rows.double(), weights.double()
    want = r64.T @ (r64 * w64[:, None]) / w64.sum()
    assert den == pytest.approx(float(w64.sum()), rel=1e-12)
    assert got.device.type == "cpu" and got.dtype == torch.float32
    assert _frob_rel(got, want) < 1e-5
    assert torch.equal(got, got.T)
