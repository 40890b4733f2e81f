"""Covariance producers: the weighted covariance (reference
tests/test_candidate_hessian.py), the identity shrinkage pinned to
scikit-learn's OAS and to its closed form, and the post-activation H2 as the
down projection's routed SSE (reference tests/test_blockldlq_proof.py:125-153)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from sklearn.covariance import oas

from qsrt_amd import candidate_hessian as ch

CPU = torch.device("cpu")


def test_weighted_covariance_matches_direct_definition():
    rows = torch.tensor([[1.0, 2.0], [3.0, 4.0], [-1.0, 2.0]])
    weights = torch.tensor([1.0, 2.0, 3.0])
    actual, denominator = ch.weighted_covariance(rows, weights, device=CPU, chunk_rows=2)
    # sum w x x^T by hand: w=1: [1 2;2 4], w=2: [18 24;24 32], w=3: [3 -6;-6 12]
    expected = torch.tensor([[22.0, 20.0], [20.0, 48.0]]) / 6.0
    assert denominator == 6.0
    torch.testing.assert_close(actual, expected)
    torch.testing.assert_close(actual, actual.T)


def test_weighted_covariance_chunking_and_integer_weights_equal_repetition():
    g = torch.Generator().manual_seed(5)
    rows = torch.randn(41, 6, generator=g, dtype=torch.float64)
    counts = torch.randint(0, 4, (41,), generator=g)
    counts[0] = 1
    repeated = rows.repeat_interleave(counts, dim=0)
    ref = repeated.T @ repeated / counts.sum()
    for chunk in (1, 7, 41, 1000):
        got, den = ch.weighted_covariance(rows, counts.double(), device=CPU, chunk_rows=chunk)
        assert den == float(counts.sum())
        torch.testing.assert_close(got.double(), ref, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("rows,weights,error", [
    (torch.empty(0, 2), torch.empty(0), "nonempty"),
    (torch.ones(2, 2), torch.ones(3), "shapes"),
    (torch.ones(2, 2), torch.tensor([1.0, -1.0]), "nonnegative"),
    (torch.ones(2, 2), torch.zeros(2), "positive"),
    (torch.tensor([[1.0, float("nan")]]), torch.ones(1), "finite"),
])
def test_weighted_covariance_rejects_bad_samples(rows, weights, error):
    with pytest.raises(ValueError, match=error):
        ch.weighted_covariance(rows, weights, device=CPU)


def test_adaptive_shrinkage_equals_sklearn_oas_at_unit_weights():
    rng = np.random.default_rng(17)
    for n, d in ((40, 6), (400, 12), (9, 30)):
        x = rng.standard_normal((n, d)) @ rng.standard_normal((d, d))
        local, _ = ch.weighted_covariance(torch.from_numpy(x), torch.ones(n, dtype=torch.float64), device=CPU)
        shrunk, ev = ch.oas_identity_shrinkage(local, torch.ones(n), max_local_alpha=1.0)
        _, expected = oas(x.astype(np.float32).astype(np.float64), assume_centered=True)
        assert ev["effective_sample_size"] == pytest.approx(n)
        assert ev["oas_shrinkage"] == pytest.approx(float(expected), rel=1e-5, abs=1e-7)
        assert ev["local_alpha"] == pytest.approx(1.0 - ev["oas_shrinkage"])
        torch.testing.assert_close(torch.trace(shrunk), torch.trace(local))


def test_adaptive_shrinkage_cap_and_identity_target():
    rows = torch.tensor([[3.0, 0.0], [0.0, 1.0], [2.0, -1.0], [-2.0, 1.0]])
    weights = torch.tensor([1.0, 2.0, 1.0, 0.5])
    local, _ = ch.weighted_covariance(rows, weights, device=CPU, return_cpu=False)
    actual, ev = ch.oas_identity_shrinkage(local, weights)
    scale = float(torch.trace(local) / 2)
    torch.testing.assert_close(actual, torch.lerp(torch.eye(2) * scale, local, ev["local_alpha"]))
    assert 0.0 <= ev["local_alpha"] <= 0.75
    # very well supported, strongly non-spherical: the cap binds
    g = torch.Generator().manual_seed(3)
    x = torch.randn(20000, 4, generator=g) * torch.tensor([1.0, 2.0, 4.0, 8.0])
    loc, _ = ch.weighted_covariance(x, torch.ones(20000), device=CPU)
    _, ev = ch.oas_identity_shrinkage(loc, torch.ones(20000), max_local_alpha=0.6)
    assert ev["local_alpha"] == 0.6
    # isotropic covariance: the denominator vanishes and the target takes over
    _, ev = ch.oas_identity_shrinkage(torch.eye(3), torch.ones(5))
    assert ev["oas_shrinkage"] == 1.0 and ev["local_alpha"] == 0.0


def test_oas_closed_form_and_weights():
    """The trace form on a hand-sized covariance, and the Kish effective
    sample size standing in for n under unequal weights."""

    g = torch.Generator().manual_seed(23)
    x = torch.randn(50, 5, generator=g, dtype=torch.float64) * torch.tensor([1.0, 1.5, 2.0, 3.0, 5.0],
                                                                             dtype=torch.float64)
    w = torch.rand(50, generator=g, dtype=torch.float64) + 0.2
    S = x.T @ (x * w[:, None]) / w.sum()
    n_eff = float(w.sum() ** 2 / (w ** 2).sum())
    p = 5
    tr, tr_s2 = float(torch.trace(S)), float(torch.trace(S @ S))
    rho = min(1.0, (tr_s2 + tr ** 2) / ((n_eff + 1.0) * (tr_s2 - tr ** 2 / p)))
    shrunk, ev = ch.oas_identity_shrinkage(S, w, max_local_alpha=1.0)
    assert ev["effective_sample_size"] == pytest.approx(n_eff, rel=1e-12)
    assert ev["oas_shrinkage"] == pytest.approx(rho, rel=1e-12)
    want = rho * tr / p * torch.eye(p, dtype=torch.float64) + (1 - rho) * S
    torch.testing.assert_close(shrunk.double(), want, rtol=1e-6, atol=1e-6)


def test_conditional_h2_is_the_down_projection_sse():
    g = torch.Generator().manual_seed(10)
    rows = torch.randn((53, 17), generator=g, dtype=torch.float64)
    gates = torch.rand(53, generator=g, dtype=torch.float64)
    wg = torch.randn((23, 17), generator=g, dtype=torch.float64)
    wu = torch.randn((23, 17), generator=g, dtype=torch.float64)
    err = torch.randn((9, 23), generator=g, dtype=torch.float64)
    middle, h2 = ch.conditional_h2(rows, gates, wg, wu)
    proxy = torch.einsum("oi,ij,oj->", err, h2, err)
    direct = ((middle @ err.T).square() * gates.square()[:, None]).sum() / gates.square().sum()
    assert float(abs(proxy - direct) / direct) < 1e-13
    _, h2b = ch.conditional_h2(rows, gates, wg * torch.tensor([1.5] + [1.0] * 22, dtype=torch.float64)[:, None], wu)
    assert float((h2b - h2).norm() / h2.norm()) > 1e-4
