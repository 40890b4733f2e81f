"""Covariance producers: weighted covariance, shrinkage, document splits and
the expert H13/H2 builder (reference tests/test_candidate_hessian.py,
tests/test_blockldlq_proof.py:125-153).  The shrinkage estimators are also
pinned to scikit-learn's OAS and to the closed form of Chen, Wiesel, Eldar
and Hero (2010), Eq. 23."""

from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch
from sklearn.covariance import oas

from qsrt_amd import candidate_hessian as ch
from qsrt_amd import pooled_calibration as pc

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


def test_shrinkage_endpoints_and_diagnostics():
    global_h = torch.eye(3)
    local_h = torch.diag(torch.tensor([2.0, 3.0, 4.0]))
    torch.testing.assert_close(ch.shrink_covariance(global_h, local_h, 0), global_h)
    torch.testing.assert_close(ch.shrink_covariance(global_h, local_h, 1), local_h)
    torch.testing.assert_close(ch.shrink_covariance(global_h, local_h, 0.25), 0.75 * global_h + 0.25 * local_h)
    d = ch.covariance_comparison(global_h, local_h)
    assert d["trace_ratio"] == 3.0
    assert d["relative_frobenius_difference"] == pytest.approx(float(torch.tensor([1.0, 2.0, 3.0]).norm()) / 3 ** 0.5)
    assert d["diagonal_cosine_similarity"] == pytest.approx(9.0 / (3 ** 0.5 * 29 ** 0.5))
    assert d["candidate_symmetry_max_abs"] == 0
    with pytest.raises(ValueError, match="alpha"):
        ch.shrink_covariance(torch.eye(2), torch.eye(2), 1.1)
    with pytest.raises(ValueError, match="equal-size"):
        ch.shrink_covariance(torch.eye(2), torch.eye(3), 0.5)


def test_effective_sample_size():
    assert ch.weighted_effective_sample_size(torch.ones(8)) == pytest.approx(8.0)
    assert ch.weighted_effective_sample_size(torch.tensor([10.0, 1, 1, 1])) == pytest.approx(169.0 / 103.0)
    assert ch.weighted_effective_sample_size(torch.tensor([0.0, 3.0, 0.0])) == pytest.approx(1.0)
    with pytest.raises(ValueError):
        ch.weighted_effective_sample_size(torch.zeros(3))


def test_adaptive_shrinkage_equals_sklearn_oas_at_unit_weights():
    rng = np.random.default_rng(17)
    for n, d in ((40, 6), (400, 12), (9, 30)):
        x = rng.standard_normal((n, d)) @ rng.standard_normal((d, d))
        local, _ = ch.weighted_covariance(torch.from_numpy(x), torch.ones(n, dtype=torch.float64), device=CPU)
        shrunk, ev = ch.adaptive_identity_shrinkage(local, torch.ones(n), max_local_alpha=1.0)
        _, expected = oas(x.astype(np.float32).astype(np.float64), assume_centered=True)
        assert ev["effective_sample_size"] == pytest.approx(n)
        assert ev["oas_shrinkage"] == pytest.approx(float(expected), rel=1e-5, abs=1e-7)
        assert ev["local_alpha"] == pytest.approx(1.0 - ev["oas_shrinkage"])
        torch.testing.assert_close(torch.trace(shrunk), torch.trace(local))


def test_adaptive_shrinkage_cap_and_identity_target():
    rows = torch.tensor([[3.0, 0.0], [0.0, 1.0], [2.0, -1.0], [-2.0, 1.0]])
    weights = torch.tensor([1.0, 2.0, 1.0, 0.5])
    local, _ = ch.weighted_covariance(rows, weights, device=CPU, return_cpu=False)
    actual, ev = ch.adaptive_identity_shrinkage(local, weights)
    scale = float(torch.trace(local) / 2)
    torch.testing.assert_close(actual, torch.lerp(torch.eye(2) * scale, local, ev["local_alpha"]))
    assert 0.0 <= ev["local_alpha"] <= 0.75
    # very well supported, strongly non-spherical: the cap binds
    g = torch.Generator().manual_seed(3)
    x = torch.randn(20000, 4, generator=g) * torch.tensor([1.0, 2.0, 4.0, 8.0])
    loc, _ = ch.weighted_covariance(x, torch.ones(20000), device=CPU)
    _, ev = ch.adaptive_identity_shrinkage(loc, torch.ones(20000), max_local_alpha=0.6)
    assert ev["local_alpha"] == 0.6
    # isotropic covariance: the denominator vanishes and the target takes over
    _, ev = ch.adaptive_identity_shrinkage(torch.eye(3), torch.ones(5))
    assert ev["oas_shrinkage"] == 1.0 and ev["local_alpha"] == 0.0


def test_candidate_h2_equals_chen_wiesel_eldar_hero_eq23():
    rng = np.random.default_rng(9173)
    x = rng.standard_normal((4096, 11))
    x[:, 0] *= 3.0
    stats = pc.CandidateHiddenStatistics.zeros(11)
    stats.update(torch.from_numpy(x), torch.from_numpy(x), torch.ones(4096, dtype=torch.float64))
    h2, ev = pc.candidate_h2(stats, max_local_alpha=1.0)
    s = x.T @ x / 4096
    p, n = 11, 4096
    tr_s2, tr2 = np.trace(s @ s), np.trace(s) ** 2
    rho = min(1.0, ((1 - 2 / p) * tr_s2 + tr2) / ((n + 1 - 2 / p) * (tr_s2 - tr2 / p)))
    assert ev["oas_shrinkage"] == pytest.approx(rho, rel=1e-10)
    expected = (1 - ev["local_alpha"]) * np.trace(s) / p * np.eye(p) + ev["local_alpha"] * s
    np.testing.assert_allclose(h2.numpy(), expected, rtol=1e-12, atol=1e-12)


def test_document_partition_and_request_mask():
    docs = [f"document-{i}" for i in range(16)]
    fit, confirmation = ch.partition_documents(docs, modulus=4, confirmation_index=0)
    assert set(fit).isdisjoint(confirmation) and set(fit) | set(confirmation) == set(docs)
    for doc in docs:
        bucket = int.from_bytes(hashlib.blake2b(doc.encode(), digest_size=8).digest(), "little") % 4
        assert (doc in confirmation) == (bucket == 0)
    assert ch.partition_documents(docs, modulus=4, confirmation_index=0) == (fit, confirmation)
    requests = {i + 1: d for i, d in enumerate(docs)}
    fit_requests = ch.subset_request_documents(requests, fit)
    assert set(fit_requests.values()) == set(fit)
    obs = torch.tensor([(1 << 32) | 7, (2 << 32) | 9, (99 << 32) | 1, (16 << 32)], dtype=torch.int64)
    expected = torch.tensor([1 in fit_requests, 2 in fit_requests, False, 16 in fit_requests])
    assert torch.equal(ch.request_mask(obs, fit_requests), expected)
    with pytest.raises(ValueError):
        ch.partition_documents(["same", "same"], modulus=4, confirmation_index=0)
    with pytest.raises(ValueError):
        ch.partition_documents(docs, modulus=1, confirmation_index=0)
    with pytest.raises(ValueError):
        ch.subset_request_documents({1: "present"}, ["missing"])
    with pytest.raises(ValueError):
        ch.request_mask(torch.zeros((1, 1), dtype=torch.int64), {1: "doc"})


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


def test_build_expert_hessians_policies():
    g = torch.Generator().manual_seed(2)
    inputs = torch.randn(300, 8, generator=g)
    gates = torch.rand(300, generator=g)
    middle = torch.randn(300, 6, generator=g)
    global_h13 = torch.eye(8) * 2.0
    h13, h2, ev = ch.build_expert_hessians(inputs, gates, middle, global_h13=global_h13, global_h2=torch.zeros(6, 6),
                                           device=CPU)
    assert torch.equal(h13, global_h13)
    local_h2, _ = ch.weighted_covariance(middle, gates.square(), device=CPU)
    expected, s = ch.adaptive_identity_shrinkage(local_h2, gates.square(), max_local_alpha=0.75)
    torch.testing.assert_close(h2, expected)
    assert ev["h2_shrinkage_policy"] == ch.PHASE1_H2_SHRINKAGE_POLICY
    assert ev["gate_square_sum"] == pytest.approx(float(gates.double().square().sum()))
    h13, h2, ev = ch.build_expert_hessians(inputs, gates, middle, global_h13=global_h13, global_h2=torch.zeros(6, 6),
                                           device=CPU, h13_alpha=0.5, h2_alpha=0.25)
    local_h13, _ = ch.weighted_covariance(inputs, gates.square(), device=CPU)
    torch.testing.assert_close(h13, 0.5 * global_h13 + 0.5 * local_h13)
    scale = float(torch.trace(local_h2) / 6)
    torch.testing.assert_close(h2, 0.75 * scale * torch.eye(6) + 0.25 * local_h2)
    assert ev["h2_shrinkage_policy"] == "fixed_alpha_scaled_identity"
    with pytest.raises(ValueError, match="dimension"):
        ch.build_expert_hessians(inputs, gates, middle, global_h13=global_h13, global_h2=torch.zeros(5, 5), device=CPU)


def test_conditional_h2_per_upstream_rate():
    from types import SimpleNamespace

    from qsrt_amd.qsrt_coupled import situ

    inputs = torch.tensor([[1.0, 0.0], [0.0, 1.0], [1.0, 1.0], [-1.0, 0.5]])
    gates = torch.tensor([1.0, 0.75, 0.5, 0.25])
    upstream = {"w1": {0: SimpleNamespace(reconstruction=torch.eye(2)),
                       1: SimpleNamespace(reconstruction=2.0 * torch.eye(2))},
                "w3": {0: SimpleNamespace(reconstruction=torch.eye(2)),
                       1: SimpleNamespace(reconstruction=torch.tensor([[1.0, 1.0], [0.0, 1.0]]))}}
    middle = ch._candidate_middle_by_r13(inputs, upstream, (0, 1))
    torch.testing.assert_close(middle[0], situ(inputs, inputs))
    torch.testing.assert_close(middle[1], situ(2.0 * inputs, inputs @ torch.tensor([[1.0, 1.0], [0.0, 1.0]]).T))
    mask = torch.tensor([True, True, False, True])
    h2, ev = ch._conditional_h2_by_r13(inputs, gates, mask, middle, global_h13=torch.eye(2), global_h2=torch.eye(2),
                                       device=CPU, hessian_policy="captured_blend", have_local_support=True)
    assert set(h2) == {0, 1} and not torch.allclose(h2[0], h2[1])
    for r in (0, 1):
        local, _ = ch.weighted_covariance(middle[r][mask], gates[mask].square(), device=CPU)
        want, s = ch.adaptive_identity_shrinkage(local, gates[mask].square())
        torch.testing.assert_close(h2[r], want)
        assert ev[f"R{r}"]["h2_shrinkage_policy"] == "weighted_oas_scaled_identity"
    assert ev["R1"]["h2_effective_sample_size"] == pytest.approx(ev["R0"]["h2_effective_sample_size"])
    # pooled global H2 values never enter
    other, _ = ch._conditional_h2_by_r13(inputs, gates, mask, middle, global_h13=torch.eye(2),
                                         global_h2=5.0 * torch.ones(2, 2), device=CPU,
                                         hessian_policy="captured_blend", have_local_support=True)
    torch.testing.assert_close(other[0], h2[0])
    for policy, support in (("identity", True), ("captured_blend", False)):
        fallback, ev = ch._conditional_h2_by_r13(inputs, gates, mask, middle, global_h13=torch.eye(2),
                                                 global_h2=torch.eye(2), device=CPU, hessian_policy=policy,
                                                 have_local_support=support)
        assert torch.equal(fallback[1], torch.eye(2)) and ev["R1"]["h2_shrinkage_policy"] == "identity_fallback"
