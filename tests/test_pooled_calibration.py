"""Pooled calibration statistics and the expert Hessian policy on the CPU.

Every quantity is pinned by an identity that holds for the mathematics,
not by restating the code's formula:

* the stacked Gram's blocks are the five cross-products of the rows,
  computed directly in float64;
* ``decoded_down_sse`` equals the routed-output SSE of the rows computed
  explicitly, and ``decoded_down_sse_difference`` the difference of two such
  SSEs (a swapped block or a dropped term fails either);
* statistics of two disjoint row partitions merge into the statistics of
  all rows;
* ``candidate_h2`` takes the identity for a spherical covariance and the
  closed form of the original OAS on a two-level spectrum; ``build_expert_
  hessians``' H2 equals scikit-learn's OAS of the same rows when the weight
  cap does not bind;
* the ridge refit solves its normal equations and tends to least squares as
  the ridge vanishes;
* the upstream metric's entries are the squared route-weighted derivatives
  of SiTU, checked by finite differences;
* the blockwise conditioning coefficients on constructed 2 x 2 metrics.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from qsrt_amd import candidate_hessian as ch
from qsrt_amd import pooled_calibration as pc
from qsrt_amd.qsrt import PHASE1_H2_EXPERT_LOCAL_ALPHA
from qsrt_amd.qsrt_coupled import CoupledHadamardSpec, coupled_execution, situ


def _rows(n, w, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, w, generator=g, dtype=torch.float64) * scale


def _stats(C, S, route, dtype=torch.float64, retain=True):
    st = pc.CandidateHiddenStatistics.zeros(C.shape[1], dtype=dtype, retain_source_gram=retain)
    st.update(C, S, route)
    return st


def test_stacked_gram_blocks_are_the_five_cross_products():
    n, w = 200, 24
    S = _rows(n, w, 1)
    C = S + 0.01 * _rows(n, w, 2)
    route = torch.rand(n, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    st = _stats(C, S, route)
    W = route.square()[:, None]
    R = C - S
    checks = {
        "candidate_gram": C.T @ (C * W), "candidate_source_cross": C.T @ (S * W), "source_gram": S.T @ (S * W),
        "candidate_residual_cross": C.T @ (R * W), "hidden_residual_gram": R.T @ (R * W),
    }
    for name, want in checks.items():
        got = getattr(st, name)
        assert torch.allclose(got, want, rtol=1e-12, atol=1e-12 * float(want.abs().max())), name
    assert st.rows == n and math.isclose(st.weight_sum, float(route.square().sum()), rel_tol=1e-12)
    assert math.isclose(st.effective_sample_size, float(route.square().sum() ** 2 / route.pow(4).sum()), rel_tol=1e-12)
    bare = _stats(C, S, route, retain=False)
    assert bare.source_gram is None and bare.hidden_residual_gram is None
    with pytest.raises(ValueError, match="retained source Gram"):
        pc.decoded_down_sse(bare, torch.zeros(w, 5, dtype=torch.float64), torch.zeros(w, 5, dtype=torch.float64))


def test_decoded_down_sse_equals_explicit_routed_sse():
    n, w, out = 300, 32, 20
    S = _rows(n, w, 4)
    C = S + 0.05 * _rows(n, w, 5)
    route = torch.rand(n, generator=torch.Generator().manual_seed(6), dtype=torch.float64) + 0.1
    src = _rows(w, out, 7)
    cand = src + 0.02 * _rows(w, out, 8)
    base = src + 0.03 * _rows(w, out, 9)
    st = _stats(C, S, route)

    def explicit(down):
        err = (C @ down - S @ src) * route[:, None]
        return float(err.square().sum())

    got = float(pc.decoded_down_sse(st, cand, src))
    assert math.isclose(got, explicit(cand), rel_tol=1e-10)
    assert math.isclose(float(pc.decoded_down_sse(st, src, src)), explicit(src), rel_tol=1e-10)
    diff = float(pc.decoded_down_sse_difference(st, cand, base, src))
    assert math.isclose(diff, explicit(cand) - explicit(base), rel_tol=1e-8, abs_tol=1e-10 * explicit(base))


def test_partition_statistics_merge_to_the_whole():
    n, w = 160, 16
    S = _rows(n, w, 10)
    C = S + 0.1 * _rows(n, w, 11)
    route = torch.rand(n, generator=torch.Generator().manual_seed(12), dtype=torch.float64)
    whole = _stats(C, S, route)
    part = _stats(C[:70], S[:70], route[:70])
    part.merge_(_stats(C[70:], S[70:], route[70:]))
    assert torch.allclose(part.stacked, whole.stacked, rtol=1e-12, atol=1e-12)
    assert part.rows == n and math.isclose(part.weight_square_sum, whole.weight_square_sum, rel_tol=1e-12)
    moved = part.to(device="cpu", dtype=torch.float32)
    assert moved.stacked.dtype == torch.float32 and moved.rows == n


def test_candidate_h2_spherical_and_two_level_closed_form():
    # spherical covariance: tr(S^2) = tr(S)^2 / p, so the OAS denominator is zero and the identity is taken
    p = 8
    st = pc.CandidateHiddenStatistics.zeros(p)
    st.stacked[:p, :p] = torch.eye(p, dtype=torch.float64) * 3.0 * 10.0
    st.weight_sum, st.weight_square_sum, st.rows = 10.0, 10.0, 10
    h2, ev = pc.candidate_h2(st)
    assert ev["oas_shrinkage"] == 1.0 and ev["local_alpha"] == 0.0
    assert torch.allclose(h2, torch.eye(p, dtype=torch.float64) * 3.0)
    # two-level spectrum: S = diag(a,...,a, b,...,b) with k entries a; closed form of the original OAS
    a, b, k, n_eff = 5.0, 1.0, 3, 40.0
    S = torch.diag(torch.tensor([a] * k + [b] * (p - k), dtype=torch.float64))
    st.stacked[:p, :p] = S * 100.0
    st.weight_sum = 100.0
    st.weight_square_sum = 100.0 ** 2 / n_eff
    tr = k * a + (p - k) * b
    tr2 = k * a * a + (p - k) * b * b
    rho = min(1.0, ((1 - 2 / p) * tr2 + tr * tr) / ((n_eff + 1 - 2 / p) * (tr2 - tr * tr / p)))
    h2, ev = pc.candidate_h2(st, max_local_alpha=1.0)
    assert math.isclose(ev["oas_shrinkage"], rho, rel_tol=1e-12)
    want = (1 - (1 - rho)) * (tr / p) * torch.eye(p, dtype=torch.float64) + (1 - rho) * S
    assert torch.allclose(h2, want, rtol=1e-12)
    capped, ev = pc.candidate_h2(st, max_local_alpha=0.1)
    assert ev["local_alpha"] == 0.1 and torch.allclose(capped, 0.9 * (tr / p) * torch.eye(p, dtype=torch.float64)
                                                      + 0.1 * S)


def test_build_expert_hessians_matches_sklearn_oas_and_keeps_global_h13():
    from sklearn.covariance import oas

    n, hidden, inter = 24, 12, 16  # a low-support expert: OAS shrinks hard and the 0.75 cap does not bind
    x = _rows(n, hidden, 20).float()
    mid = (_rows(n, inter, 21) * torch.linspace(0.5, 1.5, inter, dtype=torch.float64)).float()
    gates = torch.ones(n)
    g13 = torch.eye(hidden) * 2.0
    h13, h2, ev = ch.build_expert_hessians(x, gates, mid, global_h13=g13, global_h2=torch.eye(inter),
                                           device="cpu")
    assert torch.equal(h13, g13)  # local weight 0: the layer's global H13
    shrunk, rho = oas(mid.double().numpy(), assume_centered=True)
    assert 1 - rho <= PHASE1_H2_EXPERT_LOCAL_ALPHA  # the cap does not bind here
    assert math.isclose(ev["h2_oas_shrinkage"], rho, rel_tol=1e-6)
    assert np.allclose(h2.double().numpy(), shrunk, rtol=1e-5, atol=1e-6)
    # a local H13 weight blends toward the local covariance
    h13b, _, _ = ch.build_expert_hessians(x, gates, mid, global_h13=g13, global_h2=torch.eye(inter), device="cpu",
                                          h13_alpha=0.5)
    local = (x.double().T @ x.double() / n).float()
    assert torch.allclose(h13b, 0.5 * g13 + 0.5 * local, rtol=1e-5, atol=1e-6)
    assert ch.adaptive_identity_shrinkage is ch.oas_identity_shrinkage
    assert math.isclose(ch.weighted_effective_sample_size(torch.tensor([1.0, 1.0, 2.0])), 16.0 / 6.0)
    assert torch.allclose(ch.shrink_covariance(torch.eye(3), 3 * torch.eye(3), 0.25), 1.5 * torch.eye(3))


def test_conditional_h2_by_rate_uses_each_candidates_rows():
    n, hidden, inter = 300, 16, 8
    x = _rows(n, hidden, 30).float()
    gates = torch.rand(n, generator=torch.Generator().manual_seed(31)) + 0.2
    mask = torch.ones(n, dtype=torch.bool)
    mask[::5] = False
    recon = {r: (_rows(inter, hidden, 40 + r).float() * 0.3, _rows(inter, hidden, 50 + r).float() * 0.3)
             for r in (0, 1, 2)}
    h2s, ev = ch.conditional_h2_by_rate(x, gates, mask, recon, global_h13=torch.eye(hidden),
                                        global_h2=torch.eye(inter), device="cpu")
    assert set(h2s) == {0, 1, 2} and set(ev) == {"R0", "R1", "R2"}
    for r, (w1, w3) in recon.items():
        mid = situ(x[mask] @ w1.T, x[mask] @ w3.T)
        _, want, _ = ch.build_expert_hessians(x[mask], gates[mask], mid, global_h13=torch.eye(hidden),
                                              global_h2=torch.eye(inter), device="cpu")
        assert torch.allclose(h2s[r], want, rtol=1e-5, atol=1e-7)
    ident, ev = ch.conditional_h2_by_rate(x, gates, mask, recon, global_h13=torch.eye(hidden),
                                          global_h2=torch.eye(inter), device="cpu", hessian_policy="identity")
    assert all(torch.equal(h, torch.eye(inter)) for h in ident.values())
    assert ev["R1"]["h2_shrinkage_policy"] == "identity_fallback"


def test_ridge_refit_solves_its_normal_equations():
    n, w, out = 500, 12, 7
    S = _rows(n, w, 60)
    C = S + 0.2 * _rows(n, w, 61)
    route = torch.rand(n, generator=torch.Generator().manual_seed(62), dtype=torch.float64) + 0.5
    src = _rows(w, out, 63)
    st = _stats(C, S, route)
    refit, ev = pc.ridge_refit_down_from_statistics(st, src, regularization_ratio=0.3)
    lam = ev["regularization"]
    Wt = route.square()[:, None]
    lhs = C.T @ (C * Wt) @ refit + lam * refit
    rhs = C.T @ (S * Wt) @ src + lam * src
    assert torch.allclose(lhs, rhs, rtol=1e-9, atol=1e-9 * float(rhs.abs().max()))
    # vanishing ridge: the weighted least-squares fit of S src from C
    tiny, _ = pc.ridge_refit_down_from_statistics(st, src, regularization_ratio=1e-12)
    ls = torch.linalg.lstsq(C * route[:, None], (S @ src) * route[:, None]).solution
    assert torch.allclose(tiny, ls, rtol=1e-6, atol=1e-8)


def test_upstream_metric_is_route_weighted_squared_situ_derivatives():
    hidden, inter, n = 16, 8, 50
    g = torch.Generator().manual_seed(70)
    src = pc.CoupledTriplet(torch.randn(inter, hidden, generator=g), torch.randn(inter, hidden, generator=g),
                            torch.randn(hidden, inter, generator=g))
    x = torch.randn(n, hidden, generator=g)
    route = torch.rand(n, generator=g) + 0.1
    batches = [{"input": x[:20], "route_weight": route[:20], "row_index": torch.arange(20)},
               {"input": x[20:], "route_weight": route[20:], "row_index": torch.arange(20, n) + 100}]
    stats = pc.collect_upstream_functional_statistics(batches, source=src, device="cpu")
    # central differences of SiTU's definition, h = 4 tanh(g / 4) sigmoid(g) * 25 tanh(u / 25), in float64
    # (the product's situ rounds through FP32)
    def situ64(a, b):
        return 4.0 * torch.tanh(a / 4.0) * torch.sigmoid(a) * (25.0 * torch.tanh(b / 25.0))

    gate = (x.double() @ src.gate.double().T)
    up = (x.double() @ src.up.double().T)
    eps = 1e-5
    dg = (situ64(gate + eps, up) - situ64(gate - eps, up)) / (2 * eps)
    du = (situ64(gate, up + eps) - situ64(gate, up - eps)) / (2 * eps)
    assert torch.allclose(situ(gate.float(), up.float()).double(), situ64(gate, up), rtol=1e-5, atol=1e-6)
    w = route.double().square()
    e = src.down.double().square().sum(dim=0)
    assert torch.allclose(stats.derivative_metric[:, 0, 0], (w[:, None] * dg * dg).sum(0) * e, rtol=1e-4)
    assert torch.allclose(stats.derivative_metric[:, 0, 1], (w[:, None] * dg * du).sum(0) * e, rtol=1e-4)
    assert torch.allclose(stats.derivative_metric[:, 1, 1], (w[:, None] * du * du).sum(0) * e, rtol=1e-4)
    assert torch.allclose(stats.hidden_energy, (w[:, None] * situ64(gate, up).square()).sum(0), rtol=1e-4)
    assert stats.rows == n
    with pytest.raises(ValueError, match="increasing"):
        pc.collect_upstream_functional_statistics(batches[::-1], source=src, device="cpu")


def test_blockwise_coefficients_on_constructed_metrics():
    # block of two neurons: metrics sum to [[4, 2], [2, 8]] -> gate_from_up 0.5, up_from_gate 0.25
    m = torch.tensor([[[1.0, 0.5], [0.5, 3.0]], [[3.0, 1.5], [1.5, 5.0]],
                      [[2.0, -1.0], [-1.0, 1.0]], [[2.0, -1.0], [-1.0, 1.0]]], dtype=torch.float64)
    gfu, ufg, ev = pc.blockwise_upstream_conditioning_coefficients(m, block_size=2)
    assert torch.allclose(gfu, torch.tensor([0.5, 0.5, -0.5, -0.5], dtype=torch.float64))
    assert torch.allclose(ufg, torch.tensor([0.25, 0.25, -1.0, -1.0], dtype=torch.float64))
    assert ev["blocks"] == 2.0
    with pytest.raises(ValueError, match="semidefinite"):
        pc.blockwise_upstream_conditioning_coefficients(torch.tensor([[[1.0, 2.0], [2.0, 1.0]]]), block_size=1)


def test_expert_evaluation_scores_match_explicit_forward():
    hidden, inter, n = 512, 128, 64
    g = torch.Generator().manual_seed(80)
    spec = CoupledHadamardSpec()
    src = pc.CoupledTriplet(0.05 * torch.randn(inter, hidden, generator=g), 0.05 * torch.randn(inter, hidden, generator=g),
                            0.05 * torch.randn(hidden, inter, generator=g))
    from qsrt_amd.qsrt_coupled import encode_coupled_weights

    coords = encode_coupled_weights(src.tensors(), spec)
    cand = pc.CoupledTriplet(*(c + 0.003 * torch.randn(c.shape, generator=g) for c in coords))
    ex = coupled_execution(src.tensors(), spec)
    x = torch.randn(n, hidden, generator=g)
    route = torch.rand(n, generator=g) + 0.2
    batches = [{"input": x, "route_weight": route, "row_index": torch.arange(n) * 3}]
    ev = pc.evaluate_coupled_expert_batches(batches, source=src, candidate_coordinates=cand, execution=ex,
                                            prefix_row_limits=(30,), retain_source_gram=True,
                                            statistics_dtype=torch.float64)
    teacher = situ(x @ src.gate.T, x @ src.up.T) @ src.down.T
    output = ex.execute(x, cand.tensors())
    want = float(((output - teacher) * route[:, None]).double().square().sum())
    assert math.isclose(ev.sse, want, rel_tol=1e-6)
    assert ev.routed_occurrences == n and ev.prefix_scores[30][2] == 10
    # the portfolio path scores the same candidate identically
    port = pc.evaluate_coupled_candidate_portfolio_batches(batches, source=src, candidate_coordinates={"a": cand},
                                                           executions={"a": ex})
    assert math.isclose(port.candidate_sse["a"], ev.sse, rel_tol=1e-6)
    # the statistics score the candidate's own down projection as the explicit forward does (in the coupled
    # basis, whose output transform is orthogonal)
    sse = float(pc.decoded_down_sse(ev.statistics, cand.down.T.double(), coords[2].T.double()))
    src_hidden = ex.decode_middle(ex.transform_inputs(x), coords[0], coords[1])
    cand_hidden = ex.decode_middle(ex.transform_inputs(x), cand.gate, cand.up)
    direct = float(((cand_hidden @ cand.down.T - src_hidden @ coords[2].T) * route[:, None]).double().square().sum())
    assert math.isclose(sse, direct, rel_tol=1e-5)
