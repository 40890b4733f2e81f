"""Pooled sufficient statistics (reference tests/test_pooled_calibration.py):
every statistic-derived score is checked against the explicit routed-output
computation it replaces."""

from __future__ import annotations

import pytest
import torch

from qsrt_amd import pooled_calibration as pc
from qsrt_amd.qsrt_coupled import (CoupledHadamardExecution, CoupledHadamardSpec, encode_coupled_weights, situ,
                                   situ_derivatives)


def _samples():
    g = torch.Generator().manual_seed(7819)
    source = torch.randn(37, 7, generator=g, dtype=torch.float64)
    candidate = source + 0.08 * torch.randn(37, 7, generator=g, dtype=torch.float64)
    gates = torch.rand(37, generator=g, dtype=torch.float64)
    down = torch.randn(7, 5, generator=g, dtype=torch.float64)
    return source, candidate, gates, down


def _explicit_sse(candidate, source, gates, cand_down, src_down):
    return (gates[:, None] * (candidate @ cand_down - source @ src_down)).square().sum(dtype=torch.float64)


def test_statistics_are_the_weighted_cross_products():
    source, candidate, gates, _ = _samples()
    st = pc.CandidateHiddenStatistics.zeros(7)
    st.update(candidate, source, gates)
    w = gates.square()
    res = candidate - source
    torch.testing.assert_close(st.candidate_gram, sum(w[i] * torch.outer(candidate[i], candidate[i]) for i in range(37)))
    torch.testing.assert_close(st.candidate_source_cross, sum(w[i] * torch.outer(candidate[i], source[i]) for i in range(37)))
    torch.testing.assert_close(st.source_gram, sum(w[i] * torch.outer(source[i], source[i]) for i in range(37)))
    torch.testing.assert_close(st.candidate_residual_cross, sum(w[i] * torch.outer(candidate[i], res[i]) for i in range(37)))
    torch.testing.assert_close(st.hidden_residual_gram, sum(w[i] * torch.outer(res[i], res[i]) for i in range(37)))
    assert st.weight_sum == pytest.approx(float(w.sum()))
    assert st.effective_sample_size == pytest.approx(float(w.sum() ** 2 / w.square().sum()))
    assert st.rows == 37


def test_pooled_down_sse_matches_explicit_weighted_outputs():
    source, candidate, gates, down = _samples()
    st = pc.CandidateHiddenStatistics.zeros(7)
    st.update(candidate, source, gates)
    decoded = down + 0.04
    torch.testing.assert_close(pc.decoded_down_sse(st, decoded, down), _explicit_sse(candidate, source, gates, decoded, down),
                               rtol=2e-12, atol=2e-12)
    # identical hidden rows and projections: zero error
    same = pc.CandidateHiddenStatistics.zeros(7)
    same.update(source, source, gates)
    assert float(pc.decoded_down_sse(same, down, down)) == 0.0


def test_chunked_statistics_match_one_pass_and_to_roundtrips():
    source, candidate, gates, _ = _samples()
    full = pc.CandidateHiddenStatistics.zeros(7)
    full.update(candidate, source, gates)
    chunked = pc.CandidateHiddenStatistics.zeros(7)
    for a, b in ((0, 5), (5, 5), (5, 19), (19, 37)):
        part = pc.CandidateHiddenStatistics.zeros(7)
        part.update(candidate[a:b], source[a:b], gates[a:b])
        chunked.merge_(part)
    for x, y in zip(chunked._matrices(), full._matrices()):
        torch.testing.assert_close(x, y)
    assert chunked.weight_sum == pytest.approx(full.weight_sum)
    assert chunked.weight_square_sum == pytest.approx(full.weight_square_sum)
    assert chunked.rows == full.rows
    f32 = full.to(device="cpu", dtype=torch.float32)
    assert f32.candidate_gram.dtype == torch.float32 and f32.rows == full.rows
    with pytest.raises(ValueError, match="retention"):
        full.merge_(pc.CandidateHiddenStatistics.zeros(7, retain_source_gram=False))
    with pytest.raises(ValueError, match="widths"):
        full.merge_(pc.CandidateHiddenStatistics.zeros(6))
    with pytest.raises(TypeError):
        pc.CandidateHiddenStatistics.zeros(7, dtype=torch.float16)


def test_candidate_h2_uses_only_candidate_gram_and_scaled_identity():
    source, candidate, gates, _ = _samples()
    st = pc.CandidateHiddenStatistics.zeros(7)
    st.update(candidate, source, gates)
    h2, ev = pc.candidate_h2(st)
    local = st.candidate_gram / st.weight_sum
    expected = (1 - ev["local_alpha"]) * torch.eye(7, dtype=torch.float64) * torch.trace(local) / 7 + ev["local_alpha"] * local
    torch.testing.assert_close(h2, expected)
    torch.testing.assert_close(torch.trace(h2), torch.trace(local))
    assert 0 <= ev["local_alpha"] <= 0.75


def test_ridge_refit_improves_objective_and_difference_matches():
    source, candidate, gates, down = _samples()
    st = pc.CandidateHiddenStatistics.zeros(7)
    st.update(candidate, source, gates)
    refit, ev = pc.ridge_refit_down_from_statistics(st, down, regularization_ratio=1e-5)
    assert ev["regularization"] > 0
    # the refit is the normal-equation solution of the explicit ridge problem
    lam = ev["regularization"]
    w = gates.square()
    lhs = candidate.T @ (candidate * w[:, None]) + lam * torch.eye(7, dtype=torch.float64)
    rhs = candidate.T @ ((source @ down) * w[:, None]) + lam * down
    torch.testing.assert_close(refit, torch.linalg.solve(lhs, rhs))
    assert pc.decoded_down_sse(st, refit, down) < pc.decoded_down_sse(st, down, down)
    sparse = pc.CandidateHiddenStatistics.zeros(7, retain_source_gram=False)
    sparse.update(candidate, source, gates)
    diff = pc.decoded_down_sse_difference(sparse, refit, down, down)
    explicit = _explicit_sse(candidate, source, gates, refit, down) - _explicit_sse(candidate, source, gates, down, down)
    torch.testing.assert_close(diff, explicit)
    with pytest.raises(ValueError, match="source Gram"):
        pc.decoded_down_sse(sparse, refit, down)


def _cancellation_case(seed):
    g = torch.Generator().manual_seed(seed)
    source = 16.0 * torch.randn(2048, 64, generator=g)
    candidate = source + 2e-3 * torch.randn(2048, 64, generator=g)
    gates = torch.rand(2048, generator=g)
    source_down = 8.0 * torch.randn(64, 48, generator=g)
    baseline_down = source_down + 2e-3 * torch.randn(64, 48, generator=g)
    candidate_down = baseline_down + 1e-3 * torch.randn(64, 48, generator=g)
    return source, candidate, gates, source_down, baseline_down, candidate_down


def test_fp32_statistics_avoid_energy_cancellation():
    source, candidate, gates, source_down, baseline_down, candidate_down = _cancellation_case(13084)
    st = pc.CandidateHiddenStatistics.zeros(64, dtype=torch.float32)
    st.update(candidate, source, gates)
    explicit = _explicit_sse(candidate.double(), source.double(), gates.double(), candidate_down.double(),
                             source_down.double())
    torch.testing.assert_close(pc.decoded_down_sse(st, candidate_down, source_down).double(), explicit, rtol=2e-4, atol=2e-4)
    sparse = pc.CandidateHiddenStatistics.zeros(64, dtype=torch.float32, retain_source_gram=False)
    sparse.update(candidate, source, gates)
    e_c = candidate.double() @ candidate_down.double() - source.double() @ source_down.double()
    e_b = candidate.double() @ baseline_down.double() - source.double() @ source_down.double()
    expected = (gates.double()[:, None].square() * (e_c.square() - e_b.square())).sum()
    torch.testing.assert_close(pc.decoded_down_sse_difference(sparse, candidate_down, baseline_down, source_down).double(),
                               expected, rtol=2e-4, atol=2e-4)


def _tiny_expert(seed):
    g = torch.Generator().manual_seed(seed)
    return g, pc.CoupledTriplet(torch.randn(3, 4, generator=g), torch.randn(3, 4, generator=g),
                                torch.randn(4, 3, generator=g))


def test_pooled_coupled_evaluation_matches_explicit_routed_function():
    g, source = _tiny_expert(4051)
    spec = CoupledHadamardSpec(residual_block_size=2, preactivation_block_size=2, postactivation_block_size=1,
                               intermediate_draw=3)
    execution = CoupledHadamardExecution(hidden=4, intermediate=3, spec=spec)
    enc = pc.CoupledTriplet(*encode_coupled_weights(source.tensors(), spec))
    candidate = pc.CoupledTriplet(enc.gate + 0.015, enc.up - 0.02, enc.down + 0.01)
    inputs = torch.randn(11, 4, generator=g)
    gates = torch.rand(11, generator=g)
    idx = torch.tensor([0, 2, 3, 7, 8, 11, 13, 18, 20, 22, 29])
    batches = [{"input": inputs[:6], "route_weight": gates[:6], "row_index": idx[:6]},
               {"input": inputs[6:6], "route_weight": gates[6:6], "row_index": idx[6:6]},
               {"input": inputs[6:], "route_weight": gates[6:], "row_index": idx[6:]}]
    res = pc.evaluate_coupled_expert_batches(batches, source=source, candidate_coordinates=candidate, execution=execution,
                                             prefix_row_limits=(10, 21, 30), statistics_dtype=torch.float64,
                                             retain_source_gram=True)
    # the explicit function over the same batch partition: FP32 products over
    # a different number of rows round differently
    src_out = torch.cat([situ(b["input"] @ source.gate.T, b["input"] @ source.up.T) @ source.down.T for b in batches])
    cand_out = torch.cat([execution.execute(b["input"], candidate.tensors()) for b in batches])
    err = ((cand_out - src_out) * gates[:, None]).square().sum(dim=1).double()
    energy = (src_out * gates[:, None]).square().sum(dim=1).double()
    assert res.routed_occurrences == 11
    assert res.sse == pytest.approx(float(err.sum()), rel=2e-6)
    assert res.source_energy == pytest.approx(float(energy.sum()), rel=2e-6)
    assert res.nmse == pytest.approx(res.sse / res.source_energy)
    for limit, n in ((10, 5), (21, 9), (30, 11)):
        s, e, count = res.prefix_scores[limit]
        assert count == n
        assert s == pytest.approx(float(err[:n].sum()), rel=2e-6)
        assert e == pytest.approx(float(energy[:n].sum()), rel=2e-6)
    t = execution.transform_inputs(inputs)
    explicit = ((execution.decode_middle(t, candidate.gate, candidate.up) @ candidate.down.T
                 - execution.decode_middle(t, enc.gate, enc.up) @ enc.down.T) * gates[:, None]).square().sum()
    torch.testing.assert_close(pc.decoded_down_sse(res.statistics, candidate.down.T, enc.down.T), explicit.double(),
                               rtol=2e-6, atol=2e-6)
    hidden = pc.collect_coupled_hidden_statistics(batches, source=source, candidate_coordinates=candidate,
                                                  execution=execution, statistics_dtype=torch.float64,
                                                  retain_source_gram=True)
    for x, y in zip(hidden._matrices(), res.statistics._matrices()):
        torch.testing.assert_close(x, y)
    assert hidden.rows == res.statistics.rows
    with pytest.raises(ValueError, match="increasing"):
        pc.evaluate_coupled_expert_batches([batches[2], batches[0]], source=source, candidate_coordinates=candidate,
                                           execution=execution)
    with pytest.raises(TypeError, match="int64"):
        pc.collect_coupled_hidden_statistics([{**batches[0], "row_index": idx[:6].int()}], source=source,
                                             candidate_coordinates=candidate, execution=execution)


def test_portfolio_matches_independent_candidate_scores():
    g, source = _tiny_expert(1987)
    inputs = torch.randn(13, 4, generator=g)
    route = torch.rand(13, generator=g)
    idx = torch.arange(2, 28, 2, dtype=torch.int64)
    batches = [{"input": inputs[:7], "route_weight": route[:7], "row_index": idx[:7]},
               {"input": inputs[7:], "route_weight": route[7:], "row_index": idx[7:]}]
    candidates, executions = {}, {}
    for draw, off in ((0, 0.01), (3, -0.015)):
        spec = CoupledHadamardSpec(residual_block_size=2, preactivation_block_size=2, postactivation_block_size=1,
                                   intermediate_draw=draw)
        enc = pc.CoupledTriplet(*encode_coupled_weights(source.tensors(), spec))
        candidates[str(draw)] = pc.CoupledTriplet(enc.gate + off, enc.up - 0.5 * off, enc.down + 0.25 * off)
        executions[str(draw)] = CoupledHadamardExecution(4, 3, spec)
    port = pc.evaluate_coupled_candidate_portfolio_batches(iter(batches), source=source, candidate_coordinates=candidates,
                                                           executions=executions)
    for name, cand in candidates.items():
        one = pc.evaluate_coupled_expert_batches(iter(batches), source=source, candidate_coordinates=cand,
                                                 execution=executions[name])
        assert port.candidate_sse[name] == pytest.approx(one.sse, rel=2e-6)
        assert port.source_energy == pytest.approx(one.source_energy, rel=2e-6)
        assert port.routed_occurrences == one.routed_occurrences == 13


def test_situ_derivatives_match_autograd():
    g = torch.Generator().manual_seed(5)
    gate = (6 * torch.randn(200, generator=g, dtype=torch.float64)).requires_grad_()
    up = (40 * torch.randn(200, generator=g, dtype=torch.float64)).requires_grad_()
    f = 4.0 * torch.tanh(gate / 4.0) * torch.sigmoid(gate) * 25.0 * torch.tanh(up / 25.0)
    dg, du = torch.autograd.grad(f.sum(), (gate, up))
    ag, au = situ_derivatives(gate.detach(), up.detach())
    # evaluated in FP32, derivatives of magnitude up to ~25
    torch.testing.assert_close(ag.double(), dg, rtol=2e-5, atol=2e-5)
    torch.testing.assert_close(au.double(), du, rtol=2e-5, atol=2e-5)


def test_upstream_functional_statistics_match_explicit_outer_products():
    g, source = _tiny_expert(903)
    inputs = torch.randn(9, 4, generator=g)
    route = torch.rand(9, generator=g)
    st = pc.collect_upstream_functional_statistics(
        [{"input": inputs[:4], "route_weight": route[:4], "row_index": torch.arange(4)},
         {"input": inputs[4:], "route_weight": route[4:], "row_index": torch.arange(4, 9)}], source=source, device="cpu")
    gate, up = inputs @ source.gate.T, inputs @ source.up.T
    dg, du = situ_derivatives(gate, up)
    w = route.double().square()
    down_energy = source.down.double().square().sum(dim=0)
    expected = torch.zeros(3, 2, 2, dtype=torch.float64)
    for r in range(9):
        for n in range(3):
            d = torch.tensor([dg[r, n], du[r, n]], dtype=torch.float64)
            expected[n] += w[r] * torch.outer(d, d) * down_energy[n]
    torch.testing.assert_close(st.derivative_metric, expected)
    torch.testing.assert_close(st.hidden_energy, (situ(gate, up).double().square() * w[:, None]).sum(dim=0))
    assert st.rows == 9 and st.effective_sample_size > 0


def test_blockwise_conditioning_coefficients_sum_metrics_before_ratio():
    metric = torch.tensor([[[4.0, 2.0], [2.0, 9.0]], [[1.0, -0.5], [-0.5, 1.0]],
                           [[2.0, 1.0], [1.0, 8.0]], [[6.0, 3.0], [3.0, 4.0]]], dtype=torch.float64)
    gate_from_up, up_from_gate, ev = pc.blockwise_upstream_conditioning_coefficients(metric, block_size=2)
    torch.testing.assert_close(gate_from_up, torch.tensor((0.3, 0.3, 0.5, 0.5), dtype=torch.float64))
    torch.testing.assert_close(up_from_gate, torch.tensor((0.15, 0.15, 1 / 3, 1 / 3), dtype=torch.float64))
    assert ev["block_size"] == 2 and ev["blocks"] == 2
    with pytest.raises(ValueError, match="positive semidefinite"):
        pc.blockwise_upstream_conditioning_coefficients(torch.tensor([[[1.0, 2.0], [2.0, 1.0]]]), block_size=1)
    with pytest.raises(ValueError, match="divide"):
        pc.blockwise_upstream_conditioning_coefficients(metric, block_size=3)


def test_scaled_row_accumulation_equals_weighted_definition():
    """The device path's algebra (rows scaled by |route|, residual formed
    before scaling), run through the gemm module's CPU branch."""

    source, candidate, gates, down = _samples()
    signed = gates * torch.where(torch.arange(37) % 3 == 0, -1.0, 1.0).double()
    st = pc.CandidateHiddenStatistics.zeros(7, dtype=torch.float32)
    st._update_matrix_cores(candidate.float(), source.float(), signed.float())
    ref = pc.CandidateHiddenStatistics.zeros(7)
    ref.update(candidate, source, signed)
    for x, y in zip(st._matrices(), ref._matrices()):
        torch.testing.assert_close(x.double(), y, rtol=1e-5, atol=1e-5)
