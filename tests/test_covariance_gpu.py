"""Covariance producers on the GPU: weighted covariance and pooled candidate
statistics accumulate on the FP32 matrix cores (qsrt_gemm_tn) and must agree
with float64 CPU evaluations of the same definitions."""

from __future__ import annotations

import sys

import pytest
import torch

from qsrt_amd import candidate_hessian as ch
from qsrt_amd import pooled_calibration as pc
from qsrt_amd.qsrt_coupled import CoupledHadamardExecution, CoupledHadamardSpec, encode_coupled_weights

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


def test_candidate_statistics_on_matrix_cores_match_float64():
    print("[cov] candidate statistics 3001x512", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(71)
    source = torch.randn(3001, 512, generator=g)
    candidate = source + 0.05 * torch.randn(3001, 512, generator=g)
    route = torch.rand(3001, generator=g) * torch.where(torch.rand(3001, generator=g) < 0.5, -1.0, 1.0)
    gpu = pc.CandidateHiddenStatistics.zeros(512, device=DEV, dtype=torch.float32)
    for a, b in ((0, 1000), (1000, 1000), (1000, 3001)):
        gpu.update(candidate[a:b].to(DEV), source[a:b].to(DEV), route[a:b].to(DEV))
    cpu = pc.CandidateHiddenStatistics.zeros(512)
    cpu.update(candidate.double(), source.double(), route.double())
    for name in ("candidate_gram", "candidate_source_cross", "source_gram", "candidate_residual_cross",
                 "hidden_residual_gram"):
        err = _frob_rel(getattr(gpu, name), getattr(cpu, name))
        assert err < 1e-5, (name, err)
    assert gpu.weight_sum == pytest.approx(cpu.weight_sum, rel=1e-6)
    assert gpu.rows == 3001
    h_gpu, ev_gpu = pc.candidate_h2(gpu)
    h_cpu, ev_cpu = pc.candidate_h2(cpu)
    assert ev_gpu["local_alpha"] == pytest.approx(ev_cpu["local_alpha"], rel=1e-5)
    assert _frob_rel(h_gpu, h_cpu) < 1e-5


def test_matrix_core_statistics_avoid_energy_cancellation():
    print("[cov] cancellation 2048x64", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(13084)
    source = 16.0 * torch.randn(2048, 64, generator=g)
    candidate = source + 2e-3 * torch.randn(2048, 64, generator=g)
    gates = torch.rand(2048, generator=g)
    source_down = 8.0 * torch.randn(64, 48, generator=g)
    candidate_down = source_down + 1e-3 * torch.randn(64, 48, generator=g)
    st = pc.CandidateHiddenStatistics.zeros(64, device=DEV, dtype=torch.float32)
    st.update(candidate.to(DEV), source.to(DEV), gates.to(DEV))
    explicit = (gates.double()[:, None] * (candidate.double() @ candidate_down.double()
                                           - source.double() @ source_down.double())).square().sum()
    got = pc.decoded_down_sse(st, candidate_down, source_down).double().cpu()
    torch.testing.assert_close(got, explicit, rtol=2e-4, atol=2e-4)


def test_build_expert_hessians_on_device():
    print("[cov] build_expert_hessians 2000 rows", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(9)
    inputs = torch.randn(2000, 1024, generator=g)
    gates = torch.rand(2000, generator=g)
    middle = torch.randn(2000, 256, generator=g)
    global_h13 = torch.eye(1024)
    h13, h2, ev = ch.build_expert_hessians(inputs.to(DEV), gates.to(DEV), middle.to(DEV), global_h13=global_h13,
                                           global_h2=torch.zeros(256, 256), device=DEV, h13_alpha=0.3)
    w = gates.double().square()
    local_h13 = inputs.double().T @ (inputs.double() * w[:, None]) / w.sum()
    local_h2 = middle.double().T @ (middle.double() * w[:, None]) / w.sum()
    assert _frob_rel(h13, 0.7 * global_h13.double() + 0.3 * local_h13) < 1e-5
    want_h2, s = ch.adaptive_identity_shrinkage(local_h2, w, max_local_alpha=0.75)
    assert ev["h2_local_alpha"] == pytest.approx(s["local_alpha"], rel=1e-5)
    assert _frob_rel(h2, want_h2) < 1e-5


def test_coupled_evaluation_on_device_matches_cpu():
    print("[cov] coupled evaluation hidden 1024 intermediate 256", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(4)
    hidden, inter = 1024, 256
    source = pc.CoupledTriplet(torch.randn(inter, hidden, generator=g) / 32, torch.randn(inter, hidden, generator=g) / 32,
                               torch.randn(hidden, inter, generator=g) / 16)
    spec = CoupledHadamardSpec(intermediate_draw=2)
    execution = CoupledHadamardExecution(hidden, inter, spec)
    enc = pc.CoupledTriplet(*encode_coupled_weights(source.tensors(), spec))
    candidate = pc.CoupledTriplet(*(t + 0.002 * torch.randn(t.shape, generator=g) for t in enc.tensors()))
    inputs = torch.randn(700, hidden, generator=g)
    route = torch.rand(700, generator=g)
    idx = torch.arange(0, 1400, 2, dtype=torch.int64)
    batches = [{"input": inputs[a:b], "route_weight": route[a:b], "row_index": idx[a:b]} for a, b in ((0, 300), (300, 700))]
    cpu = pc.evaluate_coupled_expert_batches(batches, source=source, candidate_coordinates=candidate,
                                             execution=execution, prefix_row_limits=(500,),
                                             statistics_dtype=torch.float64, retain_source_gram=True)
    gpu = pc.evaluate_coupled_expert_batches(batches, source=source, candidate_coordinates=candidate.to(DEV),
                                             execution=execution, prefix_row_limits=(500,),
                                             statistics_dtype=torch.float32, retain_source_gram=True)
    assert gpu.routed_occurrences == cpu.routed_occurrences == 700
    assert gpu.sse == pytest.approx(cpu.sse, rel=1e-4)
    assert gpu.source_energy == pytest.approx(cpu.source_energy, rel=1e-5)
    assert gpu.prefix_scores[500][2] == cpu.prefix_scores[500][2] == 250
    assert _frob_rel(gpu.statistics.candidate_gram, cpu.statistics.candidate_gram) < 1e-5
    sse_gpu = float(pc.decoded_down_sse(gpu.statistics, candidate.down.T, enc.down.T))
    sse_cpu = float(pc.decoded_down_sse(cpu.statistics, candidate.down.T, enc.down.T))
    assert sse_gpu == pytest.approx(sse_cpu, rel=1e-4)
