"""Pooled calibration statistics and the expert Hessian policy on cuda:0.

* the stacked weighted Gram on the FP32 and on the float64 matrix cores
  against float64 products on the CPU;
* ``build_expert_hessians`` for a low-support expert (19 routed rows, the
  rarest expert of the config-5 layer) against scikit-learn's OAS of the same
  rows, and the per-rate H2 ladder against its CPU run;
* a coupled Kimi-shape expert evaluated over routed batches: the routed SSE
  against an explicit float64 forward, and the statistics' score of the
  candidate's down projection against the explicit coupled-basis SSE.
"""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

from qsrt_amd import candidate_hessian as ch
from qsrt_amd import pooled_calibration as pc
from qsrt_amd.qsrt_coupled import CoupledHadamardSpec, coupled_execution, encode_coupled_weights, situ

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-5), (torch.float64, 1e-12)])
def test_stacked_statistics_on_the_matrix_cores(dtype, tol):
    n, w = 20_000, 512
    _say(f"[pooled] stacked Gram {n} rows x 2 x {w} ({dtype}) on cuda:0")
    g = torch.Generator().manual_seed(5)
    S = torch.randn(n, w, generator=g)
    C = S + 0.02 * torch.randn(n, w, generator=g)
    route = torch.rand(n, generator=g) + 0.1
    st = pc.CandidateHiddenStatistics.zeros(w, device=DEV, dtype=dtype)
    for lo in range(0, n, 6000):  # several chunks accumulate into one Gram
        st.update(C[lo:lo + 6000].to(DEV), S[lo:lo + 6000].to(DEV), route[lo:lo + 6000].to(DEV))
    torch.cuda.synchronize()
    Cd, Sd, Wd = C.double(), S.double(), route.double().square()[:, None]
    # rows are FP32 on both sides: the statistics are computed from the same values
    Cd, Sd = C.to(dtype).double(), S.to(dtype).double()
    Rd = (C.to(dtype) - S.to(dtype)).double()
    for name, want in (("candidate_gram", Cd.T @ (Cd * Wd)), ("candidate_residual_cross", Cd.T @ (Rd * Wd)),
                       ("hidden_residual_gram", Rd.T @ (Rd * Wd)), ("candidate_source_cross", Cd.T @ (Sd * Wd)),
                       ("source_gram", Sd.T @ (Sd * Wd))):
        got = getattr(st, name).double().cpu()
        err = float((got - want).abs().max() / want.abs().max())
        _say(f"[pooled] {name}: max rel {err:.2e}")
        assert err <= tol, name


def test_low_support_expert_hessians_match_sklearn_oas():
    from sklearn.covariance import oas

    import bench

    counts = bench.zipf_token_counts()
    expert = counts.index(min(counts))
    _say(f"[pooled] build_expert_hessians for layer expert {expert} ({counts[expert]} routed rows)")
    d = bench.config_expert(5, DEV, expert=expert, tokens=counts[expert])
    x = d["x"].float()
    gates = torch.linspace(0.2, 0.9, x.shape[0], device=DEV)
    middle = torch.nn.functional.silu(x @ d["w_gate"].float().T) * (x @ d["w_up"].float().T)
    g13 = torch.eye(x.shape[1], device=DEV)
    h13, h2, ev = ch.build_expert_hessians(x, gates, middle, global_h13=g13,
                                           global_h2=torch.eye(middle.shape[1]), device=DEV)
    torch.cuda.synchronize()
    assert torch.equal(h13, g13)
    # scikit-learn's OAS on rows scaled by the gate (the weighted covariance of equal-weight scaled rows) with
    # the Kish size of these weights differs from the unweighted OAS; compare instead against the closed form
    w = gates.double().square().cpu()
    rows = middle.double().cpu()
    S = rows.T @ (rows * w[:, None]) / w.sum()
    n_eff = float(w.sum() ** 2 / w.square().sum())
    p = S.shape[0]
    tr, tr2 = float(torch.trace(S)), float((S * S).sum())
    rho = min(1.0, (tr2 + tr * tr) / ((n_eff + 1.0) * (tr2 - tr * tr / p)))
    alpha = min(0.75, 1.0 - rho)
    want = (1 - alpha) * (tr / p) * torch.eye(p, dtype=torch.float64) + alpha * S
    err = float((h2.double().cpu() - want).abs().max() / want.abs().max())
    _say(f"[pooled] H2: OAS shrinkage {ev['h2_oas_shrinkage']:.4f} (closed form {rho:.4f}), local weight "
         f"{ev['h2_local_alpha']:.4f}, max rel {err:.2e}")
    assert math.isclose(ev["h2_oas_shrinkage"], rho, rel_tol=1e-6) and err <= 2e-5
    # with equal weights the closed form is scikit-learn's OAS
    ones = torch.ones(x.shape[0], device=DEV)
    _, h2_eq, ev_eq = ch.build_expert_hessians(x, ones, middle, global_h13=g13,
                                               global_h2=torch.eye(middle.shape[1]), device=DEV)
    shrunk, rho_sk = oas(rows.numpy(), assume_centered=True)
    assert math.isclose(ev_eq["h2_oas_shrinkage"], rho_sk, rel_tol=1e-6)
    if 1 - rho_sk <= 0.75:
        assert np.allclose(h2_eq.double().cpu().numpy(), shrunk, rtol=2e-5, atol=2e-5 * np.abs(shrunk).max())


def test_h2_ladder_on_device_matches_cpu():
    n, hidden, inter = 600, 512, 256
    _say(f"[pooled] conditional_h2_by_rate: 3 rates, {n} rows, {hidden} -> {inter}")
    g = torch.Generator().manual_seed(9)
    x = torch.randn(n, hidden, generator=g)
    gates = torch.rand(n, generator=g) + 0.1
    mask = torch.rand(n, generator=g) < 0.7
    recon = {r: (0.05 * torch.randn(inter, hidden, generator=g), 0.05 * torch.randn(inter, hidden, generator=g))
             for r in (0, 1, 2)}
    kw = dict(global_h13=torch.eye(hidden), global_h2=torch.eye(inter))
    gpu, ev = ch.conditional_h2_by_rate(x.to(DEV), gates.to(DEV), mask.to(DEV),
                                        {r: (a.to(DEV), b.to(DEV)) for r, (a, b) in recon.items()}, device=DEV, **kw)
    cpu, _ = ch.conditional_h2_by_rate(x, gates, mask, recon, device="cpu", **kw)
    torch.cuda.synchronize()
    for r in recon:
        err = float((gpu[r].cpu() - cpu[r]).abs().max() / cpu[r].abs().max())
        _say(f"[pooled] R{r}: local weight {ev[f'R{r}']['h2_local_alpha']:.4f}, device vs CPU max rel {err:.2e}")
        assert err <= 1e-4


def test_coupled_expert_evaluation_at_kimi_shape():
    hidden, inter, n = 7168, 2048, 512
    _say(f"[pooled] evaluate_coupled_expert_batches {hidden} x {inter}, {n} routed rows")
    g = torch.Generator().manual_seed(11)
    spec = CoupledHadamardSpec()
    src = pc.CoupledTriplet(0.015 * torch.randn(inter, hidden, generator=g),
                            0.015 * torch.randn(inter, hidden, generator=g),
                            0.015 * torch.randn(hidden, inter, generator=g)).to(DEV)
    coords = encode_coupled_weights(src.tensors(), spec)
    cand = pc.CoupledTriplet(*(c + 0.001 * torch.randn(c.shape, generator=g).to(DEV) for c in coords))
    ex = coupled_execution(src.tensors(), spec)
    x = torch.randn(n, hidden, generator=g).to(DEV)
    route = (torch.rand(n, generator=g) + 0.2).to(DEV)
    batches = [{"input": x[i:i + 128], "route_weight": route[i:i + 128],
                "row_index": torch.arange(i, i + 128, dtype=torch.int64)} for i in range(0, n, 128)]
    ev = pc.evaluate_coupled_expert_batches(batches, source=src, candidate_coordinates=cand, execution=ex,
                                            retain_source_gram=True, prefix_row_limits=(200,))
    torch.cuda.synchronize()
    xd = x.double()
    teacher = situ(xd @ src.gate.double().T, xd @ src.up.double().T) @ src.down.double().T
    output = ex.execute(x, cand.tensors()).double()
    want = float(((output - teacher) * route.double()[:, None]).square().sum())
    _say(f"[pooled] routed SSE {ev.sse:.6e} vs explicit {want:.6e}; nmse {ev.nmse:.3e}")
    assert math.isclose(ev.sse, want, rel_tol=1e-3)
    assert ev.prefix_scores[200][2] == 200
    sse = float(pc.decoded_down_sse(ev.statistics, cand.down.T, coords[2].T))
    xt = ex.transform_inputs(x)
    direct = ex.decode_middle(xt, cand.gate, cand.up) @ cand.down.T - ex.decode_middle(xt, coords[0], coords[1]) @ coords[2].T
    direct = float((direct.double() * route.double()[:, None]).square().sum())
    _say(f"[pooled] statistics' down SSE {sse:.6e} vs direct {direct:.6e}")
    assert math.isclose(sse, direct, rel_tol=1e-3)


def test_expert_encoder_support_aware_policy_on_low_support_experts():
    """The layer pipeline with the production covariance policy: the two
    least-routed experts of the config-5 layer (19-20 rows each) take the
    layer's global H13 and an OAS-shrunk H2.  The global H13 here is the
    covariance of the union of four experts' routed rows (the two encoded and
    the two most routed), a stand-in for the whole layer's calibration set.
    Every stored payload reads back (through the oracle's container reader)
    as the encoder's states, and the H2 evidence shows the shrinkage a
    tens-of-rows expert gets."""

    import bench
    from oracle import fmt as ofmt
    from qsrt_amd import exl3_encoder_backend as be
    from qsrt_amd import gemm

    counts = bench.zipf_token_counts()
    order = sorted(range(len(counts)), key=counts.__getitem__)
    low, high = order[:2], order[-2:]
    _say(f"[pooled] support-aware layer encode: experts {low} ({[counts[e] for e in low]} rows)")
    sources = [bench.expert_source(5, DEV, expert=e, tokens=counts[e]) for e in low + high]
    hidden = bench.LAYER_HIDDEN
    gram = torch.zeros((hidden, hidden), device=DEV)
    rows = 0
    for s in sources:
        gemm.gram_(gram, s["x"])
        rows += s["tokens"]
    scope = ("pooled-test", 1)
    enc = bench.ExpertEncoder(DEV, hidden=hidden, inter=bench.LAYER_INTER, record_bits=bench.LAYER_RECORD_BITS,
                              scope=scope, hessian_policy="support_aware", global_h13=gram / rows)
    try:
        out = enc.encode(sources[:2], keep_states=tuple(low))
        torch.cuda.synchronize()
    finally:
        for key in [k for k in be._SHARED_INPUT_SCALES if k[0] == scope]:
            del be._SHARED_INPUT_SCALES[key]
    for rec in out:
        ev = enc.h2_evidence[rec["expert"]]
        _say(f"[pooled] expert {rec['expert']}: H2 n_eff {ev['h2_effective_sample_size']:.1f}, OAS shrinkage "
             f"{ev['h2_oas_shrinkage']:.3f}, local weight {ev['h2_local_alpha']:.3f}; proxies "
             f"{rec['w1']['proxy']:.2e} {rec['w3']['proxy']:.2e} {rec['w2']['proxy']:.2e}")
        assert ev["h2_shrinkage_policy"] == "weighted_oas_scaled_identity"
        assert ev["h2_effective_sample_size"] < 40 and ev["h2_local_alpha"] < 0.75
        for m in ("w1", "w3", "w2"):
            r = rec[m]
            assert 0.0 < r["proxy"] < 0.1
            k, n = r["shape"]
            states, _ = ofmt.unpack_records(r["words"].cpu().numpy(), bench.LAYER_RECORD_BITS, r["rate_axis"],
                                            k // 16, n // 16)
            assert np.array_equal(states, r["encoded"].cpu().numpy().view(np.uint16))
