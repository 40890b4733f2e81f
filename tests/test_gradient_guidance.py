"""Linear-objective guidance (``qsrt_amd.gradient_guided_viterbi``,
reference ``qsrt/gradient_guided_viterbi.py``) pinned by completing the
square: a shifted target must change a quadratic objective by a constant,
whatever the candidate, so that both objectives share their minimiser."""

from __future__ import annotations

import pytest
import torch

from qsrt_amd.gradient_guided_viterbi import (LowRankViterbiGradientGuidance, ViterbiGradientGuidance,
                                              shift_elementwise_target, shift_two_sided_target,
                                              two_sided_guided_objective)


def _spd(n: int, g: torch.Generator) -> torch.Tensor:
    a = torch.randn(n, n, generator=g, dtype=torch.float64)
    return a @ a.T + n * torch.eye(n, dtype=torch.float64)


@pytest.mark.parametrize("per_element", [False, True])
def test_elementwise_shift_keeps_the_guided_minimiser(per_element):
    g = torch.Generator().manual_seed(1)
    t = torch.randn(8, 16, generator=g)
    grad = torch.randn(8, 16, generator=g)
    a = torch.rand(8, 16, generator=g) + 0.5 if per_element else 1.7
    s = 0.6
    t2 = shift_elementwise_target(t, grad, strength=s, quadratic_weight=a).double()
    a64 = torch.as_tensor(a, dtype=torch.float64)
    consts = []
    for _ in range(4):
        q = torch.randn(8, 16, generator=g, dtype=torch.float64)
        guided = a64 * (q - t.double()) ** 2 + s * grad.double() * q
        shifted = a64 * (q - t2) ** 2
        consts.append(guided - shifted)
    for c in consts[1:]:
        assert torch.allclose(c, consts[0], atol=1e-5)


def test_two_sided_shift_keeps_the_guided_minimiser():
    g = torch.Generator().manual_seed(2)
    hr, hc = _spd(12, g), _spd(8, g)
    t = torch.randn(12, 8, generator=g, dtype=torch.float64)
    grad = torch.randn(12, 8, generator=g, dtype=torch.float64)
    anchor = torch.randn(12, 8, generator=g, dtype=torch.float64)
    s = 0.9
    t2 = shift_two_sided_target(t, grad, hr, hc, strength=s)
    deltas = []
    for _ in range(4):
        q = torch.randn(12, 8, generator=g, dtype=torch.float64)
        _, _, guided = two_sided_guided_objective(t, q, anchor, grad, hr, hc, strength=s)
        e = q - t2
        deltas.append(float(guided - torch.sum(e * (hr @ e @ hc))))
    assert max(deltas) - min(deltas) <= 1e-9 * max(abs(d) for d in deltas)
    # the quadratic term is tr(E^T H_row E H_col) and the linear one s <g, Q - anchor>
    q = torch.randn(12, 8, generator=g, dtype=torch.float64)
    quad, lin, tot = two_sided_guided_objective(t, q, anchor, grad, hr, hc, strength=s)
    e = q - t
    assert torch.allclose(quad, torch.trace(e.T @ hr @ e @ hc))
    assert torch.allclose(lin, s * torch.sum(grad * (q - anchor)))
    assert torch.allclose(tot, quad + lin)


def test_low_rank_guidance_equals_dense_guidance():
    g = torch.Generator().manual_seed(3)
    left, right = torch.randn(32, 3, generator=g, dtype=torch.float64), torch.randn(3, 16, generator=g,
                                                                                   dtype=torch.float64)
    anchor = torch.randn(32, 16, generator=g, dtype=torch.float64)
    low = LowRankViterbiGradientGuidance(left, right, anchor, "anchor", "obj", strength=0.7)
    dense = ViterbiGradientGuidance(left @ right, anchor, "anchor", "obj", strength=0.7)
    low.validate((32, 16))
    dense.validate((32, 16))
    q = torch.randn(32, 16, generator=g, dtype=torch.float64)
    assert abs(low.linear_term(q, dtype=torch.float64) - dense.linear_term(q, dtype=torch.float64)) <= 1e-9
    assert torch.allclose(low.rows(slice(16, 32), device="cpu", dtype=torch.float64), (left @ right)[16:32])


def test_guidance_validation_errors():
    z = torch.zeros(4, 4)
    with pytest.raises(ValueError, match="nonnegative"):
        ViterbiGradientGuidance(z, z, "a", "o", strength=-1.0).validate((4, 4))
    with pytest.raises(ValueError, match="identities"):
        ViterbiGradientGuidance(z, z, "", "o").validate((4, 4))
    with pytest.raises(ValueError, match="do not match"):
        ViterbiGradientGuidance(z, z, "a", "o").validate((4, 8))
    with pytest.raises(ValueError, match="finite"):
        ViterbiGradientGuidance(torch.full((4, 4), float("nan")), z, "a", "o").validate((4, 4))
    with pytest.raises(ValueError, match="geometry"):
        LowRankViterbiGradientGuidance(torch.zeros(4, 2), torch.zeros(3, 4), z, "a", "o").validate((4, 4))
    with pytest.raises(ValueError, match="matching"):
        shift_elementwise_target(z, torch.zeros(4, 5), strength=1.0)
    with pytest.raises(ValueError, match="positive"):
        shift_elementwise_target(z, z, strength=1.0, quadratic_weight=0.0)
    with pytest.raises(ValueError, match="geometry"):
        shift_two_sided_target(z, z, torch.eye(3), torch.eye(4), strength=1.0)
