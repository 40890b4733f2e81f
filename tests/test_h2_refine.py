"""Dense-H path refinement and gradient guidance (reference
tests/test_h2_viterbi_refine.py): objective definitions, monotone sweeps,
no-op cases and the completed-square target shifts."""

from __future__ import annotations

import pytest
import torch

from qsrt_amd.gradient_guided_viterbi import (LowRankViterbiGradientGuidance, ViterbiGradientGuidance,
                                              shift_elementwise_target, shift_two_sided_target,
                                              two_sided_guided_objective)
from qsrt_amd.exl3_reference import tensor_core_permutation
from qsrt_amd.h2_viterbi_refine import (H2ViterbiRefineConfig, config_from_quant_args, dense_h_guided_objective,
                                        dense_h_objective, refine_h2_viterbi_paths)


class NearestGrid:
    def __init__(self, levels):
        self.levels = levels

    def __call__(self, tiles):
        levels = self.levels.to(device=tiles.device, dtype=tiles.dtype)
        code = (tiles[..., None] - levels).abs().argmin(dim=-1)
        return levels[code], code.to(torch.int16)


def _spd(n, cond, seed):
    g = torch.Generator().manual_seed(seed)
    q, _ = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
    ev = torch.exp(torch.linspace(-0.5, 0.5, n, dtype=torch.float64) * torch.log(torch.tensor(cond)))
    h = q @ torch.diag(ev) @ q.T + 0.025 * torch.eye(n, dtype=torch.float64)
    return (h / torch.diag(h).mean()).float()


PERM = tensor_core_permutation("cpu")


def _independent(weight, quantizer):
    """Per-tile encode in the tensor-core order the refinement uses."""

    r, c = weight.shape
    flat = weight.reshape(r // 16, 16, c // 16, 16).permute(0, 2, 1, 3).reshape(-1, 256)[:, PERM]
    recon, code = quantizer(flat)
    recon = recon[:, torch.argsort(PERM)]
    return (recon.reshape(r // 16, c // 16, 16, 16).permute(0, 2, 1, 3).reshape(r, c),
            code.reshape(r // 16, c // 16, *code.shape[1:]))


def _decode(levels, encoded, r, c):
    tiles = levels[encoded.long()].reshape(-1, 256)[:, torch.argsort(PERM)]
    return tiles.reshape(r // 16, c // 16, 16, 16).permute(0, 2, 1, 3).reshape(r, c)


def test_dense_objective_and_column_weights():
    g = torch.Generator().manual_seed(9)
    w, q = torch.randn(32, 16, generator=g), torch.randn(32, 16, generator=g)
    h = _spd(32, 3.0, 10)
    e = (w - q).double()
    assert dense_h_objective(w, q, h) == pytest.approx(float(torch.sum(e * (h.double() @ e))), rel=1e-10)
    s_in, s_out = torch.exp(0.2 * torch.randn(32, generator=g)), torch.exp(0.2 * torch.randn(16, generator=g))
    src_e = s_in[:, None] * (w - q) * s_out[None]
    explicit = float(torch.sum(src_e.double() * (h.double() @ src_e.double())))
    enc_h = s_in[:, None] * h * s_in[None, :]
    assert dense_h_objective(w, q, enc_h, column_weights=s_out.square()) == pytest.approx(explicit, rel=1e-6)
    assert dense_h_objective(w, q, h, chunk_columns=3) == pytest.approx(dense_h_objective(w, q, h), rel=1e-12)


@pytest.mark.parametrize("score_dtype", [torch.float64, torch.float32])
def test_refinement_is_monotone_and_improves(score_dtype):
    torch.manual_seed(3)
    w = torch.randn(64, 32)
    h = _spd(64, 5.0, 4)
    quant = NearestGrid(torch.tensor([-1.5, -0.5, 0.5, 1.5]))
    initial, payload = _independent(w, quant)
    before = dense_h_objective(w, initial, h)
    res = refine_h2_viterbi_paths(w, h, initial, payload, quant,
                                  H2ViterbiRefineConfig(sweeps=2, dither_scales=(0.02, 0.04), num_dither_patterns=2,
                                                        score_dtype=score_dtype))
    after = dense_h_objective(w, res.weight_q, h)
    assert res.weight_q.shape == initial.shape and res.encoded.shape == payload.shape
    assert after < before
    assert all(s.objective_after <= s.objective_before + 1e-6 for s in res.sweep_stats)
    # the payload still encodes the reconstruction
    assert torch.equal(_decode(torch.tensor([-1.5, -0.5, 0.5, 1.5]), res.encoded, 64, 32), res.weight_q)


def test_identity_hessian_is_a_no_op():
    torch.manual_seed(5)
    w = torch.randn(32, 16)
    quant = NearestGrid(torch.tensor([-1.0, 0.0, 1.0]))
    initial, payload = _independent(w, quant)
    res = refine_h2_viterbi_paths(w, torch.eye(32), initial, payload, quant, H2ViterbiRefineConfig())
    assert res.sweep_stats[0].accepted_tiles == 0
    assert torch.equal(res.weight_q, initial) and torch.equal(res.encoded, payload)


def test_packed_payload_shape_is_preserved():
    torch.manual_seed(7)

    class Packed(NearestGrid):
        def __call__(self, tiles):
            r, code = super().__call__(tiles)
            return r, code.reshape(code.shape[0], 128, 2)

    w = torch.randn(32, 16)
    quant = Packed(torch.tensor([-1.0, 0.0, 1.0]))
    initial, payload = _independent(w, quant)
    assert payload.shape == (2, 1, 128, 2)
    res = refine_h2_viterbi_paths(w, _spd(32, 2.0, 8), initial, payload, quant,
                                  H2ViterbiRefineConfig(dither_scales=(0.02,), num_dither_patterns=1))
    assert res.encoded.shape == payload.shape


def test_zero_strength_guidance_equals_plain_refinement():
    torch.manual_seed(11)
    w = torch.randn(48, 32)
    h = _spd(48, 4.0, 12)
    quant = NearestGrid(torch.tensor([-1.5, -0.5, 0.5, 1.5]))
    initial, payload = _independent(w, quant)
    cfg = H2ViterbiRefineConfig(sweeps=2, score_dtype=torch.float64)
    control = refine_h2_viterbi_paths(w, h, initial, payload, quant, cfg)
    guided = refine_h2_viterbi_paths(w, h, initial, payload, quant, cfg, guidance=ViterbiGradientGuidance(
        torch.randn_like(w), initial, "anchor", "objective", strength=0.0))
    assert torch.equal(guided.weight_q, control.weight_q) and guided.stats_dict() == control.stats_dict()


def test_guided_refinement_is_monotone_and_low_rank_matches_dense():
    torch.manual_seed(13)
    w = torch.randn(32, 32)
    h = _spd(32, 2.5, 14)
    quant = NearestGrid(torch.tensor([-1.0, 0.0, 1.0]))
    initial, payload = _independent(w, quant)
    left, right = torch.randn(32, 3), torch.randn(3, 32)
    dense = ViterbiGradientGuidance(left @ right, initial, "a", "o", strength=0.35)
    low = LowRankViterbiGradientGuidance(left, right, initial, "a", "o", strength=0.35)
    before = dense_h_guided_objective(w, initial, h, dense)
    assert before[1] == 0.0
    cfg = H2ViterbiRefineConfig(sweeps=3, score_dtype=torch.float64)
    r_dense = refine_h2_viterbi_paths(w, h, initial, payload, quant, cfg, guidance=dense)
    r_low = refine_h2_viterbi_paths(w, h, initial, payload, quant, cfg, guidance=low)
    after = dense_h_guided_objective(w, r_dense.weight_q, h, dense)
    assert after[2] <= before[2] + 1e-6
    assert torch.equal(r_dense.weight_q, r_low.weight_q)
    # the dense gradient was formed in FP32, the low-rank term contracts in FP64
    assert low.linear_term(r_low.weight_q, dtype=torch.float64) == pytest.approx(after[1], rel=1e-6)


def test_target_shifts_complete_the_square():
    g = torch.Generator().manual_seed(2)
    t, grad = torch.randn(4, 6, generator=g), torch.randn(4, 6, generator=g)
    a = torch.rand(4, 6, generator=g) + 0.5
    shifted = shift_elementwise_target(t, grad, strength=0.7, quadratic_weight=a)
    # a (q - t)^2 + 0.7 g q and a (q - shifted)^2 differ by a constant in q
    q1, q2 = torch.randn(4, 6, generator=g), torch.randn(4, 6, generator=g)
    f = lambda q: a * (q - t) ** 2 + 0.7 * grad * q
    s = lambda q: a * (q - shifted) ** 2
    torch.testing.assert_close(f(q1) - s(q1), f(q2) - s(q2), rtol=1e-4, atol=1e-4)
    h_row, h_col = _spd(16, 2.0, 3).double(), _spd(16, 3.0, 4).double()
    T, G, anchor = (torch.randn(16, 16, generator=g, dtype=torch.float64) for _ in range(3))
    shifted2 = shift_two_sided_target(T, G, h_row, h_col, strength=0.4)
    Q1, Q2 = (torch.randn(16, 16, generator=g, dtype=torch.float64) for _ in range(2))
    obj = lambda Q: two_sided_guided_objective(T, Q, anchor, G, h_row, h_col, strength=0.4)[2]
    sq = lambda Q: torch.sum((Q - shifted2) * (h_row @ (Q - shifted2) @ h_col))
    torch.testing.assert_close(obj(Q1) - sq(Q1), obj(Q2) - sq(Q2), rtol=1e-9, atol=1e-9)


def test_config_from_quant_args():
    cfg = config_from_quant_args({"h2_viterbi_refine_sweeps": 3, "h2_viterbi_refine_dither_scales": [0.1],
                                  "h2_viterbi_refine_patterns": 2, "h2_viterbi_refine_fp64_score": True})
    assert cfg.sweeps == 3 and cfg.dither_scales == (0.1,) and cfg.num_dither_patterns == 2
    assert cfg.score_dtype == torch.float64 and cfg.max_quantizer_batch == 256
