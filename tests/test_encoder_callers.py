"""Matrix encode plans (qsrt_amd.qsrt_encoder.plan_qsrt_matrix) on the CPU:
the LDLQ traversal, the stored P24/P33 order and the whole-record repack that
maps one onto the other (reference qsrt/pack/qsrt_encoder.py:300-365)."""

from __future__ import annotations

import pytest
import torch

from qsrt_amd import qsrt_encoder as enc
from qsrt_amd.qsrt import KIMI_K3, Geometry, expand_record_order, record_bits, resolve_mode


def _contexts(records: int, seed: int) -> torch.Tensor:
    """A shuffled one-context-per-record map over four-channel groups."""

    g = torch.Generator().manual_seed(seed)
    ctx = torch.arange(records).repeat_interleave(32)
    return ctx[torch.randperm(ctx.numel(), generator=g)]


@pytest.mark.parametrize("mode", ["R0", "R1", "R2"])
@pytest.mark.parametrize("matrix", ["w1", "w2"])
def test_plan_orders_and_repack_are_consistent(mode, matrix):
    ctx = _contexts(24, 5)
    plan = enc.plan_qsrt_matrix(ctx, mode, matrix=matrix)
    spec = resolve_mode(mode)
    n = KIMI_K3.intermediate_channels
    for perm in (plan.encoder_permutation, plan.physical_permutation):
        assert torch.equal(torch.sort(perm).values, torch.arange(n))
    # whole records move: physical channel order = encoder order read through the record repack
    assert torch.equal(plan.encoder_permutation[expand_record_order(plan.record_repack_order)],
                       plan.physical_permutation)
    # the stored tile rates follow the mode's serialized record schedule; the traversal is low to high
    assert plan.physical_tile_bits == tuple(b for b in record_bits(spec) for _ in range(8))
    assert list(plan.encoder_tile_bits) == sorted(plan.encoder_tile_bits)
    assert plan.physical_pair_bpw == (3.0,) * 12
    assert plan.rate_axis == ("k" if matrix == "w2" else "n")
    # every channel keeps its context's rate under both orders
    rates = torch.tensor(spec.context_bits)[ctx.repeat_interleave(4)]
    assert rates[plan.encoder_permutation].reshape(-1, 16)[:, 0].tolist() == list(plan.encoder_tile_bits)


def test_prefix_reuse_layout_keeps_the_stored_order():
    ctx = _contexts(24, 9)
    for mode in ("R0", "R1", "R2"):
        a = enc.plan_qsrt_matrix(ctx, mode, matrix="w2")
        b = enc.plan_qsrt_matrix(ctx, mode, matrix="w2", layout="qsrt_pair_prefix_reuse")
        assert torch.equal(a.physical_permutation, b.physical_permutation)
        assert b.physical_tile_bits == a.physical_tile_bits
    # the four transfer records come first in the traversal, the K3 middle is shared by every candidate
    r2 = enc.plan_qsrt_matrix(ctx, "R2", matrix="w2", layout="qsrt_pair_prefix_reuse")
    r0 = enc.plan_qsrt_matrix(ctx, "R0", matrix="w2", layout="qsrt_pair_prefix_reuse")
    assert r2.encoder_tile_bits[:32] == (2,) * 8 + (4,) * 8 + (2,) * 8 + (4,) * 8
    assert torch.equal(r2.encoder_permutation, r0.encoder_permutation)
    with pytest.raises(ValueError):
        enc.plan_qsrt_matrix(ctx, "H308", matrix="w2", layout="qsrt_pair_prefix_reuse")


def test_generic_geometry_and_argument_checks():
    geo = Geometry(512, 256)
    ctx = _contexts(4, 1)
    assert enc.geometry_for(ctx, 256) == geo
    plan = enc.plan_qsrt_matrix(ctx, "R1", matrix="w3", geometry=geo)
    assert plan.physical_tile_bits == (2,) * 8 + (4,) * 8 + (3,) * 16
    with pytest.raises(ValueError):
        enc.plan_qsrt_matrix(ctx, "R1", matrix="w9", geometry=geo)
    with pytest.raises(ValueError):
        enc.plan_qsrt_matrix(ctx[:-1], "R1", matrix="w1", geometry=geo)
    qa = enc._qsrt_quant_args(plan, matrix="w3", layer=3, device=torch.device("cpu"), shared_scale_scope="s")
    assert qa["mixed_tile_bits"] == plan.encoder_tile_bits and qa["mixed_rate_axis"] == "n"
    assert qa["shared_input_scales_key"] == ("s", "w3") and qa["g_scale_into_sv"] is True
    assert qa["seed"] == 3_000_001 and qa["sv_seed"] == 3_000_001 + 499_979
    assert set(qa["sqg_e4m3_luts_by_bits"]) == {2, 3, 4}
    with pytest.raises(ValueError):
        enc._qsrt_quant_args(plan, matrix="w3", layer=3, device=torch.device("cpu"), shared_scale_scope="s",
                             g_scale_override=-1.0)
    m = enc.comparison_metrics(torch.ones(4), torch.ones(4) * 1.5)
    assert m["relative_l2"] == pytest.approx(0.5) and m["max_abs"] == pytest.approx(0.5)
    assert m["cosine"] == pytest.approx(1.0)
