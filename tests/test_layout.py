"""Record layout and layer metadata of the QSRT format (qsrt_amd.qsrt):
pair placement, per-expert format codes, metadata sections, context orders
and record repacking.  Known answers follow the reference's own tests
(tests/test_qsrt.py:108-232, :414-520)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from qsrt_amd import qsrt as Q
from qsrt_amd.qsrt_coupled import situ


def test_pair_rotation_is_a_per_expert_bijection():
    for layer, expert in ((1, 0), (1, 17), (40, 285), (92, 895)):
        phys = [Q.physical_pair_slot(layer, expert, p) for p in range(Q.PAIRS_PER_EXPERT)]
        assert sorted(phys) == list(range(Q.PAIRS_PER_EXPERT))
        assert [Q.logical_pair_for_slot(layer, expert, s) for s in phys] == list(range(Q.PAIRS_PER_EXPERT))
    with pytest.raises(ValueError):
        Q.pair_rotation(0, 1)


def test_pair_rotation_balances_p24_ownership():
    counts = [0] * Q.PAIRS_PER_EXPERT
    for expert in range(Q.EXPERTS_PER_LAYER):
        for rank in range(Q.PAIRS_PER_EXPERT):
            counts[rank] += Q.logical_pair_for_slot(24, expert, rank) < 2
    assert max(counts) - min(counts) <= 1


def test_format_table_codes_and_names():
    formats = ["X4T", Q.R0, Q.R1, (1, 2)] * (Q.EXPERTS_PER_LAYER // 4)
    packed = Q.pack_qsrt_format_table(formats)
    assert packed.dtype == torch.uint8 and packed.shape == (Q.FORMAT_TABLE_BYTES,)
    assert packed[:4].tolist() == [0xFF, 0x00, 0x11, 0x12]
    assert Q.unpack_qsrt_format_table(packed) == tuple(["X4T", "R0", "R1", "R1/R2"] * (Q.EXPERTS_PER_LAYER // 4))
    bad = packed.clone()
    bad[0] = 0xD0
    with pytest.raises(ValueError, match="invalid rate code"):
        Q.unpack_qsrt_format_table(bad)
    assert Q.ExpertFormatSpec.compressed(3).name == "H308"
    assert Q.ExpertFormatSpec.from_code(0x44).name == "K2"
    with pytest.raises(ValueError, match="896 experts"):
        Q.pack_qsrt_format_table([Q.R0])
    with pytest.raises(ValueError):
        Q.ExpertFormatSpec(3, 1)  # H308 must cover both axes


def test_format_section_and_hot_metadata():
    formats = ["X4T", Q.R0, Q.R1, (1, 2)] * (Q.EXPERTS_PER_LAYER // 4)
    section = Q.pack_qsrt_format_section(formats)
    codes, slots = Q.expand_qsrt_hot_metadata(formats)
    assert section.shape == (Q.FORMAT_SECTION_BYTES,)
    assert torch.count_nonzero(section[Q.FORMAT_TABLE_BYTES:]) == 0
    assert codes[:8].tolist() == [255, 0, 17, 18, 255, 0, 17, 18]
    assert slots[:8].tolist() == [0, 0, 1, 2, 1, 3, 4, 5]
    assert codes.numel() + slots.numel() * slots.element_size() == Q.HOT_METADATA_BYTES
    bad = section.clone()
    bad[-1] = 1
    with pytest.raises(ValueError, match="nonzero alignment padding"):
        Q.unpack_qsrt_format_section(bad)


def test_shared_scale_section_round_trips():
    shared = tuple(torch.linspace(-1 + i, 1 + i, 3584, dtype=torch.float16) for i in range(3))
    section = Q.pack_qsrt_shared_scale_section(*shared)
    assert section.numel() == Q.SHARED_SCALE_SECTION_BYTES
    assert all(torch.equal(a, b) for a, b in zip(shared, Q.unpack_qsrt_shared_scale_section(section)))
    geo = Q.Geometry(2048, 7168)
    vecs = tuple(torch.full((7168,), 0.5 + i, dtype=torch.float16) for i in range(3))
    sec = Q.pack_qsrt_shared_scale_section(*vecs, geometry=geo)
    assert all(torch.equal(a, b) for a, b in zip(vecs, Q.unpack_qsrt_shared_scale_section(sec, geo)))


def test_context_orders_form_homogeneous_records():
    block_contexts = torch.arange(24).repeat_interleave(32)
    importance = Q.importance_group_order(block_contexts, Q.R2)
    storage = Q.storage_group_order(block_contexts, Q.R2)
    ch = block_contexts.index_select(0, storage).repeat_interleave(4)
    assert Q.expand_group_order(storage).shape == (Q.INTERMEDIATE_CHANNELS,)
    assert torch.all(ch.reshape(Q.RECORDS_PER_EXPERT, 128).diff(dim=1) == 0)
    assert ch.reshape(Q.RECORDS_PER_EXPERT, 128)[:, 0].tolist() == list(Q.record_contexts(Q.R2))
    order = Q.record_repack_order(importance, storage)
    encoded = torch.arange(Q.RECORDS_PER_EXPERT).repeat_interleave(8 * 256).reshape(192, 1, 256)
    repacked = Q.repack_encoded_records(encoded, order, "k")
    assert repacked.reshape(Q.RECORDS_PER_EXPERT, -1)[:, 0].tolist() == order.tolist()
    bad = importance.clone()
    bad[31], bad[32] = bad[32].clone(), bad[31].clone()
    with pytest.raises(ValueError, match="splits or changes"):
        Q.record_repack_order(importance, bad)


def test_shared_record_map_folds_into_common_permutation():
    g = torch.Generator().manual_seed(47)
    base = torch.arange(Q.RECORDS_PER_EXPERT).repeat_interleave(32)
    base = base[torch.randperm(base.numel(), generator=g)]
    donors, recipients = (7, 2), (19, 11)
    order = Q.rate_transfer_record_order(donors, recipients)
    relabeled = Q.relabel_block_contexts_for_record_order(base, order)
    importance = Q.importance_group_order(relabeled, Q.R2)
    assert order[:2] == donors and order[-2:] == tuple(reversed(recipients))
    assert base.index_select(0, importance).reshape(Q.RECORDS_PER_EXPERT, 32)[:, 0].tolist() == list(order)
    storage = Q.storage_group_order(relabeled, Q.R2)
    phys = base.index_select(0, storage).reshape(Q.RECORDS_PER_EXPERT, 32)[:, 0]
    assert list(zip(phys[0:4:2].tolist(), phys[1:4:2].tolist())) == list(zip(donors, recipients))
    for d, r, m, err in (((1,), (), None, "counts must match"), ((1,), (1,), None, "unique and disjoint"),
                         ((24,), (1,), None, "record IDs"), ((1,), (2,), tuple(range(21)), "middle_records")):
        with pytest.raises(ValueError, match=err):
            Q.rate_transfer_record_order(d, r, middle_records=m)


def test_record_repack_moves_scale_and_weight_axes():
    order = torch.arange(Q.RECORDS_PER_EXPERT - 1, -1, -1)
    channels = Q.expand_record_order(order)
    vector = torch.arange(Q.INTERMEDIATE_CHANNELS)
    assert torch.equal(Q.repack_rate_axis(vector, order, 0), vector[channels])
    matrix = vector.repeat(3, 1)
    assert torch.equal(Q.repack_rate_axis(matrix, order, 1), matrix.index_select(1, channels))
    geo = Q.Geometry(2048, 7168)
    o2 = torch.arange(geo.records - 1, -1, -1)
    v2 = torch.arange(2048)
    assert torch.equal(Q.repack_rate_axis(v2, o2, 0, geo), v2.reshape(16, 128).flip(0).flatten())


def test_coupled_permutation_preserves_the_expert_function():
    g = torch.Generator().manual_seed(300)
    x = torch.randn(5, 7, dtype=torch.float64, generator=g)
    w1 = torch.randn(64, 7, dtype=torch.float64, generator=g)
    w3 = torch.randn(64, 7, dtype=torch.float64, generator=g)
    w2 = torch.randn(7, 64, dtype=torch.float64, generator=g)
    perm = torch.randperm(64, generator=g)
    ref = F.linear(situ(F.linear(x, w1), F.linear(x, w3)), w2)
    p1, p3, p2 = Q.coupled_intermediate_permutation(w1, w3, w2, perm)
    assert torch.allclose(F.linear(situ(F.linear(x, p1), F.linear(x, p3)), p2), ref)
    assert torch.equal(Q.invert_permutation(perm)[perm], torch.arange(64))
