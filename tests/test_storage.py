"""Balanced atoms and the atom-major layer file (qsrt_amd.qsrt_storage).

Invariants follow tests/test_qsrt_storage.py:51-217 of the reference; the
atom content is additionally checked tile by tile against the packed words
of the tiles each atom must hold, so a swapped side, stripe or axis fails.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from qsrt_amd import qsrt_storage as st
from qsrt_amd.qsrt import (
    EXPERT_TRELLIS_BYTES,
    GENERIC_SCHEMA,
    INTERMEDIATE_CHANNELS,
    LOCAL_SCALE_VECTORS,
    R0,
    R1,
    R2,
    SCALE_BYTES,
    STORAGE_ALIGNMENT,
    Geometry,
    PackedQSRTTrellis,
    QSRTTrellisDescriptor,
    pack_qsrt_trellis,
    pair_rotation,
    rate_transfer_mode,
    record_bits,
)
from oracle import fmt as ofmt


def test_atoms_enumerate_every_pair_stripe_once():
    atoms = [st.logical_atom_index(p, s) for p in range(12) for s in range(st.ATOMS_PER_RECORD_PAIR)]
    assert atoms == list(range(st.ATOMS_PER_EXPERT)) and st.ATOMS_PER_EXPERT == 96
    assert [st.atom_components(a) for a in atoms] == [(p, s) for p in range(12) for s in range(8)]
    assert st.atom_record_indices(17) == (4, 5)
    with pytest.raises(ValueError):
        st.atom_components(96)
    with pytest.raises(TypeError):
        st.logical_atom_index(True, 0)


@pytest.mark.parametrize("mode,shifted", ((R0, 0), (R1, 1), (R2, 2)))
def test_every_atom_carries_six_bits(mode, shifted):
    pairs = [st.atom_rates(mode, p * 8) for p in range(12)]
    assert pairs == [(2, 4)] * shifted + [(3, 3)] * (12 - shifted)
    assert all(sum(st.atom_rates(mode, a)) == 6 for a in range(96))
    # the rates agree with the serialized record schedule
    bits = record_bits(mode)
    assert all(st.atom_rates(mode, a) == bits[2 * (a // 8):2 * (a // 8) + 2] for a in range(96))


@pytest.mark.parametrize("layer,expert", ((1, 0), (1, 17), (40, 285), (92, 895)))
def test_physical_rotation_is_a_bijection_keeping_pairs_contiguous(layer, expert):
    physical = [st.physical_atom_slot(layer, expert, a) for a in range(96)]
    assert sorted(physical) == list(range(96))
    assert [st.logical_atom_for_slot(layer, expert, s) for s in physical] == list(range(96))
    for shard in range(12):
        logical = [st.logical_atom_for_slot(layer, expert, 8 * shard + s) for s in range(8)]
        assert [st.atom_components(a) for a in logical] == [((shard - pair_rotation(layer, expert)) % 12, s)
                                                             for s in range(8)]


def test_atom_bundles_hold_the_exact_expert_bytes():
    expected = EXPERT_TRELLIS_BYTES + LOCAL_SCALE_VECTORS * INTERMEDIATE_CHANNELS * SCALE_BYTES
    assert st.ATOMS_PER_EXPERT * st.ATOM_BUNDLE_BYTES == expected == 12_404_736
    assert st.K2_STRIPE_BYTES + st.K4_STRIPE_BYTES == 2 * st.K3_STRIPE_BYTES == st.MATRIX_ATOM_TRELLIS_BYTES


@pytest.mark.parametrize("compressed", (1, 512, 700, 800, 896))
def test_equal_shards_are_contiguous_aligned_extents(compressed):
    layout = st.QSRTLayerLayout(compressed, 896 - compressed)
    assert st.EQUAL_SHARD_COUNTS == (1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 96)
    for count in st.EQUAL_SHARD_COUNTS:
        ext = [layout.shard_extent(count, i, require_equal=True) for i in range(count)]
        assert {e.atom_slots for e in ext} == {96 // count}
        assert {e.intermediate_channels for e in ext} == {INTERMEDIATE_CHANNELS // count}
        assert {e.extent_bytes for e in ext} == {(96 // count) * layout.atom_slot_stride_bytes}
        assert all(e.offset_bytes % STORAGE_ALIGNMENT == 0 for e in ext)
        assert all(a.offset_bytes + a.extent_bytes == b.offset_bytes for a, b in zip(ext, ext[1:]))
        assert ext[-1].offset_bytes + ext[-1].extent_bytes == layout.disk_bytes
        assert sum(e.payload_bytes for e in ext) == layout.compressed_payload_bytes


def test_uneven_partitions_cover_every_atom_once():
    layout = st.QSRTLayerLayout(800, 96)
    e = layout.shard_extent(12, 7)
    assert (e.first_atom_slot, e.atom_slots, e.intermediate_channels) == (56, 8, 256)
    for count in (5, 17, 64):
        ext = [layout.shard_extent(count, i) for i in range(count)]
        assert [(x.first_atom_slot, x.atom_slots) for x in ext] == [st.balanced_atom_partition(count, i)
                                                                     for i in range(count)]
        assert sum(x.atom_slots for x in ext) == 96
        assert max(x.atom_slots for x in ext) - min(x.atom_slots for x in ext) <= 1
        # earlier shards take the extra atoms
        assert sorted((x.atom_slots for x in ext), reverse=True) == [x.atom_slots for x in ext]
        assert all(a.offset_bytes + a.extent_bytes == b.offset_bytes for a, b in zip(ext, ext[1:]))
    with pytest.raises(ValueError, match="do not divide"):
        layout.shard_extent(64, 0, require_equal=True)
    with pytest.raises(ValueError):
        st.QSRTLayerLayout(800, 95)


def test_layer_header_round_trip_offsets_and_rejections():
    layout = st.QSRTLayerLayout(700, 196)
    header = st.QSRTLayerHeader(24, layout)
    blob = header.to_bytes()
    assert len(blob) == 4096 and int.from_bytes(blob[:8], "little") == 4088
    assert st.QSRTLayerHeader.from_bytes(blob) == header
    assert "tp_size" not in layout.to_manifest()
    assert layout.atom_bundle_offset(0, 0) % STORAGE_ALIGNMENT == 0
    assert layout.atom_bundle_offset(1, 0) % STORAGE_ALIGNMENT == 0
    assert layout.atom_bundle_offset(4, 17) == layout.shard_extent(24, 1).offset_bytes + 17 * st.ATOM_BUNDLE_BYTES
    # safetensors-compatible: a JSON header whose tensors tile the file after it
    import json
    doc = json.loads(blob[8:])
    ends = sorted(v["data_offsets"] for k, v in doc.items() if k != "__metadata__")
    assert ends[0][0] == 0 and all(a[1] == b[0] for a, b in zip(ends, ends[1:]))
    assert 4096 + ends[-1][1] == layout.disk_bytes
    with pytest.raises(ValueError):
        st.QSRTLayerHeader.from_bytes(blob[:-1])
    relabelled = bytearray(blob)
    relabelled[blob.index(b'"layer":"24"') + 10] = ord("5")
    assert st.QSRTLayerHeader.from_bytes(bytes(relabelled)).layer == 25
    bad = bytearray(blob)
    pos = blob.index(b"qsrt_atoms")
    bad[pos] = ord("Q")
    with pytest.raises(ValueError, match="noncanonical"):
        st.QSRTLayerHeader.from_bytes(bytes(bad))
    with pytest.raises(ValueError):
        st.QSRTLayerHeader(93, layout)


@pytest.mark.parametrize("mode", (R0, R1, R2))
@pytest.mark.parametrize("rate_axis", ("k", "n"))
def test_matrix_atom_transpose_is_bit_exact(mode, rate_axis):
    d = QSRTTrellisDescriptor(mode_id=mode.mode_id, rate_axis=rate_axis,
                              k_tiles=192 if rate_axis == "k" else 224, n_tiles=224 if rate_axis == "k" else 192)
    g = torch.Generator().manual_seed(1000 + mode.mode_id)
    payload = torch.randint(-(1 << 15), 1 << 15, (d.payload_words,), dtype=torch.int16, generator=g)
    atoms = st.pack_matrix_atoms(PackedQSRTTrellis(d, payload))
    assert atoms.shape == (96, st.MATRIX_ATOM_TRELLIS_BYTES // 2)
    assert torch.equal(st.unpack_matrix_atoms(atoms, d).payload, payload)


@pytest.mark.parametrize("rate_axis", ("k", "n"))
def test_atom_holds_the_packed_words_of_its_stripe_tiles(rate_axis):
    """Each atom = stripe s of the low record then stripe s of the high record,
    every stripe the packed tiles at rate-tile 8*record + s in orthogonal order."""

    geo = Geometry(512, 64)  # 4 records, 2 pairs, 4 orthogonal tiles
    mode = rate_transfer_mode(1, geo)
    rate_tiles, orth = geo.intermediate_channels // 16, geo.latent_channels // 16
    shape = (rate_tiles, orth) if rate_axis == "k" else (orth, rate_tiles)
    bits = record_bits(mode)
    enc = torch.empty((*shape, 256), dtype=torch.int64)
    rng = np.random.default_rng(7)
    for r in range(geo.records):
        edges = rng.integers(0, 1 << bits[r], size=(8, orth, 256))
        paths = torch.from_numpy(ofmt.cyclic_states(edges, bits[r]).astype(np.int64))
        if rate_axis == "k":
            enc[8 * r:8 * r + 8] = paths
        else:
            enc[:, 8 * r:8 * r + 8] = paths.transpose(0, 1)
    packed = pack_qsrt_trellis(enc, mode, rate_axis=rate_axis, schema=GENERIC_SCHEMA)
    atoms = st.pack_matrix_atoms(packed)
    for atom in range(st.atoms_per_expert(geo)):
        pair, stripe = st.atom_components(atom, geo)
        want = []
        for rec in (2 * pair, 2 * pair + 1):
            rt = 8 * rec + stripe
            tiles = enc[rt] if rate_axis == "k" else enc[:, rt]
            words = ofmt.pack_words(tiles.numpy(), bits[rec]).view(np.int16)
            want.append(torch.from_numpy(words.reshape(-1).copy()))
        assert torch.equal(atoms[atom], torch.cat(want)), atom
    assert torch.equal(st.unpack_matrix_atoms(atoms, packed.descriptor).payload, packed.payload)


def test_non_balanced_modes_and_bad_shapes_are_rejected():
    from qsrt_amd.qsrt import H308
    d = QSRTTrellisDescriptor(mode_id=H308.mode_id, rate_axis="k", k_tiles=192, n_tiles=224)
    with pytest.raises(ValueError, match="six-bit"):
        st.pack_matrix_atoms(PackedQSRTTrellis(d, torch.zeros(d.payload_words, dtype=torch.int16)))
    d1 = QSRTTrellisDescriptor(mode_id=1, rate_axis="k", k_tiles=192, n_tiles=224)
    with pytest.raises(ValueError):
        st.unpack_matrix_atoms(torch.zeros((96, 10), dtype=torch.int16), d1)


def test_scale_atoms_are_bit_exact_and_place_stripes():
    scale = torch.arange(INTERMEDIATE_CHANNELS, dtype=torch.int16).view(torch.float16)
    atoms = st.pack_local_scale_atoms(scale)
    assert torch.equal(st.unpack_local_scale_atoms(atoms).view(torch.int16), scale.view(torch.int16))
    ch = atoms.view(torch.int16).to(torch.int64)
    for atom in (0, 9, 95):
        pair, stripe = st.atom_components(atom)
        lo = 2 * pair * 128 + 16 * stripe
        assert ch[atom].tolist() == list(range(lo, lo + 16)) + list(range(lo + 128, lo + 144))
    with pytest.raises(ValueError):
        st.pack_local_scale_atoms(scale.float())


def test_rotation_round_trip_preserves_payload():
    logical = torch.arange(96 * 7, dtype=torch.int64).reshape(96, 7)
    physical = st.rotate_expert_atoms(logical, 24, 285)
    assert torch.equal(st.unrotate_expert_atoms(physical, 24, 285), logical)
    for slot in range(96):
        assert int(physical[slot, 0]) == 7 * st.logical_atom_for_slot(24, 285, slot)
