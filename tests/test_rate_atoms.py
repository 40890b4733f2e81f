"""Rate-record layer files (``qsrt_amd.qsrt_rate_atoms``): accounting at
BASELINE config 5, byte-exact round trips, atom contents pinned by direct
tile indexing, and rejection of malformed or inconsistent input."""

from __future__ import annotations

import os

import pytest
import torch

from qsrt_amd.qsrt import Geometry, align_up
from qsrt_amd.qsrt_rate_atoms import (
    HEADER_BYTES,
    MATRICES,
    QSRTRateLayerHeader,
    QSRTRateLayerLayout,
    QSRTRateLayerReader,
    RateSchedule,
    assemble_expert_bundles,
    materialize_rate_layer,
)

CONFIG5 = RateSchedule(Geometry(2048, 7168), (3,) * 14 + (4,) * 2)
SMALL = RateSchedule(Geometry(512, 64), (3, 4, 2, 3))


def _expert(schedule: RateSchedule, seed: int, shared: dict) -> dict:
    g = torch.Generator().manual_seed(seed)
    n_i, n_l = schedule.geometry.intermediate_channels, schedule.geometry.latent_channels
    out = {}
    for m in MATRICES:
        words = torch.randint(-32768, 32768, (schedule.matrix_words,), generator=g, dtype=torch.int32).to(torch.int16)
        local = (torch.rand(n_i, generator=g) + 0.5).half()
        if m == "w2":
            out[m] = {"trellis": words, "suh": local, "svh": shared[m]}
        else:
            out[m] = {"trellis": words, "suh": shared[m], "svh": local}
    return out


def _shared(schedule: RateSchedule, seed: int = 99) -> dict:
    g = torch.Generator().manual_seed(seed)
    n = schedule.geometry.latent_channels
    return {m: (torch.rand(n, generator=g) - 0.5).half() for m in MATRICES}


def test_config5_accounting():
    s = CONFIG5
    assert s.pair_records == ((14, 13), (15, 12), (0, 11), (1, 10), (2, 9), (3, 8), (4, 7), (5, 6))
    assert [s.pair_bits(p) for p in range(s.pairs)] == [7, 7] + [6] * 6
    # 3 matrices x 7168 x 2048 x 3.125 bits + 3 local FP16 scale vectors of 2048
    assert s.expert_bytes == 3 * 7168 * 2048 * 25 // 64 + 3 * 2048 * 2
    lay = QSRTRateLayerLayout(24, s, tuple(range(384)))
    assert lay.payload_bytes == 384 * s.expert_bytes
    assert lay.disk_bytes == HEADER_BYTES + align_up(3 * 7168 * 2) + sum(
        lay.row_stride_bytes(i) for i in range(s.atoms))
    # the per-expert pair rotation spreads the two P43 pairs evenly: every row holds the same bytes
    assert len({lay.row_payload_bytes(i) for i in range(s.atoms)}) == 1
    assert all(lay.row_offset(i) % 4096 == 0 for i in range(s.atoms))
    doc = QSRTRateLayerHeader(lay).to_bytes()
    assert len(doc) == HEADER_BYTES and QSRTRateLayerHeader.from_bytes(doc).layout == lay


@pytest.mark.parametrize("shards", range(1, 9))
def test_shard_extents_partition_the_slab(shards):
    lay = QSRTRateLayerLayout(5, SMALL, (3, 7, 11))
    cursor, slot = lay.slab_offset, 0
    for i in range(shards):
        first, slots, off, n = lay.shard_extent(shards, i)
        assert (first, off) == (slot, cursor)
        assert n == sum(lay.row_stride_bytes(s) for s in range(first, first + slots))
        cursor, slot = off + n, first + slots
    assert (slot, cursor) == (SMALL.atoms, lay.disk_bytes)


def test_round_trip_is_byte_exact(tmp_path):
    shared = _shared(SMALL)
    experts = {e: _expert(SMALL, e, shared) for e in (3, 7, 11)}
    lay = QSRTRateLayerLayout(5, SMALL, tuple(experts))
    path = tmp_path / "layer.safetensors"
    info = materialize_rate_layer(path, lay, experts.items())
    assert info["disk_bytes"] == os.path.getsize(path)
    with QSRTRateLayerReader(path) as rd:
        assert rd.layout == lay
        for e, want in experts.items():
            got = rd.read_expert(e)
            for m in MATRICES:
                for part in ("trellis", "suh", "svh"):
                    assert torch.equal(got[m][part], want[m][part]), (e, m, part)
        first, rows = rd.read_shard(2, 1)
        assert first == SMALL.atoms // 2 and len(rows) == SMALL.atoms // 2
        for i, row in enumerate(rows):
            assert row.numel() == lay.row_payload_bytes(first + i)
    # the file reads back with the safetensors loader as its two U8 tensors
    from safetensors import safe_open
    with safe_open(str(path), framework="pt") as f:
        assert set(f.keys()) == {"_qsrt_shared_scale_section", "qsrt_atoms"}
        assert f.get_tensor("qsrt_atoms").numel() == lay.slab_bytes


def _tile_words(words: torch.Tensor, schedule: RateSchedule, axis: str, tile_row: int, tile_col: int) -> torch.Tensor:
    """Words of one tile of a record-major payload, located by arithmetic on
    the container's definition (records of 8 tile columns -- or rows for a
    k-axis matrix -- each record's tiles row-major, 16 K words per tile)."""

    lt = schedule.geometry.latent_channels // 16
    rate_tile = tile_col if axis == "n" else tile_row
    record, within = divmod(rate_tile, 8)
    offset = sum(schedule.record_words(r) for r in range(record))
    bits = schedule.record_bits[record]
    index = tile_row * 8 + within if axis == "n" else within * lt + tile_col
    return words[offset + index * 16 * bits: offset + (index + 1) * 16 * bits]


def test_atom_holds_the_matching_stripes_of_its_pair():
    shared = _shared(SMALL)
    tensors = _expert(SMALL, 4, shared)
    lay = QSRTRateLayerLayout(5, SMALL, (4,))
    bundles = assemble_expert_bundles(lay, 4, tensors)
    lt = SMALL.geometry.latent_channels // 16
    for slot in range(SMALL.atoms):
        pair = lay.logical_pair(4, slot // 8)
        stripe = slot % 8
        lo, hi = SMALL.pair_records[pair]
        parts = []
        for m, axis in (("w1", "n"), ("w3", "n"), ("w2", "k")):
            for rec in (lo, hi):
                for t in range(lt):
                    if axis == "n":
                        parts.append(_tile_words(tensors[m]["trellis"], SMALL, axis, t, 8 * rec + stripe))
                    else:
                        parts.append(_tile_words(tensors[m]["trellis"], SMALL, axis, 8 * rec + stripe, t))
        for m, part in (("w1", "svh"), ("w3", "svh"), ("w2", "suh")):
            for rec in (lo, hi):
                c0 = 128 * rec + 16 * stripe
                parts.append(tensors[m][part][c0:c0 + 16].view(torch.int16))
        want = torch.cat(parts).view(torch.uint8)
        assert torch.equal(bundles[slot], want), slot


def test_inconsistent_input_is_rejected(tmp_path):
    shared = _shared(SMALL)
    experts = {e: _expert(SMALL, e, shared) for e in (1, 2)}
    other = _shared(SMALL, seed=5)
    experts[2]["w1"]["suh"] = other["w1"]
    lay = QSRTRateLayerLayout(5, SMALL, (1, 2))
    with pytest.raises(ValueError, match="differs between experts"):
        materialize_rate_layer(tmp_path / "a.safetensors", lay, experts.items())
    assert not any(p.name.endswith(".partial") for p in tmp_path.iterdir())
    good = {e: _expert(SMALL, e, shared) for e in (1, 2)}
    with pytest.raises(ValueError, match="order"):
        materialize_rate_layer(tmp_path / "b.safetensors", lay, [(2, good[2]), (1, good[1])])
    bad = _expert(SMALL, 1, shared)
    bad["w3"]["trellis"] = bad["w3"]["trellis"][:-1]
    with pytest.raises(ValueError, match="record-major payload"):
        assemble_expert_bundles(QSRTRateLayerLayout(5, SMALL, (1,)), 1, bad)
    with pytest.raises(ValueError):
        RateSchedule(Geometry(512, 64), (3, 4, 5, 3))
    with pytest.raises(ValueError):
        RateSchedule(Geometry(384, 64), (3, 3, 3))


def test_noncanonical_header_is_rejected():
    lay = QSRTRateLayerLayout(5, SMALL, (0, 1, 2, 9))
    raw = QSRTRateLayerHeader(lay).to_bytes()
    assert b'"experts":"0-2,9"' in raw
    key = f'"atom_slots":"{SMALL.atoms}"'.encode()
    tampered = raw.replace(key, f'"atom_slots":"{SMALL.atoms + 1}"'.encode())
    assert tampered != raw and len(tampered) == len(raw)
    with pytest.raises(ValueError, match="noncanonical"):
        QSRTRateLayerHeader.from_bytes(tampered)
    with pytest.raises(ValueError, match="malformed"):
        QSRTRateLayerHeader.from_bytes(raw.replace(b'"record_bits":"3423"', b'"record_bits":"3523"'))
    with pytest.raises(ValueError):
        QSRTRateLayerHeader.from_bytes(bytes(4095))
