"""Layer files for mixed-rate record schedules at any expert geometry.

The balanced-atom layer (``qsrt_storage`` / ``qsrt_atoms``) stores six
trellis bits per record pair, so it holds the Kimi-K3 R0/R1/R2 modes only.
A layer whose matrices mix K3 and K4 records: 384
SwiGLU experts of 7168 x 2048 with 14 K3 + 2 K4 records per matrix -- has
record pairs of different widths.  This module stores such layers, keeping
the reference's revision-two atom concepts (``qsrt/qsrt_atoms_v2.py:1-8``,
``qsrt/pack/qsrt_atoms_v2.py:180-420``) and generalising them to the
geometry and schedule of the layer:

* records pair as (low, high): the i-th highest-rate record with the i-th
  lowest-rate one (ties by record index), so every K4 record sits in its own
  pair (a P43 pair; the rest P33);
* an atom is stripe ``t`` (16 intermediate channels) of a pair's low record
  followed by stripe ``t`` of its high record -- eight atoms per pair -- for
  each of w1, w3, w2, plus the atom's 32 channels of the three expert-local
  FP16 scale vectors (w1.svh, w3.svh, w2.suh);
* expert ``e`` rotates its pairs by ``pair_rotation(layer, e)`` over the
  physical pair slots, so the wide P43 atoms spread evenly over the slots;
* physical atom slot ``s`` is one 4 KiB-aligned row holding slot ``s`` of
  every stored expert, in order.  Rows of different widths follow one
  another (the reference serialises its coupled H308 extents the same way),
  so a tensor-parallel shard of whole atom slots is still one contiguous
  read.

File: a 4 KiB safetensors header (JSON, sorted keys, space padded), the
layer-shared FP16 hidden-side scales (w1.suh, w3.suh, w2.svh), then the atom
rows.  Nothing is decoded or repacked bit-wise: atoms move whole packed tile
paths.  ``QSRTRateLayerReader`` returns a stored expert's record-major
payloads, which the fused HIP decode takes as they are.
"""

from __future__ import annotations

import fcntl
import json
import os
import struct
from dataclasses import dataclass
from functools import cached_property
from pathlib import Path

import torch

from .qsrt import (
    MOE_LAYERS,
    SCALE_BYTES,
    STORAGE_ALIGNMENT,
    TILE_CHANNELS,
    Geometry,
    align_up,
    logical_pair_for_slot,
)

SCHEMA = "qsrt_amd_rate_record_atoms_v1"
VERSION = 1
ENCODING = "qsrt_sqg_e4m3"
CODEBOOK = "sqg_xor_cheb_t12"
HEADER_BYTES = STORAGE_ALIGNMENT
MATRICES = ("w1", "w3", "w2")
RATE_AXIS = {"w1": "n", "w3": "n", "w2": "k"}
LOCAL_PART = {"w1": "svh", "w3": "svh", "w2": "suh"}   # intermediate-axis scales, stored per atom
SHARED_PART = {"w1": "suh", "w3": "suh", "w2": "svh"}  # hidden-axis scales, one per layer
STRIPES_PER_RECORD = 8  # 128-channel records, 16-channel stripes
_HEADER_LENGTH = struct.Struct("<Q")
_SHARED_TENSOR = "_qsrt_shared_scale_section"
_ATOM_TENSOR = "qsrt_atoms"


def _ranges(values) -> str:
    """Sorted distinct integers as ``a-b,c,...`` runs."""

    out, values = [], sorted(values)
    i = 0
    while i < len(values):
        j = i
        while j + 1 < len(values) and values[j + 1] == values[j] + 1:
            j += 1
        out.append(str(values[i]) if i == j else f"{values[i]}-{values[j]}")
        i = j + 1
    return ",".join(out)


def _parse_ranges(text: str) -> tuple[int, ...]:
    out: list[int] = []
    for part in filter(None, text.split(",")):
        lo, _, hi = part.partition("-")
        out.extend(range(int(lo), int(hi or lo) + 1))
    return tuple(out)


@dataclass(frozen=True)
class RateSchedule:
    """One record rate per 128 intermediate channels, the same for w1, w3
    and w2 (their shared rate axis)."""

    geometry: Geometry
    record_bits: tuple[int, ...]

    def __post_init__(self) -> None:
        if self.geometry.record_channels != 16 * STRIPES_PER_RECORD:
            raise ValueError("rate-record atoms need 128-channel records")
        bits = tuple(int(b) for b in self.record_bits)
        object.__setattr__(self, "record_bits", bits)
        if len(bits) != self.geometry.records or len(bits) % 2:
            raise ValueError(f"need an even number of records, one rate each ({self.geometry.records} here)")
        if any(b not in (2, 3, 4) for b in bits):
            raise ValueError("record rates must be K2, K3 or K4")

    @property
    def pairs(self) -> int:
        return len(self.record_bits) // 2

    @cached_property
    def pair_records(self) -> tuple[tuple[int, int], ...]:
        """(low, high) logical records of every logical pair."""

        order = sorted(range(len(self.record_bits)), key=lambda r: (-self.record_bits[r], r))
        n = len(order)
        return tuple((order[p], order[n - 1 - p]) for p in range(self.pairs))

    def pair_bits(self, pair: int) -> int:
        lo, hi = self.pair_records[pair]
        return self.record_bits[lo] + self.record_bits[hi]

    def matrix_atom_bytes(self, pair: int) -> int:
        """One matrix's trellis bytes in an atom of ``pair``: 16 channels of
        each record over the whole latent axis."""

        return TILE_CHANNELS * self.geometry.latent_channels * self.pair_bits(pair) // 8

    def bundle_bytes(self, pair: int) -> int:
        return 3 * self.matrix_atom_bytes(pair) + 3 * 2 * TILE_CHANNELS * SCALE_BYTES

    @property
    def atoms(self) -> int:
        return self.pairs * STRIPES_PER_RECORD

    @property
    def expert_bytes(self) -> int:
        return STRIPES_PER_RECORD * sum(self.bundle_bytes(p) for p in range(self.pairs))

    def record_words(self, record: int) -> int:
        """int16 words of one record of one matrix in the record-major container."""

        tiles = STRIPES_PER_RECORD * self.geometry.latent_channels // TILE_CHANNELS
        return tiles * TILE_CHANNELS * self.record_bits[record]

    @property
    def matrix_words(self) -> int:
        return sum(self.record_words(r) for r in range(len(self.record_bits)))


@dataclass(frozen=True)
class QSRTRateLayerLayout:
    """Byte layout of one layer: header, shared scales, then one aligned row
    per physical atom slot holding that slot of every stored expert."""

    layer: int
    schedule: RateSchedule
    experts: tuple[int, ...]

    def __post_init__(self) -> None:
        if self.layer not in MOE_LAYERS:
            raise ValueError(f"layer must be in {MOE_LAYERS.start}..{MOE_LAYERS.stop - 1}")
        experts = tuple(int(e) for e in self.experts)
        object.__setattr__(self, "experts", experts)
        if not experts or len(set(experts)) != len(experts) or min(experts) < 0:
            raise ValueError("experts must be distinct non-negative expert ids")
        # the per-expert pair rotation validates each id
        for e in experts:
            logical_pair_for_slot(self.layer, e, 0, self.schedule.geometry)

    def logical_pair(self, expert: int, pair_slot: int) -> int:
        return logical_pair_for_slot(self.layer, expert, pair_slot, self.schedule.geometry)

    @property
    def shared_section_bytes(self) -> int:
        return align_up(3 * self.schedule.geometry.latent_channels * SCALE_BYTES)

    @property
    def slab_offset(self) -> int:
        return HEADER_BYTES + self.shared_section_bytes

    @cached_property
    def _rows(self) -> tuple[tuple[int, ...], tuple[int, ...], tuple[int, ...], tuple[tuple[int, ...], ...]]:
        """Per slot: payload bytes, stride, file offset, and every stored
        expert's offset inside the row."""

        s = self.schedule
        sizes = [s.bundle_bytes(p) for p in range(s.pairs)]
        pairs = [[self.logical_pair(e, ps) for ps in range(s.pairs)] for e in self.experts]
        payload, stride, offset, inner = [], [], [], []
        cursor = self.slab_offset
        for slot in range(s.atoms):
            ps, within, run = slot // STRIPES_PER_RECORD, [], 0
            for i in range(len(self.experts)):
                within.append(run)
                run += sizes[pairs[i][ps]]
            payload.append(run)
            stride.append(align_up(run))
            offset.append(cursor)
            inner.append(tuple(within))
            cursor += stride[-1]
        return tuple(payload), tuple(stride), tuple(offset), tuple(inner)

    def row_payload_bytes(self, slot: int) -> int:
        return self._rows[0][slot]

    def row_stride_bytes(self, slot: int) -> int:
        return self._rows[1][slot]

    def row_offset(self, slot: int) -> int:
        return self._rows[2][slot]

    @property
    def slab_bytes(self) -> int:
        return sum(self._rows[1])

    @property
    def disk_bytes(self) -> int:
        return self.slab_offset + self.slab_bytes

    @property
    def payload_bytes(self) -> int:
        return len(self.experts) * self.schedule.expert_bytes

    @cached_property
    def _slot_of(self) -> dict[int, int]:
        return {e: i for i, e in enumerate(self.experts)}

    def bundle_offset(self, slot: int, expert: int) -> tuple[int, int]:
        """``(file offset, bytes)`` of ``expert``'s bundle in atom slot ``slot``."""

        if not 0 <= slot < self.schedule.atoms:
            raise ValueError(f"atom slot must be in 0..{self.schedule.atoms - 1}")
        index = self._slot_of.get(expert)
        if index is None:
            raise ValueError(f"expert {expert} is not stored in this layer")
        pair = self.logical_pair(expert, slot // STRIPES_PER_RECORD)
        return self.row_offset(slot) + self._rows[3][slot][index], self.schedule.bundle_bytes(pair)

    def shard_extent(self, shard_count: int, shard_index: int) -> tuple[int, int, int, int]:
        """``(first slot, slots, file offset, bytes)`` of a whole-slot shard
        (quotient/remainder split, earlier shards take the extra slots)."""

        atoms = self.schedule.atoms
        if not 1 <= shard_count <= atoms or not 0 <= shard_index < shard_count:
            raise ValueError(f"need 1 <= shard_count <= {atoms} and 0 <= shard_index < shard_count")
        q, r = divmod(atoms, shard_count)
        first = shard_index * q + min(shard_index, r)
        slots = q + int(shard_index < r)
        off = self.row_offset(first)
        return first, slots, off, sum(self._rows[1][first:first + slots])


@dataclass(frozen=True)
class QSRTRateLayerHeader:
    """Canonical 4 KiB safetensors header: two U8 tensors (shared scales,
    atom slab) and the metadata the layout is rebuilt from."""

    layout: QSRTRateLayerLayout

    def _document(self) -> dict:
        lay, s = self.layout, self.layout.schedule
        g = s.geometry
        meta = {
            "format": "pt",
            "schema": SCHEMA,
            "version": str(VERSION),
            "encoding": ENCODING,
            "codebook": CODEBOOK,
            "layer": str(lay.layer),
            "intermediate_channels": str(g.intermediate_channels),
            "latent_channels": str(g.latent_channels),
            "record_channels": str(g.record_channels),
            "record_bits": "".join(str(b) for b in s.record_bits),
            "experts": _ranges(lay.experts),
            "atom_slots": str(s.atoms),
            "expert_bytes": str(s.expert_bytes),
            "alignment_bytes": str(STORAGE_ALIGNMENT),
        }
        s0, s1 = 0, lay.shared_section_bytes
        return {
            "__metadata__": meta,
            _SHARED_TENSOR: {"dtype": "U8", "shape": [lay.shared_section_bytes], "data_offsets": [s0, s1]},
            _ATOM_TENSOR: {"dtype": "U8", "shape": [lay.slab_bytes], "data_offsets": [s1, s1 + lay.slab_bytes]},
        }

    def to_bytes(self) -> bytes:
        capacity = HEADER_BYTES - _HEADER_LENGTH.size
        doc = json.dumps(self._document(), sort_keys=True, separators=(",", ":")).encode("utf-8")
        if len(doc) > capacity:
            raise ValueError("rate-record layer header exceeds its 4 KiB budget (expert list too ragged)")
        return _HEADER_LENGTH.pack(capacity) + doc + b" " * (capacity - len(doc))

    @classmethod
    def from_bytes(cls, payload: bytes) -> "QSRTRateLayerHeader":
        if len(payload) != HEADER_BYTES or _HEADER_LENGTH.unpack_from(payload)[0] != HEADER_BYTES - _HEADER_LENGTH.size:
            raise ValueError("rate-record layer header must occupy exactly 4 KiB")
        try:
            doc = json.loads(payload[_HEADER_LENGTH.size:].decode("utf-8"))
            meta = doc["__metadata__"]
            if meta.get("schema") != SCHEMA or meta.get("version") != str(VERSION):
                raise ValueError("not a rate-record atom layer")
            geometry = Geometry(int(meta["intermediate_channels"]), int(meta["latent_channels"]),
                                int(meta["record_channels"]))
            schedule = RateSchedule(geometry, tuple(int(c) for c in meta["record_bits"]))
            result = cls(QSRTRateLayerLayout(int(meta["layer"]), schedule, _parse_ranges(meta["experts"])))
        except (UnicodeDecodeError, json.JSONDecodeError, KeyError, TypeError, ValueError) as exc:
            raise ValueError(f"rate-record layer header is malformed: {exc}") from exc
        if doc != result._document():
            raise ValueError("rate-record layer header is noncanonical")
        return result


# ---------------------------------------------------------------------------
# atom assembly (moves whole packed tile paths; decodes nothing)
# ---------------------------------------------------------------------------


def _record_views(words: torch.Tensor, schedule: RateSchedule, axis: str) -> list[torch.Tensor]:
    """``[stripes, latent tiles, 16 K]`` view of every record of a
    record-major payload (a rate-axis ``n`` record is ``[latent tiles][8]``
    tiles, a ``k`` record ``[8][latent tiles]``, both row-major)."""

    if words.dtype != torch.int16 or words.dim() != 1 or words.numel() != schedule.matrix_words:
        raise ValueError(f"record-major payload must be flat int16 of {schedule.matrix_words} words")
    lt = schedule.geometry.latent_channels // TILE_CHANNELS
    out, cursor = [], 0
    for r, bits in enumerate(schedule.record_bits):
        n = schedule.record_words(r)
        rec = words.narrow(0, cursor, n)
        cursor += n
        if axis == "k":
            out.append(rec.view(STRIPES_PER_RECORD, lt, TILE_CHANNELS * bits))
        else:
            out.append(rec.view(lt, STRIPES_PER_RECORD, TILE_CHANNELS * bits).transpose(0, 1))
    return out


def _check_scale(t: torch.Tensor, n: int, name: str) -> torch.Tensor:
    t = t.reshape(-1)
    if t.dtype != torch.float16 or t.numel() != n:
        raise ValueError(f"{name} must hold {n} float16 values")
    if not bool(torch.isfinite(t).all()):
        raise ValueError(f"{name} contains non-finite values")
    return t


def assemble_expert_bundles(layout: QSRTRateLayerLayout, expert: int, tensors: dict) -> list[torch.Tensor]:
    """One expert's bundles in physical slot order (uint8, on the payload's
    device).  ``tensors[m]`` holds ``trellis`` (record-major int16 words),
    ``suh`` and ``svh`` (float16) of matrix ``m`` in ``w1``, ``w3``, ``w2``."""

    s = layout.schedule
    g = s.geometry
    if set(tensors) != set(MATRICES):
        raise ValueError("an expert needs w1, w3 and w2")
    records, local = {}, {}
    for m in MATRICES:
        parts = tensors[m]
        records[m] = _record_views(parts["trellis"].reshape(-1), s, RATE_AXIS[m])
        local[m] = _check_scale(parts[LOCAL_PART[m]], g.intermediate_channels, f"{m}.{LOCAL_PART[m]}").view(
            s.pairs * 2, STRIPES_PER_RECORD, TILE_CHANNELS)
    bundles = []
    for slot in range(s.atoms):
        pair, stripe = layout.logical_pair(expert, slot // STRIPES_PER_RECORD), slot % STRIPES_PER_RECORD
        lo, hi = s.pair_records[pair]
        pieces = [torch.cat([records[m][lo][stripe].reshape(-1), records[m][hi][stripe].reshape(-1)]).view(torch.uint8)
                  for m in MATRICES]
        pieces += [torch.cat([local[m][lo][stripe], local[m][hi][stripe]]).view(torch.uint8) for m in MATRICES]
        b = torch.cat(pieces)
        if b.numel() != s.bundle_bytes(pair):
            raise AssertionError("rate-record bundle accounting drifted")
        bundles.append(b)
    return bundles


def disassemble_expert_bundles(layout: QSRTRateLayerLayout, expert: int, bundles: list[torch.Tensor],
                               shared: dict) -> dict:
    """Invert :func:`assemble_expert_bundles`; ``shared`` supplies the
    layer-shared hidden-side scales (``w1.suh``, ``w3.suh``, ``w2.svh``)."""

    s = layout.schedule
    g = s.geometry
    lt = g.latent_channels // TILE_CHANNELS
    words = {m: torch.empty(s.matrix_words, dtype=torch.int16, device=bundles[0].device) for m in MATRICES}
    local = {m: torch.empty(g.intermediate_channels, dtype=torch.float16, device=bundles[0].device) for m in MATRICES}
    views = {m: _record_views(words[m], s, RATE_AXIS[m]) for m in MATRICES}
    lviews = {m: local[m].view(s.pairs * 2, STRIPES_PER_RECORD, TILE_CHANNELS) for m in MATRICES}
    for slot in range(s.atoms):
        pair, stripe = layout.logical_pair(expert, slot // STRIPES_PER_RECORD), slot % STRIPES_PER_RECORD
        lo, hi = s.pair_records[pair]
        b = bundles[slot]
        if b.dtype != torch.uint8 or b.numel() != s.bundle_bytes(pair):
            raise ValueError(f"bundle {slot} must be {s.bundle_bytes(pair)} bytes")
        cursor = 0
        for m in MATRICES:
            n = s.matrix_atom_bytes(pair)
            w = b.narrow(0, cursor, n).view(torch.int16)
            cursor += n
            n_lo = lt * TILE_CHANNELS * s.record_bits[lo]
            views[m][lo][stripe].copy_(w[:n_lo].view(lt, -1))
            views[m][hi][stripe].copy_(w[n_lo:].view(lt, -1))
        for m in MATRICES:
            v = b.narrow(0, cursor, 2 * TILE_CHANNELS * SCALE_BYTES).view(torch.float16)
            cursor += 2 * TILE_CHANNELS * SCALE_BYTES
            lviews[m][lo][stripe].copy_(v[:TILE_CHANNELS])
            lviews[m][hi][stripe].copy_(v[TILE_CHANNELS:])
    out = {}
    for m in MATRICES:
        sh = shared[f"{m}.{SHARED_PART[m]}"].to(bundles[0].device)
        out[m] = {"trellis": words[m], LOCAL_PART[m]: local[m], SHARED_PART[m]: sh}
    return out


def pack_shared_section(layout: QSRTRateLayerLayout, shared: dict) -> torch.Tensor:
    n = layout.schedule.geometry.latent_channels
    out = torch.zeros(layout.shared_section_bytes, dtype=torch.uint8)
    parts = [_check_scale(shared[k].cpu(), n, k).view(torch.uint8) for k in ("w1.suh", "w3.suh", "w2.svh")]
    body = torch.cat(parts)
    out[:body.numel()] = body
    return out


def unpack_shared_section(layout: QSRTRateLayerLayout, raw: torch.Tensor) -> dict:
    n = layout.schedule.geometry.latent_channels
    v = raw[:3 * n * SCALE_BYTES].contiguous().view(torch.float16)
    if bool(raw[3 * n * SCALE_BYTES:].any()):
        raise ValueError("shared-scale section padding must be zero")
    return {"w1.suh": v[:n].clone(), "w3.suh": v[n:2 * n].clone(), "w2.svh": v[2 * n:].clone()}


# ---------------------------------------------------------------------------
# file I/O
# ---------------------------------------------------------------------------


def _pwrite_exact(fd: int, data: bytes, offset: int) -> None:
    done = 0
    while done < len(data):
        n = os.pwrite(fd, data[done:], offset + done)
        if n <= 0:
            raise OSError("short rate-record layer write")
        done += n


def materialize_rate_layer(destination: str | Path, layout: QSRTRateLayerLayout, experts, *,
                           discard_partial: bool = False) -> dict:
    """Write one layer atomically (a locked ``.partial`` file renamed into
    place), one expert at a time.  ``experts`` yields ``(expert id,
    tensors)`` in ``layout.experts`` order, ``tensors`` as for
    :func:`assemble_expert_bundles`; every expert must carry the same
    layer-shared hidden-side scales."""

    destination = Path(destination)
    destination.parent.mkdir(parents=True, exist_ok=True)
    if destination.exists():
        raise FileExistsError(destination)
    partial = destination.with_name(f".{destination.name}.partial")
    if partial.exists():
        if not discard_partial:
            raise FileExistsError(partial)
        partial.unlink()
    fd = os.open(partial, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o644)
    shared: dict[str, torch.Tensor] = {}
    seen = []
    try:
        fcntl.flock(fd, fcntl.LOCK_EX | fcntl.LOCK_NB)
        os.ftruncate(fd, layout.disk_bytes)
        _pwrite_exact(fd, QSRTRateLayerHeader(layout).to_bytes(), 0)
        for expert, tensors in experts:
            seen.append(int(expert))
            for m in MATRICES:
                key = f"{m}.{SHARED_PART[m]}"
                v = _check_scale(tensors[m][SHARED_PART[m]], layout.schedule.geometry.latent_channels, key).cpu()
                if not torch.equal(shared.setdefault(key, v.clone()), v):
                    raise ValueError(f"layer-shared transform {key} differs between experts")
            bundles = assemble_expert_bundles(layout, int(expert), tensors)
            host = torch.cat(bundles).cpu()
            cursor = 0
            for slot, b in enumerate(bundles):
                off, n = layout.bundle_offset(slot, int(expert))
                _pwrite_exact(fd, host[cursor:cursor + n].numpy().tobytes(), off)
                cursor += n
        if tuple(seen) != layout.experts:
            raise ValueError("experts must arrive in the layout's order, each once")
        _pwrite_exact(fd, pack_shared_section(layout, shared).numpy().tobytes(), HEADER_BYTES)
        os.fsync(fd)
    except BaseException:
        os.close(fd)
        partial.unlink(missing_ok=True)
        raise
    os.close(fd)
    partial.replace(destination)
    return {"schema": SCHEMA, "layer": layout.layer, "experts": len(layout.experts), "disk_bytes": layout.disk_bytes,
            "payload_bytes": layout.payload_bytes}


class QSRTRateLayerReader:
    """Bounded reader of one rate-record layer file."""

    def __init__(self, path: str | Path) -> None:
        self.path = Path(path)
        self._fd = os.open(self.path, os.O_RDONLY)
        try:
            self.header = QSRTRateLayerHeader.from_bytes(os.pread(self._fd, HEADER_BYTES, 0))
            self.layout = self.header.layout
            if self.path.stat().st_size != self.layout.disk_bytes:
                raise ValueError("rate-record layer size disagrees with its header")
            raw = os.pread(self._fd, self.layout.shared_section_bytes, HEADER_BYTES)
            self.shared = unpack_shared_section(self.layout, torch.frombuffer(bytearray(raw), dtype=torch.uint8))
        except BaseException:
            os.close(self._fd)
            raise

    def close(self) -> None:
        if self._fd >= 0:
            os.close(self._fd)
            self._fd = -1

    def __enter__(self) -> "QSRTRateLayerReader":
        return self

    def __exit__(self, *_exc) -> None:
        self.close()

    def _pread(self, n: int, off: int) -> bytes:
        if self._fd < 0:
            raise RuntimeError("rate-record layer reader is closed")
        raw = os.pread(self._fd, n, off)
        if len(raw) != n:
            raise ValueError("short rate-record layer read")
        return raw

    def read_shard(self, shard_count: int, shard_index: int) -> tuple[int, list[torch.Tensor]]:
        """One contiguous whole-slot shard: ``(first slot, [row payload bytes
        per slot])``, padding dropped."""

        first, slots, off, n = self.layout.shard_extent(shard_count, shard_index)
        raw = torch.frombuffer(bytearray(self._pread(n, off)), dtype=torch.uint8)
        rows, cursor = [], 0
        for slot in range(first, first + slots):
            rows.append(raw[cursor:cursor + self.layout.row_payload_bytes(slot)])
            cursor += self.layout.row_stride_bytes(slot)
        return first, rows

    def read_expert(self, expert: int, *, device="cpu") -> dict:
        """A stored expert's three matrices: record-major ``trellis`` words
        and FP16 ``suh`` / ``svh``."""

        bundles = []
        for slot in range(self.layout.schedule.atoms):
            off, n = self.layout.bundle_offset(slot, expert)
            bundles.append(torch.frombuffer(bytearray(self._pread(n, off)), dtype=torch.uint8).to(device))
        return disassemble_expert_bundles(self.layout, expert, bundles, self.shared)


__all__ = [
    "QSRTRateLayerHeader",
    "QSRTRateLayerLayout",
    "QSRTRateLayerReader",
    "RateSchedule",
    "assemble_expert_bundles",
    "disassemble_expert_bundles",
    "materialize_rate_layer",
]
