"""Tensor-parallel-independent storage of QSRT layers: balanced atoms
(mirrors ``qsrt/qsrt_storage.py``).

An atom is 32 intermediate channels: the matching 16-channel stripes of the
low and high record of one rate pair, so every atom carries six trellis bits
per coefficient pair (K2 + K4 for a P24 pair, K3 + K3 for P33) plus the
matching fragments of the three expert-local FP16 scale vectors.  Shards own
whole atoms and never split, decode or repack a trellis stream.  Packing
moves complete packed 16x16 tile paths; it never decodes edges.

The module-level constants are the Kimi-K3 preset; every function takes the
geometry from the descriptor (or an explicit :class:`Geometry`), so the
other BASELINE shapes atomize with the same code.
"""

from __future__ import annotations

import json
import struct
from dataclasses import dataclass

import torch

from .qsrt import (
    EXPERTS_PER_LAYER,
    FORMAT_SECTION_BYTES,
    KIMI_K3,
    LAYER_HEADER_BYTES,
    LOCAL_SCALE_VECTORS,
    SCALE_BYTES,
    SHARED_SCALE_SECTION_BYTES,
    STORAGE_ALIGNMENT,
    TILE_CHANNELS,
    Geometry,
    ModeSpec,
    PackedQSRTTrellis,
    align_up,
    pair_rotation,
    record_bits,
    resolve_mode,
)

SCHEMA = "qsrt_kimi_k3_qsrt_atoms_v1"
VERSION = 1
ENCODING_QSRT_SQG_E4M3 = "qsrt_sqg_e4m3"
PROFILE_ID_QSRT_SQG_E4M3 = 1
_HEADER_LENGTH = struct.Struct("<Q")
_FORMAT_TENSOR_NAME = "_qsrt_format_section"
_SHARED_SCALE_TENSOR_NAME = "_qsrt_shared_scale_section"
_ATOM_TENSOR_NAME = "qsrt_atoms"

ATOM_SIDE_CHANNELS = TILE_CHANNELS
ATOM_CHANNELS = 2 * ATOM_SIDE_CHANNELS
ATOMS_PER_RECORD_PAIR = 128 // ATOM_SIDE_CHANNELS


def atoms_per_expert(geometry: Geometry = KIMI_K3) -> int:
    return (geometry.records // 2) * ATOMS_PER_RECORD_PAIR


def matrix_atom_trellis_bytes(geometry: Geometry = KIMI_K3) -> int:
    """Six bits per coefficient pair over a 32 x latent atom."""

    return ATOM_CHANNELS * geometry.latent_channels * 3 // 8


ATOMS_PER_EXPERT = atoms_per_expert()
K2_STRIPE_BYTES = ATOM_SIDE_CHANNELS * KIMI_K3.latent_channels * 2 // 8
K3_STRIPE_BYTES = ATOM_SIDE_CHANNELS * KIMI_K3.latent_channels * 3 // 8
K4_STRIPE_BYTES = ATOM_SIDE_CHANNELS * KIMI_K3.latent_channels * 4 // 8
MATRIX_ATOM_TRELLIS_BYTES = matrix_atom_trellis_bytes()
MATRIX_ATOM_SCALE_BYTES = ATOM_CHANNELS * SCALE_BYTES
ATOM_TRELLIS_BYTES = 3 * MATRIX_ATOM_TRELLIS_BYTES
ATOM_SCALE_BYTES = LOCAL_SCALE_VECTORS * MATRIX_ATOM_SCALE_BYTES
ATOM_BUNDLE_BYTES = ATOM_TRELLIS_BYTES + ATOM_SCALE_BYTES
MATRIX_ATOM_TRELLIS_OFFSETS = {"w1": 0, "w3": MATRIX_ATOM_TRELLIS_BYTES, "w2": 2 * MATRIX_ATOM_TRELLIS_BYTES}
MATRIX_ATOM_SCALE_OFFSETS = {
    "w1": ATOM_TRELLIS_BYTES,
    "w3": ATOM_TRELLIS_BYTES + MATRIX_ATOM_SCALE_BYTES,
    "w2": ATOM_TRELLIS_BYTES + 2 * MATRIX_ATOM_SCALE_BYTES,
}
ATOM_SLAB_OFFSET = LAYER_HEADER_BYTES + FORMAT_SECTION_BYTES + SHARED_SCALE_SECTION_BYTES
# shard counts that divide the atom axis (equal-width direct loads)
EQUAL_SHARD_COUNTS = tuple(n for n in range(1, ATOMS_PER_EXPERT + 1) if ATOMS_PER_EXPERT % n == 0)


def _int_in(value, lo: int, hi: int, name: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int):
        raise TypeError(f"{name} must be an integer")
    if not lo <= value < hi:
        raise ValueError(f"{name} must be in {lo}..{hi - 1}")
    return value


def balanced_atom_partition(shard_count: int, shard_index: int, geometry: Geometry = KIMI_K3) -> tuple[int, int]:
    """``(first_atom, atom_count)`` of one whole-atom shard: the quotient /
    remainder rule, earlier shards take the extra atoms."""

    atoms = atoms_per_expert(geometry)
    _int_in(shard_count, 1, atoms + 1, "shard_count")
    _int_in(shard_index, 0, shard_count, "shard_index")
    quotient, remainder = divmod(atoms, shard_count)
    return shard_index * quotient + min(shard_index, remainder), quotient + int(shard_index < remainder)


def logical_atom_index(record_pair: int, stripe: int, geometry: Geometry = KIMI_K3) -> int:
    _int_in(record_pair, 0, geometry.records // 2, "record_pair")
    _int_in(stripe, 0, ATOMS_PER_RECORD_PAIR, "stripe")
    return record_pair * ATOMS_PER_RECORD_PAIR + stripe


def atom_components(logical_atom: int, geometry: Geometry = KIMI_K3) -> tuple[int, int]:
    _int_in(logical_atom, 0, atoms_per_expert(geometry), "logical_atom")
    return divmod(logical_atom, ATOMS_PER_RECORD_PAIR)


def atom_record_indices(logical_atom: int, geometry: Geometry = KIMI_K3) -> tuple[int, int]:
    pair, _ = atom_components(logical_atom, geometry)
    return 2 * pair, 2 * pair + 1


def atom_rates(mode: ModeSpec | str | int, logical_atom: int, geometry: Geometry = KIMI_K3) -> tuple[int, int]:
    pair, _ = atom_components(logical_atom, geometry)
    spec = resolve_mode(mode, geometry)
    return (2, 4) if pair < spec.mode_id else (3, 3)


def physical_atom_rotation(layer: int, expert: int, geometry: Geometry = KIMI_K3) -> int:
    return ATOMS_PER_RECORD_PAIR * pair_rotation(layer, expert, geometry)


def physical_atom_slot(layer: int, expert: int, logical_atom: int, geometry: Geometry = KIMI_K3) -> int:
    atom_components(logical_atom, geometry)
    return (logical_atom + physical_atom_rotation(layer, expert, geometry)) % atoms_per_expert(geometry)


def logical_atom_for_slot(layer: int, expert: int, physical_slot: int, geometry: Geometry = KIMI_K3) -> int:
    atoms = atoms_per_expert(geometry)
    _int_in(physical_slot, 0, atoms, "physical_slot")
    return (physical_slot - physical_atom_rotation(layer, expert, geometry)) % atoms


def _record_word_ranges(packed: PackedQSRTTrellis) -> tuple[tuple[int, int, int], ...]:
    """``(offset, words, K)`` of every stored record."""

    packed.validate()
    if packed.descriptor.mode.mode_id not in (0, 1, 2):
        raise ValueError("balanced atoms need six-bit record pairs (modes R0..R2)")
    out, cursor = [], 0
    for bits in record_bits(packed.descriptor.mode):
        words = packed.descriptor.tiles_per_record * TILE_CHANNELS * bits
        out.append((cursor, words, bits))
        cursor += words
    if cursor != packed.payload.numel():
        raise AssertionError("candidate record accounting drifted")
    return tuple(out)


def _record_stripes(record_words: torch.Tensor, rate_axis: str, orthogonal: int, words_per_tile: int) -> torch.Tensor:
    """``[stripes, orthogonal, words_per_tile]`` view-or-copy of one record."""

    if rate_axis == "k":
        return record_words.reshape(ATOMS_PER_RECORD_PAIR, orthogonal, words_per_tile)
    return record_words.reshape(orthogonal, ATOMS_PER_RECORD_PAIR, words_per_tile).transpose(0, 1)


def pack_matrix_atoms(packed: PackedQSRTTrellis) -> torch.Tensor:
    """Regroup packed tile words into ``[atoms, words_per_atom]`` (stripe ``s``
    of the low record followed by stripe ``s`` of the high record of each
    pair), without decoding a symbol."""

    d = packed.descriptor
    geo = d.geometry
    ranges = _record_word_ranges(packed)
    words_per_atom = matrix_atom_trellis_bytes(geo) // 2
    out = torch.empty((atoms_per_expert(geo), words_per_atom), dtype=torch.int16, device=packed.payload.device)
    orth = d.orthogonal_tiles
    for pair in range(geo.records // 2):
        sides = []
        for record in (2 * pair, 2 * pair + 1):
            offset, words, bits = ranges[record]
            sides.append(_record_stripes(packed.payload.narrow(0, offset, words), d.rate_axis, orth, TILE_CHANNELS * bits))
        joined = torch.cat([side.reshape(ATOMS_PER_RECORD_PAIR, -1) for side in sides], dim=1)
        out[pair * ATOMS_PER_RECORD_PAIR:(pair + 1) * ATOMS_PER_RECORD_PAIR].copy_(joined)
    return out


def unpack_matrix_atoms(atoms: torch.Tensor, descriptor) -> PackedQSRTTrellis:
    """Invert :func:`pack_matrix_atoms`."""

    geo = descriptor.geometry
    n_atoms, words_per_atom = atoms_per_expert(geo), matrix_atom_trellis_bytes(geo) // 2
    if atoms.dtype != torch.int16 or tuple(atoms.shape) != (n_atoms, words_per_atom) or not atoms.is_contiguous():
        raise ValueError(f"matrix atoms must be contiguous int16 [{n_atoms}, {words_per_atom}]")
    payload = torch.empty(descriptor.payload_words, dtype=torch.int16, device=atoms.device)
    packed = PackedQSRTTrellis(descriptor=descriptor, payload=payload)
    ranges = _record_word_ranges(packed)
    orth = descriptor.orthogonal_tiles
    for pair in range(geo.records // 2):
        block = atoms[pair * ATOMS_PER_RECORD_PAIR:(pair + 1) * ATOMS_PER_RECORD_PAIR]
        cursor = 0
        for record in (2 * pair, 2 * pair + 1):
            offset, words, bits = ranges[record]
            side_words = orth * TILE_CHANNELS * bits
            src = block[:, cursor:cursor + side_words].reshape(ATOMS_PER_RECORD_PAIR, orth, TILE_CHANNELS * bits)
            _record_stripes(payload.narrow(0, offset, words), descriptor.rate_axis, orth, TILE_CHANNELS * bits).copy_(src)
            cursor += side_words
        if cursor != words_per_atom:
            raise AssertionError("atom inverse did not consume its payload")
    packed.validate()
    return packed


def pack_local_scale_atoms(scale: torch.Tensor, geometry: Geometry = KIMI_K3) -> torch.Tensor:
    """One intermediate-axis FP16 scale vector -> ``[atoms, 32]``."""

    n = geometry.intermediate_channels
    if scale.dtype != torch.float16 or tuple(scale.shape) != (n,) or not scale.is_contiguous():
        raise ValueError(f"local scale must be contiguous float16 [{n}]")
    rec = scale.reshape(geometry.records // 2, 2, ATOMS_PER_RECORD_PAIR, ATOM_SIDE_CHANNELS)
    return rec.permute(0, 2, 1, 3).reshape(atoms_per_expert(geometry), ATOM_CHANNELS).contiguous()


def unpack_local_scale_atoms(atoms: torch.Tensor, geometry: Geometry = KIMI_K3) -> torch.Tensor:
    n_atoms = atoms_per_expert(geometry)
    if atoms.dtype != torch.float16 or tuple(atoms.shape) != (n_atoms, ATOM_CHANNELS) or not atoms.is_contiguous():
        raise ValueError(f"scale atoms must be contiguous float16 [{n_atoms}, {ATOM_CHANNELS}]")
    a = atoms.reshape(geometry.records // 2, ATOMS_PER_RECORD_PAIR, 2, ATOM_SIDE_CHANNELS)
    return a.permute(0, 2, 1, 3).reshape(geometry.intermediate_channels).contiguous()


def rotate_expert_atoms(logical_atoms: torch.Tensor, layer: int, expert: int, geometry: Geometry = KIMI_K3) -> torch.Tensor:
    """One expert's logical atoms in global physical-slot order."""

    n = atoms_per_expert(geometry)
    if logical_atoms.ndim < 1 or logical_atoms.shape[0] != n:
        raise ValueError(f"logical_atoms must have leading dimension {n}")
    order = torch.tensor([logical_atom_for_slot(layer, expert, s, geometry) for s in range(n)], dtype=torch.long,
                         device=logical_atoms.device)
    return logical_atoms.index_select(0, order).contiguous()


def unrotate_expert_atoms(physical_atoms: torch.Tensor, layer: int, expert: int, geometry: Geometry = KIMI_K3) -> torch.Tensor:
    n = atoms_per_expert(geometry)
    if physical_atoms.ndim < 1 or physical_atoms.shape[0] != n:
        raise ValueError(f"physical_atoms must have leading dimension {n}")
    order = torch.tensor([physical_atom_slot(layer, expert, a, geometry) for a in range(n)], dtype=torch.long,
                         device=physical_atoms.device)
    return physical_atoms.index_select(0, order).contiguous()


@dataclass(frozen=True)
class QSRTShardExtent:
    """One shard's single contiguous atom-slab read."""

    shard_count: int
    shard_index: int
    first_atom_slot: int
    atom_slots: int
    intermediate_channels: int
    offset_bytes: int
    extent_bytes: int
    payload_bytes: int
    padding_bytes: int


@dataclass(frozen=True)
class QSRTLayerLayout:
    """Atom-major compressed layer: ``[atoms, compressed_experts, bundle]``
    with each atom row padded to 4 KiB."""

    compressed_experts: int
    x4t_experts: int

    def __post_init__(self) -> None:
        for name, value in (("compressed_experts", self.compressed_experts), ("x4t_experts", self.x4t_experts)):
            if isinstance(value, bool) or not isinstance(value, int) or value < 0:
                raise ValueError(f"{name} must be a non-negative integer")
        if self.compressed_experts + self.x4t_experts != EXPERTS_PER_LAYER:
            raise ValueError(f"a layer must account for exactly {EXPERTS_PER_LAYER} experts")

    @property
    def atom_slot_payload_bytes(self) -> int:
        return self.compressed_experts * ATOM_BUNDLE_BYTES

    @property
    def atom_slot_stride_bytes(self) -> int:
        return align_up(self.atom_slot_payload_bytes, STORAGE_ALIGNMENT)

    @property
    def atom_slot_padding_bytes(self) -> int:
        return self.atom_slot_stride_bytes - self.atom_slot_payload_bytes

    @property
    def compressed_payload_bytes(self) -> int:
        return self.compressed_experts * ATOMS_PER_EXPERT * ATOM_BUNDLE_BYTES

    @property
    def disk_bytes(self) -> int:
        return ATOM_SLAB_OFFSET + ATOMS_PER_EXPERT * self.atom_slot_stride_bytes

    def atom_bundle_offset(self, physical_slot: int, compressed_slot: int) -> int:
        if isinstance(physical_slot, bool) or not isinstance(physical_slot, int) or not 0 <= physical_slot < ATOMS_PER_EXPERT:
            raise ValueError(f"physical_slot must be in 0..{ATOMS_PER_EXPERT - 1}")
        if (isinstance(compressed_slot, bool) or not isinstance(compressed_slot, int)
                or not 0 <= compressed_slot < self.compressed_experts):
            raise ValueError(f"compressed_slot must be in 0..{self.compressed_experts - 1}")
        return ATOM_SLAB_OFFSET + physical_slot * self.atom_slot_stride_bytes + compressed_slot * ATOM_BUNDLE_BYTES

    def shard_extent(self, shard_count: int, shard_index: int, *, require_equal: bool = False) -> QSRTShardExtent:
        first, slots = balanced_atom_partition(shard_count, shard_index)
        if require_equal and shard_count not in EQUAL_SHARD_COUNTS:
            raise ValueError(f"{shard_count} shards do not divide the QSRT atom axis; "
                             f"equal partitions are {EQUAL_SHARD_COUNTS}")
        extent = slots * self.atom_slot_stride_bytes
        payload = slots * self.atom_slot_payload_bytes
        return QSRTShardExtent(shard_count, shard_index, first, slots, slots * ATOM_CHANNELS,
                               ATOM_SLAB_OFFSET + first * self.atom_slot_stride_bytes, extent, payload, extent - payload)

    def to_manifest(self) -> dict:
        return {
            "schema": SCHEMA,
            "alignment_bytes": STORAGE_ALIGNMENT,
            "compressed_experts": self.compressed_experts,
            "x4t_experts": self.x4t_experts,
            "atom_channels": ATOM_CHANNELS,
            "atom_slots": ATOMS_PER_EXPERT,
            "atom_bundle_bytes": ATOM_BUNDLE_BYTES,
            "atom_slot_payload_bytes": self.atom_slot_payload_bytes,
            "atom_slot_stride_bytes": self.atom_slot_stride_bytes,
            "atom_slot_padding_bytes": self.atom_slot_padding_bytes,
            "compressed_payload_bytes": self.compressed_payload_bytes,
            "atom_slab_offset": ATOM_SLAB_OFFSET,
            "disk_bytes": self.disk_bytes,
            "equal_shard_counts": list(EQUAL_SHARD_COUNTS),
        }


@dataclass(frozen=True)
class QSRTLayerHeader:
    """Canonical 4 KiB safetensors header of one atom-major layer: format
    section, shared-scale section and the padded atom slab as three U8
    tensors, JSON with sorted keys, space padded."""

    layer: int
    layout: QSRTLayerLayout
    profile_id: int = PROFILE_ID_QSRT_SQG_E4M3

    def __post_init__(self) -> None:
        if isinstance(self.layer, bool) or not isinstance(self.layer, int):
            raise TypeError("layer must be an integer")
        if not 1 <= self.layer <= 92:
            raise ValueError("K3 MoE layer must be in 1..92")
        if self.profile_id != PROFILE_ID_QSRT_SQG_E4M3:
            raise ValueError("unsupported QSRT reconstruction profile")

    def _document(self) -> dict:
        slab = ATOMS_PER_EXPERT * self.layout.atom_slot_stride_bytes
        meta = {
            "format": "pt",
            "schema": SCHEMA,
            "version": str(VERSION),
            "encoding": ENCODING_QSRT_SQG_E4M3,
            "layer": str(self.layer),
            "profile_id": str(self.profile_id),
            "experts": str(EXPERTS_PER_LAYER),
            "compressed_experts": str(self.layout.compressed_experts),
            "x4t_experts": str(self.layout.x4t_experts),
            "intermediate_channels": str(KIMI_K3.intermediate_channels),
            "latent_channels": str(KIMI_K3.latent_channels),
            "atom_channels": str(ATOM_CHANNELS),
            "atom_slots": str(ATOMS_PER_EXPERT),
            "atom_bundle_bytes": str(ATOM_BUNDLE_BYTES),
            "atom_slot_payload_bytes": str(self.layout.atom_slot_payload_bytes),
            "atom_slot_stride_bytes": str(self.layout.atom_slot_stride_bytes),
            "alignment_bytes": str(STORAGE_ALIGNMENT),
        }
        f0, f1 = 0, FORMAT_SECTION_BYTES
        s1 = f1 + SHARED_SCALE_SECTION_BYTES
        return {
            "__metadata__": meta,
            _FORMAT_TENSOR_NAME: {"dtype": "U8", "shape": [FORMAT_SECTION_BYTES], "data_offsets": [f0, f1]},
            _SHARED_SCALE_TENSOR_NAME: {"dtype": "U8", "shape": [SHARED_SCALE_SECTION_BYTES], "data_offsets": [f1, s1]},
            _ATOM_TENSOR_NAME: {"dtype": "U8", "shape": [ATOMS_PER_EXPERT, self.layout.atom_slot_stride_bytes],
                                "data_offsets": [s1, s1 + slab]},
        }

    def to_bytes(self) -> bytes:
        capacity = LAYER_HEADER_BYTES - _HEADER_LENGTH.size
        document = json.dumps(self._document(), sort_keys=True, separators=(",", ":")).encode("utf-8")
        if len(document) > capacity:
            raise AssertionError("QSRT safetensors header exceeds its 4 KiB budget")
        return _HEADER_LENGTH.pack(capacity) + document + b" " * (capacity - len(document))

    @classmethod
    def from_bytes(cls, payload: bytes) -> "QSRTLayerHeader":
        if len(payload) != LAYER_HEADER_BYTES:
            raise ValueError(f"QSRT layer header must contain {LAYER_HEADER_BYTES} bytes")
        if _HEADER_LENGTH.unpack_from(payload)[0] != LAYER_HEADER_BYTES - _HEADER_LENGTH.size:
            raise ValueError("QSRT safetensors header must occupy exactly 4 KiB")
        try:
            document = json.loads(payload[_HEADER_LENGTH.size:].decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as exc:
            raise ValueError("QSRT safetensors header is invalid JSON") from exc
        if not isinstance(document, dict) or not isinstance(document.get("__metadata__"), dict):
            raise ValueError("QSRT safetensors header omits metadata")
        meta = document["__metadata__"]
        try:
            result = cls(layer=int(meta["layer"]),
                         layout=QSRTLayerLayout(int(meta["compressed_experts"]), int(meta["x4t_experts"])),
                         profile_id=int(meta["profile_id"]))
        except (KeyError, TypeError, ValueError) as exc:
            raise ValueError("QSRT safetensors metadata is malformed") from exc
        if document != result._document():
            raise ValueError("QSRT safetensors header is noncanonical")
        return result


# accounting invariants of the Kimi-K3 preset
if ATOMS_PER_EXPERT != 96:
    raise AssertionError("Kimi-K3 QSRT must contain 96 balanced atoms")
if K2_STRIPE_BYTES + K4_STRIPE_BYTES != 2 * K3_STRIPE_BYTES:
    raise AssertionError("P24 and P33 atom payloads must have equal size")
if MATRIX_ATOM_TRELLIS_BYTES != K2_STRIPE_BYTES + K4_STRIPE_BYTES:
    raise AssertionError("matrix atom trellis accounting drifted")
