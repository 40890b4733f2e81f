"""QSRT matrix format: rate modes, EXL word packing, descriptors, decode.

Mirrors ``qsrt/qsrt.py``.  The reference hard-codes the Kimi-K3 geometry
(3072 intermediate x 3584 latent channels, ``qsrt.py:33-47``); here the
geometry is a parameter (:class:`Geometry`) and the Kimi-K3 values are the
default preset ``KIMI_K3``, so the BASELINE shapes (256/512, 5120/1536,
7168/2048) pack and decode with the same code.

Packing of GPU tensors runs in the HIP kernels ``qsrt_pack_edges`` /
``qsrt_unpack_states``; CPU tensors use the reference's torch formulation
(the two are checked against each other and against the reference's
known-answer words, ``tests/test_qsrt.py:242-258``).
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass, field
from typing import Literal

import torch

from .exl3_reference import (
    CODEBOOK_SQG_XOR_CHEB_T12,
    decode_qsrt_weight,
    reconstruct_trellis_states,
)

TILE_CHANNELS = 16
TILE_VALUES = TILE_CHANNELS * TILE_CHANNELS
RECORD_CHANNELS = 128
TILES_PER_RECORD_AXIS = RECORD_CHANNELS // TILE_CHANNELS
STORAGE_ALIGNMENT = 4096
SCHEMA = "qsrt_kimi_k3_qsrt_candidate_v1"
GENERIC_SCHEMA = "qsrt_amd_qsrt_candidate_v1"
LOGICAL_CANDIDATE_SCHEMAS = (SCHEMA, GENERIC_SCHEMA)

RateAxis = Literal["k", "n"]
PairKind = Literal["P22", "P24", "P33"]

MATRIX_RATE_AXIS: dict[str, RateAxis] = {"w1": "n", "w3": "n", "w2": "k"}


@dataclass(frozen=True)
class Geometry:
    """Expert geometry: the shared intermediate (rate) axis and the latent
    (orthogonal) axis, in channels."""

    intermediate_channels: int
    latent_channels: int
    record_channels: int = RECORD_CHANNELS

    def __post_init__(self) -> None:
        if self.record_channels % TILE_CHANNELS or self.record_channels <= 0:
            raise ValueError("record_channels must be a positive multiple of 16")
        if self.intermediate_channels % self.record_channels or self.intermediate_channels <= 0:
            raise ValueError("the intermediate axis must hold whole records")
        if self.latent_channels % TILE_CHANNELS or self.latent_channels <= 0:
            raise ValueError("the latent axis must hold whole 16-channel tiles")

    @property
    def records(self) -> int:
        return self.intermediate_channels // self.record_channels

    @property
    def tiles_per_record_axis(self) -> int:
        return self.record_channels // TILE_CHANNELS


KIMI_K3 = Geometry(3072, 3584)
INTERMEDIATE_CHANNELS = KIMI_K3.intermediate_channels
LATENT_CHANNELS = KIMI_K3.latent_channels
RECORDS_PER_EXPERT = KIMI_K3.records
PAIRS_PER_EXPERT = RECORDS_PER_EXPERT // 2
FIXED_HIGH_RATE_RECORD_BITS = (3,) * 22 + (4,) * 2

# Layer-level format constants (reference qsrt.py:33-90).
EXPERTS_PER_LAYER = 896
MOE_LAYERS = range(1, 93)
CONTEXT_GROUP_CHANNELS = 4
PAIR_CHANNELS = 2 * RECORD_CHANNELS
PAIR_ROTATION_EXPERT_MULTIPLIER = 5
FORMAT_BITS = 8
FORMAT_X4T = 0xFF
FORMAT_NIBBLE_MASK = 0x0F
LAYER_HEADER_BYTES = STORAGE_ALIGNMENT
FORMAT_TABLE_BYTES = (EXPERTS_PER_LAYER * FORMAT_BITS + 7) // 8
FORMAT_SECTION_BYTES = STORAGE_ALIGNMENT
HOT_FORMAT_BYTES = EXPERTS_PER_LAYER
HOT_SLOT_BYTES = EXPERTS_PER_LAYER * 2
HOT_METADATA_BYTES = HOT_FORMAT_BYTES + HOT_SLOT_BYTES
SHARED_SCALE_VECTORS = 3
LOCAL_SCALE_VECTORS = 3
SHARED_SCALE_ORDER = ("w1.suh", "w3.suh", "w2.svh")
LOCAL_SCALE_ORDER = ("w1.svh", "w3.svh", "w2.suh")
SCALE_BYTES = 2
SHARED_SCALE_BYTES = SHARED_SCALE_VECTORS * LATENT_CHANNELS * SCALE_BYTES
SHARED_SCALE_SECTION_BYTES = 6 * STORAGE_ALIGNMENT
PAIR_BYTES = PAIR_CHANNELS * LATENT_CHANNELS * 3 // 8
MATRIX_TRELLIS_BYTES = PAIRS_PER_EXPERT * PAIR_BYTES
EXPERT_TRELLIS_BYTES = 3 * MATRIX_TRELLIS_BYTES
FIXED_HIGH_RATE_TRELLIS_BYTES = (
    INTERMEDIATE_CHANNELS * LATENT_CHANNELS * sum(FIXED_HIGH_RATE_RECORD_BITS) // (RECORDS_PER_EXPERT * 8)
)
PURE_K2_MATRIX_TRELLIS_BYTES = INTERMEDIATE_CHANNELS * LATENT_CHANNELS * 2 // 8
PURE_K2_EXPERT_TRELLIS_BYTES = 3 * PURE_K2_MATRIX_TRELLIS_BYTES


# ---------------------------------------------------------------------------
# Rate modes (reference qsrt.py:143-236, :516-561)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class ModeSpec:
    """A record-rate schedule: ``context_bits`` holds one K per context,
    ordered from low to high importance.  IDs 0..2 are the equal-rate
    K2/K4 transfer modes R0..R2, 3 is H308 (22 x K3 + 2 x K4), 4 is K2."""

    mode_id: int
    name: str
    context_bits: tuple[int, ...]
    geometry: Geometry = field(default=KIMI_K3, compare=False)

    def __post_init__(self) -> None:
        if isinstance(self.mode_id, bool) or not isinstance(self.mode_id, int):
            raise TypeError("mode_id must be an integer")
        if not 0 <= self.mode_id <= 4:
            raise ValueError("QSRT mode_id must identify R0, R1, R2, H308, or K2")
        if not self.name:
            raise ValueError("mode name must not be empty")
        pure_k2 = self.mode_id == 4
        high_rate = self.mode_id == 3
        if not self.context_bits or (len(self.context_bits) % 2 and not pure_k2):
            raise ValueError("a mode must contain an even, nonzero context count")
        if any(b not in (2, 3, 4) for b in self.context_bits):
            raise ValueError("QSRT supports only K2, K3, and K4")
        records = self.geometry.records
        if high_rate:
            if self.name != "H308" or self.context_bits != FIXED_HIGH_RATE_RECORD_BITS:
                raise ValueError("H308 must contain exactly 22 K3 and 2 K4 records")
            if records != len(FIXED_HIGH_RATE_RECORD_BITS):
                raise ValueError("H308 needs exactly 24 records on the rate axis")
        elif pure_k2:
            if self.name != "K2" or self.context_bits != (2,):
                raise ValueError("K2 must contain one uniform two-bit context")
        elif sum(self.context_bits) != 3 * len(self.context_bits):
            raise ValueError("a rate-transfer mode must average exactly three bits")
        if records % len(self.context_bits):
            raise ValueError("contexts must divide the rate axis records")
        if tuple(sorted(self.context_bits)) != self.context_bits:
            raise ValueError("context rates must be monotone from K2 through K4")
        if high_rate or pure_k2:
            return
        per_context = records // len(self.context_bits)
        k2 = self.context_bits.count(2) * per_context
        k4 = self.context_bits.count(4) * per_context
        if k2 != k4:
            raise ValueError("K2 and K4 record counts must match")
        if self.mode_id != k2:
            raise ValueError(f"mode_id must equal the rate-transfer count {k2}")

    @property
    def context_count(self) -> int:
        return len(self.context_bits)

    @property
    def records_per_context(self) -> int:
        return self.geometry.records // self.context_count


def rate_transfer_mode(r: int, geometry: Geometry = KIMI_K3) -> ModeSpec:
    n = geometry.records
    return ModeSpec(r, f"R{r}", (2,) * r + (3,) * (n - 2 * r) + (4,) * r, geometry)


def high_rate_mode(geometry: Geometry = KIMI_K3) -> ModeSpec:
    return ModeSpec(3, "H308", FIXED_HIGH_RATE_RECORD_BITS, geometry)


def pure_k2_mode(geometry: Geometry = KIMI_K3) -> ModeSpec:
    return ModeSpec(4, "K2", (2,), geometry)


RATE_TRANSFER_MODES = tuple(rate_transfer_mode(r) for r in range(3))
R0, R1, R2 = RATE_TRANSFER_MODES
H308 = high_rate_mode()
K2 = pure_k2_mode()
_ALL_MODES = (*RATE_TRANSFER_MODES, H308, K2)

# Phase-1 covariance policy of the expert encode (reference qsrt/qsrt.py:220-233): H13 is the layer's
# global input covariance (local weight 0); H2 is the expert's decoded post-activation covariance shrunk
# toward its trace-scaled identity by weighted OAS, its local weight capped at 0.75.  Offline encoder
# controls: they consume no format bits.
PHASE1_H13_EXPERT_LOCAL_ALPHA = 0.0
PHASE1_H2_EXPERT_LOCAL_ALPHA = 0.75
PHASE1_H2_LOCAL_BASIS = "decoded_candidate_post_situ"
PHASE1_H2_SHRINKAGE_POLICY = "weighted_oas_scaled_identity"


def modes_for(geometry: Geometry) -> dict[str, ModeSpec]:
    """The named modes that exist for a geometry (H308 needs 24 records)."""

    out = {f"R{r}": rate_transfer_mode(r, geometry) for r in range(min(3, geometry.records // 2 + 1))}
    out["K2"] = pure_k2_mode(geometry)
    if geometry.records == len(FIXED_HIGH_RATE_RECORD_BITS):
        out["H308"] = high_rate_mode(geometry)
    return out


def resolve_mode(mode: ModeSpec | str | int, geometry: Geometry = KIMI_K3) -> ModeSpec:
    if isinstance(mode, ModeSpec):
        return mode
    table = modes_for(geometry)
    if isinstance(mode, str):
        try:
            return table[mode.upper()]
        except KeyError as exc:
            raise ValueError(f"unknown QSRT mode: {mode}") from exc
    if isinstance(mode, int) and not isinstance(mode, bool):
        for spec in table.values():
            if spec.mode_id == mode:
                return spec
        raise ValueError(f"unknown QSRT mode ID: {mode}")
    raise TypeError("mode must be a ModeSpec, name, or integer ID")


def matrix_rate_axis(matrix: str) -> RateAxis:
    try:
        return MATRIX_RATE_AXIS[matrix]
    except KeyError as exc:
        raise ValueError(f"unknown expert matrix: {matrix}") from exc


def record_contexts(mode: ModeSpec | str | int) -> tuple[int, ...]:
    """Serialized record order: low/high contexts interleaved so records
    pair into P24/P33 (reference qsrt.py:516-532)."""

    spec = resolve_mode(mode)
    records = spec.geometry.records
    if spec.mode_id == 3:
        return tuple(range(records))
    if spec.mode_id == 4:
        return (0,) * records
    contexts: list[int] = []
    for low in range(spec.context_count // 2):
        high = spec.context_count - 1 - low
        for _ in range(spec.records_per_context):
            contexts.extend((low, high))
    return tuple(contexts)


def record_bits(mode: ModeSpec | str | int) -> tuple[int, ...]:
    spec = resolve_mode(mode)
    return tuple(spec.context_bits[c] for c in record_contexts(spec))


def pair_bits(mode: ModeSpec | str | int) -> tuple[tuple[int, int], ...]:
    spec = resolve_mode(mode)
    records = record_bits(spec)
    pairs = tuple(zip(records[0::2], records[1::2], strict=True))
    expected = 4 if spec.mode_id == 4 else 6
    if any(sum(p) != expected for p in pairs):
        raise ValueError("QSRT record pairs do not match the mode rate sum")
    return pairs


def pair_kinds(mode: ModeSpec | str | int) -> tuple[PairKind, ...]:
    kinds = {(2, 2): "P22", (2, 4): "P24", (3, 3): "P33"}
    out = []
    for pair in pair_bits(mode):
        if pair not in kinds:
            raise ValueError(f"unsupported QSRT pair schedule: {pair}")
        out.append(kinds[pair])
    return tuple(out)


# ---------------------------------------------------------------------------
# EXL word packing and cyclic states (reference qsrt.py:861-913)
# ---------------------------------------------------------------------------


def _validate_k(bits: int) -> None:
    if isinstance(bits, bool) or not isinstance(bits, int) or bits not in (2, 3, 4):
        raise ValueError("QSRT supports K=2, K=3, or K=4")


def pack_trellis_edges(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """Low K bits of each of 256 symbols -> 16K int16 words per tile: one
    MSB-first bitstream over the tile, 16 bits per word, adjacent words
    swapped (the EXL ``pack_trellis`` order with SWAP16)."""

    _validate_k(bits)
    if indices.ndim < 1 or indices.shape[-1] != TILE_VALUES:
        raise ValueError("indices must have a final dimension of 256")
    if indices.dtype == torch.bool or indices.is_floating_point():
        raise TypeError("indices must use an integer dtype")
    if indices.is_cuda:
        from .codec import pack_edges_gpu

        return pack_edges_gpu(indices, bits)
    values = indices.to(torch.int64) & ((1 << bits) - 1)
    lead = values.shape[:-1]
    shifts = torch.arange(bits - 1, -1, -1)
    stream = ((values[..., None] >> shifts) & 1).reshape(*lead, TILE_VALUES * bits)
    words = (stream.reshape(*lead, 16 * bits, 16) << torch.arange(15, -1, -1)).sum(-1)
    swapped = words.reshape(*lead, -1, 2).flip(-1).reshape(*lead, 16 * bits)
    return swapped.to(torch.int16).contiguous()


def unpack_trellis_edges(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """Inverse of :func:`pack_trellis_edges`: the stored K-bit symbols."""

    _validate_k(bits)
    if packed.ndim < 1 or packed.shape[-1] != TILE_CHANNELS * bits:
        raise ValueError(f"packed tiles must end in {TILE_CHANNELS * bits} int16 words")
    if packed.dtype != torch.int16:
        raise TypeError("packed trellis words must use torch.int16")
    lead = packed.shape[:-1]
    words = (packed.to(torch.int64) & 0xFFFF).reshape(*lead, -1, 2).flip(-1).reshape(*lead, 16 * bits)
    stream = ((words[..., None] >> torch.arange(15, -1, -1, device=packed.device)) & 1).reshape(*lead, TILE_VALUES, bits)
    values = (stream << torch.arange(bits - 1, -1, -1, device=packed.device)).sum(-1)
    return values.to(torch.int16).contiguous()


def unpack_trellis_states(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """Unpack words and rebuild every cyclic 16-bit state."""

    if packed.is_cuda:
        _validate_k(bits)
        if packed.ndim < 1 or packed.shape[-1] != TILE_CHANNELS * bits:
            raise ValueError(f"packed tiles must end in {TILE_CHANNELS * bits} int16 words")
        if packed.dtype != torch.int16:
            raise TypeError("packed trellis words must use torch.int16")
        from .codec import unpack_states_gpu

        return unpack_states_gpu(packed, bits)
    return reconstruct_trellis_states(unpack_trellis_edges(packed, bits), bits)


# ---------------------------------------------------------------------------
# Matrix payloads (reference qsrt.py:916-1172), geometry-parameterised
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class QSRTTrellisDescriptor:
    """One complete packed expert matrix, independent of tensor parallelism."""

    mode_id: int
    rate_axis: RateAxis
    k_tiles: int
    n_tiles: int
    schema: str = SCHEMA
    intermediate_channels: int = INTERMEDIATE_CHANNELS
    record_channels: int = RECORD_CHANNELS
    latent_channels: int = LATENT_CHANNELS

    def __post_init__(self) -> None:
        if self.schema not in LOGICAL_CANDIDATE_SCHEMAS:
            raise ValueError(f"unsupported QSRT schema: {self.schema}")
        if self.schema == SCHEMA and (
            self.intermediate_channels != INTERMEDIATE_CHANNELS or self.latent_channels != LATENT_CHANNELS
        ):
            raise ValueError("the Kimi-K3 schema requires a 3072-channel intermediate axis and 3584 latent channels")
        if self.record_channels != RECORD_CHANNELS:
            raise ValueError("QSRT requires 128-channel records")
        if self.rate_axis not in ("k", "n"):
            raise ValueError("rate_axis must be 'k' or 'n'")
        if self.k_tiles <= 0 or self.n_tiles <= 0:
            raise ValueError("tile dimensions must be positive")
        self.mode  # validates mode against the geometry
        rate_tiles = self.k_tiles if self.rate_axis == "k" else self.n_tiles
        if rate_tiles * TILE_CHANNELS != self.intermediate_channels:
            raise ValueError(f"rate axis must contain exactly {self.intermediate_channels} channels")
        orth = self.n_tiles if self.rate_axis == "k" else self.k_tiles
        if orth * TILE_CHANNELS != self.latent_channels:
            raise ValueError(f"orthogonal axis must contain exactly {self.latent_channels} channels")

    @property
    def geometry(self) -> Geometry:
        return Geometry(self.intermediate_channels, self.latent_channels, self.record_channels)

    @property
    def mode(self) -> ModeSpec:
        return resolve_mode(self.mode_id, self.geometry)

    @property
    def orthogonal_tiles(self) -> int:
        return self.n_tiles if self.rate_axis == "k" else self.k_tiles

    @property
    def tiles_per_record(self) -> int:
        return TILES_PER_RECORD_AXIS * self.orthogonal_tiles

    @property
    def words_per_record(self) -> tuple[int, ...]:
        unit = self.tiles_per_record * TILE_CHANNELS
        return tuple(unit * b for b in record_bits(self.mode))

    @property
    def words_per_pair(self) -> int:
        if self.mode.mode_id == 3:
            raise ValueError("H308 has no fixed six-bit record-pair contract")
        return self.tiles_per_record * TILE_CHANNELS * sum(pair_bits(self.mode)[0])

    @property
    def payload_words(self) -> int:
        return sum(self.words_per_record)

    @property
    def payload_bytes(self) -> int:
        return self.payload_words * 2

    @property
    def weight_count(self) -> int:
        return self.k_tiles * self.n_tiles * TILE_VALUES

    def to_manifest(self) -> dict[str, object]:
        high = self.mode.mode_id == 3
        return {
            "schema": self.schema,
            "mode_id": self.mode_id,
            "mode": self.mode.name,
            "rate_axis": self.rate_axis,
            "k_tiles": self.k_tiles,
            "n_tiles": self.n_tiles,
            "intermediate_channels": self.intermediate_channels,
            "latent_channels": self.latent_channels,
            "record_channels": self.record_channels,
            "pair_channels": 2 * self.record_channels,
            "record_bits": list(record_bits(self.mode)),
            "pair_kinds": None if high else list(pair_kinds(self.mode)),
            "words_per_pair": None if high else self.words_per_pair,
            "words_per_record": list(self.words_per_record),
            "payload_words": self.payload_words,
            "payload_bytes": self.payload_bytes,
        }


@dataclass(frozen=True)
class PackedQSRTTrellis:
    descriptor: QSRTTrellisDescriptor
    payload: torch.Tensor

    def validate(self) -> None:
        if self.payload.dtype != torch.int16:
            raise TypeError("QSRT trellis payload must use torch.int16")
        if self.payload.ndim != 1:
            raise ValueError("QSRT trellis payload must be one-dimensional")
        if self.payload.numel() != self.descriptor.payload_words:
            raise ValueError("QSRT trellis payload length does not match its descriptor")


def _record_tiles(encoded: torch.Tensor, record: int, rate_axis: RateAxis) -> torch.Tensor:
    begin = record * TILES_PER_RECORD_AXIS
    axis = 0 if rate_axis == "k" else 1
    return encoded.narrow(axis, begin, TILES_PER_RECORD_AXIS).reshape(-1, TILE_VALUES)


def _descriptor_for(encoded: torch.Tensor, spec: ModeSpec, rate_axis: RateAxis, schema: str | None) -> QSRTTrellisDescriptor:
    if encoded.ndim != 3 or encoded.shape[-1] != TILE_VALUES:
        raise ValueError("encoded states must have shape [K/16, N/16, 256]")
    if encoded.dtype == torch.bool or encoded.is_floating_point():
        raise TypeError("encoded states must use an integer dtype")
    if rate_axis not in ("k", "n"):
        raise ValueError("rate_axis must be 'k' or 'n'")
    rate_tiles, orth_tiles = (encoded.shape[0], encoded.shape[1]) if rate_axis == "k" else (encoded.shape[1], encoded.shape[0])
    geometry = spec.geometry
    if rate_tiles * TILE_CHANNELS != geometry.intermediate_channels:
        raise ValueError(f"encoded rate axis must contain exactly {geometry.intermediate_channels} channels")
    if schema is None:
        schema = SCHEMA if geometry == KIMI_K3 else GENERIC_SCHEMA
    return QSRTTrellisDescriptor(
        mode_id=spec.mode_id,
        rate_axis=rate_axis,
        k_tiles=encoded.shape[0],
        n_tiles=encoded.shape[1],
        schema=schema,
        intermediate_channels=geometry.intermediate_channels,
        latent_channels=orth_tiles * TILE_CHANNELS,
    )


def pack_qsrt_trellis(
    encoded: torch.Tensor,
    mode: ModeSpec | str | int,
    *,
    rate_axis: RateAxis,
    schema: str | None = None,
    validate_states: bool = True,
    geometry: Geometry | None = None,
) -> PackedQSRTTrellis:
    """Record-major concatenation of per-tile EXL words; with
    ``validate_states`` every record must unpack to the same closed cyclic
    states (reference qsrt.py:1051-1082)."""

    if geometry is None:
        axis_tiles = encoded.shape[0] if rate_axis == "k" else encoded.shape[1]
        orth_tiles = encoded.shape[1] if rate_axis == "k" else encoded.shape[0]
        geometry = Geometry(axis_tiles * TILE_CHANNELS, orth_tiles * TILE_CHANNELS) if not isinstance(mode, ModeSpec) else mode.geometry
    spec = mode if isinstance(mode, ModeSpec) else resolve_mode(mode, geometry)
    descriptor = _descriptor_for(encoded, spec, rate_axis, schema)
    pieces = []
    for record, bits in enumerate(record_bits(spec)):
        states = _record_tiles(encoded, record, rate_axis)
        words = pack_trellis_edges(states, bits)
        if validate_states and not torch.equal(unpack_trellis_states(words, bits), states.to(torch.int16)):
            raise ValueError("encoded input is not a closed cyclic trellis path")
        pieces.append(words.reshape(-1))
    packed = PackedQSRTTrellis(descriptor, torch.cat(pieces).contiguous())
    packed.validate()
    return packed


def _unpack_records(packed: PackedQSRTTrellis, fn) -> torch.Tensor:
    packed.validate()
    d = packed.descriptor
    out = torch.empty((d.k_tiles, d.n_tiles, TILE_VALUES), dtype=torch.int16, device=packed.payload.device)
    axis = 0 if d.rate_axis == "k" else 1
    cursor = 0
    for record, bits in enumerate(record_bits(d.mode)):
        count = d.tiles_per_record * TILE_CHANNELS * bits
        words = packed.payload.narrow(0, cursor, count).reshape(d.tiles_per_record, TILE_CHANNELS * bits)
        tiles = fn(words, bits)
        shape = (TILES_PER_RECORD_AXIS, d.n_tiles, TILE_VALUES) if axis == 0 else (d.k_tiles, TILES_PER_RECORD_AXIS, TILE_VALUES)
        out.narrow(axis, record * TILES_PER_RECORD_AXIS, TILES_PER_RECORD_AXIS).copy_(tiles.reshape(shape))
        cursor += count
    if cursor != packed.payload.numel():
        raise ValueError("QSRT trellis payload has trailing data")
    return out


def unpack_qsrt_trellis_edges(packed: PackedQSRTTrellis) -> torch.Tensor:
    return _unpack_records(packed, unpack_trellis_edges)


def unpack_qsrt_trellis_states(packed: PackedQSRTTrellis) -> torch.Tensor:
    """Physical-order 16-bit states of a complete payload.  States never
    cross tiles, so each record's tiles are rebuilt independently."""

    return _unpack_records(packed, unpack_trellis_states)


def _validate_scale_vector(scale: torch.Tensor, length: int, name: str, device=None) -> None:
    if scale.dtype != torch.float16:
        raise TypeError(f"{name} must use torch.float16")
    if scale.ndim != 1 or scale.numel() != length:
        raise ValueError(f"{name} must contain exactly {length} values")
    if not scale.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if device is not None and scale.device != device:
        raise ValueError(f"{name} must be on {device}")
    if not bool(torch.all(torch.isfinite(scale))):
        raise ValueError(f"{name} contains non-finite values")


def decode_qsrt_exl3_weight(
    packed: PackedQSRTTrellis,
    suh: torch.Tensor,
    svh: torch.Tensor,
    *,
    codebook: str = CODEBOOK_SQG_XOR_CHEB_T12,
) -> torch.Tensor:
    """Decode a complete payload to its EXL-oriented ``[K, N]`` FP32 weight
    (reference qsrt.py:1175-1209)."""

    packed.validate()
    d = packed.descriptor
    _validate_scale_vector(suh, d.k_tiles * TILE_CHANNELS, "suh", packed.payload.device)
    _validate_scale_vector(svh, d.n_tiles * TILE_CHANNELS, "svh", packed.payload.device)
    tile_bits = tuple(b for rate in record_bits(d.mode) for b in (rate,) * TILES_PER_RECORD_AXIS)
    return decode_qsrt_weight(
        unpack_qsrt_trellis_states(packed), suh, svh, rate_axis=d.rate_axis, tile_bits=tile_bits, codebook=codebook
    )


def repack_encoded_records(encoded: torch.Tensor, record_order: torch.Tensor, rate_axis: RateAxis) -> torch.Tensor:
    """Reorder complete 128-channel records of ``[K/16, N/16, 256]`` states
    (reference qsrt.py:824-853)."""

    if encoded.ndim != 3 or encoded.shape[-1] != TILE_VALUES:
        raise ValueError("encoded states must have shape [K/16, N/16, 256]")
    order = record_order.to(device=encoded.device, dtype=torch.long)
    axis = 0 if rate_axis == "k" else 1
    records = encoded.shape[axis] // TILES_PER_RECORD_AXIS
    if order.numel() != records or not torch.equal(torch.sort(order).values, torch.arange(records, device=order.device)):
        raise ValueError(f"record_order must be a permutation of {records} records")
    if axis == 0:
        r = encoded.reshape(records, TILES_PER_RECORD_AXIS, encoded.shape[1], TILE_VALUES)
        return r.index_select(0, order).reshape(encoded.shape).contiguous()
    r = encoded.reshape(encoded.shape[0], records, TILES_PER_RECORD_AXIS, TILE_VALUES)
    return r.index_select(1, order).reshape(encoded.shape).contiguous()


def align_up(value: int, alignment: int = STORAGE_ALIGNMENT) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise ValueError("value must be a non-negative integer")
    if isinstance(alignment, bool) or not isinstance(alignment, int) or alignment <= 0 or alignment & (alignment - 1):
        raise ValueError("alignment must be a positive power of two")
    return (value + alignment - 1) & -alignment


def mode_from_context_bits(context_bits: Sequence[int], geometry: Geometry = KIMI_K3) -> ModeSpec:
    """Resolve a record-rate allocation to its canonical mode
    (reference qsrt.py:239-253)."""

    bits = tuple(context_bits)
    if bits == FIXED_HIGH_RATE_RECORD_BITS:
        return high_rate_mode(geometry)
    if bits == (2,):
        return pure_k2_mode(geometry)
    if not bits or geometry.records % len(bits):
        raise ValueError("allocation contexts must divide the records")
    r = bits.count(2) * (geometry.records // len(bits))
    ModeSpec(r, "candidate", bits, geometry)
    return rate_transfer_mode(r, geometry)


# ---------------------------------------------------------------------------
# Physical pair placement (reference qsrt.py:101-141)
# ---------------------------------------------------------------------------


def _check_int(value, lo: int, hi: int, message: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or not lo <= value < hi:
        raise ValueError(message)
    return value


def pair_rotation(layer: int, expert: int, geometry: Geometry = KIMI_K3) -> int:
    """Cyclic logical-pair placement balancing physical atom slots:
    ``(5 expert + layer) mod pairs``."""

    _check_int(layer, 1, 93, "K3 MoE layer must be in 1..92")
    _check_int(expert, 0, EXPERTS_PER_LAYER, f"expert must be in 0..{EXPERTS_PER_LAYER - 1}")
    return (PAIR_ROTATION_EXPERT_MULTIPLIER * expert + layer) % (geometry.records // 2)


def logical_pair_for_slot(layer: int, expert: int, pair_slot: int, geometry: Geometry = KIMI_K3) -> int:
    pairs = geometry.records // 2
    _check_int(pair_slot, 0, pairs, f"pair_slot must be in 0..{pairs - 1}")
    return (pair_slot - pair_rotation(layer, expert, geometry)) % pairs


def physical_pair_slot(layer: int, expert: int, logical_pair: int, geometry: Geometry = KIMI_K3) -> int:
    pairs = geometry.records // 2
    _check_int(logical_pair, 0, pairs, f"logical_pair must be in 0..{pairs - 1}")
    return (logical_pair + pair_rotation(layer, expert, geometry)) % pairs


# ---------------------------------------------------------------------------
# Per-expert format codes and layer metadata sections (reference :257-491)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class ExpertFormatSpec:
    """Per-expert tier: ``None/None`` is the exact X4T tier, else the w1/w3
    (``r13``) and w2 (``r2``) mode IDs packed as one byte ``r13 << 4 | r2``."""

    r13: int | None
    r2: int | None

    def __post_init__(self) -> None:
        if (self.r13 is None) != (self.r2 is None):
            raise ValueError("r13 and r2 must both be absent or both be present")
        for name, value in (("r13", self.r13), ("r2", self.r2)):
            if value is None:
                continue
            if isinstance(value, bool) or not isinstance(value, int):
                raise TypeError(f"{name} must be an integer")
            if not 0 <= value <= 4:
                raise ValueError(f"{name} must identify R0, R1, R2, H308, or K2")
        if self.r13 is not None:
            fixed = {H308.mode_id, K2.mode_id}
            if (self.r13 in fixed or self.r2 in fixed) and self.r13 != self.r2:
                raise ValueError("H308 and K2 must be selected for both matrix rate axes")

    @classmethod
    def x4t(cls) -> "ExpertFormatSpec":
        return cls(None, None)

    @classmethod
    def compressed(cls, r13: int, r2: int | None = None) -> "ExpertFormatSpec":
        return cls(r13, r13 if r2 is None else r2)

    @property
    def is_x4t(self) -> bool:
        return self.r13 is None

    @property
    def name(self) -> str:
        if self.is_x4t:
            return "X4T"
        if self.r13 == self.r2 == H308.mode_id:
            return H308.name
        if self.r13 == self.r2 == K2.mode_id:
            return K2.name
        return f"R{self.r13}" if self.r13 == self.r2 else f"R{self.r13}/R{self.r2}"

    @property
    def code(self) -> int:
        return FORMAT_X4T if self.is_x4t else (self.r13 << 4) | self.r2

    @classmethod
    def from_code(cls, code: int) -> "ExpertFormatSpec":
        if code == FORMAT_X4T:
            return cls.x4t()
        r13, r2 = code >> 4, code & FORMAT_NIBBLE_MASK
        if r13 > 4 or r2 > 4:
            raise ValueError(f"format table contains invalid rate code 0x{code:02x}")
        return cls.compressed(r13, r2)


def resolve_expert_format(value) -> ExpertFormatSpec:
    if isinstance(value, ExpertFormatSpec):
        return value
    if isinstance(value, ModeSpec):
        return ExpertFormatSpec.compressed(value.mode_id)
    if isinstance(value, tuple):
        if len(value) != 2:
            raise ValueError("expert format tuple must be (r13, r2)")
        return ExpertFormatSpec.compressed(value[0], value[1])
    if not isinstance(value, str):
        raise TypeError("expert format must be a name, ModeSpec, ExpertFormatSpec, or pair")
    name = value.upper()
    if name == "X4T":
        return ExpertFormatSpec.x4t()
    if "/" in name:
        left, right = name.split("/", 1)
        return ExpertFormatSpec.compressed(resolve_mode(left).mode_id, resolve_mode(right).mode_id)
    return ExpertFormatSpec.compressed(resolve_mode(name).mode_id)


def pack_qsrt_format_table(formats: Sequence) -> torch.Tensor:
    """One byte per expert of the layer."""

    if len(formats) != EXPERTS_PER_LAYER:
        raise ValueError(f"format table must contain {EXPERTS_PER_LAYER} experts")
    return torch.tensor([resolve_expert_format(v).code for v in formats], dtype=torch.uint8)


def unpack_qsrt_format_table(payload: torch.Tensor) -> tuple[str, ...]:
    if payload.dtype != torch.uint8:
        raise TypeError("format table must use torch.uint8")
    if payload.ndim != 1 or payload.numel() != FORMAT_TABLE_BYTES:
        raise ValueError(f"format table must contain exactly {FORMAT_TABLE_BYTES} bytes")
    return tuple(ExpertFormatSpec.from_code(code).name for code in payload.cpu().tolist())


def pack_qsrt_format_section(formats: Sequence) -> torch.Tensor:
    """The 4 KiB on-disk format section: the table, zero padded."""

    section = torch.zeros(FORMAT_SECTION_BYTES, dtype=torch.uint8)
    section[:FORMAT_TABLE_BYTES].copy_(pack_qsrt_format_table(formats))
    return section


def unpack_qsrt_format_section(payload: torch.Tensor) -> tuple[str, ...]:
    if payload.dtype != torch.uint8:
        raise TypeError("format section must use torch.uint8")
    if payload.ndim != 1 or payload.numel() != FORMAT_SECTION_BYTES:
        raise ValueError(f"format section must contain exactly {FORMAT_SECTION_BYTES} bytes")
    if bool(torch.any(payload[FORMAT_TABLE_BYTES:] != 0)):
        raise ValueError("format section has nonzero alignment padding")
    return unpack_qsrt_format_table(payload[:FORMAT_TABLE_BYTES])


def expand_qsrt_hot_metadata(formats: Sequence) -> tuple[torch.Tensor, torch.Tensor]:
    """Format codes and int16 tier-local slots (X4T and compressed experts
    are numbered separately, in expert order)."""

    codes = pack_qsrt_format_table(formats)
    unpack_qsrt_format_table(codes)
    slots = torch.empty(EXPERTS_PER_LAYER, dtype=torch.int16)
    kept = compressed = 0
    for expert, code in enumerate(codes.tolist()):
        if code == FORMAT_X4T:
            slots[expert] = kept
            kept += 1
        else:
            slots[expert] = compressed
            compressed += 1
    return codes, slots


def pack_qsrt_shared_scale_section(w1_suh: torch.Tensor, w3_suh: torch.Tensor, w2_svh: torch.Tensor,
                                   geometry: Geometry = KIMI_K3) -> torch.Tensor:
    """The three layer-shared hidden-side FP16 vectors, zero padded to six
    4 KiB pages."""

    scales = (w1_suh, w3_suh, w2_svh)
    device = scales[0].device
    for name, scale in zip(SHARED_SCALE_ORDER, scales, strict=True):
        _validate_scale_vector(scale, geometry.latent_channels, name, device)
    shared = SHARED_SCALE_VECTORS * geometry.latent_channels * SCALE_BYTES
    section = torch.zeros(align_up(shared) if geometry != KIMI_K3 else SHARED_SCALE_SECTION_BYTES,
                          dtype=torch.uint8, device=device)
    cursor = 0
    for scale in scales:
        raw = scale.view(torch.uint8)
        section[cursor:cursor + raw.numel()].copy_(raw)
        cursor += raw.numel()
    return section


def unpack_qsrt_shared_scale_section(payload: torch.Tensor, geometry: Geometry = KIMI_K3):
    shared = SHARED_SCALE_VECTORS * geometry.latent_channels * SCALE_BYTES
    size = align_up(shared) if geometry != KIMI_K3 else SHARED_SCALE_SECTION_BYTES
    if payload.dtype != torch.uint8:
        raise TypeError("shared scale section must use torch.uint8")
    if payload.ndim != 1 or payload.numel() != size:
        raise ValueError(f"shared scale section must contain exactly {size} bytes")
    if bool(torch.any(payload[shared:] != 0)):
        raise ValueError("shared scale section has nonzero alignment padding")
    out, cursor, nbytes = [], 0, geometry.latent_channels * SCALE_BYTES
    for name in SHARED_SCALE_ORDER:
        vector = payload[cursor:cursor + nbytes].clone().view(torch.float16).contiguous()
        _validate_scale_vector(vector, geometry.latent_channels, name)
        out.append(vector)
        cursor += nbytes
    return tuple(out)


# ---------------------------------------------------------------------------
# Context groups, record orders and channel permutations (reference :564-853)
# ---------------------------------------------------------------------------


def _validate_block_contexts(block_contexts: torch.Tensor, mode: ModeSpec) -> None:
    groups = mode.geometry.intermediate_channels // CONTEXT_GROUP_CHANNELS
    if block_contexts.ndim != 1 or block_contexts.numel() != groups:
        raise ValueError(f"block_contexts must contain {groups} four-channel groups")
    if block_contexts.dtype == torch.bool or block_contexts.is_floating_point():
        raise TypeError("block_contexts must use an integer dtype")
    if int(block_contexts.min()) < 0 or int(block_contexts.max()) >= mode.context_count:
        raise ValueError("block_contexts contains an out-of-range context ID")
    counts = torch.bincount(block_contexts.to(torch.long), minlength=mode.context_count)
    if counts.tolist() != [groups // mode.context_count] * mode.context_count:
        raise ValueError("every context must have equal population")


def importance_group_order(block_contexts: torch.Tensor, mode) -> torch.Tensor:
    """Stable low-to-high context order of the four-channel groups (the LDLQ
    traversal order)."""

    spec = resolve_mode(mode)
    _validate_block_contexts(block_contexts, spec)
    return torch.argsort(block_contexts, stable=True)


def storage_group_order(block_contexts: torch.Tensor, mode) -> torch.Tensor:
    """Physical group order: records of context ``c`` interleaved with
    records of ``count - 1 - c`` so consecutive records form P24/P33 pairs."""

    spec = resolve_mode(mode)
    _validate_block_contexts(block_contexts, spec)
    if spec.mode_id in (H308.mode_id, K2.mode_id):
        return torch.argsort(block_contexts, stable=True)
    per_record = spec.geometry.record_channels // CONTEXT_GROUP_CHANNELS
    by_context = [torch.nonzero(block_contexts == ctx).flatten().reshape(-1, per_record)
                  for ctx in range(spec.context_count)]
    chunks = []
    for low in range(spec.context_count // 2):
        lo, hi = by_context[low], by_context[spec.context_count - 1 - low]
        if lo.shape != hi.shape:
            raise ValueError("paired contexts have different record populations")
        for record in range(lo.shape[0]):
            chunks.extend((lo[record], hi[record]))
    return torch.cat(chunks)


def rate_transfer_record_order(donor_records: Sequence[int], recipient_records: Sequence[int], *,
                               middle_records: Sequence[int] | None = None,
                               geometry: Geometry = KIMI_K3) -> tuple[int, ...]:
    """Low-to-high record order for an equal-rate exchange: donors first
    (K2 end), recipients reversed last (K4 end), so donor ``i`` and recipient
    ``i`` land in one physical P24 pair."""

    donors, recipients = tuple(donor_records), tuple(recipient_records)
    records = geometry.records
    if len(donors) != len(recipients):
        raise ValueError("donor and recipient record counts must match")
    if len(donors) > records // 2:
        raise ValueError(f"at most {records // 2} rate exchanges are allowed")
    selected = donors + recipients
    if any(isinstance(r, bool) or not isinstance(r, int) or not 0 <= r < records for r in selected):
        raise ValueError(f"record IDs must be integers in 0..{records - 1}")
    if len(set(selected)) != len(selected):
        raise ValueError("donor and recipient records must be unique and disjoint")
    remaining = tuple(r for r in range(records) if r not in set(selected))
    if middle_records is None:
        middle = remaining
    else:
        middle = tuple(middle_records)
        if len(middle) != len(remaining) or set(middle) != set(remaining):
            raise ValueError("middle_records must be a permutation of all unselected records")
    return donors + middle + tuple(reversed(recipients))


def relabel_block_contexts_for_record_order(block_contexts: torch.Tensor, record_order: Sequence[int],
                                            geometry: Geometry = KIMI_K3) -> torch.Tensor:
    """Relabel a one-context-per-record partition so that
    :func:`importance_group_order` visits records in ``record_order``."""

    records = geometry.records
    _validate_block_contexts(block_contexts, rate_transfer_mode(0, geometry) if geometry.records != 24
                             else R0)
    order = tuple(record_order)
    if len(order) != records:
        raise ValueError(f"record_order must contain {records} records")
    if any(isinstance(r, bool) or not isinstance(r, int) or not 0 <= r < records for r in order) or len(set(order)) != records:
        raise ValueError("record_order must be a permutation of all record IDs")
    inverse = torch.empty(records, dtype=torch.long, device=block_contexts.device)
    inverse[torch.tensor(order, dtype=torch.long, device=block_contexts.device)] = torch.arange(
        records, device=block_contexts.device)
    return inverse[block_contexts.to(torch.long)]


def _validate_permutation(permutation: torch.Tensor, length: int, name: str = "permutation") -> None:
    if permutation.ndim != 1 or permutation.numel() != length:
        raise ValueError(f"{name} must contain exactly {length} entries")
    if permutation.dtype == torch.bool or permutation.is_floating_point():
        raise TypeError(f"{name} must use an integer dtype")
    values = permutation.to(torch.long)
    if not torch.equal(torch.sort(values).values, torch.arange(length, device=values.device)):
        raise ValueError(f"{name} must be a bijection over 0..{length - 1}")


def invert_permutation(permutation: torch.Tensor) -> torch.Tensor:
    _validate_permutation(permutation, permutation.numel())
    return torch.argsort(permutation.to(torch.long))


def expand_group_order(group_order: torch.Tensor, geometry: Geometry = KIMI_K3) -> torch.Tensor:
    """Four-channel group IDs -> new-channel -> old-channel permutation."""

    groups = geometry.intermediate_channels // CONTEXT_GROUP_CHANNELS
    if group_order.ndim != 1 or group_order.numel() != groups:
        raise ValueError(f"group_order must contain {groups} groups")
    _validate_permutation(group_order, groups, "group_order")
    offsets = torch.arange(CONTEXT_GROUP_CHANNELS, device=group_order.device)
    return (group_order.to(torch.long)[:, None] * CONTEXT_GROUP_CHANNELS + offsets[None]).flatten()


def coupled_intermediate_permutation(w1: torch.Tensor, w3: torch.Tensor, w2: torch.Tensor,
                                     permutation: torch.Tensor):
    """One exact neuron permutation of an expert: ``w1[P]``, ``w3[P]``,
    ``w2[:, P]`` (``permutation[new] = old``)."""

    if w1.ndim != 2 or w3.ndim != 2 or w2.ndim != 2:
        raise ValueError("expert weights must all be two-dimensional")
    if w1.shape != w3.shape:
        raise ValueError("w1 and w3 must have identical shapes")
    intermediate, hidden = w1.shape
    if tuple(w2.shape) != (hidden, intermediate):
        raise ValueError("w2 must have shape [hidden, intermediate]")
    _validate_permutation(permutation, intermediate)
    p = permutation.to(torch.long)
    return (w1.index_select(0, p.to(w1.device)).contiguous(), w3.index_select(0, p.to(w3.device)).contiguous(),
            w2.index_select(1, p.to(w2.device)).contiguous())


def record_repack_order(source_group_order: torch.Tensor, destination_group_order: torch.Tensor,
                        geometry: Geometry = KIMI_K3) -> torch.Tensor:
    """Destination record -> source record, refusing to split a record."""

    groups = geometry.intermediate_channels // CONTEXT_GROUP_CHANNELS
    _validate_permutation(source_group_order, groups, "source_group_order")
    _validate_permutation(destination_group_order, groups, "destination_group_order")
    per_record = geometry.record_channels // CONTEXT_GROUP_CHANNELS
    src = source_group_order.cpu().reshape(-1, per_record)
    dst = destination_group_order.cpu().reshape(-1, per_record)
    lookup = {tuple(r.tolist()): i for i, r in enumerate(src)}
    if len(lookup) != geometry.records:
        raise ValueError("source order contains duplicate or malformed records")
    try:
        order = [lookup[tuple(r.tolist())] for r in dst]
    except KeyError as exc:
        raise ValueError("destination order splits or changes a source record") from exc
    return torch.tensor(order, dtype=torch.long, device=source_group_order.device)


def expand_record_order(record_order: torch.Tensor, geometry: Geometry = KIMI_K3) -> torch.Tensor:
    _validate_permutation(record_order, geometry.records, "record_order")
    offsets = torch.arange(geometry.record_channels, device=record_order.device)
    return (record_order.to(torch.long)[:, None] * geometry.record_channels + offsets[None]).flatten()


def repack_rate_axis(tensor: torch.Tensor, record_order: torch.Tensor, axis: int,
                     geometry: Geometry = KIMI_K3) -> torch.Tensor:
    """Move whole 128-channel blocks along a tensor's rate axis."""

    if tensor.ndim == 0:
        raise ValueError("cannot repack a scalar tensor")
    axis = axis % tensor.ndim
    if tensor.shape[axis] != geometry.intermediate_channels:
        raise ValueError(f"rate axis must contain exactly {geometry.intermediate_channels} channels")
    return tensor.index_select(axis, expand_record_order(record_order, geometry).to(tensor.device)).contiguous()
