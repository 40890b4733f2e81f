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
