"""Materialise and read canonical atom-major QSRT layer files (mirrors
``qsrt/pack/qsrt_atoms.py``), and decode them on the GPU.

A layer file is the 4 KiB safetensors header of :class:`QSRTLayerHeader`,
the 4 KiB per-expert format section, the six-page layer-shared scale
section, then one 4 KiB-aligned row per physical atom slot holding that
atom's bundle for every compressed expert.  A tensor-parallel shard is one
contiguous read; nothing is decoded or repacked while writing.  Beyond the
reference, :meth:`QSRTAtomLayerReader.decode_expert` turns a compressed
expert of the file back into its three weight matrices with the fused HIP
decode, so the stored layer is directly the decode kernel's input.
"""

from __future__ import annotations

import fcntl
import os
from dataclasses import dataclass
from pathlib import Path

import torch

from .qsrt import (
    EXPERTS_PER_LAYER,
    FORMAT_SECTION_BYTES,
    INTERMEDIATE_CHANNELS,
    LAYER_HEADER_BYTES,
    LATENT_CHANNELS,
    MATRIX_RATE_AXIS,
    MATRIX_TRELLIS_BYTES,
    MOE_LAYERS,
    SHARED_SCALE_SECTION_BYTES,
    ExpertFormatSpec,
    PackedQSRTTrellis,
    QSRTTrellisDescriptor,
    pack_qsrt_format_section,
    pack_qsrt_shared_scale_section,
    resolve_expert_format,
    unpack_qsrt_format_section,
    unpack_qsrt_shared_scale_section,
)
from .qsrt_storage import (
    ATOM_BUNDLE_BYTES,
    ATOM_TRELLIS_BYTES,
    ATOMS_PER_EXPERT,
    MATRIX_ATOM_SCALE_BYTES,
    MATRIX_ATOM_SCALE_OFFSETS,
    MATRIX_ATOM_TRELLIS_BYTES,
    MATRIX_ATOM_TRELLIS_OFFSETS,
    SCHEMA,
    QSRTLayerHeader,
    QSRTLayerLayout,
    pack_local_scale_atoms,
    pack_matrix_atoms,
    rotate_expert_atoms,
    unpack_local_scale_atoms,
    unpack_matrix_atoms,
    unrotate_expert_atoms,
)
from .transform_seeds import MATRICES

LAYER_PREFIX = "qsrt-layer-"
LAYER_SUFFIX = ".safetensors"


def layer_filename(layer: int) -> str:
    if isinstance(layer, bool) or not isinstance(layer, int) or not 1 <= layer <= 92:
        raise ValueError("Kimi-K3 MoE layer must lie in 1..92")
    return f"{LAYER_PREFIX}{layer:05d}{LAYER_SUFFIX}"


def candidate_layer_path(root: str | Path, layer: int) -> Path:
    return Path(root) / "candidates" / f"qsrt-layer-{layer:05d}.safetensors"


def candidate_tensor_name(layer: int, expert: int, matrix: str, part: str) -> str:
    """Tensor name of one selected candidate component in a candidate file
    (reference qsrt/pack/qsrt_candidates.py:1599-1607)."""

    if matrix not in MATRICES or part not in ("trellis", "suh", "svh"):
        raise ValueError("invalid QSRT candidate tensor component")
    return f"language_model.model.layers.{layer}.block_sparse_moe.experts.{expert}.{matrix}.qsrt_{part}"


def _flat(tensor: torch.Tensor, *, dtype: torch.dtype, values: int, name: str) -> torch.Tensor:
    out = tensor.detach().cpu().contiguous().reshape(-1)
    if out.dtype != dtype or out.numel() != values:
        raise ValueError(f"{name} must contain {values} contiguous {dtype} values, got {out.numel()} {out.dtype} values")
    if dtype != torch.int16 and not bool(torch.all(torch.isfinite(out))):
        raise ValueError(f"{name} contains non-finite values")
    return out


def _matrix_descriptor(matrix: str, mode_id: int) -> QSRTTrellisDescriptor:
    axis = MATRIX_RATE_AXIS[matrix]
    rate_tiles, orth_tiles = INTERMEDIATE_CHANNELS // 16, LATENT_CHANNELS // 16
    return QSRTTrellisDescriptor(mode_id=mode_id, rate_axis=axis,
                                 k_tiles=rate_tiles if axis == "k" else orth_tiles,
                                 n_tiles=orth_tiles if axis == "k" else rate_tiles)


def _mode_of(format_spec: ExpertFormatSpec, matrix: str) -> int:
    return format_spec.r2 if matrix == "w2" else format_spec.r13


def assemble_candidate_atoms(*, layer: int, expert: int, format_spec, tensors: dict) -> tuple[torch.Tensor, dict]:
    """One expert as physical ``[96, bundle]`` byte atoms plus its three
    layer-shared hidden-side scale vectors (reference qsrt_atoms.py:96-164).
    Moves whole packed tile paths; decodes nothing."""

    format_spec = resolve_expert_format(format_spec)
    if format_spec.is_x4t:
        raise ValueError("X4T experts do not have QSRT atoms")
    if set(tensors) != set(MATRICES):
        raise ValueError("candidate must contain w1, w3, and w2")
    logical = torch.empty((ATOMS_PER_EXPERT, ATOM_BUNDLE_BYTES), dtype=torch.uint8)
    shared: dict[str, torch.Tensor] = {}
    for matrix in MATRICES:
        parts = tensors[matrix]
        if set(parts) != {"trellis", "suh", "svh"}:
            raise ValueError(f"{matrix} candidate components are incomplete")
        trellis = _flat(parts["trellis"], dtype=torch.int16, values=MATRIX_TRELLIS_BYTES // 2, name=f"{matrix}.trellis")
        atoms = pack_matrix_atoms(PackedQSRTTrellis(_matrix_descriptor(matrix, _mode_of(format_spec, matrix)), trellis))
        t0 = MATRIX_ATOM_TRELLIS_OFFSETS[matrix]
        logical[:, t0:t0 + MATRIX_ATOM_TRELLIS_BYTES].copy_(atoms.view(torch.uint8).reshape(ATOMS_PER_EXPERT, -1))
        shared_part, local_part = ("svh", "suh") if matrix == "w2" else ("suh", "svh")
        shared[f"{matrix}.{shared_part}"] = _flat(parts[shared_part], dtype=torch.float16, values=LATENT_CHANNELS,
                                                  name=f"{matrix}.{shared_part}")
        local = _flat(parts[local_part], dtype=torch.float16, values=INTERMEDIATE_CHANNELS, name=f"{matrix}.{local_part}")
        s0 = MATRIX_ATOM_SCALE_OFFSETS[matrix]
        logical[:, s0:s0 + MATRIX_ATOM_SCALE_BYTES].copy_(
            pack_local_scale_atoms(local).view(torch.uint8).reshape(ATOMS_PER_EXPERT, -1))
    if ATOM_TRELLIS_BYTES + 3 * MATRIX_ATOM_SCALE_BYTES != ATOM_BUNDLE_BYTES:
        raise AssertionError("atom bundle accounting drifted")
    return rotate_expert_atoms(logical, layer, expert), shared


@dataclass(frozen=True)
class QSRTAtomLayerSpec:
    """Which experts of a layer are compressed (atoms) and which are X4T."""

    layer: int
    formats: tuple
    compressed: tuple[int, ...]
    x4t: tuple[int, ...]

    def __post_init__(self) -> None:
        if self.layer not in MOE_LAYERS:
            raise ValueError("atom layer must be a Kimi-K3 MoE layer")
        if len(self.formats) != EXPERTS_PER_LAYER:
            raise ValueError(f"atom layer must describe {EXPERTS_PER_LAYER} experts")
        specs = [resolve_expert_format(f) for f in self.formats]
        if (self.compressed != tuple(e for e, f in enumerate(specs) if not f.is_x4t)
                or self.x4t != tuple(e for e, f in enumerate(specs) if f.is_x4t)):
            raise ValueError("atom layer tiers disagree with its format table")

    @property
    def layout(self) -> QSRTLayerLayout:
        return QSRTLayerLayout(len(self.compressed), len(self.x4t))


def _pwrite_exact(fd: int, payload, offset: int) -> None:
    data = payload if isinstance(payload, bytes) else payload.contiguous().numpy().tobytes()
    done = 0
    while done < len(data):
        n = os.pwrite(fd, data[done:], offset + done)
        if n <= 0:
            raise OSError("short QSRT atom write")
        done += n


def materialize_atom_layer(candidate_root: str | Path, destination: str | Path, spec: QSRTAtomLayerSpec, *,
                           discard_partial: bool = False) -> dict:
    """Write one canonical atom layer from a candidate file, atomically (a
    locked ``.partial`` file renamed into place) and one expert at a time
    (reference qsrt_atoms.py:202-295)."""

    from safetensors import safe_open

    source = candidate_layer_path(candidate_root, spec.layer)
    if not source.is_file():
        raise FileNotFoundError(source)
    destination = Path(destination)
    destination.parent.mkdir(parents=True, exist_ok=True)
    if destination.exists():
        raise FileExistsError(destination)
    partial = destination.with_name(f".{destination.name}.partial")
    if partial.exists():
        if not discard_partial:
            raise FileExistsError(partial)
        partial.unlink()
    layout = spec.layout
    fd = os.open(partial, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o644)
    try:
        fcntl.flock(fd, fcntl.LOCK_EX | fcntl.LOCK_NB)
        if hasattr(os, "posix_fallocate"):
            os.posix_fallocate(fd, 0, layout.disk_bytes)
        else:
            os.ftruncate(fd, layout.disk_bytes)
        _pwrite_exact(fd, QSRTLayerHeader(spec.layer, layout).to_bytes(), 0)
        _pwrite_exact(fd, pack_qsrt_format_section(spec.formats), LAYER_HEADER_BYTES)
        reference: dict[str, torch.Tensor] = {}
        with safe_open(str(source), framework="pt", device="cpu") as handle:
            for slot, expert in enumerate(spec.compressed):
                tensors = {m: {p: handle.get_tensor(candidate_tensor_name(spec.layer, expert, m, p))
                               for p in ("trellis", "suh", "svh")} for m in MATRICES}
                atoms, shared = assemble_candidate_atoms(layer=spec.layer, expert=expert,
                                                         format_spec=spec.formats[expert], tensors=tensors)
                for name, value in shared.items():
                    if not torch.equal(reference.setdefault(name, value.clone()), value):
                        raise ValueError(f"layer-shared transform {name} drifted")
                for physical in range(ATOMS_PER_EXPERT):
                    _pwrite_exact(fd, atoms[physical], layout.atom_bundle_offset(physical, slot))
        if spec.compressed:
            if set(reference) != {"w1.suh", "w3.suh", "w2.svh"}:
                raise AssertionError("shared transform inventory did not close")
            section = pack_qsrt_shared_scale_section(reference["w1.suh"], reference["w3.suh"], reference["w2.svh"])
        else:
            section = torch.zeros(SHARED_SCALE_SECTION_BYTES, dtype=torch.uint8)
        _pwrite_exact(fd, section, LAYER_HEADER_BYTES + FORMAT_SECTION_BYTES)
        os.fsync(fd)
    except BaseException:
        os.close(fd)
        partial.unlink(missing_ok=True)
        raise
    os.close(fd)
    partial.replace(destination)
    return {"schema": SCHEMA, "layer": spec.layer, "compressed_experts": len(spec.compressed),
            "x4t_experts": len(spec.x4t), "disk_bytes": layout.disk_bytes}


class QSRTAtomLayerReader:
    """Bounded reader of one atom layer file; the serving read is one
    contiguous shard extent (reference qsrt_atoms.py:298-455)."""

    def __init__(self, path: str | Path) -> None:
        self.path = Path(path)
        self._fd = os.open(self.path, os.O_RDONLY)
        try:
            self.header = QSRTLayerHeader.from_bytes(os.pread(self._fd, LAYER_HEADER_BYTES, 0))
            if self.path.stat().st_size != self.header.layout.disk_bytes:
                raise ValueError("QSRT atom layer size disagrees with its header")
            raw = os.pread(self._fd, FORMAT_SECTION_BYTES, LAYER_HEADER_BYTES)
            self.formats = unpack_qsrt_format_section(torch.frombuffer(bytearray(raw), dtype=torch.uint8))
            self.format_specs = tuple(resolve_expert_format(f) for f in self.formats)
            self.compressed = tuple(e for e, f in enumerate(self.format_specs) if not f.is_x4t)
            self.x4t = tuple(e for e, f in enumerate(self.format_specs) if f.is_x4t)
            if (len(self.compressed), len(self.x4t)) != (self.header.layout.compressed_experts,
                                                         self.header.layout.x4t_experts):
                raise ValueError("QSRT format section disagrees with the layer header")
            self._slots = {e: s for s, e in enumerate(self.compressed)}
            raw = os.pread(self._fd, SHARED_SCALE_SECTION_BYTES, LAYER_HEADER_BYTES + FORMAT_SECTION_BYTES)
            self.shared_scales = unpack_qsrt_shared_scale_section(torch.frombuffer(bytearray(raw), dtype=torch.uint8))
        except BaseException:
            os.close(self._fd)
            raise

    def close(self) -> None:
        if self._fd >= 0:
            os.close(self._fd)
            self._fd = -1

    def __enter__(self) -> "QSRTAtomLayerReader":
        return self

    def __exit__(self, *_exc) -> None:
        self.close()

    def _open(self) -> int:
        if self._fd < 0:
            raise RuntimeError("QSRT atom reader is closed")
        return self._fd

    def read_shard(self, shard_count: int, shard_index: int, *, require_equal: bool = False) -> torch.Tensor:
        """One contiguous whole-atom shard, de-padded:
        ``[atom slots, compressed experts, bundle]`` bytes."""

        fd = self._open()
        layout = self.header.layout
        extent = layout.shard_extent(shard_count, shard_index, require_equal=require_equal)
        raw = os.pread(fd, extent.extent_bytes, extent.offset_bytes)
        if len(raw) != extent.extent_bytes:
            raise ValueError("short QSRT atom extent")
        rows = torch.frombuffer(bytearray(raw), dtype=torch.uint8).reshape(extent.atom_slots,
                                                                           layout.atom_slot_stride_bytes)
        return rows[:, :layout.atom_slot_payload_bytes].reshape(extent.atom_slots, layout.compressed_experts,
                                                                 ATOM_BUNDLE_BYTES).contiguous()

    def read_expert_atoms(self, compressed_slot: int) -> torch.Tensor:
        """One expert's physical atoms (validation, not serving)."""

        fd = self._open()
        out = torch.empty((ATOMS_PER_EXPERT, ATOM_BUNDLE_BYTES), dtype=torch.uint8)
        for slot in range(ATOMS_PER_EXPERT):
            raw = os.pread(fd, ATOM_BUNDLE_BYTES, self.header.layout.atom_bundle_offset(slot, compressed_slot))
            if len(raw) != ATOM_BUNDLE_BYTES:
                raise ValueError("short QSRT expert atom")
            out[slot].copy_(torch.frombuffer(bytearray(raw), dtype=torch.uint8))
        return out

    def read_compressed_matrix(self, expert: int, matrix: str) -> dict[str, torch.Tensor]:
        """One matrix's full candidate payload and scales, rebuilt from the
        expert's atoms."""

        try:
            slot = self._slots[expert]
        except KeyError as exc:
            raise ValueError(f"expert {expert} is not in the QSRT tier") from exc
        if matrix not in MATRICES:
            raise ValueError(f"unknown expert matrix: {matrix}")
        logical = unrotate_expert_atoms(self.read_expert_atoms(slot), self.header.layer, expert)
        t0 = MATRIX_ATOM_TRELLIS_OFFSETS[matrix]
        trellis_atoms = logical[:, t0:t0 + MATRIX_ATOM_TRELLIS_BYTES].contiguous().view(torch.int16)
        descriptor = _matrix_descriptor(matrix, _mode_of(self.format_specs[expert], matrix))
        trellis = unpack_matrix_atoms(trellis_atoms.contiguous(), descriptor).payload
        s0 = MATRIX_ATOM_SCALE_OFFSETS[matrix]
        local = unpack_local_scale_atoms(logical[:, s0:s0 + MATRIX_ATOM_SCALE_BYTES].contiguous().view(torch.float16))
        w1_suh, w3_suh, w2_svh = self.shared_scales
        suh, svh = {"w1": (w1_suh, local), "w3": (w3_suh, local), "w2": (local, w2_svh)}[matrix]
        return {"trellis": trellis, "suh": suh.clone().contiguous(), "svh": svh.clone().contiguous()}

    def decode_expert(self, expert: int, luts_by_bits: dict, *, device="cuda:0",
                      out_dtype=torch.bfloat16) -> dict[str, torch.Tensor]:
        """The three ``[K, N]`` EXL-oriented weights of a compressed expert,
        decoded from the file by the fused HIP decode (one launch per rate)."""

        from .decode import decode_packed

        device = torch.device(device)
        out = {}
        for matrix in MATRICES:
            parts = self.read_compressed_matrix(expert, matrix)
            descriptor = _matrix_descriptor(matrix, _mode_of(self.format_specs[expert], matrix))
            packed = PackedQSRTTrellis(descriptor, parts["trellis"].to(device))
            out[matrix] = decode_packed(packed, parts["suh"].to(device), parts["svh"].to(device),
                                        {b: lut.to(device) for b, lut in luts_by_bits.items()}, out_dtype=out_dtype)
        return out


__all__ = [
    "QSRTAtomLayerReader",
    "QSRTAtomLayerSpec",
    "assemble_candidate_atoms",
    "candidate_layer_path",
    "candidate_tensor_name",
    "layer_filename",
    "materialize_atom_layer",
]
