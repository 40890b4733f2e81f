"""Matrix and expert encode callers (mirrors ``qsrt/pack/qsrt_encoder.py``).

These sit one layer above the encoder backend: plan the low-to-high LDLQ
traversal and the stored P24/P33 record order of one matrix, build the
backend's ``quant_args``, run ``quantize_qsrt`` (or the batched
``quantize_qsrt_batch`` over rate candidates and experts), repack whole
128-channel records into the stored order, pack the payload, and then prove
closure independently: every packed edge and state unpacks to the encoded
path, the stored payload decodes to the encoder's own reconstruction, and the
payload holds exactly the mode's bit budget.

Differences from the reference that a caller can see:

* the geometry is taken from the inputs (``block_contexts`` covers the
  intermediate axis in four-channel groups), so the BASELINE shapes other than
  Kimi-K3 encode through the same code; Kimi-K3 inputs get the Kimi schema;
* the default quantizer module is this package's backend (the reference loads
  an external ExLlamaV3 checkout and installs its tile op into it).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Literal, Mapping

import torch

from . import exl3_encoder_backend as _backend
from .exl3_reference import CODEBOOK_SQG_CHEB_NORMAL_E4M3, CODEBOOK_SQG_NORMAL_E4M3, CODEBOOK_SQG_XOR_CHEB_T12
from .exl3_reference import QSRT_CODEBOOKS, decode_qsrt_weight
from .ldlq import SIGMA_REG, make_shared_h
from .qsrt import (
    CONTEXT_GROUP_CHANNELS,
    GENERIC_SCHEMA,
    KIMI_K3,
    SCHEMA,
    TILE_CHANNELS,
    ExpertFormatSpec,
    Geometry,
    ModeSpec,
    PackedQSRTTrellis,
    RateAxis,
    decode_qsrt_exl3_weight,
    expand_group_order,
    importance_group_order,
    matrix_rate_axis,
    pack_qsrt_trellis,
    record_bits,
    record_repack_order,
    repack_encoded_records,
    repack_rate_axis,
    resolve_expert_format,
    resolve_mode,
    storage_group_order,
    unpack_qsrt_trellis_edges,
    unpack_qsrt_trellis_states,
)
from .sqg_e4m3 import sqg_cheb_normal_e4m3_bytes, sqg_xor_cheb_t12_bytes
from .transform_seeds import MATRICES, QSRTTransformSeeds, default_qsrt_transform_seeds

Layout = Literal["importance_ordered", "qsrt_pair_prefix_reuse"]
MIXED_LAYOUTS: tuple[Layout, ...] = ("importance_ordered", "qsrt_pair_prefix_reuse")
# R0..R2 differ only in the two least and two most important records: the
# prefix-reuse traversal keeps those four records at the low-K end of LDLQ.
QSRT_PREFIX_REUSE_MAX_MODE = 2


def comparison_metrics(reference: torch.Tensor, actual: torch.Tensor) -> dict[str, float]:
    """Relative L2, max-abs and cosine of ``actual`` against ``reference``
    (reference qsrt/tp_simulator.py:128-149), with one host transfer."""

    reference, actual = reference.float(), actual.float()
    delta = actual - reference
    denominator = reference.norm().clamp_min(torch.finfo(torch.float32).tiny)
    cosine = torch.nn.functional.cosine_similarity(reference.reshape(1, -1), actual.reshape(1, -1))
    values = torch.stack((delta.norm() / denominator, delta.abs().max(), cosine.reshape(()))).cpu()
    return {"relative_l2": float(values[0]), "max_abs": float(values[1]), "cosine": float(values[2])}


def geometry_for(block_contexts: torch.Tensor, latent_channels: int | None = None) -> Geometry:
    """The expert geometry implied by a four-channel context map (Kimi-K3 when
    it matches, else a generic geometry with the given latent width)."""

    intermediate = int(block_contexts.numel()) * CONTEXT_GROUP_CHANNELS
    if intermediate == KIMI_K3.intermediate_channels and latent_channels in (None, KIMI_K3.latent_channels):
        return KIMI_K3
    if latent_channels is None:
        raise ValueError("a non-Kimi context map needs the latent width")
    return Geometry(intermediate, int(latent_channels))


def _schema_for(geometry: Geometry) -> str:
    return SCHEMA if geometry == KIMI_K3 else GENERIC_SCHEMA


def _qsrt_pair_prefix_reuse_group_order(block_contexts: torch.Tensor, spec: ModeSpec) -> torch.Tensor:
    """Importance order with the nested donor/recipient record pairs first
    (reference qsrt_encoder.py:94-125): LDLQ walks records backwards, so the
    K3 middle is encoded first and shared by every R0..R2 candidate."""

    if spec.context_count != spec.geometry.records:
        raise ValueError("qsrt_pair_prefix_reuse requires one context per 128-channel record")
    ordered = importance_group_order(block_contexts, spec).reshape(spec.context_count, -1)
    r = min(QSRT_PREFIX_REUSE_MAX_MODE, spec.context_count // 2)
    paired = tuple(rec for t in range(r, 0, -1) for rec in (t - 1, spec.context_count - t))
    middle = tuple(range(r, spec.context_count - r))
    index = torch.tensor(paired + middle, dtype=torch.long, device=ordered.device)
    return ordered.index_select(0, index).flatten()


@dataclass(frozen=True)
class QSRTMatrixPlan:
    """Layout plan of one matrix encode: ``encoder_permutation`` is the LDLQ
    order, ``physical_permutation`` the stored P24/P33 order, and
    ``record_repack_order`` maps the former onto the latter in whole records."""

    matrix: str
    mode: ModeSpec
    rate_axis: RateAxis
    layout: Layout
    encoder_permutation: torch.Tensor
    physical_permutation: torch.Tensor
    record_repack_order: torch.Tensor
    encoder_tile_bits: tuple[int, ...]
    physical_tile_bits: tuple[int, ...]
    encoder_pair_bpw: tuple[float, ...]
    physical_pair_bpw: tuple[float, ...]

    @property
    def geometry(self) -> Geometry:
        return self.mode.geometry


def _pair_bpw(tile_bits: tuple[int, ...], geometry: Geometry) -> tuple[float, ...]:
    pair_tiles = 2 * geometry.tiles_per_record_axis
    if len(tile_bits) != geometry.intermediate_channels // TILE_CHANNELS:
        raise ValueError("rate map must cover the intermediate tile axis")
    return tuple(sum(tile_bits[b:b + pair_tiles]) / pair_tiles for b in range(0, len(tile_bits), pair_tiles))


def _tile_bits(contexts: torch.Tensor, permutation: torch.Tensor, spec: ModeSpec, what: str) -> tuple[int, ...]:
    tiles = contexts.index_select(0, permutation).reshape(-1, TILE_CHANNELS)
    if not bool(torch.all(tiles == tiles[:, :1])):
        raise ValueError(f"{what} permutation does not produce homogeneous EXL tiles")
    return tuple(spec.context_bits[int(c)] for c in tiles[:, 0].cpu().tolist())


def plan_qsrt_matrix(block_contexts: torch.Tensor, mode: ModeSpec | str | int, *, matrix: str,
                     layout: Layout = "importance_ordered", geometry: Geometry | None = None) -> QSRTMatrixPlan:
    """Plan one rate-shifted traversal and its paired-record repack
    (reference qsrt_encoder.py:300-365)."""

    geometry = geometry or geometry_for(block_contexts)
    spec = resolve_mode(mode, geometry)
    rate_axis = matrix_rate_axis(matrix)
    if layout == "importance_ordered":
        encoder_groups = importance_group_order(block_contexts, spec)
    elif layout == "qsrt_pair_prefix_reuse":
        if spec.mode_id > QSRT_PREFIX_REUSE_MAX_MODE:
            raise ValueError("qsrt_pair_prefix_reuse supports only R0 through R2")
        encoder_groups = _qsrt_pair_prefix_reuse_group_order(block_contexts, spec)
    else:
        raise ValueError(f"unsupported context layout: {layout}")
    physical_groups = storage_group_order(block_contexts, spec)
    encoder_perm = expand_group_order(encoder_groups, geometry)
    physical_perm = expand_group_order(physical_groups, geometry)
    repack = record_repack_order(encoder_groups, physical_groups, geometry)
    channel_contexts = block_contexts.to(torch.long).repeat_interleave(CONTEXT_GROUP_CHANNELS)
    encoder_bits = _tile_bits(channel_contexts, encoder_perm, spec, "context")
    physical_bits = _tile_bits(channel_contexts, physical_perm, spec, "physical")
    expected = tuple(b for b in record_bits(spec) for _ in range(geometry.tiles_per_record_axis))
    if physical_bits != expected:
        raise ValueError("physical contexts do not match the QSRT mode schedule")
    return QSRTMatrixPlan(
        matrix=matrix, mode=spec, rate_axis=rate_axis, layout=layout, encoder_permutation=encoder_perm,
        physical_permutation=physical_perm, record_repack_order=repack, encoder_tile_bits=encoder_bits,
        physical_tile_bits=physical_bits, encoder_pair_bpw=_pair_bpw(encoder_bits, geometry),
        physical_pair_bpw=_pair_bpw(physical_bits, geometry),
    )


@dataclass(frozen=True)
class QSRTMatrixEncoding:
    """One closed stored payload and its canonical-order reconstruction."""

    reconstruction: torch.Tensor
    tensors: dict[str, torch.Tensor]
    packed: PackedQSRTTrellis
    plan: QSRTMatrixPlan
    coding: dict[str, object]


@dataclass
class QSRTMatrixCandidate:
    """Unpacked rate candidate (canonical reconstruction, encoder-order
    states); packing and closure are deferred to
    :func:`finalize_qsrt_matrix_candidate`."""

    reconstruction: torch.Tensor
    encoded: torch.Tensor
    tensors: dict[str, torch.Tensor]
    plan: QSRTMatrixPlan
    proxy: float
    transform_seeds: QSRTTransformSeeds
    global_scale: float = 1.0


@dataclass
class QSRTExpertEncoding:
    """Three matrices encoded under one physical neuron permutation."""

    format: ExpertFormatSpec
    matrices: dict[str, QSRTMatrixEncoding]
    physical_permutation: torch.Tensor
    coding: dict[str, object] = field(default_factory=dict)


def _shapes(matrix: str, geometry: Geometry) -> tuple[tuple[int, int], tuple[int, int]]:
    inter, latent = geometry.intermediate_channels, geometry.latent_channels
    if matrix == "w2":
        return (latent, inter), (inter, inter)
    return (inter, latent), (latent, latent)


def _validate_source_and_hessian(source: torch.Tensor, hessian: torch.Tensor, matrix: str,
                                 geometry: Geometry) -> None:
    """Shape, dtype and finiteness checks (reference qsrt_encoder.py:368-394)."""

    if matrix not in MATRICES:
        raise ValueError(f"unknown expert matrix: {matrix}")
    want_source, want_hessian = _shapes(matrix, geometry)
    if source.ndim != 2 or tuple(source.shape) != want_source:
        raise ValueError(f"{matrix} source has shape {tuple(source.shape)}, expected {want_source}")
    if hessian.ndim != 2 or tuple(hessian.shape) != want_hessian:
        raise ValueError(f"{matrix} Hessian has shape {tuple(hessian.shape)}, expected {want_hessian}")
    if source.dtype != torch.float32:
        raise TypeError("QSRT source must use torch.float32")
    if not bool(torch.all(torch.isfinite(source))):
        raise ValueError("QSRT source contains non-finite values")
    if not bool(torch.all(torch.isfinite(hessian))):
        raise ValueError("QSRT Hessian contains non-finite values")


def _source_geometry(block_contexts: torch.Tensor, source: torch.Tensor, matrix: str) -> Geometry:
    latent = source.shape[0] if matrix == "w2" else source.shape[1]
    return geometry_for(block_contexts, int(latent))


def _load_quantizer_module(codebook: str = CODEBOOK_SQG_XOR_CHEB_T12):
    if codebook not in QSRT_CODEBOOKS:
        raise ValueError(f"unsupported QSRT codebook: {codebook!r}")
    return _backend


def make_qsrt_shared_h(block_contexts: torch.Tensor, *, matrix: str, mode: ModeSpec | str | int,
                       hessian: torch.Tensor, device: torch.device, layout: Layout = "importance_ordered",
                       geometry: Geometry | None = None) -> dict[str, object]:
    """One reusable Hessian preparation for every rate candidate of a matrix,
    signed with the matrix, layout, neuron order and source Hessian so that
    reuse with anything else fails (reference qsrt_encoder.py:411-460)."""

    if device.type != "cuda":
        raise ValueError("native QSRT quantization requires a GPU device")
    if matrix not in MATRICES:
        raise ValueError(f"unknown expert matrix: {matrix}")
    geometry = geometry or geometry_for(block_contexts, hessian.shape[0] if matrix != "w2" else None)
    _, want = _shapes(matrix, geometry)
    if hessian.ndim != 2 or tuple(hessian.shape) != want:
        raise ValueError(f"{matrix} Hessian has shape {tuple(hessian.shape)}, expected {want}")
    if not bool(torch.all(torch.isfinite(hessian))):
        raise ValueError("QSRT Hessian contains non-finite values")
    contexts = block_contexts.to(device=device, dtype=torch.long)
    plan = plan_qsrt_matrix(contexts, mode, matrix=matrix, layout=layout, geometry=geometry)
    encoder_hessian = hessian
    if matrix == "w2":
        p = plan.encoder_permutation.to(hessian.device)
        encoder_hessian = hessian.index_select(0, p).index_select(1, p)
    shared = make_shared_h(want[0], device, encoder_hessian)
    shared["_qsrt_matrix"] = matrix
    shared["_qsrt_layout"] = layout
    shared["_qsrt_permutation"] = plan.encoder_permutation.detach().cpu().contiguous()
    shared["_qsrt_source_hessian_ptr"] = int(hessian.data_ptr())
    return shared


def _validate_qsrt_shared_h(shared_h: dict, *, matrix: str, layout: Layout, plan: QSRTMatrixPlan,
                            hessian: torch.Tensor, device: torch.device) -> None:
    if shared_h.get("_qsrt_matrix") != matrix:
        raise ValueError("QSRT shared Hessian belongs to another matrix")
    if shared_h.get("_qsrt_layout") != layout:
        raise ValueError("QSRT shared Hessian belongs to another layout")
    if shared_h.get("_qsrt_source_hessian_ptr") != int(hessian.data_ptr()):
        raise ValueError("QSRT shared Hessian belongs to another source Hessian")
    perm = shared_h.get("_qsrt_permutation")
    if not isinstance(perm, torch.Tensor) or not torch.equal(perm, plan.encoder_permutation.detach().cpu()):
        raise ValueError("QSRT shared Hessian belongs to another neuron order")
    error_h = shared_h.get("error_H")
    n = hessian.shape[0]
    if not isinstance(error_h, torch.Tensor) or tuple(error_h.shape) != (n, n) or error_h.device != device:
        raise ValueError("QSRT shared Hessian has an invalid error_H tensor")


def _qsrt_quant_args(plan: QSRTMatrixPlan, *, matrix: str, layer: int, device: torch.device,
                     shared_scale_scope: object | None, codebook: str = CODEBOOK_SQG_XOR_CHEB_T12,
                     sqg_e4m3_luts_by_bits: Mapping[int, torch.Tensor | None] | None = None,
                     ldlq_tf32: bool = False, tailbite_context: int = 128,
                     transform_seeds: QSRTTransformSeeds | None = None,
                     g_scale_override: float | None = None) -> dict[str, object]:
    """Backend arguments of one matrix encode (reference qsrt_encoder.py:493-561):
    K3 regularisation and scale search, the heterogeneous tile map, seeds,
    per-rate codebooks and the layer-shared ``su`` scope of w1/w3."""

    if codebook not in QSRT_CODEBOOKS:
        raise ValueError(f"unsupported QSRT codebook {codebook!r}; expected one of {QSRT_CODEBOOKS}")
    seeds = transform_seeds or default_qsrt_transform_seeds(layer, matrix)
    quant_args: dict[str, object] = {
        "K": 3,
        "mixed_rate_axis": plan.rate_axis,
        "mixed_tile_bits": plan.encoder_tile_bits,
        "seed": seeds.input_sign,
        "sv_seed": seeds.output_sign,
        "sigma_reg": SIGMA_REG,
        "devices": [str(device)],
        "device_ratios": None,
        "apply_out_scales": False,
        "ldlq_tf32": bool(ldlq_tf32),
        "tailbite_context": int(tailbite_context),
    }
    if sqg_e4m3_luts_by_bits is None and codebook == CODEBOOK_SQG_NORMAL_E4M3:
        quant_args["sqg_e4m3_mode"] = "normal"
    else:
        if sqg_e4m3_luts_by_bits is None:
            build = sqg_xor_cheb_t12_bytes if codebook == CODEBOOK_SQG_XOR_CHEB_T12 else sqg_cheb_normal_e4m3_bytes
            if codebook not in (CODEBOOK_SQG_XOR_CHEB_T12, CODEBOOK_SQG_CHEB_NORMAL_E4M3):
                raise AssertionError("QSRT codebook dispatch is incomplete")
            sqg_e4m3_luts_by_bits = {bits: build(bits) for bits in (2, 3, 4)}
        if set(sqg_e4m3_luts_by_bits) != {2, 3, 4}:
            raise ValueError("rate-specific SQG LUTs must define K2, K3, and K4")
        quant_args["sqg_e4m3_luts_by_bits"] = dict(sqg_e4m3_luts_by_bits)
    if matrix in ("w1", "w3"):
        quant_args["shared_input_scales_key"] = (shared_scale_scope, matrix)
        quant_args["g_scale_into_sv"] = True
    if g_scale_override is not None:
        if (isinstance(g_scale_override, bool) or not isinstance(g_scale_override, (int, float))
                or not math.isfinite(float(g_scale_override)) or float(g_scale_override) <= 0.0):
            raise ValueError("g_scale_override must be positive and finite")
        quant_args["g_scale_override"] = float(g_scale_override)
    return quant_args


def _encoder_weight(source: torch.Tensor, hessian: torch.Tensor, plan: QSRTMatrixPlan):
    """EXL-oriented ``[in, out]`` weight in encoder order and its Hessian."""

    p = plan.encoder_permutation
    if plan.matrix == "w2":
        hp = p.to(hessian.device)
        return source.index_select(1, p).T.contiguous(), hessian.index_select(0, hp).index_select(1, hp)
    return source.index_select(0, p).T.contiguous(), hessian


def _closure_mask(plan: QSRTMatrixPlan, device: torch.device) -> torch.Tensor:
    bits = torch.tensor(plan.physical_tile_bits, device=device, dtype=torch.int64)
    masks = (1 << bits) - 1
    return masks[:, None, None] if plan.rate_axis == "k" else masks[None, :, None]


def _check_closure(packed: PackedQSRTTrellis, physical: torch.Tensor, plan: QSRTMatrixPlan, layer: int) -> torch.Tensor:
    """Unpack edges and states of the stored payload and require both to
    equal the encoded path; returns the decoded states."""

    edges = unpack_qsrt_trellis_edges(packed)
    edge_ok = torch.all(edges.to(torch.int64) == (physical.to(torch.int64) & _closure_mask(plan, physical.device)))
    states = unpack_qsrt_trellis_states(packed)
    state_ok = torch.all(states == physical.to(torch.int16))
    e_ok, s_ok = torch.stack((edge_ok, state_ok)).cpu().tolist()
    where = f"layer {layer} {plan.matrix} {plan.mode.name} ({plan.rate_axis}-rate, {plan.layout})"
    if not e_ok:
        raise ValueError(f"QSRT reference edge unpack failed closure for {where}")
    if not s_ok:
        mismatch = states != physical.to(torch.int16)
        first = tuple(int(v) for v in torch.nonzero(mismatch, as_tuple=False)[0].cpu().tolist())
        raise ValueError(f"QSRT state reconstruction failed exact closure for {where}: "
                         f"{int(mismatch.sum())} states differ; first at {first}, "
                         f"encoded={int(physical[first])}, decoded={int(states[first])}")
    return states


def _repack_scales(tensors: dict[str, torch.Tensor], plan: QSRTMatrixPlan) -> dict[str, torch.Tensor]:
    out = dict(tensors)
    name = "suh" if plan.rate_axis == "k" else "svh"
    out[name] = repack_rate_axis(out[name], plan.record_repack_order, 0, plan.geometry)
    return {k: v.contiguous() for k, v in out.items()}


def _place(reconstruction: torch.Tensor, decoded_physical: torch.Tensor, plan: QSRTMatrixPlan) -> None:
    if plan.matrix == "w2":
        reconstruction[:, plan.physical_permutation] = decoded_physical.T
    else:
        reconstruction[plan.physical_permutation] = decoded_physical.T


def _bit_accounting(tensors: dict[str, torch.Tensor], plan: QSRTMatrixPlan, weights: int) -> tuple[int, int]:
    index_bits = tensors["trellis"].numel() * tensors["trellis"].element_size() * 8
    scale_bits = sum(tensors[n].numel() * tensors[n].element_size() * 8 for n in ("suh", "svh"))
    if index_bits != weights * sum(plan.mode.context_bits) // len(plan.mode.context_bits):
        raise ValueError("QSRT payload does not match its fixed record-rate schedule")
    return index_bits, scale_bits


def _coding(plan: QSRTMatrixPlan, packed: PackedQSRTTrellis, tensors: dict, *, proxy: float, index_bits: int,
            scale_bits: int, codebook: str, tailbite_context: int, seeds: QSRTTransformSeeds,
            stored_vs_encoder: dict) -> dict[str, object]:
    return {
        "proxy": float(proxy),
        "scale_bits": scale_bits,
        "index_bits": index_bits,
        "matrix": plan.matrix,
        "codebook": codebook,
        "tailbite_context": int(tailbite_context),
        "mode": plan.mode.name,
        "mode_id": plan.mode.mode_id,
        "rate_axis": plan.rate_axis,
        "layout": plan.layout,
        "encoder_pair_trellis_bpw": list(plan.encoder_pair_bpw),
        "stored_pair_trellis_bpw": list(plan.physical_pair_bpw),
        "postpack_moves_complete_128_channel_records": True,
        "reference_edge_roundtrip": True,
        "reference_state_roundtrip": True,
        "stored_decode_vs_encoder": stored_vs_encoder,
        "trellis_descriptor": packed.descriptor.to_manifest(),
        "permutation_is_128_context_aligned": True,
        "scale_tensor_shapes": {n: list(tensors[n].shape) for n in ("suh", "svh")},
        "shared_hidden_scale_tensor": "svh" if plan.matrix == "w2" else "suh",
        "expert_local_intermediate_scale_tensor": "suh" if plan.matrix == "w2" else "svh",
        "transform_seeds": {"input_sign": seeds.input_sign, "output_sign": seeds.output_sign},
    }


def quantize_qsrt_matrix(source: torch.Tensor, block_contexts: torch.Tensor, *, matrix: str,
                         mode: ModeSpec | str | int, hessian: torch.Tensor, layer: int, device: torch.device,
                         layout: Layout = "importance_ordered", quantizer_module=None,
                         shared_scale_scope: object | None = None, shared_h_data: dict | None = None,
                         logical_trellis_schema: str | None = None, codebook: str = CODEBOOK_SQG_XOR_CHEB_T12,
                         ldlq_tf32: bool = False, tailbite_context: int = 128,
                         transform_seeds: QSRTTransformSeeds | None = None) -> QSRTMatrixEncoding:
    """Dense-H heterogeneous LDLQ of one matrix, closed into its stored
    payload (reference qsrt_encoder.py:1426-1661).  ``shared_scale_scope`` is
    required for w1/w3, whose hidden ``suh`` is stored once per layer."""

    if not 1 <= layer <= 92:
        raise ValueError("Kimi-K3 MoE layer must be in 1..92")
    if device.type != "cuda":
        raise ValueError("native QSRT quantization requires a GPU device")
    if source.device != device:
        raise ValueError(f"QSRT source must be resident on {device}, got {source.device}")
    geometry = _source_geometry(block_contexts, source, matrix)
    _validate_source_and_hessian(source, hessian, matrix, geometry)
    if matrix in ("w1", "w3") and shared_scale_scope is None:
        raise ValueError(f"{matrix} requires a shared_scale_scope for layer-shared suh")
    if shared_scale_scope is not None:
        try:
            hash(shared_scale_scope)
        except TypeError as exc:
            raise TypeError("shared_scale_scope must be hashable") from exc
    schema = logical_trellis_schema or _schema_for(geometry)

    contexts = block_contexts.to(device=source.device, dtype=torch.long)
    plan = plan_qsrt_matrix(contexts, mode, matrix=matrix, layout=layout, geometry=geometry)
    weight, encoder_hessian = _encoder_weight(source, hessian, plan)
    if shared_h_data is None:
        shared_h = make_shared_h(weight.shape[0], device, encoder_hessian)
    else:
        _validate_qsrt_shared_h(shared_h_data, matrix=matrix, layout=layout, plan=plan, hessian=hessian,
                                device=device)
        shared_h = shared_h_data
    seeds = transform_seeds or default_qsrt_transform_seeds(layer, matrix)
    quant_args = _qsrt_quant_args(plan, matrix=matrix, layer=layer, device=device,
                                  shared_scale_scope=shared_scale_scope, codebook=codebook, ldlq_tf32=ldlq_tf32,
                                  tailbite_context=tailbite_context, transform_seeds=seeds)

    holder: dict[str, PackedQSRTTrellis] = {}

    def pack_qsrt(encoded: torch.Tensor, _quant_args: dict) -> torch.Tensor:
        physical = repack_encoded_records(encoded, plan.record_repack_order, plan.rate_axis)
        packed = pack_qsrt_trellis(physical, plan.mode, rate_axis=plan.rate_axis, schema=schema,
                                   validate_states=False)
        _check_closure(packed, physical, plan, layer)
        holder["packed"] = packed
        return packed.payload

    quant_args["pack_trellis_fn"] = pack_qsrt
    module = _load_quantizer_module(codebook) if quantizer_module is None else quantizer_module
    quantized, proxy, raw = module.quantize_qsrt(weight, shared_h, quant_args, True, progress_str="")
    packed = holder.get("packed")
    if packed is None:
        raise ValueError("QSRT packer was not called; fallback encoding is unsupported")
    tensors = _repack_scales({n: raw[n] for n in ("trellis", "suh", "svh")}, plan)
    decoded_physical = decode_qsrt_exl3_weight(packed, tensors["suh"], tensors["svh"], codebook=codebook)
    encoder_physical = repack_rate_axis(quantized, plan.record_repack_order, 0 if plan.rate_axis == "k" else 1,
                                        geometry)
    stored_vs_encoder = comparison_metrics(encoder_physical, decoded_physical)
    if not all(math.isfinite(v) for v in stored_vs_encoder.values()):
        raise ValueError("stored QSRT decode produced non-finite values")
    reconstruction = torch.empty_like(source)
    _place(reconstruction, decoded_physical, plan)
    placed = (reconstruction.index_select(1, plan.physical_permutation) if matrix == "w2"
              else reconstruction.index_select(0, plan.physical_permutation))
    if not torch.equal(placed, decoded_physical.T):
        raise ValueError(f"{matrix} physical permutation failed exact matrix closure")
    index_bits, scale_bits = _bit_accounting(tensors, plan, source.numel())
    if not torch.equal(tensors["trellis"], packed.payload):
        raise ValueError("quantizer returned a different trellis payload")
    coding = _coding(plan, packed, tensors, proxy=proxy, index_bits=index_bits, scale_bits=scale_bits,
                     codebook=codebook, tailbite_context=tailbite_context, seeds=seeds,
                     stored_vs_encoder=stored_vs_encoder)
    return QSRTMatrixEncoding(reconstruction=reconstruction, tensors=tensors, packed=packed, plan=plan,
                              coding=coding)


def finalize_qsrt_matrix_candidate(candidate: QSRTMatrixCandidate, *, layer: int,
                                   logical_trellis_schema: str | None = None,
                                   codebook: str = CODEBOOK_SQG_XOR_CHEB_T12,
                                   tailbite_context: int = 128) -> QSRTMatrixEncoding:
    """Pack and independently decode one selected candidate
    (reference qsrt_encoder.py:1257-1423)."""

    plan = candidate.plan
    geometry = plan.geometry
    physical = repack_encoded_records(candidate.encoded, plan.record_repack_order, plan.rate_axis)
    packed = pack_qsrt_trellis(physical, plan.mode, rate_axis=plan.rate_axis,
                               schema=logical_trellis_schema or _schema_for(geometry), validate_states=False)
    states = _check_closure(packed, physical, plan, layer)
    tensors = _repack_scales({"trellis": packed.payload, "suh": candidate.tensors["suh"],
                              "svh": candidate.tensors["svh"]}, plan)
    decoded_physical = decode_qsrt_weight(states, tensors["suh"], tensors["svh"], rate_axis=plan.rate_axis,
                                          tile_bits=plan.physical_tile_bits, codebook=codebook)
    p = plan.encoder_permutation
    encoder_weight = (candidate.reconstruction.index_select(1, p).T.contiguous() if plan.matrix == "w2"
                      else candidate.reconstruction.index_select(0, p).T.contiguous())
    encoder_physical = repack_rate_axis(encoder_weight, plan.record_repack_order,
                                        0 if plan.rate_axis == "k" else 1, geometry)
    stored_vs_encoder = comparison_metrics(encoder_physical, decoded_physical)
    if not all(math.isfinite(v) for v in stored_vs_encoder.values()):
        raise ValueError("stored QSRT decode produced non-finite values")
    reconstruction = torch.empty_like(candidate.reconstruction)
    _place(reconstruction, decoded_physical, plan)
    scoring_vs_stored = comparison_metrics(candidate.reconstruction, reconstruction)
    if not all(math.isfinite(v) for v in scoring_vs_stored.values()):
        raise ValueError("selected QSRT scoring reconstruction did not close")
    index_bits, scale_bits = _bit_accounting(tensors, plan, reconstruction.numel())
    coding = _coding(plan, packed, tensors, proxy=candidate.proxy, index_bits=index_bits, scale_bits=scale_bits,
                     codebook=codebook, tailbite_context=tailbite_context, seeds=candidate.transform_seeds,
                     stored_vs_encoder=stored_vs_encoder)
    coding["scoring_reconstruction_vs_stored"] = scoring_vs_stored
    return QSRTMatrixEncoding(reconstruction=reconstruction, tensors=tensors, packed=packed, plan=plan,
                              coding=coding)


def quantize_qsrt_matrix_expert_batch(
    sources_by_expert: list[dict[str, torch.Tensor]], block_contexts_by_expert: list[torch.Tensor], *,
    modes_by_expert: list[tuple[ModeSpec, ...]], hessians_by_expert: list[dict[str, torch.Tensor]], layer: int,
    device: torch.device, quantizer_module=None, shared_scale_scope: object | None = None,
    layout: Layout = "importance_ordered", codebook: str = CODEBOOK_SQG_XOR_CHEB_T12,
    sqg_e4m3_luts_by_bits: Mapping[int, torch.Tensor | None] | None = None, ldlq_tf32: bool = False,
    tailbite_context: int = 128, transform_seeds_by_expert: list[Mapping[str, QSRTTransformSeeds]] | None = None,
    intermediate_conditioning_by_expert: list[torch.Tensor | None] | None = None,
    g_scale_overrides_by_expert: list[float | None] | None = None,
) -> list[dict[str, dict[int, QSRTMatrixCandidate]]]:
    """Every requested rate mode of same-shape matrices of several experts in
    one backend batch (reference qsrt_encoder.py:963-1254).  Experts keep
    their own permutations, Hessians, transforms and feedback; the batch only
    fills the tile launches."""

    n = len(sources_by_expert)
    if n <= 0 or len(block_contexts_by_expert) != n or len(modes_by_expert) != n or len(hessians_by_expert) != n:
        raise ValueError("expert-batched QSRT inputs must have equal nonzero lengths")
    if transform_seeds_by_expert is None:
        transform_seeds_by_expert = [{} for _ in range(n)]
    elif len(transform_seeds_by_expert) != n:
        raise ValueError("expert-batched transform seed maps have the wrong length")
    if intermediate_conditioning_by_expert is None:
        intermediate_conditioning_by_expert = [None] * n
    elif len(intermediate_conditioning_by_expert) != n:
        raise ValueError("expert-batched conditioning profiles have the wrong length")
    if g_scale_overrides_by_expert is None:
        g_scale_overrides_by_expert = [None] * n
    elif len(g_scale_overrides_by_expert) != n:
        raise ValueError("expert-batched global-scale overrides have the wrong length")

    entries, plans, weights, shared, groups = [], [], [], [], []
    common_shape = None
    residual_seeds: dict[str, int] = {}
    for e, (sources, contexts_raw, modes, hessians, seed_map, cond_raw, g_override) in enumerate(zip(
            sources_by_expert, block_contexts_by_expert, modes_by_expert, hessians_by_expert,
            transform_seeds_by_expert, intermediate_conditioning_by_expert, g_scale_overrides_by_expert)):
        if not sources or set(sources) != set(hessians):
            raise ValueError("batched QSRT sources and Hessians must share nonempty keys")
        if not modes or len({resolve_mode(m).mode_id if not isinstance(m, ModeSpec) else m.mode_id
                             for m in modes}) != len(modes):
            raise ValueError("batched QSRT modes must be nonempty and unique")
        matrices = [m for m in MATRICES if m in sources]
        if set(matrices) != set(sources):
            raise ValueError("batched QSRT sources contain an unknown matrix")
        shapes = {tuple(s.shape) for s in sources.values()}
        if len(shapes) != 1:
            raise ValueError("one QSRT batch may contain only same-shape matrices")
        shape = next(iter(shapes))
        if common_shape is None:
            common_shape = shape
        elif shape != common_shape:
            raise ValueError("expert-batched QSRT matrices must share one shape")
        contexts = contexts_raw.to(device=device, dtype=torch.long)
        geometry = _source_geometry(contexts, next(iter(sources.values())), matrices[0])
        specs = tuple(resolve_mode(m, geometry) for m in modes)
        cond = None
        if cond_raw is not None:
            cond = cond_raw.to(device=device, dtype=torch.float32)
            if cond.ndim != 1 or cond.numel() != geometry.intermediate_channels:
                raise ValueError(f"intermediate conditioning must cover {geometry.intermediate_channels} channels")
            if not bool(torch.all(torch.isfinite(cond))) or bool(torch.any(cond <= 0)):
                raise ValueError("intermediate conditioning must be finite and positive")
        unknown = set(seed_map) - set(MATRICES)
        if unknown:
            raise ValueError(f"transform seed map contains unknown matrices: {sorted(unknown)}")
        for matrix in matrices:
            source, hessian = sources[matrix], hessians[matrix]
            _validate_source_and_hessian(source, hessian, matrix, geometry)
            if source.device != device:
                raise ValueError(f"batched QSRT source {e}.{matrix} is not on {device}")
            if matrix in ("w1", "w3") and shared_scale_scope is None:
                raise ValueError(f"{matrix} requires a shared_scale_scope")
            seeds = seed_map.get(matrix) or default_qsrt_transform_seeds(layer, matrix)
            if not isinstance(seeds, QSRTTransformSeeds):
                raise TypeError("transform seed overrides must use QSRTTransformSeeds")
            residual = seeds.output_sign if matrix == "w2" else seeds.input_sign
            if residual_seeds.setdefault(matrix, residual) != residual:
                side = "output" if matrix == "w2" else "input"
                raise ValueError(f"{matrix} {side}-sign seed must be layer-shared within a batch")
            mplans = {s.mode_id: plan_qsrt_matrix(contexts, s, matrix=matrix, layout=layout, geometry=geometry)
                      for s in specs}
            ref = mplans[specs[0].mode_id]
            for p in mplans.values():
                if not torch.equal(p.encoder_permutation, ref.encoder_permutation):
                    raise ValueError("rate candidates changed the encoder neuron order")
                if not torch.equal(p.physical_permutation, ref.physical_permutation):
                    raise ValueError("rate candidates changed the physical neuron order")
            weight, _ = _encoder_weight(source, hessian, ref)
            enc_cond = None
            if cond is not None and matrix in ("w1", "w3"):
                enc_cond = cond.index_select(0, ref.encoder_permutation)
                blocks = enc_cond.reshape(-1, 128)
                if not bool(torch.all(blocks == blocks[:, :1])):
                    raise ValueError("folded conditioning must be constant in each Hadamard block")
                weight = weight / enc_cond.unsqueeze(0)
            entries.append((e, matrix, source, specs, enc_cond))
            plans.append(mplans)
            weights.append(weight)
            shared.append(make_qsrt_shared_h(contexts, matrix=matrix, mode=specs[0], hessian=hessian, device=device,
                                             layout=layout, geometry=geometry))
            groups.append([_qsrt_quant_args(mplans[s.mode_id], matrix=matrix, layer=layer, device=device,
                                            shared_scale_scope=shared_scale_scope, codebook=codebook,
                                            sqg_e4m3_luts_by_bits=sqg_e4m3_luts_by_bits, ldlq_tf32=ldlq_tf32,
                                            tailbite_context=tailbite_context, transform_seeds=seeds,
                                            g_scale_override=g_override) for s in specs])

    module = _load_quantizer_module(codebook) if quantizer_module is None else quantizer_module
    batch_api = getattr(module, "quantize_qsrt_batch", None)
    if batch_api is None:
        raise ValueError("QSRT encoder backend lacks mixed-rate batch support")
    raw_groups = batch_api(weights, shared, groups, return_weight_q=True)
    if len(raw_groups) != len(entries):
        raise ValueError("QSRT batch returned the wrong source count")

    result: list[dict[str, dict[int, QSRTMatrixCandidate]]] = [{} for _ in range(n)]
    finite_checks, labels = [], []
    for i, ((e, matrix, source, specs, enc_cond), raw_group) in enumerate(zip(entries, raw_groups)):
        if len(raw_group) != len(specs):
            raise ValueError("QSRT batch returned the wrong candidate count")
        out: dict[int, QSRTMatrixCandidate] = {}
        for spec, raw in zip(specs, raw_group):
            plan = plans[i][spec.mode_id]
            encoder_weight = raw["weight_q"]
            if not isinstance(encoder_weight, torch.Tensor):
                raise ValueError("QSRT batch omitted its reconstruction")
            suh, svh = raw["suh"], raw["svh"]
            if enc_cond is not None:
                # fold the conditioning back into the stored fp16 sv; scale the
                # reconstruction by what fp16 actually kept
                original = svh.float()
                svh = (original * enc_cond).to(torch.float16)
                ratio = torch.ones_like(original)
                nz = original != 0
                ratio[nz] = svh.float()[nz] / original[nz]
                encoder_weight = encoder_weight * ratio.unsqueeze(0)
            reconstruction = torch.empty_like(source)
            if matrix == "w2":
                reconstruction[:, plan.encoder_permutation] = encoder_weight.T
            else:
                reconstruction[plan.encoder_permutation] = encoder_weight.T
            finite_checks.append(torch.all(torch.isfinite(reconstruction)))
            labels.append((e, matrix, spec.mode_id))
            proxy = float(raw["proxy"])
            if not math.isfinite(proxy):
                raise ValueError(f"QSRT batch produced a non-finite proxy for batch expert {e}, {matrix}, "
                                 f"mode {spec.mode_id}: {proxy!r}")
            out[spec.mode_id] = QSRTMatrixCandidate(
                reconstruction=reconstruction, encoded=raw["encoded"], tensors={"suh": suh, "svh": svh}, plan=plan,
                proxy=proxy, transform_seeds=QSRTTransformSeeds(int(groups[i][0]["seed"]), int(groups[i][0]["sv_seed"])),
                global_scale=float(raw.get("g_scale", 1.0)))
        result[e][matrix] = out
    finite = torch.stack(finite_checks).cpu()
    if not bool(torch.all(finite)):
        e, matrix, mode_id = labels[int(torch.nonzero(~finite, as_tuple=False)[0])]
        raise ValueError(f"QSRT batch produced a non-finite reconstruction for expert-index {e} {matrix} R{mode_id}")
    return result


def quantize_qsrt_matrix_candidates_batched(sources: dict[str, torch.Tensor], block_contexts: torch.Tensor, *,
                                            modes: tuple[ModeSpec, ...], hessians: dict[str, torch.Tensor],
                                            layer: int, device: torch.device, quantizer_module=None,
                                            shared_scale_scope: object | None = None,
                                            layout: Layout = "importance_ordered",
                                            codebook: str = CODEBOOK_SQG_XOR_CHEB_T12,
                                            sqg_e4m3_luts_by_bits=None, ldlq_tf32: bool = False,
                                            tailbite_context: int = 128, transform_seeds=None,
                                            intermediate_conditioning: torch.Tensor | None = None,
                                            g_scale_override: float | None = None):
    """One expert's same-shape matrices over several rate modes
    (reference qsrt_encoder.py:916-960)."""

    return quantize_qsrt_matrix_expert_batch(
        [sources], [block_contexts], modes_by_expert=[modes], hessians_by_expert=[hessians], layer=layer,
        device=device, quantizer_module=quantizer_module, shared_scale_scope=shared_scale_scope, layout=layout,
        codebook=codebook, sqg_e4m3_luts_by_bits=sqg_e4m3_luts_by_bits, ldlq_tf32=ldlq_tf32,
        tailbite_context=tailbite_context, transform_seeds_by_expert=[transform_seeds or {}],
        intermediate_conditioning_by_expert=[intermediate_conditioning],
        g_scale_overrides_by_expert=[g_scale_override])[0]


def quantize_qsrt_expert(sources: dict[str, torch.Tensor], block_contexts: torch.Tensor, *, format_spec,
                         h13: torch.Tensor, h2: torch.Tensor, layer: int, device: torch.device,
                         shared_scale_scope: object, quantizer_module=None, logical_trellis_schema: str | None = None,
                         codebook: str = CODEBOOK_SQG_XOR_CHEB_T12, ldlq_tf32: bool = False,
                         tailbite_context: int = 128,
                         transform_seeds: Mapping[str, QSRTTransformSeeds] | None = None) -> QSRTExpertEncoding:
    """All three matrices of one expert under one physical neuron order
    (reference qsrt_encoder.py:1664-1747)."""

    format_spec = resolve_expert_format(format_spec)
    if format_spec.is_x4t:
        raise ValueError("quantize_qsrt_expert requires a compressed format")
    if set(sources) != set(MATRICES):
        raise ValueError(f"sources must contain exactly {MATRICES}")
    geometry = _source_geometry(block_contexts, sources["w1"], "w1")
    modes = {"w1": resolve_mode(format_spec.r13, geometry), "w3": resolve_mode(format_spec.r13, geometry),
             "w2": resolve_mode(format_spec.r2, geometry)}
    hessians = {"w1": h13, "w3": h13, "w2": h2}
    encodings = {
        m: quantize_qsrt_matrix(sources[m], block_contexts, matrix=m, mode=modes[m], hessian=hessians[m],
                                layer=layer, device=device, quantizer_module=quantizer_module,
                                shared_scale_scope=shared_scale_scope, logical_trellis_schema=logical_trellis_schema,
                                codebook=codebook, ldlq_tf32=ldlq_tf32, tailbite_context=tailbite_context,
                                transform_seeds=(transform_seeds or {}).get(m))
        for m in MATRICES
    }
    perm = encodings["w1"].plan.physical_permutation
    for m in ("w3", "w2"):
        if not torch.equal(encodings[m].plan.physical_permutation, perm):
            raise ValueError("expert matrices do not share one physical permutation")
    trellis_bytes = sum(x.tensors["trellis"].numel() * x.tensors["trellis"].element_size() for x in encodings.values())
    scale_bytes = sum(x.tensors[n].numel() * x.tensors[n].element_size()
                      for x in encodings.values() for n in ("suh", "svh"))
    return QSRTExpertEncoding(
        format=format_spec, matrices=encodings, physical_permutation=perm,
        coding={"format": format_spec.name, "format_code": format_spec.code, "r13": format_spec.r13,
                "r2": format_spec.r2, "common_physical_permutation": True, "trellis_bytes": trellis_bytes,
                "raw_scale_bytes": scale_bytes,
                "matrices": {m: x.coding for m, x in encodings.items()}})
