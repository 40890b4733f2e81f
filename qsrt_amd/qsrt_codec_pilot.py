"""Uniform-rate codec entry points (mirrors the uniform part of
``qsrt/qsrt_codec_pilot.py``): encode one matrix at a single tile rate
K2..K6 through ``quantize_qsrt``, decode its own payload, and report the
payload's identity and bit accounting.

The uniform payload is the EXL word stream at any K (packed and unpacked by
``qsrt_amd.codec``); the QSRT container format stays K2..K4.  Procedural MCG
and FP16 experimental tables are research controls here and raise
``NotImplementedError``, as the encoder backend does.
"""

from __future__ import annotations

import hashlib
import math
import time
from collections.abc import Mapping
from typing import Any

import torch

from . import exl3_encoder_backend
from .codec import pack_words, unpack_words
from .exl3_reference import CODEBOOK_SQG_CHEB_NORMAL_E4M3, CODEBOOK_SQG_XOR_CHEB_T12, decode_exl3_weight
from .ldlq import SIGMA_REG, make_shared_h
from .sqg_e4m3 import sqg_codebook_bytes

CODEBOOK_MCG = "mcg"
SQG_FP16_D3L = "sqg_fp16_d3l"
UNIFORM_CODEBOOKS = (CODEBOOK_MCG, CODEBOOK_SQG_XOR_CHEB_T12, CODEBOOK_SQG_CHEB_NORMAL_E4M3, SQG_FP16_D3L)


def tensor_sha256(value: torch.Tensor) -> str:
    """SHA-256 of a tensor's bytes (host copy, contiguous)."""

    return hashlib.sha256(value.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def _check_uniform_rate(bits: int, what: str) -> None:
    if isinstance(bits, bool) or not isinstance(bits, int) or bits not in range(2, 7):
        raise ValueError(f"{what} must be K2 through K6")


def unpack_uniform_trellis_states(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """EXL words ``[..., 16 K]`` -> cyclic states ``[..., 256]`` (reference
    qsrt_codec_pilot.py:220-244)."""

    _check_uniform_rate(bits, "uniform trellis rate")
    if packed.dtype != torch.int16 or packed.ndim != 3:
        raise TypeError("packed uniform trellis must be a rank-three int16 tensor")
    if packed.shape[-1] != 16 * bits:
        raise ValueError("packed uniform trellis has the wrong word width")
    return unpack_words(packed, bits)


def pack_uniform_trellis_edges(edges: torch.Tensor, bits: int) -> torch.Tensor:
    """Edge symbols ``[..., 256]`` -> EXL words (reference :247-281)."""

    _check_uniform_rate(bits, "uniform trellis rate")
    return pack_words(edges, bits)


def _canonical_metric(hessian: torch.Tensor, dimension: int, name: str, axis: str) -> torch.Tensor:
    if (hessian.ndim != 2 or tuple(hessian.shape) != (dimension, dimension) or not torch.is_floating_point(hessian)
            or not bool(torch.isfinite(hessian).all())):
        raise ValueError(f"{name} must be a finite floating-point square matrix matching the {axis} dimension")
    metric = hessian.float()
    if not torch.allclose(metric, metric.T, atol=1e-5, rtol=1e-5):
        raise ValueError(f"{name} must be symmetric")
    if float(metric.diagonal().mean().item()) <= 0.0:
        raise ValueError(f"{name} must have a positive mean diagonal")
    return metric


def encode_uniform_candidate(source: torch.Tensor, *, bits: int, codebook: str, device: torch.device,
                             quantizer_module: Any = exl3_encoder_backend, input_sign_seed: int,
                             output_sign_seed: int, rate_axis: str | None = None,
                             scale_scope_key: object | None = None, g_scale_into_sv: bool = False,
                             sigma_reg: float = SIGMA_REG, tailbite_context: int = 128, ldlq_tf32: bool = True,
                             g_scale_override: float | None = None, ldlq_feedback_multiplier: float = 1.0,
                             codebook_values: torch.Tensor | None = None, hessian: torch.Tensor | None = None,
                             input_hessian: torch.Tensor | None = None, output_hessian: torch.Tensor | None = None,
                             use_two_sided_traversal_without_output_feedback: bool = False,
                             return_replay_state: bool = False,
                             return_trellis_diagnostics: bool = False) -> dict[str, Any]:
    """Encode one ``[out, in]`` matrix at uniform rate K2..K6 and decode its
    payload (reference qsrt_codec_pilot.py:284-584).  ``reconstruction`` is
    the decoded matrix in the source orientation (fp16 values, host)."""

    if source.ndim != 2 or not torch.is_floating_point(source):
        raise TypeError("source must be a floating-point matrix")
    m = ldlq_feedback_multiplier
    if isinstance(m, bool) or not isinstance(m, (int, float)) or not math.isfinite(float(m)) or not 0.0 <= float(m) <= 1.0:
        raise ValueError("ldlq_feedback_multiplier must be a real number in [0, 1]")
    _check_uniform_rate(bits, "uniform codec rate")
    if not isinstance(use_two_sided_traversal_without_output_feedback, bool):
        raise TypeError("use_two_sided_traversal_without_output_feedback must be a boolean")
    if use_two_sided_traversal_without_output_feedback and output_hessian is not None:
        raise ValueError("the zero-output-feedback traversal control cannot be combined with an output Hessian")
    if codebook_values is None and codebook not in UNIFORM_CODEBOOKS:
        raise ValueError(f"unsupported uniform codebook {codebook!r}")
    if codebook in (CODEBOOK_MCG, SQG_FP16_D3L) or codebook_values is not None:
        raise NotImplementedError("procedural MCG and FP16 experimental tables are research controls outside the "
                                  "MI355X encoder hot path")
    if return_trellis_diagnostics:
        raise NotImplementedError("trellis diagnostics are a research feature outside the MI355X encoder hot path")
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("uniform codec encoding requires a GPU device")
    out_metric = None
    out_role, out_sha = "identity_implicit", None
    if output_hessian is not None:
        out_metric = _canonical_metric(output_hessian, source.shape[0], "output_hessian", "source output")
        out_role, out_sha = "caller_supplied_downstream_curvature", tensor_sha256(out_metric)
    encoder_weight = source.T.float().contiguous().to(device)
    if hessian is not None and input_hessian is not None:
        raise ValueError("supply either hessian or input_hessian, not both")
    chosen = input_hessian if input_hessian is not None else hessian
    if chosen is None:
        shared_h = make_shared_h(encoder_weight.shape[0], device)
        in_role, in_sha = "identity_control", None
    else:
        in_metric = _canonical_metric(chosen, encoder_weight.shape[0], "input_hessian", "encoder input")
        shared_h = make_shared_h(encoder_weight.shape[0], device, in_metric)
        in_role, in_sha = "caller_supplied_curvature", tensor_sha256(in_metric)
    quant_args: dict[str, Any] = {
        "K": bits, "seed": int(input_sign_seed), "sv_seed": int(output_sign_seed), "sigma_reg": float(sigma_reg),
        "devices": [str(device)], "device_ratios": None, "apply_out_scales": False, "ldlq_tf32": bool(ldlq_tf32),
        "tailbite_context": int(tailbite_context), "ldlq_feedback_multiplier": float(m),
        "sqg_e4m3_lut": sqg_codebook_bytes(bits, codebook, rate_axis=rate_axis),
    }
    if scale_scope_key is not None:
        quant_args["shared_input_scales_key"] = scale_scope_key
    if g_scale_into_sv:
        quant_args["g_scale_into_sv"] = True
    if g_scale_override is not None:
        quant_args["g_scale_override"] = float(g_scale_override)
    if out_metric is not None:
        quant_args["output_hessian"] = out_metric
    if use_two_sided_traversal_without_output_feedback:
        quant_args["use_two_sided_traversal_without_output_feedback"] = True

    torch.cuda.synchronize(device)
    started = time.monotonic()
    _, proxy, tensors = quantizer_module.quantize_qsrt(encoder_weight, shared_h, quant_args, False, progress_str="")
    torch.cuda.synchronize(device)
    elapsed = time.monotonic() - started
    trellis, suh, svh = (tensors[k].contiguous() for k in ("trellis", "suh", "svh"))
    k_in, n_out = encoder_weight.shape
    if trellis.dtype != torch.int16 or tuple(trellis.shape) != (k_in // 16, n_out // 16, 16 * bits):
        raise ValueError("uniform encoder returned an invalid trellis payload")
    if suh.dtype != torch.float16 or tuple(suh.shape) != (k_in,):
        raise ValueError("uniform encoder returned an invalid suh vector")
    if svh.dtype != torch.float16 or tuple(svh.shape) != (n_out,):
        raise ValueError("uniform encoder returned an invalid svh vector")
    states = unpack_uniform_trellis_states(trellis, bits)
    decoded = decode_exl3_weight(states, suh, svh, codebook=codebook, bits=bits).half()
    logical_bytes = trellis.numel() * trellis.element_size()
    bpw = logical_bytes * 8.0 / source.numel()
    if bpw != float(bits):
        raise ValueError("uniform trellis payload does not match its declared rate")
    proxy_value = float(proxy)
    if not math.isfinite(proxy_value):
        raise ValueError("uniform encoder returned a non-finite proxy")
    result: dict[str, Any] = {
        "reconstruction": decoded.T.contiguous().cpu(),
        "payload": {
            "profile": "qsrt_sqg_e4m3" if codebook == CODEBOOK_SQG_XOR_CHEB_T12 else "offline_sqg_control",
            "codebook": codebook, "rate": bits, "trellis_bytes": logical_bytes, "trellis_bpw": bpw,
            "scale_bytes": suh.numel() * suh.element_size() + svh.numel() * svh.element_size(),
            "trellis_sha256": tensor_sha256(trellis), "suh_sha256": tensor_sha256(suh),
            "svh_sha256": tensor_sha256(svh), "mcg_multiplier": None, "proxy_relative_error": proxy_value,
            "encode_seconds": elapsed, "input_sign_seed": int(input_sign_seed),
            "output_sign_seed": int(output_sign_seed), "rate_axis": rate_axis, "g_scale": float(quant_args["g_scale"]),
            "codebook_values_sha256": None, "input_hessian_role": in_role, "input_hessian_sha256": in_sha,
            "output_hessian_role": out_role, "output_hessian_sha256": out_sha,
            "two_sided_feedback": out_metric is not None,
            "output_hessian_factorization": quant_args.get("output_hessian_record"),
            "two_sided_traversal_without_output_feedback": use_two_sided_traversal_without_output_feedback,
            "ldlq_feedback_multiplier": float(m),
        },
    }
    if return_replay_state:
        result["replay_state"] = {"bits": bits, "trellis": trellis.cpu(), "suh": suh.cpu(), "svh": svh.cpu()}
    return result


@torch.no_grad()
def replay_uniform_candidate(replay_state: Mapping[str, Any], *, codebook_values: torch.Tensor) -> torch.Tensor:
    """Decode a stored uniform path and scales through another state-indexed
    fp16 table, in the source orientation (reference :587-627)."""

    bits = replay_state.get("bits")
    trellis, suh, svh = (replay_state.get(k) for k in ("trellis", "suh", "svh"))
    _check_uniform_rate(bits, "replay state rate")
    if not all(isinstance(v, torch.Tensor) for v in (trellis, suh, svh)):
        raise TypeError("replay state must contain trellis, suh, and svh tensors")
    if (codebook_values.dtype != torch.float16 or codebook_values.ndim != 1 or codebook_values.numel() != 65536
            or not bool(torch.isfinite(codebook_values).all())):
        raise ValueError("replay codebook must contain 65,536 finite FP16 values")
    states = unpack_uniform_trellis_states(trellis, bits)
    return decode_exl3_weight(states, suh, svh, codebook_values=codebook_values).half().T.contiguous().cpu()


__all__ = [
    "CODEBOOK_MCG",
    "SQG_FP16_D3L",
    "UNIFORM_CODEBOOKS",
    "encode_uniform_candidate",
    "pack_uniform_trellis_edges",
    "replay_uniform_candidate",
    "tensor_sha256",
    "unpack_uniform_trellis_states",
]
