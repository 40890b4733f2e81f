"""L2 tile-quantizer operator: ``quantize_tiles(tiles, quant_args)`` on MI355X.

Mirrors ``qsrt/sqg_quantizer.py`` (reference ``install_sqg_quantizer`` at
:459-657): the same ``quant_args`` keys select the reconstruction table and
the same validation messages are raised; the call is executed by the HIP
kernel behind ``qsrt_viterbi_tiles`` (``include/qsrt_amd.h``).

Differences, all deliberate:

* path metrics are FP32 (the reference kernel uses FP16);
* the state-indexed LUT is handed to the kernel as is -- the kernel widens
  each thread's labels into registers once, so no predecessor-major
  transpose (reference :612-633) is needed;
* the boundary argmin follows the reference's per-K dispatch
  (``sqg_quantize.cu:730-749``): the K2 fast kernel scores the final primer
  step, the generic K3/K4 kernel the step before it.  ``quant_args
  ["tailbite_boundary"]`` ("reference" | "final" | "penultimate") overrides;
* research controls that are outside the encoder hot path (periodic rate
  schedules, FP16 tables, procedural MCG/MUL1 codebooks, on-GPU trellis
  diagnostics) raise ``NotImplementedError`` instead of running.
"""

from __future__ import annotations

import math
import os
from collections.abc import Mapping

import torch

from . import _native
from .exl3_reference import reconstruct_trellis_states
from .sqg_e4m3 import sqg_e4m3_bytes

# Largest label magnitude for which the reference routes K2 to its dedicated
# kernel (qsrt_quantize_tiles_k2_kernel.cuh:45).
K2_FAST_MAX_LABEL = 16.0

_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def _workspace(device: torch.device, bits: int, n_tiles: int) -> torch.Tensor:
    """Traceback workspace of the current stream on ``device``.  Each stream
    has its own buffer (sized once for the widest grid), so launches queued
    on different streams never share decision rows; launches on one stream
    are ordered and reuse it."""

    need = int(_native.lib().qsrt_viterbi_workspace_bytes(bits, n_tiles))
    if need == 0:
        raise _native.NativeError(
            "qsrt_viterbi_workspace_bytes failed: " + _native.lib().qsrt_last_error().decode()
        )
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, torch.cuda.current_stream(device).cuda_stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < need:
        # Size for the widest grid (one workgroup per CU) once.
        full = max(int(_native.lib().qsrt_viterbi_workspace_bytes(b, 1 << 30)) for b in range(1, 7))
        ws = torch.empty(max(need, full), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def _lut_abs_max(lut: torch.Tensor) -> float:
    """Largest label magnitude of an E4M3 LUT, remembered on the tensor
    object itself (with its version counter) so that neither a reused device
    address nor an in-place edit can return another table's value."""

    hit = getattr(lut, "_qsrt_abs_max", None)
    if hit is not None and hit[0] == lut._version:
        return hit[1]
    value = float(lut.view(torch.float8_e4m3fn).to(torch.float32).abs().amax())
    lut._qsrt_abs_max = (lut._version, value)
    return value


def _lut_on(lut: torch.Tensor, device: torch.device) -> torch.Tensor:
    """``lut`` as a contiguous uint8 tensor on ``device``; the device copy of a
    host table is made once per source tensor and version."""

    if lut.device == device and lut.dtype == torch.uint8 and lut.is_contiguous():
        return lut
    copies = getattr(lut, "_qsrt_device_copies", None)
    if copies is None:
        copies = {}
        lut._qsrt_device_copies = copies
    hit = copies.get(str(device))
    if hit is None or hit[0] != lut._version:
        hit = (lut._version, lut.to(device=device, dtype=torch.uint8).contiguous())
        copies[str(device)] = hit
    return hit[1]


def boundary_lag(bits: int, lut_abs_max: float, policy: str = "reference") -> int:
    """0: argmin over the primer's final costs; 1: over the step before."""

    if policy == "final":
        return 0
    if policy == "penultimate":
        return 1
    if policy != "reference":
        raise ValueError("tailbite_boundary must be 'reference', 'final' or 'penultimate'")
    fast_k2 = bits == 2 and math.isfinite(lut_abs_max) and 0.0 < lut_abs_max <= K2_FAST_MAX_LABEL
    return 0 if fast_k2 else 1


def viterbi_tiles(
    tiles: torch.Tensor,
    lut: torch.Tensor,
    bits: int,
    *,
    tailbite_context: int = 128,
    lag: int = 0,
    out: tuple[torch.Tensor, torch.Tensor] | None = None,
    max_workgroups: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Run the HIP tile Viterbi.  ``tiles`` FP32 ``[T, 256]`` (tensor-core
    order), ``lut`` the state-indexed uint8 E4M3 table on the same device.
    ``max_workgroups`` caps the grid (0: one workgroup per CU).
    Returns ``(recon f32 [T, 256], states int16 [T, 256])``."""

    if not tiles.is_cuda:
        raise ValueError("the MI355X tile quantizer requires a GPU tensor")
    if bits not in (1, 2, 3, 4, 5, 6):
        raise ValueError(f"K{bits} is not supported by the MI355X tile kernel (K1..K6)")
    tiles = tiles.contiguous()
    if tiles.dtype != torch.float32 or tiles.ndim != 2 or tiles.shape[1] != 256:
        raise ValueError("SQG tiles must be contiguous FP32 [N, 256]")
    if lut.dtype != torch.uint8 or lut.numel() != 65536:
        raise ValueError("codebook must contain 65,536 uint8 E4M3 values")
    lut = lut.to(device=tiles.device).contiguous()
    if out is None:
        recon = torch.empty_like(tiles)
        states = torch.empty(tiles.shape, dtype=torch.int16, device=tiles.device)
    else:
        recon, states = out
    n = tiles.shape[0]
    if n == 0:
        return recon, states
    ws = _workspace(tiles.device, bits, n)
    with torch.cuda.device(tiles.device):
        rc = _native.lib().qsrt_viterbi_tiles_ex(
            tiles.data_ptr(), recon.data_ptr(), states.data_ptr(), n, int(bits), int(tailbite_context),
            lut.data_ptr(), int(lag), int(max_workgroups), ws.data_ptr(), ws.numel(),
            _native.stream_handle(tiles.device),
        )
    _native.check(rc, "qsrt_viterbi_tiles_ex")
    return recon, states


def debug_check_trellis_closure(indices: torch.Tensor, bits: int) -> None:
    """Raise if a tile's states are not a closed cyclic path
    (reference sqg_quantizer.py:304-331, opt-in via QSRT_DEBUG_TILE_CLOSURE=1)."""

    expected = reconstruct_trellis_states(indices.to(torch.int64) & ((1 << bits) - 1), bits)
    mismatch = indices != expected
    if bool(torch.any(mismatch)):
        first = tuple(int(v) for v in torch.nonzero(mismatch)[0].cpu().tolist())
        raise RuntimeError(
            "SQG tile kernel emitted a non-closing trellis state: "
            f"K{bits}, {int(mismatch.sum())} states differ; first at {first}, "
            f"encoded={int(indices[first])}, reconstructed={int(expected[first])}"
        )


_R44_LUTS: dict[tuple[str, int], torch.Tensor] = {}


def _resolve_codebook(quant_args: dict, bits: int, device: torch.device) -> torch.Tensor:
    if quant_args.get("periodic_rate_schedules") is not None:
        raise NotImplementedError("periodic rate schedules are a research control outside the MI355X hot path")
    codebook = quant_args.get("sqg_e4m3_lut")
    fp16_codebook = quant_args.get("sqg_fp16_lut")
    rate_codebooks = quant_args.get("sqg_e4m3_luts_by_bits")
    mode = quant_args.get("sqg_e4m3_mode")
    if fp16_codebook is not None:
        if codebook is not None or rate_codebooks is not None or mode is not None:
            raise ValueError("an FP16 SQG table cannot be combined with another codebook")
        raise NotImplementedError("FP16 SQG tables are a research control outside the MI355X hot path")
    if rate_codebooks is not None:
        if codebook is not None or mode is not None:
            raise ValueError("rate-specific SQG LUTs cannot be combined with another SQG law")
        if not isinstance(rate_codebooks, Mapping):
            raise TypeError("sqg_e4m3_luts_by_bits must be a mapping")
        if set(rate_codebooks) - {1, 2, 3, 4}:
            raise ValueError("rate-specific SQG LUT keys must be K1 through K4")
        try:
            codebook = rate_codebooks[bits]
        except KeyError as exc:
            raise ValueError(f"missing rate-specific SQG K{bits} LUT") from exc
        if codebook is None:
            raise NotImplementedError("procedural MCG/MUL1 control codebooks are not part of the MI355X hot path")
    elif codebook is None:
        if mode != "normal":
            raise ValueError("the supported R44 mode is 'normal'")
        key = (str(device), bits)
        codebook = _R44_LUTS.get(key)
        if codebook is None:
            codebook = sqg_e4m3_bytes(bits, mode, device=device)
            _R44_LUTS[key] = codebook
    return _lut_on(codebook, device)


def has_sqg_codebook(quant_args: dict) -> bool:
    return any(
        quant_args.get(key) is not None
        for key in ("periodic_rate_schedules", "sqg_e4m3_lut", "sqg_fp16_lut", "sqg_e4m3_luts_by_bits", "sqg_e4m3_mode")
    )


def quantize_tiles_sqg(tiles: torch.Tensor, quant_args: dict) -> tuple[torch.Tensor, torch.Tensor]:
    """The patched ``quantize_tiles`` body (reference sqg_quantizer.py:478-654)."""

    devices = quant_args.get("devices", [tiles.device])
    if len(devices) != 1:
        raise ValueError("the SQG validation hook currently requires one CUDA device")
    tiles = tiles.contiguous()
    if tiles.dtype != torch.float32 or tiles.ndim != 2 or tiles.shape[1] != 256:
        raise ValueError("SQG tiles must be contiguous FP32 [N, 256]")
    if quant_args.get("return_trellis_diagnostics"):
        raise NotImplementedError("on-GPU trellis diagnostics are a research feature outside the MI355X hot path")
    bits = int(quant_args["K"])
    if bits not in (1, 2, 3, 4, 5, 6):
        raise ValueError(f"SQG tile quantization supports K1 through K6, not K{bits}")
    lut = _resolve_codebook(quant_args, bits, tiles.device)
    lag = boundary_lag(bits, _lut_abs_max(lut), quant_args.get("tailbite_boundary", "reference"))
    context = int(quant_args.get("tailbite_context", 128))
    if not 1 <= context <= 128:
        raise ValueError("tailbite_context must be in 1..128")
    output, indices = viterbi_tiles(tiles, lut, bits, tailbite_context=context, lag=lag,
                                    max_workgroups=int(quant_args.get("tile_workgroups", 0)))
    if os.environ.get("QSRT_DEBUG_TILE_CLOSURE") == "1":
        debug_check_trellis_closure(indices, bits)
    return output, indices


def install_sqg_quantizer(quantizer_module) -> None:
    """Route ``quantizer_module.quantize_tiles`` through the MI355X kernel
    for every call that names an SQG codebook; other calls keep the
    module's original function (reference sqg_quantizer.py:459-471)."""

    if getattr(quantizer_module, "_qsrt_sqg_installed", False):
        return
    original = quantizer_module.quantize_tiles

    def quantize_tiles(tiles: torch.Tensor, quant_args: dict):
        if not has_sqg_codebook(quant_args):
            return original(tiles, quant_args)
        return quantize_tiles_sqg(tiles, quant_args)

    quantizer_module.quantize_tiles = quantize_tiles
    quantizer_module._qsrt_sqg_installed = True


def _overlap(a: torch.Tensor, b: torch.Tensor) -> bool:
    a0, b0 = a.data_ptr(), b.data_ptr()
    return a0 < b0 + b.numel() * b.element_size() and b0 < a0 + a.numel() * a.element_size()


def apply_bakron_block_update(workspace: torch.Tensor, quantized: torch.Tensor, output_factor: torch.Tensor,
                              input_factor: torch.Tensor, intermediate: torch.Tensor, *, first_diagonal: int,
                              middle_diagonal: int, last_diagonal: int, block_size: int,
                              block_lower: bool = False) -> None:
    """One fused FP32 band propagation of the recursive BaKron rounding on the
    GPU (reference ``qsrt/sqg_quantizer.py:383-407`` over
    ``qsrt/csrc/sqg_quantize.cu:991-1100``): the intermediate receives
    ``Lout (Q - T)`` restricted to the finished band [first, middle) on the
    diagonals [first, last), and the workspace gains
    ``intermediate Lin^T`` on the next band [middle, last).  Runs the HIP
    kernel behind ``qsrt_bakron_band_update_f32`` on the current stream; the
    checks and their messages follow the reference launcher's.
    ``block_lower=True`` (not in the reference) promises a block-lower output
    factor and runs ``qsrt_bakron_band_update_lower_f32``, which skips its
    zero blocks; the result is the same for such factors."""

    if not workspace.is_cuda:
        raise ValueError("workspace must be CUDA")
    if workspace.dtype != torch.float32:
        raise ValueError("workspace must be FP32")
    if workspace.ndim not in (2, 3) or not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous matrix or matrix batch")
    if quantized.shape != workspace.shape or quantized.dtype != torch.float32 or not quantized.is_contiguous():
        raise ValueError("quantized matrix must match workspace")
    if (intermediate.shape != workspace.shape or intermediate.dtype != torch.float32
            or not intermediate.is_contiguous()):
        raise ValueError("intermediate matrix must match workspace")
    for factor, name in ((output_factor, "output factor"), (input_factor, "input factor")):
        if (not factor.is_cuda or factor.device != workspace.device or factor.dtype != torch.float32
                or factor.ndim not in (2, 3) or not factor.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous CUDA FP32 matrix")
    if quantized.device != workspace.device or intermediate.device != workspace.device:
        raise ValueError("BaKron matrices must share one CUDA device")
    # the left launch writes the intermediate while reading the others, the right one writes the workspace
    for other, name in ((workspace, "workspace"), (quantized, "quantized matrix"), (output_factor, "output factor"),
                        (input_factor, "input factor")):
        if _overlap(intermediate, other):
            raise ValueError(f"intermediate matrix must not overlap the {name}")
    for other, name in ((quantized, "quantized matrix"), (output_factor, "output factor"),
                        (input_factor, "input factor")):
        if _overlap(workspace, other):
            raise ValueError(f"workspace must not overlap the {name}")
    if block_size != 16:
        raise ValueError("fused BaKron updates require 16x16 blocks")
    n_out, n_in = map(int, workspace.shape[-2:])
    batch = 1 if workspace.ndim == 2 else int(workspace.shape[0])
    if n_out % 16 or n_in % 16:
        raise ValueError("BaKron dimensions must be divisible by 16")
    if tuple(output_factor.shape[-2:]) != (n_out, n_out) or (output_factor.ndim == 3
                                                            and output_factor.shape[0] != batch):
        raise ValueError("output factor shape mismatch")
    if tuple(input_factor.shape[-2:]) != (n_in, n_in) or (input_factor.ndim == 3 and input_factor.shape[0] != batch):
        raise ValueError("input factor shape mismatch")
    diagonals = n_out // 16 + n_in // 16 - 1
    first, middle, last = int(first_diagonal), int(middle_diagonal), int(last_diagonal)
    if not 0 <= first < middle < last <= diagonals:
        raise ValueError("invalid recursive BaKron diagonal range")
    lib = _native.lib()
    with torch.cuda.device(workspace.device):
        fn = lib.qsrt_bakron_band_update_lower_f32 if block_lower else lib.qsrt_bakron_band_update_f32
        _native.check(fn(
            workspace.data_ptr(), quantized.data_ptr(), output_factor.data_ptr(), input_factor.data_ptr(),
            intermediate.data_ptr(), batch, n_out, n_in, 0 if output_factor.ndim == 2 else n_out * n_out,
            0 if input_factor.ndim == 2 else n_in * n_in, first, middle, last,
            _native.stream_handle(workspace.device)), "qsrt_bakron_band_update_f32")
