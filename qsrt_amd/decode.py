"""Fused trellis decode on MI355X: packed EXL words -> bf16 (or f32) weights.

``decode_words`` decodes one uniform-rate ``[K/16, N/16, 16 bits]`` trellis
(the ``trellis`` tensor of ``quantize_qsrt``); ``decode_packed`` decodes a
mixed-rate ``PackedQSRTTrellis`` payload record by record with one launch per
rate.  Both compute ``W = H_R(H_L(X) * su) * sv`` (reference
``qsrt/exl3_reference.py:280-330``, ``qsrt/qsrt.py:1175-1209``) in the HIP
kernel behind ``qsrt_decode`` (``include/qsrt_amd.h``).
"""

from __future__ import annotations

import ctypes

import torch

from . import _native
from .sqg_quantizer import _lut_abs_max, _lut_on

# FP8 matrix-core products are exact for labels up to this magnitude (every
# SQG table: |label| <= 5.5); larger tables use the FP32 path.
FP8_EXACT_MAX_LABEL = 6.0
_OUT = {torch.bfloat16: 0, torch.float32: 1}


def _check_lut(lut: torch.Tensor, device) -> torch.Tensor:
    if lut.dtype != torch.uint8 or lut.numel() != 1 << 16:
        raise ValueError("decode LUT must be uint8[65536] E4M3 bytes")
    lut = _lut_on(lut.reshape(-1), torch.device(device))
    if lut.data_ptr() % 16:
        lut = lut.clone()
    return lut


def _scale(v: torch.Tensor, n: int, device, divide: float = 1.0) -> torch.Tensor:
    if v.ndim != 1 or v.numel() != n:
        raise ValueError(f"scale vector must contain exactly {n} values")
    return (v.to(device=device, dtype=torch.float32) / divide).contiguous()


def _run(jobs: list, bits: int, lut: torch.Tensor, out_dtype, device) -> None:
    if not jobs:
        return
    lib = _native.lib()
    arr = (_native.DecodeJob * len(jobs))(*jobs)
    need = int(lib.qsrt_decode_workspace_bytes(len(jobs)))
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=device)
    exact_fp8 = int(_lut_abs_max(lut) <= FP8_EXACT_MAX_LABEL)
    _native.check(
        lib.qsrt_decode(ctypes.cast(arr, ctypes.c_void_p), len(jobs), bits, lut.data_ptr(), exact_fp8,
                        _OUT[out_dtype], ws.data_ptr(), ws.numel(), _native.stream_handle(device)),
        "qsrt_decode",
    )


def decode_words(words: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, bits: int, lut: torch.Tensor, *,
                 out_dtype=torch.bfloat16, out: torch.Tensor | None = None) -> torch.Tensor:
    """``[K/16, N/16, 16 bits]`` int16 EXL words + ``suh [K]``, ``svh [N]`` ->
    ``[K, N]`` weights in ``out_dtype`` (bf16 or f32)."""

    if not words.is_cuda:
        raise ValueError("decode_words runs on the GPU; move the payload to a CUDA device")
    if words.dtype != torch.int16 or words.ndim != 3 or words.shape[2] != 16 * bits:
        raise ValueError("words must be int16 [K/16, N/16, 16 * bits]")
    if out_dtype not in _OUT:
        raise ValueError("out_dtype must be torch.bfloat16 or torch.float32")
    kt, nt, _ = words.shape
    k, n = 16 * kt, 16 * nt
    if k % 128 or n % 128:
        raise ValueError("decode needs K and N multiples of 128")
    dev = words.device
    words = words.contiguous()
    lut = _check_lut(lut, dev)
    su = _scale(suh, k, dev, 128.0)
    sv = _scale(svh, n, dev)
    if out is None:
        out = torch.empty((k, n), dtype=out_dtype, device=dev)
    elif out.shape != (k, n) or out.dtype != out_dtype or out.stride(1) != 1:
        raise ValueError("out must be a row-major [K, N] tensor of out_dtype")
    job = _native.DecodeJob(words.data_ptr(), nt * 16 * bits, 16 * bits, su.data_ptr(), sv.data_ptr(),
                            out.data_ptr(), out.stride(0), k, n, 0, 0)
    _run([job], bits, lut, out_dtype, dev)
    return out


def record_jobs(words_ptr: int, record_bits, rate_axis: str, k: int, n: int, su: torch.Tensor, sv: torch.Tensor,
                out: torch.Tensor) -> tuple[dict[int, list], int]:
    """Decode jobs of one record-major payload (``pack_qsrt_trellis`` layout:
    records of 128 rate-axis channels, each ``[tiles, 16 K]`` words in
    row-major tile order), grouped by rate.  A run of consecutive same-rate
    records is one job: along K the run is a contiguous row strip, along N its
    records are the block columns (one record apart in the payload).
    Returns the jobs by rate and the number of int16 words the records use."""

    from .qsrt import TILE_CHANNELS, TILES_PER_RECORD_AXIS

    esize = out.element_size()
    kt, nt = k // TILE_CHANNELS, n // TILE_CHANNELS
    other = nt if rate_axis == "k" else kt
    runs = []  # [bits, first record, word offset, records]
    cursor = 0
    for record, bits in enumerate(record_bits):
        if runs and runs[-1][0] == bits:
            runs[-1][3] += 1
        else:
            runs.append([bits, record, cursor, 1])
        cursor += TILES_PER_RECORD_AXIS * other * 16 * bits
    by_bits: dict[int, list] = {}
    for bits, first, offset, count in runs:
        r0 = first * TILES_PER_RECORD_AXIS * TILE_CHANNELS
        wpt = 16 * bits
        if rate_axis == "k":
            job = _native.DecodeJob(words_ptr + 2 * offset, nt * wpt, wpt, su.data_ptr() + 4 * r0, sv.data_ptr(),
                                    out.data_ptr() + esize * r0 * out.stride(0), out.stride(0), 128 * count, n, 0, 0)
        else:
            job = _native.DecodeJob(words_ptr + 2 * offset, TILES_PER_RECORD_AXIS * wpt, wpt, su.data_ptr(),
                                    sv.data_ptr() + 4 * r0, out.data_ptr() + esize * r0, out.stride(0), k,
                                    128 * count, 8 * TILES_PER_RECORD_AXIS * wpt, TILES_PER_RECORD_AXIS * kt * wpt)
        by_bits.setdefault(bits, []).append(job)
    return by_bits, cursor


def decode_packed(packed, suh: torch.Tensor, svh: torch.Tensor, luts_by_bits: dict, *, out_dtype=torch.bfloat16,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """Mixed-rate ``PackedQSRTTrellis`` -> ``[K, N]`` weights: every 128-channel
    record along the rate axis is decoded at its own rate (one launch per
    rate)."""

    from .qsrt import TILE_CHANNELS, record_bits

    packed.validate()
    d = packed.descriptor
    payload = packed.payload
    if not payload.is_cuda:
        raise ValueError("decode_packed runs on the GPU; move the payload to a CUDA device")
    dev = payload.device
    k, n = d.k_tiles * TILE_CHANNELS, d.n_tiles * TILE_CHANNELS
    su = _scale(suh, k, dev, 128.0)
    sv = _scale(svh, n, dev)
    if out is None:
        out = torch.empty((k, n), dtype=out_dtype, device=dev)
    elif out.shape != (k, n) or out.dtype != out_dtype or out.stride(1) != 1:
        raise ValueError("out must be a row-major [K, N] tensor of out_dtype")
    by_bits, used = record_jobs(payload.data_ptr(), record_bits(d.mode), d.rate_axis, k, n, su, sv, out)
    if used != payload.numel():
        raise ValueError("QSRT trellis payload has trailing data")
    for bits, jobs in sorted(by_bits.items()):
        _run(jobs, bits, _check_lut(luts_by_bits[bits], dev), out_dtype, dev)
    return out


class DecodePlan:
    """A fixed set of payloads decoded again and again: the job table of each
    rate is validated and uploaded once (``qsrt_decode_prepare``) and
    ``run()`` is one launch per rate (``qsrt_decode_execute``).

    ``matrices`` is a list of ``(words [K/16, N/16, 16 bits], su f32 [K] (already
    divided by 128), sv f32 [N], out [K, N])`` at the uniform rate ``bits``;
    :meth:`for_records` builds a plan over mixed-rate record-major payloads."""

    def __init__(self, matrices: list | None, bits: int | None, lut: torch.Tensor | None, *, out_dtype=torch.bfloat16,
                 _jobs_by_bits: dict | None = None, _luts: dict | None = None, _device=None, _keep=None):
        if _jobs_by_bits is None:
            if not matrices:
                raise ValueError("empty decode plan")
            jobs = []
            for words, su, sv, out in matrices:
                kt, nt, wpt = words.shape
                if wpt != 16 * bits or out.shape != (16 * kt, 16 * nt) or out.dtype != out_dtype:
                    raise ValueError("decode plan entry does not match its output")
                jobs.append(_native.DecodeJob(words.data_ptr(), nt * 16 * bits, 16 * bits, su.data_ptr(),
                                              sv.data_ptr(), out.data_ptr(), out.stride(0), 16 * kt, 16 * nt, 0, 0))
            _jobs_by_bits = {bits: jobs}
            _device = matrices[0][0].device
            _luts = {bits: lut}
            _keep = matrices
        if out_dtype not in _OUT:
            raise ValueError("out_dtype must be torch.bfloat16 or torch.float32")
        self.device, self.out_dtype, self._keep = _device, out_dtype, _keep
        lib = _native.lib()
        stream = _native.stream_handle(_device)
        self._plans = []
        for bits, jobs in sorted(_jobs_by_bits.items()):
            lut = _check_lut(_luts[bits], _device)
            arr = (_native.DecodeJob * len(jobs))(*jobs)
            ws = torch.empty(max(int(lib.qsrt_decode_workspace_bytes(len(jobs))), 16), dtype=torch.uint8,
                             device=_device)
            plan = _native.DecodePlanStruct()
            _native.check(lib.qsrt_decode_prepare(ctypes.cast(arr, ctypes.c_void_p), len(jobs), bits, ws.data_ptr(),
                                                  ws.numel(), ctypes.byref(plan), stream), "qsrt_decode_prepare")
            self._plans.append((plan, lut, ws, int(_lut_abs_max(lut) <= FP8_EXACT_MAX_LABEL)))

    @classmethod
    def for_records(cls, payloads: list, luts_by_bits: dict, *, out_dtype=torch.bfloat16) -> "DecodePlan":
        """``payloads``: ``(words int16 (flat, record-major), record_bits, rate_axis, su f32 [K] / 128,
        sv f32 [N], out [K, N])`` tuples."""

        if not payloads:
            raise ValueError("empty decode plan")
        merged: dict[int, list] = {}
        for words, rbits, axis, su, sv, out in payloads:
            if out.dtype != out_dtype or out.stride(1) != 1:
                raise ValueError("decode plan outputs must be row-major tensors of out_dtype")
            k, n = out.shape
            jobs, used = record_jobs(words.data_ptr(), tuple(rbits), axis, k, n, su, sv, out)
            if used != words.numel():
                raise ValueError("record payload length does not match its rates")
            for bits, js in jobs.items():
                merged.setdefault(bits, []).extend(js)
        return cls(None, None, None, out_dtype=out_dtype, _jobs_by_bits=merged,
                   _luts={b: luts_by_bits[b] for b in merged}, _device=payloads[0][0].device, _keep=payloads)

    def run(self) -> None:
        lib = _native.lib()
        stream = _native.stream_handle(self.device)
        for plan, lut, _ws, fp8 in self._plans:
            _native.check(lib.qsrt_decode_execute(ctypes.byref(plan), lut.data_ptr(), fp8, _OUT[self.out_dtype],
                                                  stream), "qsrt_decode_execute")
