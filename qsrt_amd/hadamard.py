"""Blockwise normalised Hadamard rotations (128-row/column blocks for the
EXL basis, 512/128 for the coupled expert basis).

Device tensors run the HIP butterfly kernel behind ``qsrt_hadamard`` (FP32)
or ``qsrt_hadamard_f64`` (float64, the encoder's regularisation)
(``include/qsrt_amd.h``); the optional per-index vectors fuse the sign and
scale multiplies that surround each rotation.  CPU tensors use the same
matrix definition with torch (the reference's functions accept both).
"""

from __future__ import annotations

import torch

from . import _native
from .exl3_reference import normalized_hadamard

_SIDES = {"left": 0, "right": 1}
BLOCKS = (64, 128, 256, 512)


def _vec(v, n: int, x: torch.Tensor):
    if v is None:
        return None
    v = v.reshape(-1)
    if v.numel() != n:
        raise ValueError("scale vector does not align with the rotated axis")
    if v.device != x.device or v.dtype != x.dtype or not v.is_contiguous():
        v = v.to(device=x.device, dtype=x.dtype).contiguous()
    return v


def rotate_(x: torch.Tensor, block: int = 128, *, side: str, pre_mul=None, pre_div=None, post_mul=None) -> torch.Tensor:
    """In place: ``x[blk] = post_mul * (H @ (x[blk] * pre_mul / pre_div))``
    per ``block`` rows (``side="left"``), or the same per ``block`` columns
    with ``x[:, blk] @ H`` (``side="right"``).  Vectors are indexed along
    the rotated axis and taken in ``x``'s dtype (float32 or float64)."""

    if x.dtype not in (torch.float32, torch.float64) or x.ndim != 2:
        raise ValueError("Hadamard rotation expects a float32 or float64 matrix")
    if side not in _SIDES:
        raise ValueError("side must be 'left' or 'right'")
    k, n = x.shape
    ext = k if side == "left" else n
    if block not in BLOCKS:
        raise ValueError(f"Hadamard block must be one of {BLOCKS}")
    if ext % block:
        raise ValueError("row count must be a multiple of the Hadamard block" if side == "left"
                         else "column count must be a multiple of the Hadamard block")
    pre_mul, pre_div, post_mul = (_vec(v, ext, x) for v in (pre_mul, pre_div, post_mul))
    if x.is_cuda:
        if x.numel() == 0:
            return x
        if x.stride(1) != 1 or x.stride(0) % 4 or n % 4 or x.data_ptr() % 16:
            raise ValueError("device Hadamard needs a row-major, 16-byte aligned matrix with columns % 4 == 0")
        lib = _native.lib()
        entry = lib.qsrt_hadamard if x.dtype == torch.float32 else lib.qsrt_hadamard_f64
        _native.check(
            entry(
                x.data_ptr(), k, n, x.stride(0), block, _SIDES[side],
                None if pre_mul is None else pre_mul.data_ptr(),
                None if pre_div is None else pre_div.data_ptr(),
                None if post_mul is None else post_mul.data_ptr(),
                _native.stream_handle(x.device),
            ),
            "qsrt_hadamard" if x.dtype == torch.float32 else "qsrt_hadamard_f64",
        )
        return x
    shape = (ext, 1) if side == "left" else (1, ext)
    if pre_mul is not None:
        x.mul_(pre_mul.view(shape))
    if pre_div is not None:
        x.div_(pre_div.view(shape))
    h = normalized_hadamard(device=x.device, dtype=x.dtype, size=block)
    if side == "left":
        x.copy_(torch.matmul(h, x.view(k // block, block, n)).view(k, n))
    else:
        x.copy_(torch.matmul(x.view(k, n // block, block), h).view(k, n))
    if post_mul is not None:
        x.mul_(post_mul.view(shape))
    return x
