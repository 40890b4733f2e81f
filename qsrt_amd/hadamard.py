"""Blockwise normalised Hadamard rotations of 128-row or 128-column blocks."""

from __future__ import annotations

import torch

from .exl3_reference import normalized_hadamard


def rotate_(x: torch.Tensor, block: int = 128, *, side: str) -> torch.Tensor:
    """In place: ``x[blk] = H @ x[blk]`` per ``block`` rows (``side="left"``)
    or ``x[:, blk] = x[:, blk] @ H`` per ``block`` columns (``"right"``)."""

    if x.dtype != torch.float32 or x.ndim != 2:
        raise ValueError("Hadamard rotation expects a float32 matrix")
    h = normalized_hadamard(device=x.device, dtype=x.dtype, size=block)
    k, n = x.shape
    if side == "left":
        if k % block:
            raise ValueError("row count must be a multiple of the Hadamard block")
        x.copy_(torch.matmul(h, x.view(k // block, block, n)).view(k, n))
    elif side == "right":
        if n % block:
            raise ValueError("column count must be a multiple of the Hadamard block")
        x.copy_(torch.matmul(x.view(k, n // block, block), h).view(k, n))
    else:
        raise ValueError("side must be 'left' or 'right'")
    return x
