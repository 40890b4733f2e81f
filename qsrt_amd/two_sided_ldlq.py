"""Two-sided block error feedback for a fixed tile quantizer (mirrors
``qsrt/two_sided_ldlq.py``).

BlockLDLQ feeds committed error along the input coordinates only; the
two-sided recurrence adds a strict block factor along the output coordinates
(a Kronecker-factored loss metric).  Blocks are visited by anti-diagonals from
the last one: blocks on one anti-diagonal do not depend on each other, so each
anti-diagonal is one batched step —

* one batched product ``L_out[:, o]^T R[:, i]`` for all its blocks (factors
  with their on- and above-diagonal blocks zeroed, so the full-length product
  equals the sliced one),
* one call of the tile quantizer on all its targets,
* one batched input-feedback update ``R[o, :] += E (o, i) L_in[i, :]`` into
  the disjoint row blocks of the running right-compensated error ``R``.

The quantizer callback maps source-oriented ``[n, b, b]`` tiles to
``(reconstruction [n, b, b], codes [n, ...])``.
"""

from __future__ import annotations

from collections.abc import Callable
from typing import TypeAlias

import torch

TileQuantizer: TypeAlias = Callable[[torch.Tensor], tuple[torch.Tensor, torch.Tensor]]


def _validate_factor(factor: torch.Tensor, *, dimension: int, block_size: int, role: str) -> None:
    if factor.ndim != 2 or factor.shape != (dimension, dimension) or not torch.is_floating_point(factor):
        raise ValueError(f"{role} factor must be a floating-point {dimension} by {dimension} matrix")
    if factor.device.type != "meta" and not bool(torch.isfinite(factor).all()):
        raise ValueError(f"{role} factor must contain only finite values")
    blocks = factor.reshape(dimension // block_size, block_size, dimension // block_size, block_size)
    diagonal = torch.diagonal(blocks, dim1=0, dim2=2)
    if bool(torch.count_nonzero(diagonal)):
        raise ValueError(f"{role} factor must have zero {block_size}-coordinate diagonal blocks")


def validate_two_sided_inputs(source_weight: torch.Tensor, input_factor: torch.Tensor, output_factor: torch.Tensor, *,
                              block_size: int) -> None:
    """Check a source-oriented ``[output, input]`` matrix and its strict block
    factors (reference two_sided_ldlq.py:57-101)."""

    if (source_weight.ndim != 2 or not torch.is_floating_point(source_weight) or source_weight.device.type == "meta"
            or not bool(torch.isfinite(source_weight).all())):
        raise ValueError("source weight must be a finite floating-point matrix")
    if isinstance(block_size, bool) or not isinstance(block_size, int):
        raise TypeError("block_size must be an integer")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    out_dim, in_dim = source_weight.shape
    if out_dim % block_size or in_dim % block_size:
        raise ValueError("source dimensions must contain complete square blocks")
    if (source_weight.device != input_factor.device or source_weight.device != output_factor.device
            or source_weight.dtype != input_factor.dtype or source_weight.dtype != output_factor.dtype):
        raise ValueError("source weight and factors must share device and dtype")
    _validate_factor(input_factor, dimension=in_dim, block_size=block_size, role="input")
    _validate_factor(output_factor, dimension=out_dim, block_size=block_size, role="output")


def _strictly_lower_blocks(factor: torch.Tensor, block_size: int) -> torch.Tensor:
    """``factor`` with every block on or above the block diagonal set to 0."""

    n = factor.shape[0] // block_size
    block_row = torch.arange(factor.shape[0], device=factor.device) // block_size
    mask = block_row[:, None] > block_row[None, :]
    if n and bool((factor.masked_fill(mask, 0) != 0).any()):
        factor = factor * mask
    return factor.contiguous()


def _blocks(matrix: torch.Tensor, block_size: int) -> torch.Tensor:
    rows, cols = matrix.shape
    return matrix.view(rows // block_size, block_size, cols // block_size, block_size).permute(0, 2, 1, 3)


def two_sided_block_ldlq(source_weight: torch.Tensor, input_factor: torch.Tensor, output_factor: torch.Tensor,
                         quantize_tiles: TileQuantizer, *, block_size: int = 16,
                         feedback_multiplier: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize blocks with input- and output-direction error feedback
    (reference two_sided_ldlq.py:104-240).

    ``source_weight`` is ``[output, input]``; ``input_factor`` and
    ``output_factor`` are the strict lower block LDL factors of the two
    Kronecker metrics (zero diagonal blocks).  Target of block ``(o, i)``:
    ``W + m (R[o, i] + L_out[o+:, o]^T R[o+:, i])`` with ``R = E (I + L_in)``
    over the blocks committed so far.  Returns the reconstruction and the codes
    as ``[output blocks, input blocks, ...]``.
    """

    validate_two_sided_inputs(source_weight, input_factor, output_factor, block_size=block_size)
    if not callable(quantize_tiles):
        raise TypeError("quantize_tiles must be callable")
    if (isinstance(feedback_multiplier, bool) or not isinstance(feedback_multiplier, (int, float))
            or not 0.0 <= float(feedback_multiplier) <= 1.0):
        raise ValueError("feedback_multiplier must be a real number in [0, 1]")
    m = float(feedback_multiplier)
    bs = block_size
    out_dim, in_dim = source_weight.shape
    ob, ib = out_dim // bs, in_dim // bs
    device = source_weight.device
    l_out = _strictly_lower_blocks(output_factor, bs)
    l_in = _strictly_lower_blocks(input_factor, bs)
    l_out_cols = l_out.view(out_dim, ob, bs)                      # [:, o, :] = column block o
    l_in_rows = l_in.view(ib, bs, in_dim)                         # [i] = row block i
    source_blocks = _blocks(source_weight, bs)
    reconstructed = torch.zeros_like(source_weight)
    recon_blocks = _blocks(reconstructed, bs)
    right = torch.zeros_like(source_weight)                       # R = E (I + L_in), running
    right_rows = right.view(ob, bs, in_dim)
    right_cols = right.view(out_dim, ib, bs)
    stored_codes: torch.Tensor | None = None

    for diagonal in range(ob + ib - 2, -1, -1):
        outs = torch.arange(max(0, diagonal - ib + 1), min(ob, diagonal + 1), device=device)
        ins = diagonal - outs
        n = outs.numel()
        sources = source_blocks[outs, ins]                         # [n, b, b]
        if m == 0.0:
            targets = sources.contiguous()
        else:
            feedback = _blocks(right, bs)[outs, ins]               # R[o, i]
            lo = l_out_cols[:, outs].permute(1, 2, 0).contiguous()  # [n, b, out]: L_out[:, o]^T
            ri = right_cols[:, ins].permute(1, 0, 2).contiguous()   # [n, out, b]: R[:, i]
            feedback = feedback + torch.bmm(lo, ri)
            targets = sources + m * feedback
        quantized, codes = quantize_tiles(targets)
        if quantized.shape != targets.shape:
            raise ValueError("tile quantizer returned reconstructions with the wrong shape")
        if (quantized.device != device or quantized.dtype != source_weight.dtype
                or not bool(torch.isfinite(quantized).all())):
            raise ValueError("tile quantizer reconstructions must be finite and match the source")
        if codes.ndim < 1 or codes.shape[0] != n:
            raise ValueError("tile quantizer returned codes with the wrong batch size")
        if stored_codes is None:
            stored_codes = torch.empty((ob, ib, *codes.shape[1:]), dtype=codes.dtype, device=codes.device)
        elif stored_codes.shape[2:] != codes.shape[1:] or stored_codes.dtype != codes.dtype or \
                stored_codes.device != codes.device:
            raise ValueError("tile quantizer changed its code shape, dtype, or device")
        # Commit the whole anti-diagonal, then feed its error forward.
        recon_blocks[outs, ins] = quantized
        stored_codes[outs.to(codes.device), ins.to(codes.device)] = codes
        error = sources - quantized                                # [n, b, b]
        update = torch.bmm(error.contiguous(), l_in_rows[ins])    # [n, b, in]: E L_in[i, :] (zero from block i on)
        rows = right_rows[outs]
        rows += update
        rows.view(n, bs, ib, bs)[torch.arange(n, device=device), :, ins] += error
        right_rows[outs] = rows

    if stored_codes is None:
        raise AssertionError("two-sided traversal did not visit any blocks")
    return reconstructed, stored_codes


def kronecker_quadratic_loss(error: torch.Tensor, input_metric: torch.Tensor, output_metric: torch.Tensor) -> torch.Tensor:
    """``tr(H_out E H_in E^T)`` of a source-oriented error."""

    if error.ndim != 2 or not torch.is_floating_point(error):
        raise TypeError("error must be a floating-point matrix")
    out_dim, in_dim = error.shape
    if input_metric.shape != (in_dim, in_dim):
        raise ValueError("input metric does not match the error input dimension")
    if output_metric.shape != (out_dim, out_dim):
        raise ValueError("output metric does not match the error output dimension")
    return torch.sum((output_metric @ error @ input_metric) * error)


__all__ = ["kronecker_quadratic_loss", "two_sided_block_ldlq", "validate_two_sided_inputs"]
