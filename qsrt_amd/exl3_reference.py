"""Codec definitions: cyclic states, tensor-core order, Hadamard, decode.

Mirrors ``qsrt/exl3_reference.py``.  These functions define the stored
format; they accept CPU or GPU tensors like the reference.  The serving-
grade decode of a packed matrix to bf16 is the HIP kernel behind
``qsrt_decode_bf16`` (see ``qsrt_amd.decode``), which is checked against
these definitions.
"""

from __future__ import annotations

import math
from functools import lru_cache

import torch

from .sqg_e4m3 import SQG_CHEB_NORMAL_E4M3, SQG_NORMAL_E4M3, SQG_XOR_CHEB_T12, sqg_codebook

TILE_VALUES = 256
HADAMARD_BLOCK = 128
CODEBOOK_SQG_NORMAL_E4M3 = SQG_NORMAL_E4M3
CODEBOOK_SQG_XOR_CHEB_T12 = SQG_XOR_CHEB_T12
CODEBOOK_SQG_CHEB_NORMAL_E4M3 = SQG_CHEB_NORMAL_E4M3
QSRT_CODEBOOKS = (CODEBOOK_SQG_XOR_CHEB_T12, CODEBOOK_SQG_NORMAL_E4M3, CODEBOOK_SQG_CHEB_NORMAL_E4M3)


def _check_bits(bits: int) -> None:
    if isinstance(bits, bool) or not isinstance(bits, int) or not 1 <= bits <= 6:
        raise ValueError("the uniform SQG reference supports K=1 through K=6")


def reconstruct_trellis_states(edge_symbols: torch.Tensor, bits: int) -> torch.Tensor:
    """Cyclic 16-bit states from K-bit edges: state i holds edge i in its low
    K bits, edge i-1 above it, ... (reference exl3_reference.py:34-58)."""

    _check_bits(bits)
    if edge_symbols.ndim < 1 or edge_symbols.shape[-1] != TILE_VALUES:
        raise ValueError("edge_symbols must have a final dimension of 256")
    if edge_symbols.dtype == torch.bool or edge_symbols.is_floating_point():
        raise TypeError("edge_symbols must use an integer dtype")
    edges = edge_symbols.to(torch.int64) & ((1 << bits) - 1)
    states = torch.zeros_like(edges)
    for lag in range(-(-16 // bits)):
        states |= torch.roll(edges, shifts=lag, dims=-1) << (lag * bits)
    return (states & 0xFFFF).to(torch.int16).contiguous()


@lru_cache(maxsize=None)
def _tc_perm_cpu() -> torch.Tensor:
    perm = torch.empty(TILE_VALUES, dtype=torch.long)
    for lane in range(32):
        r = (lane % 4) * 2
        c = lane // 4
        rows = (r, r + 1, r + 8, r + 9)
        for half, col in enumerate((c, c + 8)):
            for i, row in enumerate(rows):
                perm[lane * 8 + half * 4 + i] = row * 16 + col
    return perm


def tensor_core_permutation(device: torch.device | str = "cpu") -> torch.Tensor:
    """Row-major 16x16 index held at each tensor-core position
    (reference exl3_reference.py:86-105)."""

    return _tc_perm_cpu().to(device)


def _decode_codebook_states(states: torch.Tensor, codebook: str, *, bits: int | None = None, rate_axis=None) -> torch.Tensor:
    if codebook not in QSRT_CODEBOOKS:
        raise ValueError(f"unsupported QSRT codebook {codebook!r}; expected one of {QSRT_CODEBOOKS}")
    if bits is None:
        raise ValueError("SQG reconstruction requires an explicit trellis rate")
    _check_bits(bits)
    values = sqg_codebook(bits, codebook, rate_axis=rate_axis, device=states.device, dtype=torch.float16)
    index = (states.to(torch.int64) & 0xFFFF).flatten()
    return values.index_select(0, index).reshape(states.shape)


def _tiles_to_matrix(decoded: torch.Tensor) -> torch.Tensor:
    inverse = torch.argsort(tensor_core_permutation(decoded.device))
    decoded = decoded.index_select(-1, inverse)
    kt, nt, _ = decoded.shape
    return decoded.reshape(kt, nt, 16, 16).permute(0, 2, 1, 3).reshape(kt * 16, nt * 16).contiguous()


def decode_regularized_weight(
    states: torch.Tensor,
    *,
    codebook: str = CODEBOOK_SQG_XOR_CHEB_T12,
    codebook_values: torch.Tensor | None = None,
    bits: int | None = None,
) -> torch.Tensor:
    """``[K/16, N/16, 256]`` states -> transformed ``[K, N]`` (reference :108-140)."""

    if states.ndim != 3 or states.shape[-1] != TILE_VALUES:
        raise ValueError("states must have shape [K/16, N/16, 256]")
    if codebook_values is None:
        decoded = _decode_codebook_states(states, codebook, bits=bits).float()
    else:
        if codebook_values.ndim != 1 or codebook_values.numel() != 1 << 16:
            raise ValueError("custom codebook must contain exactly 65,536 values")
        if not codebook_values.is_floating_point():
            raise TypeError("custom codebook must be floating point")
        if not bool(torch.isfinite(codebook_values).all()):
            raise ValueError("custom codebook must be finite")
        index = (states.to(torch.int64) & 0xFFFF).flatten()
        decoded = codebook_values.to(states.device).index_select(0, index).reshape(states.shape).float()
    return _tiles_to_matrix(decoded)


def decode_qsrt_regularized_weight(
    states: torch.Tensor, *, rate_axis: str, tile_bits: tuple[int, ...], codebook: str
) -> torch.Tensor:
    """Mixed-rate variant: each tile decodes with its own K table
    (reference exl3_reference.py:143-207)."""

    if states.ndim != 3 or states.shape[-1] != TILE_VALUES:
        raise ValueError("states must have shape [K/16, N/16, 256]")
    if rate_axis not in ("k", "n", "tile"):
        raise ValueError("rate_axis must be 'k', 'n', or 'tile'")
    axis = 0 if rate_axis == "k" else 1
    expected = states.shape[0] * states.shape[1] if rate_axis == "tile" else states.shape[axis]
    if len(tile_bits) != expected:
        raise ValueError("tile_bits length does not match the selected rate axis")
    if any(isinstance(b, bool) or not isinstance(b, int) or b not in (1, 2, 3, 4) for b in tile_bits):
        raise ValueError("tile_bits must contain only integer K1 through K4")
    if codebook not in QSRT_CODEBOOKS:
        raise ValueError(f"unsupported QSRT codebook: {codebook}")
    decoded = torch.empty(states.shape, dtype=torch.float32, device=states.device)
    bits_t = torch.tensor(tile_bits, dtype=torch.long, device=states.device)
    for bits in sorted(set(tile_bits)):
        where = torch.nonzero(bits_t == bits).flatten()
        if rate_axis == "tile":
            flat = decoded.view(-1, TILE_VALUES)
            sel = states.reshape(-1, TILE_VALUES).index_select(0, where)
            flat.index_copy_(0, where, _decode_codebook_states(sel, codebook, bits=bits).float())
        else:
            sel = states.index_select(axis, where)
            decoded.index_copy_(axis, where, _decode_codebook_states(sel, codebook, bits=bits, rate_axis=rate_axis).float())
    return _tiles_to_matrix(decoded)


def normalized_hadamard(*, device, dtype: torch.dtype = torch.float32, size: int = HADAMARD_BLOCK) -> torch.Tensor:
    """Sylvester Hadamard scaled by 1/sqrt(size) (reference :210-227)."""

    if size <= 0 or size & (size - 1):
        raise ValueError("Hadamard size must be a positive power of two")
    idx = torch.arange(size)
    parity = torch.zeros(size, size, dtype=torch.int64)
    x = idx[:, None] & idx[None, :]
    while bool(x.any()):
        parity ^= x & 1
        x = x >> 1
    h = 1.0 - 2.0 * parity.to(torch.float64)
    return (h / math.sqrt(size)).to(dtype=dtype, device=device)


def _blockwise_hadamard_left(weight: torch.Tensor) -> torch.Tensor:
    if weight.shape[0] % HADAMARD_BLOCK:
        raise ValueError("EXL K dimension must be divisible by 128")
    h = normalized_hadamard(device=weight.device, dtype=weight.dtype)
    return torch.matmul(h, weight.reshape(-1, HADAMARD_BLOCK, weight.shape[1])).reshape(weight.shape).contiguous()


def _blockwise_hadamard_right(weight: torch.Tensor) -> torch.Tensor:
    if weight.shape[1] % HADAMARD_BLOCK:
        raise ValueError("EXL N dimension must be divisible by 128")
    h = normalized_hadamard(device=weight.device, dtype=weight.dtype)
    return torch.matmul(weight.reshape(weight.shape[0], -1, HADAMARD_BLOCK), h).reshape(weight.shape).contiguous()


def qsrt_regularized_target(encoder_weight: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor) -> torch.Tensor:
    """Encoder-coordinate weight -> trellis objective basis (reference :246-277)."""

    if encoder_weight.ndim != 2:
        raise ValueError("encoder weight must be two-dimensional")
    if suh.ndim != 1 or svh.ndim != 1 or suh.numel() != encoder_weight.shape[0] or svh.numel() != encoder_weight.shape[1]:
        raise ValueError("QSRT scale vectors do not match the encoder weight")
    if not all(torch.is_floating_point(v) for v in (encoder_weight, suh, svh)):
        raise TypeError("QSRT target and scales must be floating point")
    if not all(bool(torch.isfinite(v).all()) for v in (encoder_weight, suh, svh)):
        raise ValueError("QSRT target and scales must be finite")
    if bool((suh == 0).any()) or bool((svh == 0).any()):
        raise ValueError("QSRT scales must be nonzero")
    target = _blockwise_hadamard_right(encoder_weight.float() / svh.float().unsqueeze(0))
    return _blockwise_hadamard_left(target / suh.float().unsqueeze(1)).contiguous()


def _apply_scales(weight: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor) -> torch.Tensor:
    if suh.ndim != 1 or suh.numel() != weight.shape[0]:
        raise ValueError("suh length does not match the EXL K dimension")
    if svh.ndim != 1 or svh.numel() != weight.shape[1]:
        raise ValueError("svh length does not match the EXL N dimension")
    weight = _blockwise_hadamard_left(weight)
    weight *= suh.to(device=weight.device, dtype=weight.dtype).unsqueeze(1)
    weight = _blockwise_hadamard_right(weight)
    weight *= svh.to(device=weight.device, dtype=weight.dtype).unsqueeze(0)
    return weight.contiguous()


def decode_exl3_weight(
    states: torch.Tensor,
    suh: torch.Tensor,
    svh: torch.Tensor,
    *,
    codebook: str = CODEBOOK_SQG_XOR_CHEB_T12,
    codebook_values: torch.Tensor | None = None,
    bits: int | None = None,
) -> torch.Tensor:
    """States + scales -> EXL ``[K, N]`` weight (reference :280-302)."""

    weight = decode_regularized_weight(states, codebook=codebook, codebook_values=codebook_values, bits=bits)
    return _apply_scales(weight, suh, svh)


def decode_qsrt_weight(
    states: torch.Tensor,
    suh: torch.Tensor,
    svh: torch.Tensor,
    *,
    rate_axis: str,
    tile_bits: tuple[int, ...],
    codebook: str = CODEBOOK_SQG_XOR_CHEB_T12,
) -> torch.Tensor:
    """Mixed-rate states + scales -> EXL ``[K, N]`` weight (reference :305-330)."""

    weight = decode_qsrt_regularized_weight(states, rate_axis=rate_axis, tile_bits=tile_bits, codebook=codebook)
    return _apply_scales(weight, suh, svh)
