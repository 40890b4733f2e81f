"""Payload codec: EXL word packing and cyclic-state unpacking at any tile
rate K1..K6 — the HIP kernels ``qsrt_pack_edges`` / ``qsrt_unpack_states``
for device tensors, torch for host tensors.  (The QSRT container format of
``qsrt_amd.qsrt`` admits K2..K4 only; the tile quantizer and the uniform
codec paths go to K6.)"""

from __future__ import annotations

import torch

from . import _native


def pack_edges_gpu(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """``[..., 256]`` integer states on the GPU -> ``[..., 16K]`` int16 words."""

    lead = indices.shape[:-1]
    states = indices.reshape(-1, 256)
    if states.dtype != torch.int16:
        states = (states.to(torch.int64) & 0xFFFF).to(torch.int32).to(torch.int16)
    states = states.contiguous()
    n = states.shape[0]
    words = torch.empty((n, 16 * bits), dtype=torch.int16, device=states.device)
    if n:
        with torch.cuda.device(states.device):
            rc = _native.lib().qsrt_pack_edges(states.data_ptr(), n, bits, words.data_ptr(), _native.stream_handle(states.device))
        _native.check(rc, "qsrt_pack_edges")
    return words.reshape(*lead, 16 * bits)


def unpack_states_gpu(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """``[..., 16K]`` int16 words on the GPU -> ``[..., 256]`` int16 states."""

    lead = packed.shape[:-1]
    words = packed.reshape(-1, 16 * bits).contiguous()
    n = words.shape[0]
    states = torch.empty((n, 256), dtype=torch.int16, device=words.device)
    if n:
        with torch.cuda.device(words.device):
            rc = _native.lib().qsrt_unpack_states(words.data_ptr(), n, bits, states.data_ptr(), _native.stream_handle(words.device))
        _native.check(rc, "qsrt_unpack_states")
    return states.reshape(*lead, 256)


def _check_rate(bits: int) -> None:
    if isinstance(bits, bool) or not isinstance(bits, int) or not 1 <= bits <= 6:
        raise ValueError("trellis word packing supports K1 through K6")


def pack_words(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """Low K bits of 256 symbols per tile -> ``16 K`` int16 words: one
    MSB-first bitstream, 16 bits per word, adjacent words swapped."""

    _check_rate(bits)
    if indices.ndim < 1 or indices.shape[-1] != 256:
        raise ValueError("indices must have a final dimension of 256")
    if indices.dtype == torch.bool or indices.is_floating_point():
        raise TypeError("indices must use an integer dtype")
    if indices.is_cuda:
        return pack_edges_gpu(indices, bits)
    values = indices.to(torch.int64) & ((1 << bits) - 1)
    lead = values.shape[:-1]
    stream = ((values[..., None] >> torch.arange(bits - 1, -1, -1)) & 1).reshape(*lead, 256 * bits)
    words = (stream.reshape(*lead, 16 * bits, 16) << torch.arange(15, -1, -1)).sum(-1)
    return words.reshape(*lead, -1, 2).flip(-1).reshape(*lead, 16 * bits).to(torch.int16).contiguous()


def unpack_words(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """Inverse of :func:`pack_words`: the cyclic 16-bit states, int16."""

    _check_rate(bits)
    if packed.dtype != torch.int16 or packed.ndim < 1 or packed.shape[-1] != 16 * bits:
        raise ValueError(f"packed tiles must be int16 and end in {16 * bits} words")
    if packed.is_cuda:
        return unpack_states_gpu(packed, bits)
    from .exl3_reference import reconstruct_trellis_states

    lead = packed.shape[:-1]
    words = (packed.to(torch.int64) & 0xFFFF).reshape(*lead, -1, 2).flip(-1).reshape(*lead, 16 * bits)
    stream = ((words[..., None] >> torch.arange(15, -1, -1)) & 1).reshape(*lead, 256, bits)
    edges = (stream << torch.arange(bits - 1, -1, -1)).sum(-1)
    return reconstruct_trellis_states(edges, bits)
