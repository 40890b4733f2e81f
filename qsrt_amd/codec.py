"""GPU payload codec: EXL word packing and cyclic-state unpacking via the
HIP kernels ``qsrt_pack_edges`` / ``qsrt_unpack_states``."""

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
