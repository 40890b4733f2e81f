"""Uniform-rate payload codec at K1..K6 (reference qsrt_codec_pilot.py:220-281
and the EXL word order of qsrt.py:861-883): the K-generic packer agrees with
the container packer at K2..K4 and with a bit-by-bit definition at every K,
and unpacking returns the cyclic states."""

from __future__ import annotations

import pytest
import torch

from qsrt_amd import qsrt as Q
from qsrt_amd.codec import pack_words, unpack_words
from qsrt_amd.exl3_reference import reconstruct_trellis_states
from qsrt_amd.qsrt_codec_pilot import pack_uniform_trellis_edges, unpack_uniform_trellis_states


def _bitwise(edges, bits):
    """Symbol i's K bits MSB-first at stream bits [iK, iK + K); word w holds
    stream bits [16w, 16w + 16) MSB-first; adjacent words swapped."""

    out = torch.zeros(*edges.shape[:-1], 16 * bits, dtype=torch.int64)
    flat_e, flat_o = edges.reshape(-1, 256).long(), out.view(-1, 16 * bits)
    for t in range(flat_e.shape[0]):
        for i in range(256):
            for b in range(bits):
                bit = (int(flat_e[t, i]) >> (bits - 1 - b)) & 1
                pos = i * bits + b
                w = pos // 16
                flat_o[t, w ^ 1] |= bit << (15 - pos % 16)
    return out.to(torch.int16)


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6])
def test_generic_packer_matches_the_bitwise_definition(bits):
    g = torch.Generator().manual_seed(bits)
    edges = torch.randint(0, 1 << bits, (2, 256), generator=g)
    words = pack_words(edges, bits)
    assert torch.equal(words, _bitwise(edges, bits))
    states = unpack_words(words, bits)
    assert torch.equal(states, reconstruct_trellis_states(edges, bits))
    if 2 <= bits <= 4:
        assert torch.equal(words, Q.pack_trellis_edges(edges, bits))


def test_uniform_api_rate_checks():
    edges = torch.zeros(1, 1, 256, dtype=torch.int16)
    for bits in (1, 7):
        with pytest.raises(ValueError):
            pack_uniform_trellis_edges(edges, bits)
    words = pack_uniform_trellis_edges(edges, 5)
    assert words.shape == (1, 1, 80)
    assert torch.equal(unpack_uniform_trellis_states(words, 5), torch.zeros(1, 1, 256, dtype=torch.int16))
    with pytest.raises(ValueError):
        Q.pack_trellis_edges(edges, 5)  # the container format stays K2..K4
