"""GPU payload codec kernels vs the reference formulation and the oracle."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import fmt as ofmt
from qsrt_amd import qsrt as Q
from qsrt_amd.exl3_reference import reconstruct_trellis_states

pytestmark = pytest.mark.gpu

KAT = {
    2: [6939] * 6,
    3: [30469, 1337, 1337, 14711, 14711, 30469],
    4: [17767, 291, -12817, -30293, 17767, 291],
}


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_gpu_pack_known_answer_and_round_trip(bits):
    print(f"[codec] K{bits}", file=sys.stderr, flush=True)
    idx = (torch.arange(256, dtype=torch.int16) % (1 << bits))[None]
    packed = Q.pack_trellis_edges(idx.cuda(), bits)
    assert packed.is_cuda and packed[0, :6].tolist() == KAT[bits]
    g = torch.Generator().manual_seed(10 + bits)
    edges = torch.randint(0, 1 << bits, (37, 3, 256), generator=g)
    states = reconstruct_trellis_states(edges, bits)
    gpu_words = Q.pack_trellis_edges(states.cuda(), bits).cpu()
    assert torch.equal(gpu_words, Q.pack_trellis_edges(states, bits))
    assert np.array_equal(gpu_words.numpy().view(np.uint16), ofmt.pack_words(states.numpy(), bits))
    back = Q.unpack_trellis_states(gpu_words.cuda(), bits).cpu()
    assert torch.equal(back, states)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_gpu_unpack_of_arbitrary_words_matches_reference(bits):
    g = torch.Generator().manual_seed(20 + bits)
    words = torch.randint(-32768, 32768, (513, 16 * bits), generator=g, dtype=torch.int32).to(torch.int16)
    want = Q.unpack_trellis_states(words, bits)
    got = Q.unpack_trellis_states(words.cuda(), bits).cpu()
    assert torch.equal(got, want)


def test_gpu_matrix_payload_round_trip():
    geo = Q.Geometry(512, 256)
    mode = Q.resolve_mode("R1", geo)
    g = torch.Generator().manual_seed(3)
    states = torch.empty((16, 32, 256), dtype=torch.int16)
    for r, bits in enumerate(Q.record_bits(mode)):
        e = torch.randint(0, 1 << bits, (16, 8, 256), generator=g)
        states[:, 8 * r:8 * r + 8] = reconstruct_trellis_states(e, bits)
    cpu = Q.pack_qsrt_trellis(states, mode, rate_axis="n")
    gpu = Q.pack_qsrt_trellis(states.cuda(), mode, rate_axis="n")
    assert torch.equal(gpu.payload.cpu(), cpu.payload)
    assert torch.equal(Q.unpack_qsrt_trellis_states(gpu).cpu(), states)
