"""Record-major packing of the layer's payloads (bench.pack_records): each
128-channel record's tiles, row-major within the record, packed at the
record's rate and concatenated in record order -- checked against packing
every record on its own and against the oracle's record reader, for records
along both axes and a rate schedule with runs and a lone record."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from oracle import fmt as ofmt
from qsrt_amd.exl3_reference import reconstruct_trellis_states
from qsrt_amd.qsrt import pack_trellis_edges


@pytest.mark.parametrize("axis", ["k", "n"])
def test_record_packing_equals_per_record_packing(axis):
    bits = (3, 3, 3, 4, 4, 3, 2, 3)
    tk, tn = (64, 24) if axis == "k" else (24, 64)
    g = torch.Generator().manual_seed(7)
    edges = torch.randint(0, 16, (tk, tn, 256), generator=g)
    rows = torch.arange(tk)[:, None] if axis == "k" else torch.arange(tn)[None, :]
    rate = torch.tensor(bits)[(rows // 8).expand(tk, tn)]
    states = reconstruct_trellis_states(edges & ((1 << rate) - 1)[..., None], 4)  # any 16-bit cyclic states
    states = states & 0x7FFF
    dim = 0 if axis == "k" else 1
    want = torch.cat([pack_trellis_edges(states.narrow(dim, 8 * r, 8).reshape(-1, 256), b).reshape(-1)
                      for r, b in enumerate(bits)])
    got = bench.pack_records(states, axis, bits)
    assert torch.equal(got, want)
    # the oracle's container reader recovers each tile's low K bits at its record's rate
    back, tile_bits = ofmt.unpack_records(got.numpy(), bits, axis, tk, tn)
    mask = (1 << np.asarray(tile_bits)) - 1
    assert np.array_equal(back & mask[..., None], states.numpy() & mask[..., None])
