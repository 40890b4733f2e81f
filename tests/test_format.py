"""Payload format: EXL word packing, cyclic states, tensor-core order,
matrix payloads and the reference decode (CPU).

Known answers come from the reference's own tests
(tests/test_qsrt.py:242-295, tests/test_sqg_e4m3.py:136-200)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fmt as ofmt
from oracle import tables as otables
from qsrt_amd import qsrt as Q
from qsrt_amd.exl3_reference import (
    CODEBOOK_SQG_NORMAL_E4M3,
    decode_exl3_weight,
    decode_qsrt_regularized_weight,
    decode_regularized_weight,
    normalized_hadamard,
    reconstruct_trellis_states,
    tensor_core_permutation,
)
from qsrt_amd.sqg_e4m3 import sqg_e4m3_codebook

KAT = {
    2: [6939] * 6,
    3: [30469, 1337, 1337, 14711, 14711, 30469],
    4: [17767, 291, -12817, -30293, 17767, 291],
}


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_edge_pack_known_answer_words(bits):
    indices = (torch.arange(256, dtype=torch.int16) % (1 << bits))[None]
    packed = Q.pack_trellis_edges(indices, bits)
    assert packed.shape == (1, 16 * bits)
    assert packed[0, :6].tolist() == KAT[bits]
    assert torch.equal(Q.unpack_trellis_edges(packed, bits), indices)
    oracle = ofmt.pack_words(indices.numpy(), bits).view(np.int16)
    assert oracle[0, :6].tolist() == KAT[bits]


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_edge_pack_round_trips_low_bits_and_matches_oracle(bits):
    g = torch.Generator().manual_seed(100 + bits)
    idx = torch.randint(-32768, 32768, (7, 256), generator=g)
    packed = Q.pack_trellis_edges(idx, bits)
    assert torch.equal(Q.unpack_trellis_edges(packed, bits).int(), idx.int() & ((1 << bits) - 1))
    assert np.array_equal(packed.numpy().view(np.uint16), ofmt.pack_words(idx.numpy(), bits))
    assert np.array_equal(ofmt.unpack_symbols(packed.numpy(), bits), idx.numpy() & ((1 << bits) - 1))


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_cyclic_states_closed_form_equals_scalar_recurrence(bits):
    g = torch.Generator().manual_seed(175 + bits)
    edges = torch.randint(0, 1 << bits, (3, 5, 256), generator=g)
    states = reconstruct_trellis_states(edges, bits)
    assert np.array_equal(states.numpy().view(np.uint16), ofmt.cyclic_states(edges.numpy(), bits))
    packed = Q.pack_trellis_edges(states, bits)
    assert torch.equal(Q.unpack_trellis_states(packed, bits), states)


def test_tensor_core_permutation_is_the_closed_form_bijection():
    perm = tensor_core_permutation()
    assert torch.equal(torch.sort(perm).values, torch.arange(256))
    assert np.array_equal(perm.numpy(), ofmt.tensor_core_perm())
    # a planted mistake (rows 8/9 swapped) is not the same permutation
    wrong = ofmt.tensor_core_perm().copy()
    wrong[[2, 3]] = wrong[[3, 2]]
    assert not np.array_equal(perm.numpy(), wrong)


def test_hadamard_is_orthonormal_symmetric_sylvester():
    h = normalized_hadamard(device="cpu", dtype=torch.float64, size=128)
    assert torch.allclose(h @ h.T, torch.eye(128, dtype=torch.float64), atol=1e-14)
    assert torch.equal(h, h.T)
    assert np.allclose(h.numpy(), ofmt.hadamard(128), atol=0)
    h2 = np.array([[1.0, 1.0], [1.0, -1.0]]) / np.sqrt(2.0)
    k = h2
    for _ in range(6):
        k = np.kron(k, h2)
    assert np.allclose(h.numpy(), k, atol=1e-15)


def test_reference_decoder_accepts_custom_codebook():
    # reference tests/test_sqg_e4m3.py:136-146
    states = torch.arange(256, dtype=torch.int16).reshape(1, 1, 256)
    codebook = sqg_e4m3_codebook(3, "normal")
    decoded = decode_regularized_weight(states, codebook_values=codebook)
    assert decoded.shape == (16, 16)
    assert torch.equal(torch.sort(decoded.flatten()).values, torch.sort(codebook[:256].float()).values)


@pytest.mark.parametrize("rate_axis", ("k", "n"))
def test_rate_specific_tables_compose(rate_axis):
    # reference tests/test_sqg_e4m3.py:149-173
    states = torch.arange(3 * 3 * 256, dtype=torch.int32).to(torch.int16).reshape(3, 3, 256)
    tile_bits = (1, 2, 3)
    decoded = decode_qsrt_regularized_weight(states, rate_axis=rate_axis, tile_bits=tile_bits, codebook=CODEBOOK_SQG_NORMAL_E4M3)
    axis = 0 if rate_axis == "k" else 1
    pieces = [
        decode_regularized_weight(states.narrow(axis, t, 1), codebook=CODEBOOK_SQG_NORMAL_E4M3, bits=b)
        for t, b in enumerate(tile_bits)
    ]
    assert torch.equal(decoded, torch.cat(pieces, dim=axis))


def test_decode_matches_float64_oracle():
    g = torch.Generator().manual_seed(5)
    bits = 3
    edges = torch.randint(0, 8, (16, 8, 256), generator=g)  # [K/16, N/16] = 256 x 128
    states = reconstruct_trellis_states(edges, bits)
    suh = (torch.rand(256, generator=g) + 0.5).half()
    svh = (torch.rand(128, generator=g) - 0.5).half()
    got = decode_exl3_weight(states, suh, svh, bits=bits).double().numpy()
    want = ofmt.decode(states.numpy().view(np.uint16), otables.t12_values(bits), suh.float().numpy(), svh.float().numpy())
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(want).max())


def _legal_states(shape, rbits, rate_axis, seed):
    g = torch.Generator().manual_seed(seed)
    states = torch.empty(shape, dtype=torch.int16)
    for record, bits in enumerate(rbits):
        b = record * 8
        if rate_axis == "k":
            e = torch.randint(0, 1 << bits, (8, shape[1], 256), generator=g)
            states[b:b + 8] = reconstruct_trellis_states(e, bits)
        else:
            e = torch.randint(0, 1 << bits, (shape[0], 8, 256), generator=g)
            states[:, b:b + 8] = reconstruct_trellis_states(e, bits)
    return states


@pytest.mark.parametrize(("rate_axis", "shape"), [("k", (192, 224, 256)), ("n", (224, 192, 256))])
@pytest.mark.parametrize("mode", [Q.R0, Q.R1, Q.R2, Q.H308])
def test_kimi_payload_closes_on_both_axes(rate_axis, shape, mode):
    # reference tests/test_qsrt.py:337-380
    enc = _legal_states(shape, Q.record_bits(mode), rate_axis, 200 + mode.mode_id)
    packed = Q.pack_qsrt_trellis(enc, mode, rate_axis=rate_axis)
    assert packed.descriptor.schema == Q.SCHEMA
    if mode.mode_id != 3:
        assert packed.payload.numel() == enc.numel() * 3 // 16
        assert packed.descriptor.words_per_pair * Q.PAIRS_PER_EXPERT == packed.payload.numel()
    else:
        assert packed.descriptor.payload_bytes == 3072 * 3584 * 74 // (24 * 8)
    assert torch.equal(Q.unpack_qsrt_trellis_states(packed), enc)


@pytest.mark.parametrize("inter,latent", [(2048, 7168), (512, 256), (1536, 5120)])
def test_generic_geometry_payloads_close(inter, latent):
    geo = Q.Geometry(inter, latent)
    for name, mode in Q.modes_for(geo).items():
        rbits = Q.record_bits(mode)
        shape = (latent // 16, inter // 16, 256)
        enc = _legal_states(shape, rbits, "n", inter + mode.mode_id)
        packed = Q.pack_qsrt_trellis(enc, mode, rate_axis="n")
        assert packed.descriptor.schema == Q.GENERIC_SCHEMA
        assert packed.payload.numel() * 16 == sum(rbits) * enc.numel() // len(rbits)
        assert torch.equal(Q.unpack_qsrt_trellis_states(packed), enc), name


def test_packer_rejects_noncyclic_states():
    bad = torch.zeros((192, 224, 256), dtype=torch.int16)
    bad[..., 0] = 1
    with pytest.raises(ValueError, match="closed cyclic trellis path"):
        Q.pack_qsrt_trellis(bad, Q.R2, rate_axis="k")


def test_mode_ladder_matches_reference_record_orders():
    assert Q.record_bits(Q.R0) == (3,) * 24
    assert Q.record_bits(Q.R2)[:6] == (2, 4, 2, 4, 3, 3)
    assert Q.pair_kinds(Q.R1) == ("P24",) + ("P33",) * 11
    assert Q.record_bits(Q.H308) == (3,) * 22 + (4,) * 2
    assert Q.record_bits(Q.K2) == (2,) * 24
    assert Q.mode_from_context_bits((2,) * 2 + (3,) * 20 + (4,) * 2) == Q.R2
