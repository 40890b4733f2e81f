"""SQG tables: product module and oracle, both pinned to the reference's
golden SHA-256 digests (reference tests/test_sqg_e4m3.py:30-70)."""

from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

from oracle import tables as otables
from qsrt_amd import sqg_e4m3 as sqg

# Golden digests held by the reference's own tests (tests/test_sqg_e4m3.py:30-38).
GOLDEN_SHA256 = {
    "t12": "cca11fe5744c9c93a34f4217f342fbc0f74ecc8a007c076582424a505fc9da5e",
    1: "12d404e5a107582a8b4e38f80ac51117e8519c65e8b18f59f463aa1f8442c5ee",
    2: "62027916386245a84c86156a0a08b6cf07e41548871af0e56fb40780558f6293",
    3: "afe7b3633e7d243b00b379b18ec4dca573722b3727cafef47fcb6470d7e7e6c9",
    4: "5a9620f0c4d8f0a60d0b6fbea921dcecbd193e6febf31043aaa6403c20389c2f",
    5: "a1caf5572c67d4face423478f423e1ed6149a8c920be5c28d4702946c93cae2f",
    6: "8e0edc92e20eb92f5287dbdadc8e870fc500fc03c5eed996cae0781d197ebcb0",
}


def _sha(data) -> str:
    if isinstance(data, torch.Tensor):
        data = data.contiguous().numpy()
    return hashlib.sha256(np.ascontiguousarray(data).tobytes()).hexdigest()


def test_t12_table_matches_golden_digest():
    table = sqg.sqg_xor_cheb_t12_rank_lut_bytes()
    assert table.dtype == torch.uint8 and table.shape == (4096,)
    assert _sha(table) == GOLDEN_SHA256["t12"]
    assert _sha(otables.t12_bytes()) == GOLDEN_SHA256["t12"]


@pytest.mark.parametrize("bits", (1, 2, 3, 4, 5, 6))
def test_label_maps_match_golden_digests_and_invariants(bits):
    ranks = sqg.sqg_xor_rank_permutation(bits)
    labels = sqg.sqg_xor_cheb_t12_bytes(bits)
    width = 16 - bits
    strata = (ranks >> width).reshape(1 << width, 1 << bits)
    assert torch.equal(torch.sort(ranks).values, torch.arange(1 << 16))
    assert torch.equal(torch.sort(strata, dim=1).values, torch.arange(1 << bits).expand_as(strata))
    assert torch.equal(labels, sqg.sqg_xor_cheb_t12_rank_lut_bytes()[ranks >> 4])
    assert torch.equal(labels, sqg.sqg_codebook_bytes(bits, sqg.SQG_XOR_CHEB_T12))
    assert bool(torch.isfinite(labels.view(torch.float8_e4m3fn).float()).all())
    assert not bool(((labels & 0x7F) == 0).logical_and(labels != 0).any())
    assert _sha(labels) == GOLDEN_SHA256[bits]
    # the oracle's independent restatement lands on the same bytes
    assert _sha(otables.t12_labels(bits)) == GOLDEN_SHA256[bits]
    assert np.array_equal(otables.rank_permutation(bits), ranks.numpy())


def test_k2_table_has_151_distinct_values():
    # reference tests/test_synthetic_source_distortion.py:98-109
    values = sqg.sqg_xor_cheb_t12_bytes(2).view(torch.float8_e4m3fn).float()
    assert len(torch.unique(values)) == 151
    assert 0.0 in values.tolist()


@pytest.mark.parametrize(("bits", "expected"), ((2, 2.0437), (3, 7.9062)))
def test_menu_stratum_diversity(bits, expected):
    # reference tests/test_synthetic_source_distortion.py:112-125 (the exact
    # staircase shares the carry-mixed graph of the T12 law)
    ranks = sqg.sqg_xor_rank_permutation(bits).numpy()
    strata = ranks.reshape(1 << bits, 1 << (16 - bits)).T >> (16 - bits)
    mean = np.array([len(np.unique(row)) for row in strata]).mean()
    assert mean == pytest.approx(expected, abs=5e-3)


@pytest.mark.parametrize("bits", (1, 2, 3, 4, 5, 6))
def test_r44_control_law_round_trips_and_is_a_permutation(bits):
    raw = sqg.sqg_e4m3_bytes(bits, "normal")
    cb = sqg.sqg_e4m3_codebook(bits, "normal")
    assert torch.equal(cb.to(torch.float8_e4m3fn).view(torch.uint8), raw)
    ranks = sqg.sqg_rank_permutation(bits)
    assert torch.equal(torch.sort(ranks).values, torch.arange(1 << 16))
    strata = (ranks >> (16 - bits)).reshape(1 << (16 - bits), 1 << bits)
    assert torch.equal(torch.sort(strata, dim=1).values, torch.arange(1 << bits).expand_as(strata))


@pytest.mark.parametrize("bits", (1, 2, 3, 4))
def test_shared_rank_lut_relabels_one_graph(bits):
    rank_lut = torch.arange(1 << 16, dtype=torch.int64).remainder(126).to(torch.uint8)
    raw = sqg.sqg_e4m3_bytes_from_rank_lut(bits, rank_lut)
    assert torch.equal(raw, rank_lut.index_select(0, sqg.sqg_rank_permutation(bits)))
    expected = sqg.sqg_cheb_normal_rank_e4m3_bytes().index_select(0, sqg.sqg_rank_permutation(bits))
    assert torch.equal(sqg.sqg_codebook_bytes(bits, sqg.SQG_CHEB_NORMAL_E4M3), expected)


def test_rank_lut_rejects_nonfinite():
    lut = torch.zeros(1 << 16, dtype=torch.uint8)
    lut[0] = 0x7F
    with pytest.raises(ValueError, match="finite E4M3"):
        sqg.sqg_e4m3_bytes_from_rank_lut(2, lut)


def test_oracle_e4m3_encoder_agrees_with_torch_and_round_trips():
    codes = np.arange(256, dtype=np.uint8)
    finite = (codes & 0x7F) != 0x7F
    nonzero = finite & ((codes & 0x7F) != 0)
    values = otables.e4m3_decode(codes[nonzero])
    assert np.array_equal(otables.e4m3_encode(values), codes[nonzero])
    x = torch.randn(200_000, generator=torch.Generator().manual_seed(3)) * 8
    assert np.array_equal(otables.e4m3_encode(x.numpy()), x.to(torch.float8_e4m3fn).view(torch.uint8).numpy())
    # ties to even at a midpoint between 1.0 (0x38) and 1.125 (0x39)
    assert otables.e4m3_encode(np.array([1.0625]))[0] == 0x38
    assert otables.e4m3_encode(np.array([1.1875]))[0] == 0x3A


def test_lut_abs_max_is_per_tensor_and_version():
    """The cached largest label belongs to one tensor object and version:
    another table (even one that reuses a freed address) or an in-place edit
    never sees a stale value (a stale 5.5 would route a wide table to the
    FP8 decode path)."""

    from qsrt_amd.sqg_quantizer import _lut_abs_max, _lut_on

    a = sqg.sqg_xor_cheb_t12_bytes(3).clone()
    b = a.clone()
    assert _lut_abs_max(a) == 5.5
    b[7] = 0x77  # E4M3 240
    assert _lut_abs_max(b) == 240.0 and _lut_abs_max(a) == 5.5
    a[9] = 0xF7  # -240, in place
    assert _lut_abs_max(a) == 240.0
    assert _lut_on(a, torch.device("cpu")) is a
