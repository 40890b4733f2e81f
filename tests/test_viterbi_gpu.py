"""GPU parity of the HIP tile Viterbi against the CPU oracle.

Bar: states (codewords) and reconstructions bit-exact with
oracle/viterbi_ref.c on the same seeded inputs, for K1..K6, tail-bite
contexts 1/32/128 and both boundary rules, plus the reference's own GPU
checks (closure, decode, saturated inputs; reference
tests/test_sqg_quantizer.py:178-231).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import tables as otables
from oracle import viterbi as ov
from qsrt_amd.exl3_reference import reconstruct_trellis_states
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes
from qsrt_amd.sqg_quantizer import install_sqg_quantizer, viterbi_tiles

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _gpu(tiles: np.ndarray, bits: int, context: int, lag: int):
    lut = sqg_xor_cheb_t12_bytes(bits).cuda()
    recon, states = viterbi_tiles(torch.from_numpy(tiles).cuda(), lut, bits, tailbite_context=context, lag=lag)
    torch.cuda.synchronize()
    return recon.cpu().numpy(), states.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("lag", (0, 1))
@pytest.mark.parametrize("context", (1, 32, 128))
@pytest.mark.parametrize("bits", (1, 2, 3, 4, 5, 6))
def test_gpu_matches_oracle_bit_exact(bits, context, lag):
    _say(f"[viterbi] K{bits} C{context} lag{lag}: 24 tiles")
    rng = np.random.default_rng(100 * bits + context + lag)
    tiles = rng.standard_normal((24, 256)).astype(np.float32)
    tiles[3] *= 100.0
    tiles[11] = 0.0
    tiles[17] *= -40.0
    recon, states = _gpu(tiles, bits, context, lag)
    o_recon, o_states = ov.encode(tiles, otables.t12_values(bits), K=bits, context=context, boundary_lag=lag)
    mismatch = (states != o_states).any(axis=1)
    assert not mismatch.any(), f"{int(mismatch.sum())} tiles differ, first {int(np.flatnonzero(mismatch)[0])}"
    assert np.array_equal(recon, o_recon)


@pytest.mark.parametrize("bits", (2, 3, 4))
def test_gpu_tie_heavy_tiles_match_oracle(bits):
    """Tiles drawn from a handful of the codebook's own values (and their
    negatives, and zero): many edges cost exactly the same, so the
    lowest-index rule decides most decisions.  The tournament argmin of the
    recorded steps (pair minima, the root as compare-and-select, one
    compare per level against the minimum) must pick the same predecessor
    as the oracle's scan on every tie."""

    _say(f"[viterbi] K{bits}: 32 tie-heavy tiles")
    values = np.unique(np.abs(otables.t12_values(bits).astype(np.float32)))
    rng = np.random.default_rng(300 + bits)
    pool = np.concatenate([values[rng.choice(values.size, 3, replace=False)], [0.0]]).astype(np.float32)
    pool = np.concatenate([pool, -pool])
    tiles = rng.choice(pool, size=(32, 256)).astype(np.float32)
    tiles[5] = pool[0]
    tiles[9] = 0.0
    recon, states = _gpu(tiles, bits, 128, 0 if bits == 2 else 1)
    o_recon, o_states = ov.encode(tiles, otables.t12_values(bits), K=bits, boundary_lag=0 if bits == 2 else 1)
    mismatch = (states != o_states).any(axis=1)
    assert not mismatch.any(), f"{int(mismatch.sum())} tiles differ, first {int(np.flatnonzero(mismatch)[0])}"
    assert np.array_equal(recon, o_recon)


@pytest.mark.parametrize("bits", (1, 2, 3, 4, 5, 6))
def test_gpu_many_tiles_persistent_loop(bits):
    """More tiles than workgroups: every workgroup walks several tiles."""

    n = 600
    _say(f"[viterbi] K{bits}: {n} tiles (persistent loop)")
    rng = np.random.default_rng(7 + bits)
    tiles = (rng.standard_normal((n, 256)) * 1.3).astype(np.float32)
    recon, states = _gpu(tiles, bits, 128, 0 if bits == 2 else 1)
    sample = np.arange(0, n, 37)
    o_recon, o_states = ov.encode(tiles[sample], otables.t12_values(bits), K=bits, boundary_lag=0 if bits == 2 else 1)
    assert np.array_equal(states[sample], o_states)
    assert np.array_equal(recon[sample], o_recon)
    st = torch.from_numpy(states.astype(np.int64))
    assert torch.equal(reconstruct_trellis_states(st & ((1 << bits) - 1), bits).to(torch.int64) & 0xFFFF, st)


@pytest.mark.parametrize("tailbite_context", [1, 32, 128])
def test_k2_operator_closes_trellis_and_decodes_states(tailbite_context):
    """Reference tests/test_sqg_quantizer.py:178-210 through the L2 operator."""

    from types import SimpleNamespace

    _say(f"[viterbi] operator K2 C{tailbite_context}")
    module = SimpleNamespace(quantize_tiles=lambda *_a: "upstream")
    install_sqg_quantizer(module)
    gen = torch.Generator(device="cpu").manual_seed(7)
    tiles = torch.randn((64, 256), generator=gen, dtype=torch.float32)
    tiles[3] *= 100.0
    tiles[11] = 0.0
    tiles[17] *= -40.0
    lut = sqg_xor_cheb_t12_bytes(2)
    output, states = module.quantize_tiles(
        tiles.cuda(), {"K": 2, "devices": ["cuda:0"], "sqg_e4m3_lut": lut, "tailbite_context": tailbite_context}
    )
    edges = states.to(torch.int64) & 0x3
    assert torch.equal(states, reconstruct_trellis_states(edges, 2))
    decoded = lut.view(torch.float8_e4m3fn).to(torch.float32)[states.cpu().to(torch.int64) & 0xFFFF]
    assert torch.equal(decoded, output.cpu())


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_saturated_cost_paths_stay_closed(bits):
    """Reference tests/test_sqg_quantizer.py:212-231."""

    from types import SimpleNamespace

    _say(f"[viterbi] saturated K{bits}")
    module = SimpleNamespace(quantize_tiles=lambda *_a: "upstream")
    install_sqg_quantizer(module)
    tiles = torch.full((2, 256), 1000.0, dtype=torch.float32, device="cuda")
    _output, states = module.quantize_tiles(
        tiles, {"K": bits, "devices": ["cuda:0"], "sqg_e4m3_lut": sqg_xor_cheb_t12_bytes(bits), "tailbite_context": 128}
    )
    edges = states.to(torch.int64) & ((1 << bits) - 1)
    assert torch.equal(states, reconstruct_trellis_states(edges, bits))


def test_empty_input_returns_empty():
    out, st = viterbi_tiles(torch.empty((0, 256), device="cuda"), sqg_xor_cheb_t12_bytes(2).cuda(), 2)
    assert out.shape == (0, 256) and st.shape == (0, 256)


def test_bad_arguments_raise():
    lut = sqg_xor_cheb_t12_bytes(2).cuda()
    with pytest.raises(ValueError):
        viterbi_tiles(torch.zeros((1, 128), device="cuda"), lut, 2)
    for bits in (0, 7):
        with pytest.raises(ValueError):
            viterbi_tiles(torch.zeros((1, 256), device="cuda"), lut, bits)
    with pytest.raises(ValueError):
        viterbi_tiles(torch.zeros((1, 256), device="cuda"), lut, 2, tailbite_context=129)
