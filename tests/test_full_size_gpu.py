"""The hot path at BASELINE's full sizes, through size-independent properties.

* Viterbi microbench (65,536 iid N(0,1) tiles of 256, K2 and K3, C = 128):
  every tile's states form a closed cyclic path, every reconstruction is the
  label of its state, a seeded sample of tiles is bit-exact with the CPU
  oracle, and the per-symbol MSE at the fitted global scale matches the
  reference's published coding measurement for the production SQG T12 table
  (K2 0.066435, K3 0.016814: docs/qsrt-exl3-comparative-assessment.md:94,
  measured by qsrt/synthetic_source_distortion.py:341-393 with an exact FP32
  search, windowed steady state, two-stage scale grid around 1/sigma).
* One Kimi-class matrix (7168 x 2048, K3, BlockLDLQ under an AR(1) Hessian):
  the payload closes, decodes to the encoder's reconstruction, carries
  exactly K bits per weight, and sampled tile-quantizer calls replay
  bit-exact on the CPU oracle.
* Layer decode records (config 5): a gate-shaped [7168 x 2048] payload with
  its 16 records along N and a down-shaped [2048 x 7168] one with them along
  K, 14 K3 + 2 K4 records each, decoded through one prepared plan; sampled
  128-row block rows match the float64 oracle (the decode is separable by
  block rows).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import fmt as ofmt
from oracle import tables as otables
from oracle import viterbi as ov
from qsrt_amd import decode as D
from qsrt_amd import exl3_encoder_backend as be
from qsrt_amd import qsrt as Q
from qsrt_amd.exl3_reference import decode_regularized_weight, reconstruct_trellis_states
from qsrt_amd.ldlq import make_shared_h
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes
from qsrt_amd.sqg_quantizer import _lut_abs_max, boundary_lag, quantize_tiles_sqg

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TILES = 65536
PUBLISHED_MSE = {2: 0.066435, 3: 0.016814}


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _qa(bits: int, lut: torch.Tensor) -> dict:
    return {"K": bits, "sqg_e4m3_lut": lut, "tailbite_context": 128, "devices": [str(DEV)]}


@pytest.mark.parametrize("bits", (2, 3))
def test_microbench_full_size_properties_and_published_distortion(bits):
    _say(f"[full] Viterbi microbench K{bits}: {TILES} tiles x 256")
    lut = sqg_xor_cheb_t12_bytes(bits).to(DEV)
    values = lut.view(torch.float8_e4m3fn).float()
    qa = _qa(bits, lut)
    g = torch.Generator(device=DEV).manual_seed(20261201 + bits)
    source = torch.randn((TILES, 256), device=DEV, generator=g)

    def mse_at(scale: float) -> float:
        tiles = source / scale
        recon, _ = quantize_tiles_sqg(tiles, qa)
        return float(((recon - tiles) ** 2).mean(dtype=torch.float64)) * scale * scale

    # two-stage grid around the unit-variance normalisation, as the reference measurement fits its scale
    centre = 1.0 / float(values.double().std())
    coarse = [round(float(v), 6) for v in np.linspace(0.9, 1.1, 9) * centre]
    coarse_mse = [mse_at(s) for s in coarse]
    best = int(np.argmin(coarse_mse))
    assert 0 < best < len(coarse) - 1, "fitted scale sits on the coarse grid's edge"
    fine = [round(float(v), 6) for v in np.linspace(coarse[best - 1], coarse[best + 1], 9)]
    fine_mse = [mse_at(s) for s in fine]
    k = int(np.argmin(fine_mse))
    scale, mse = fine[k], fine_mse[k]
    rel = mse / PUBLISHED_MSE[bits] - 1.0
    _say(f"[full] K{bits}: MSE {mse:.6f} at scale {scale:.6f} (published {PUBLISHED_MSE[bits]}, {100 * rel:+.2f}%)")
    # The published figure is a windowed steady state over 65,536 symbols (stderr ~0.5%) that pays nothing
    # for the path's ends; cyclic 256-symbol tiles pay for closing the cycle (here +0.87% at K2 and +0.90% at
    # K3).  A wrong label, cost or argmin moves the MSE by far more than 2%.
    assert abs(rel) < 0.02

    tiles = source / scale
    recon, states = quantize_tiles_sqg(tiles, qa)
    s64 = states.to(torch.int64) & 0xFFFF
    assert torch.equal(states, reconstruct_trellis_states(s64 & ((1 << bits) - 1), bits).to(states.dtype))
    assert torch.equal(recon, values[s64])
    pick = torch.randperm(TILES, generator=torch.Generator().manual_seed(7 + bits))[:16]
    lag = boundary_lag(bits, _lut_abs_max(lut))
    sample = tiles[pick.to(DEV)].cpu().numpy()
    o_recon, o_states = ov.encode(sample, otables.t12_values(bits), K=bits, context=128, boundary_lag=lag)
    assert np.array_equal(states[pick.to(DEV)].cpu().numpy().view(np.uint16), o_states)
    assert np.array_equal(recon[pick.to(DEV)].cpu().numpy(), o_recon)


def test_kimi_matrix_full_size_encode_closes_and_replays(monkeypatch):
    k, n, bits = 7168, 2048, 3
    _say(f"[full] quantize_qsrt {k}x{n} K{bits}, BlockLDLQ under an AR(1) Hessian")
    idx = torch.arange(k, dtype=torch.float64)
    H = (0.85 ** (idx[:, None] - idx[None, :]).abs()).float().to(DEV)  # AR(1) covariance, rho = 0.85
    shared = make_shared_h(k, DEV, H)
    shared["count"] = 1
    rng = np.random.default_rng(20261204)
    W = torch.from_numpy((rng.standard_t(5.0, size=(k, n)) * 0.015 / (5.0 / 3.0) ** 0.5).astype(np.float32)).to(DEV)
    lut = sqg_xor_cheb_t12_bytes(bits)
    qa = {"K": bits, "seed": 1_000_000, "sv_seed": 1_499_979, "sigma_reg": 0.01, "devices": [str(DEV)],
          "apply_out_scales": False, "tailbite_context": 128, "sqg_e4m3_lut": lut}
    recorded = {}
    keep = {3, 250}  # LDLQ steps (16-row blocks of n / 16 tiles); the scale search's batches are not replayed
    original = be.quantize_tiles_multigpu
    calls = [0]

    def recording(tiles, q):
        out = original(tiles, q)
        if tiles.shape[0] == n // 16:
            if calls[0] in keep:
                recorded[calls[0]] = (tiles.cpu().numpy(), out[0].cpu().numpy(), out[1].cpu().numpy())
            calls[0] += 1
        return out

    monkeypatch.setattr(be, "quantize_tiles_multigpu", recording)
    weight_q, proxy, tensors = be.quantize_qsrt(W.clone(), shared, qa, False)
    torch.cuda.synchronize()
    monkeypatch.setattr(be, "quantize_tiles_multigpu", original)
    trellis = tensors["trellis"]
    _say(f"[full] {calls[0]} LDLQ steps, proxy {proxy:.5f}, g_scale {qa['g_scale']:.4f}")
    assert calls[0] == k // 16
    assert trellis.dtype == torch.int16 and tuple(trellis.shape) == (k // 16, n // 16, 16 * bits)
    assert trellis.numel() * 16 == k * n * bits  # exactly K bits per weight
    states = Q.unpack_trellis_states(trellis, bits)
    s64 = states.to(torch.int64) & 0xFFFF
    assert torch.equal(states, reconstruct_trellis_states(s64 & ((1 << bits) - 1), bits).to(states.dtype))
    assert torch.equal(decode_regularized_weight(states.cpu(), bits=bits), weight_q.cpu())
    assert 0.0 < proxy < 0.05
    assert set(recorded) == keep
    lag = boundary_lag(bits, _lut_abs_max(lut))
    for i, (tiles, recon, st) in sorted(recorded.items()):
        o_recon, o_states = ov.encode(tiles, otables.t12_values(bits), K=bits, context=128, boundary_lag=lag)
        assert np.array_equal(st.view(np.uint16), o_states), f"call {i}"
        assert np.array_equal(recon, o_recon), f"call {i}"


LAYER_RECORD_BITS = (3,) * 14 + (4,) * 2  # config 5: 14 K3 + 2 K4 records per matrix


def _record_payload(rbits, rate_axis, other_tiles, seed):
    """Record-major words of random closed paths, one record (8 rate-axis
    tiles) per entry of ``rbits``; returns (states [kt, nt, 256], words)."""

    g = torch.Generator().manual_seed(seed)
    shape = (8 * len(rbits), other_tiles) if rate_axis == "k" else (other_tiles, 8 * len(rbits))
    states = torch.empty((*shape, 256), dtype=torch.int16)
    pieces = []
    for i, bits in enumerate(rbits):
        e = torch.randint(0, 1 << bits, (8, other_tiles, 256) if rate_axis == "k" else (other_tiles, 8, 256),
                          generator=g)
        st = reconstruct_trellis_states(e, bits)
        if rate_axis == "k":
            states[8 * i:8 * i + 8] = st
        else:
            states[:, 8 * i:8 * i + 8] = st
        pieces.append(Q.pack_trellis_edges(st.reshape(-1, 256), bits).reshape(-1))
    return states, torch.cat(pieces)


def test_layer_records_full_size_decode_matches_oracle():
    _say("[full] decode plan: gate [7168 x 2048] records along N, down [2048 x 7168] records along K")
    luts = {b: sqg_xor_cheb_t12_bytes(b).to(DEV) for b in set(LAYER_RECORD_BITS)}
    cases = [("n", 448, 61), ("k", 448, 62)]
    payloads, meta = [], []
    for axis, other, seed in cases:
        states, words = _record_payload(LAYER_RECORD_BITS, axis, other, seed)
        kt, nt = states.shape[:2]
        g = torch.Generator().manual_seed(seed + 100)
        suh = (torch.rand(16 * kt, generator=g) + 0.5).half()
        svh = (torch.rand(16 * nt, generator=g) - 0.5).half()
        out = torch.empty((16 * kt, 16 * nt), dtype=torch.float32, device=DEV)
        payloads.append((words.to(DEV), LAYER_RECORD_BITS, axis, (suh.float() / 128).to(DEV), svh.float().to(DEV),
                         out))
        meta.append((states, suh, svh, axis))
    plan = D.DecodePlan.for_records(payloads, luts, out_dtype=torch.float32)
    plan.run()
    torch.cuda.synchronize()
    for (states, suh, svh, axis), p in zip(meta, payloads):
        st = states.numpy().view(np.uint16)
        kt, nt = st.shape[:2]
        record = np.empty((kt, nt), dtype=np.int64)  # rate of every tile
        for i, bits in enumerate(LAYER_RECORD_BITS):
            if axis == "k":
                record[8 * i:8 * i + 8] = bits
            else:
                record[:, 8 * i:8 * i + 8] = bits
        tables = {b: otables.t12_values(b) for b in set(LAYER_RECORD_BITS)}
        got = p[5].cpu().double().numpy()
        rows = np.random.default_rng(len(axis) + kt).choice(kt // 8, size=4, replace=False)
        for br in sorted(rows.tolist()):
            sl = slice(8 * br, 8 * br + 8)
            labels = np.empty((8, nt, 256), dtype=np.float64)
            for b, table in tables.items():
                mask = record[sl] == b
                labels[mask] = table[st[sl][mask]]
            want = ofmt.decode_tile_values(labels, suh.float().numpy()[128 * br:128 * br + 128], svh.float().numpy())
            block = got[128 * br:128 * br + 128]
            assert np.max(np.abs(block - want)) <= 2e-6 * np.abs(want).max(), f"{axis} block row {br}"
