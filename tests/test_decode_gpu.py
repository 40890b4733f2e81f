"""Fused HIP trellis decode (qsrt_decode) against the float64 oracle
decode: packed words -> states -> E4M3 labels -> H_L, su, H_R, sv.

* f32 output within 1e-6 of the oracle (relative to the matrix maximum);
* bf16 output equal to the round-to-nearest-even bf16 of the oracle value
  except where the oracle sits within 1e-5 relative of a rounding midpoint;
* K2/K3/K4, FP8 (SQG tables) and FP32 (wide table) matrix-core paths,
  mixed-rate payloads along both rate axes, strided output, the
  ``quantize_qsrt`` payload round trip.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import fmt as ofmt
from oracle import tables as otables
from qsrt_amd import decode as D
from qsrt_amd import qsrt as Q
from qsrt_amd.exl3_reference import reconstruct_trellis_states
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _payload(bits, kt, nt, seed):
    g = torch.Generator().manual_seed(seed)
    edges = torch.randint(0, 1 << bits, (kt, nt, 256), generator=g)
    states = reconstruct_trellis_states(edges, bits)
    suh = ((torch.rand(16 * kt, generator=g) + 0.5) * torch.sign(torch.randn(16 * kt, generator=g))).half()
    svh = ((torch.rand(16 * nt, generator=g) + 0.5) * torch.sign(torch.randn(16 * nt, generator=g))).half()
    return states, suh, svh


def _bf16_ok(got_bf16: torch.Tensor, want: np.ndarray, tol: float = 1e-6):
    """Every output is the bf16 rounding of a value within ``tol * max|want|``
    of the oracle; returns the fraction equal to RNE(oracle)."""

    got = got_bf16.float().cpu().double().numpy()
    rne = torch.from_numpy(want).float().bfloat16().double().numpy()
    _, e = np.frexp(want)
    half_ulp = np.ldexp(1.0, e - 9)  # bf16 keeps 8 significant bits
    assert np.all(np.abs(got - want) <= half_ulp + tol * np.abs(want).max())
    return float((got == rne).mean())


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_decode_words_matches_oracle(bits):
    _say(f"[decode] words K{bits} 384x256")
    states, suh, svh = _payload(bits, 24, 16, 100 + bits)
    words = Q.pack_trellis_edges(states, bits).cuda()
    lut = sqg_xor_cheb_t12_bytes(bits).cuda()
    want = ofmt.decode(states.numpy().view(np.uint16), otables.t12_values(bits), suh.float().numpy(),
                       svh.float().numpy())
    f32 = D.decode_words(words, suh.cuda(), svh.cuda(), bits, lut, out_dtype=torch.float32)
    assert np.max(np.abs(f32.cpu().double().numpy() - want)) <= 1e-6 * np.abs(want).max()
    bf = D.decode_words(words, suh.cuda(), svh.cuda(), bits, lut)
    assert bf.dtype == torch.bfloat16
    assert _bf16_ok(bf, want) > 0.999


def test_decode_fp32_path_for_wide_tables():
    _say("[decode] wide-range LUT (FP32 matrix-core path)")
    bits = 3
    states, suh, svh = _payload(bits, 16, 8, 7)
    g = torch.Generator().manual_seed(8)
    lut = torch.randint(0, 0x77, (65536,), generator=g, dtype=torch.int64)  # |label| up to 240, no NaN
    lut = (lut | (torch.randint(0, 2, (65536,), generator=g) << 7)).to(torch.uint8)
    values = lut.view(torch.float8_e4m3fn).float().numpy()
    assert np.abs(values).max() > D.FP8_EXACT_MAX_LABEL
    words = Q.pack_trellis_edges(states, bits).cuda()
    want = ofmt.decode(states.numpy().view(np.uint16), values, suh.float().numpy(), svh.float().numpy())
    got = D.decode_words(words, suh.cuda(), svh.cuda(), bits, lut.cuda(), out_dtype=torch.float32)
    assert np.max(np.abs(got.cpu().double().numpy() - want)) <= 1e-6 * np.abs(want).max()


@pytest.mark.parametrize("rate_axis", ["k", "n"])
def test_decode_mixed_rate_payload(rate_axis):
    _say(f"[decode] mixed-rate payload rate_axis={rate_axis}")
    geo = Q.Geometry(512, 256)
    mode = Q.resolve_mode("R1", geo)
    rbits = Q.record_bits(mode)
    g = torch.Generator().manual_seed(3)
    shape = (32, 16) if rate_axis == "k" else (16, 32)
    states = torch.empty((*shape, 256), dtype=torch.int16)
    for r, bits in enumerate(rbits):
        e = torch.randint(0, 1 << bits, (8, shape[1], 256) if rate_axis == "k" else (shape[0], 8, 256), generator=g)
        if rate_axis == "k":
            states[8 * r:8 * r + 8] = reconstruct_trellis_states(e, bits)
        else:
            states[:, 8 * r:8 * r + 8] = reconstruct_trellis_states(e, bits)
    packed = Q.pack_qsrt_trellis(states.cuda(), mode, rate_axis=rate_axis)
    k, n = 16 * shape[0], 16 * shape[1]
    suh = (torch.rand(k, generator=g) + 0.5).half()
    svh = (torch.rand(n, generator=g) - 0.5).half()
    luts = {b: sqg_xor_cheb_t12_bytes(b) for b in set(rbits)}
    got = D.decode_packed(packed, suh.cuda(), svh.cuda(), luts, out_dtype=torch.float32)
    want = Q.decode_qsrt_exl3_weight(
        Q.PackedQSRTTrellis(packed.descriptor, packed.payload.cpu()), suh, svh).double().numpy()
    assert np.max(np.abs(got.cpu().double().numpy() - want)) <= 2e-6 * np.abs(want).max()


def _record_payload(rbits, rate_axis, other_tiles, seed):
    """Record-major words of random closed paths, one record (8 rate-axis
    tiles) per rate in ``rbits``; returns (states [kt, nt, 256], words)."""

    g = torch.Generator().manual_seed(seed)
    r = len(rbits)
    shape = (8 * r, other_tiles) if rate_axis == "k" else (other_tiles, 8 * r)
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


def test_decode_plan_over_mixed_records_matches_the_oracle():
    """Prepared plan over two record-major payloads (records along K with
    mergeable same-rate runs, records along N), run twice; the oracle looks
    every tile's labels up in its own record's table."""

    _say("[decode] prepared plan over mixed-rate records")
    cases = [((3, 3, 4, 4, 3), "k", 16, 41), ((2, 4, 3, 3), "n", 8, 42)]
    luts = {b: sqg_xor_cheb_t12_bytes(b).cuda() for b in (2, 3, 4)}
    payloads, wants = [], []
    for rbits, axis, other, seed in cases:
        states, words = _record_payload(rbits, axis, other, seed)
        kt, nt = states.shape[:2]
        g = torch.Generator().manual_seed(seed + 100)
        suh = (torch.rand(16 * kt, generator=g) + 0.5).half()
        svh = (torch.rand(16 * nt, generator=g) - 0.5).half()
        st = states.numpy().view(np.uint16)
        labels = np.empty((kt, nt, 256), dtype=np.float64)
        for i, bits in enumerate(rbits):
            sl = (slice(8 * i, 8 * i + 8), slice(None)) if axis == "k" else (slice(None), slice(8 * i, 8 * i + 8))
            labels[sl] = otables.t12_values(bits)[st[sl]]
        wants.append(ofmt.decode_tile_values(labels, suh.float().numpy(), svh.float().numpy()))
        out = torch.empty((16 * kt, 16 * nt), dtype=torch.float32, device="cuda")
        payloads.append((words.cuda(), rbits, axis, (suh.float() / 128).cuda(), svh.float().cuda(), out))
    plan = D.DecodePlan.for_records(payloads, luts, out_dtype=torch.float32)
    plan.run()
    first = [p[5].clone() for p in payloads]
    plan.run()
    for want, p, f in zip(wants, payloads, first):
        assert torch.equal(p[5], f)
        assert np.max(np.abs(p[5].cpu().double().numpy() - want)) <= 2e-6 * np.abs(want).max()


def test_decode_plan_api_edges():
    from qsrt_amd import _native
    import ctypes
    lib = _native.lib()
    plan = _native.DecodePlanStruct()
    ws = torch.empty(16, dtype=torch.uint8, device="cuda")
    _native.check(lib.qsrt_decode_prepare(None, 0, 3, ws.data_ptr(), ws.numel(), ctypes.byref(plan),
                                          _native.stream_handle(ws.device)), "prepare")
    assert plan.n_jobs == 0 and plan.total_blocks == 0
    lut = sqg_xor_cheb_t12_bytes(3).cuda()
    _native.check(lib.qsrt_decode_execute(ctypes.byref(plan), lut.data_ptr(), 1, 0, _native.stream_handle(ws.device)),
                  "execute")
    plan.K = 7
    plan.n_jobs = 1
    plan.total_blocks = 1
    assert lib.qsrt_decode_execute(ctypes.byref(plan), lut.data_ptr(), 1, 0, _native.stream_handle(ws.device)) != 0
    assert b"K7" in lib.qsrt_last_error()


def test_decode_into_strided_output_leaves_the_rest():
    bits = 2
    states, suh, svh = _payload(bits, 8, 8, 21)
    words = Q.pack_trellis_edges(states, bits).cuda()
    lut = sqg_xor_cheb_t12_bytes(bits).cuda()
    big = torch.full((128, 256), 7.0, dtype=torch.bfloat16, device="cuda")
    view = big[:, 64:192]
    D.decode_words(words, suh.cuda(), svh.cuda(), bits, lut, out=view)
    ref = D.decode_words(words, suh.cuda(), svh.cuda(), bits, lut)
    assert torch.equal(view, ref)
    assert bool((big[:, :64] == 7).all()) and bool((big[:, 192:] == 7).all())


def test_decode_rejects_bad_shapes():
    lut = sqg_xor_cheb_t12_bytes(2).cuda()
    w = torch.zeros((4, 8, 32), dtype=torch.int16, device="cuda")  # K = 64: not a multiple of 128
    with pytest.raises(ValueError):
        D.decode_words(w, torch.ones(64).half().cuda(), torch.ones(128).half().cuda(), 2, lut)
    with pytest.raises(ValueError):
        D.decode_words(torch.zeros((8, 8, 32), dtype=torch.int16, device="cuda"), torch.ones(128).half().cuda(),
                       torch.ones(128).half().cuda(), 3, lut)


def test_decode_of_encoded_payload_equals_encoder_reconstruction():
    _say("[decode] quantize_qsrt round trip 256x512 K3")
    from qsrt_amd import exl3_encoder_backend as be
    from qsrt_amd.ldlq import make_shared_h

    rng = np.random.default_rng(5)
    k, n = 256, 512
    x = rng.standard_normal((2048, k))
    H = torch.from_numpy(x.T @ x).float()
    shared = make_shared_h(k, torch.device("cuda:0"), H)
    shared["count"] = 2048
    W = torch.from_numpy((rng.standard_normal((k, n)) * 0.02).astype(np.float32)).cuda()
    qa = {"K": 3, "seed": 11, "sv_seed": 12, "sigma_reg": 0.01, "devices": ["cuda:0"], "apply_out_scales": False,
          "tailbite_context": 128, "sqg_e4m3_lut": sqg_xor_cheb_t12_bytes(3)}
    weight_q, _, tensors = be.quantize_qsrt(W, shared, qa, True)
    got = D.decode_words(tensors["trellis"], tensors["suh"], tensors["svh"], 3, sqg_xor_cheb_t12_bytes(3),
                         out_dtype=torch.float32)
    # weight_q uses the FP32 su/sv; the payload stores them in fp16
    rel = float((got - weight_q).norm() / weight_q.norm())
    assert rel < 2e-3
    from qsrt_amd.exl3_reference import decode_exl3_weight
    ref = decode_exl3_weight(Q.unpack_trellis_states(tensors["trellis"], 3), tensors["suh"], tensors["svh"], bits=3)
    assert float((got - ref).abs().max()) <= 1e-5 * float(ref.abs().max())
