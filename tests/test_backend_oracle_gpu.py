"""The encoder backend's device stages against the float64 oracle, each on
its own (cuda tensors, so every rotation and product runs on the HIP
kernels):

* ``finalize_capture_H`` (damping, sign congruence through the HIP
  Hadamard, rocsolver block LDL) and the conditioned two-stage preparation
  against ``oracle.encode.prepare_hessian`` + ``oracle.encode.factor``;
* ``regularize`` at a fixed global scale against ``oracle.ldlq.regularize``,
  also with a layer-shared input profile and the scale folded into ``sv``;
* ``ldlq_mixed`` and ``ldlq_mixed_batched`` teacher-forced: every tile call
  replays bit-exactly on the C oracle at its own rate, and every target
  equals the float64 recursion ``W + L0^T (W - Q)`` on the GPU's own ``Q``;
* the L4 caller's stored record-major payload decodes, through the oracle's
  own container reader and float64 decode, to what the product decodes.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import bench
from oracle import encode as oenc
from oracle import fmt as ofmt
from oracle import ldlq as oldlq
from oracle import tables as otables
from oracle import viterbi as ov
from qsrt_amd import exl3_encoder_backend as be
from qsrt_amd.ldlq import make_shared_h
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _signs(n: int, seed: int) -> np.ndarray:
    g = torch.Generator().manual_seed(int(seed))
    return (torch.randn(n, generator=g).sign() + 1e-5).sign().double().numpy()


def _rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.abs(b).max(), 1e-30))


def _hessian_sum(k: int, rows: int, rho: float, seed: int) -> torch.Tensor:
    x = bench.ar1_scan(rows, k, rho, torch.Generator().manual_seed(seed)).double()
    return (x.T @ x).float()


def test_finalize_capture_H_on_device_matches_float64_congruence_and_block_ldl():
    k, rows = 512, 2048
    _say(f"[backend-oracle] finalize_capture_H {k} x {k} on cuda:0")
    H_sum = _hessian_sum(k, rows, 0.8, 61)
    shared = make_shared_h(k, DEV, H_sum)
    shared["count"] = rows
    qa = {"seed": 1_000_001, "sigma_reg": 0.01}
    q_fallback, H, L, su, diag = be.finalize_capture_H(shared, qa, False)
    torch.cuda.synchronize()
    assert not q_fallback and H.is_cuda and L.is_cuda
    Hp = oenc.prepare_hessian(H_sum.double().numpy(), rows, 0.01)
    s = _signs(k, qa["seed"])
    H_c, L0 = oenc.factor(Hp, s)
    errs = (_rel(diag.cpu(), np.diag(Hp)), _rel(H.cpu(), H_c), _rel(L.cpu(), L0))
    _say(f"[backend-oracle] diag {errs[0]:.2e}, conditioned H {errs[1]:.2e}, L {errs[2]:.2e} (max rel)")
    assert np.array_equal(su.cpu().numpy().reshape(-1), s)
    assert L.dtype == torch.float64  # the factor stays float64; the metric is the FP32 rounding of H_c
    assert errs[0] <= 1e-6 and errs[1] <= 1e-6 and errs[2] <= 1e-11

    # the conditioned (two-stage) preparation with a scaled su
    shared2 = make_shared_h(k, DEV, H_sum)
    shared2["count"] = rows
    be.prepare_capture_H_for_conditioning(shared2, qa, False)
    su_full = torch.from_numpy(s * np.linspace(0.5, 2.0, k)).float().reshape(k, 1)
    _, H2, L2, _, _ = be.finalize_capture_H_with_conditioning(shared2, su_full.to(DEV), qa, False)
    H_c2, L02 = oenc.factor(Hp, su_full.double().numpy())
    e2 = (_rel(H2.cpu(), H_c2), _rel(L2.cpu(), L02))
    _say(f"[backend-oracle] conditioned with scaled su: H {e2[0]:.2e}, L {e2[1]:.2e}")
    assert e2[0] <= 1e-6 and e2[1] <= 1e-11


def _regularize_gpu(W, su, sv, qa):
    out = be.regularize(W.to(DEV).clone(), torch.from_numpy(su).float().reshape(-1, 1).to(DEV),
                        torch.from_numpy(sv).float().reshape(1, -1).to(DEV), qa, False, None, None)
    torch.cuda.synchronize()
    return out


def test_regularize_on_device_matches_oracle_at_fixed_scale():
    k, n = 512, 768
    _say(f"[backend-oracle] regularize [{k} x {n}] at g = 0.87")
    gen = torch.Generator().manual_seed(71)
    W = bench.student_t_like((k, n), std=0.02, gen=gen)
    su, sv = _signs(k, 5), _signs(n, 6)
    qa = {"apply_out_scales": False, "g_scale_override": 0.87}
    apply_out, W_r, g, su_r, sv_r = _regularize_gpu(W, su, sv, qa)
    assert apply_out is False and g == pytest.approx(0.87) and qa["zeros"] is False
    assert W_r.dtype == su_r.dtype == sv_r.dtype == torch.float64
    W_o, su_o, sv_o = oldlq.regularize(W.double().numpy(), su, sv, 0.87)
    errs = (_rel(W_r.cpu(), W_o), _rel(su_r.cpu(), su_o), _rel(sv_r.cpu(), sv_o))
    _say(f"[backend-oracle] W_r {errs[0]:.2e}, su {errs[1]:.2e}, sv {errs[2]:.2e} (max rel)")
    assert errs[0] <= 1e-13 and errs[1] <= 1e-14 and errs[2] == 0.0

    # w1/w3: a layer-shared input profile (taken from the first matrix) and g folded into sv
    key = ("backend-oracle-test", "w1")
    W3 = bench.student_t_like((k, n), std=0.02, gen=gen)
    sv3 = _signs(n, 7)
    shared_profile = oldlq.input_rms(W.double().numpy(), sv)
    for Wm, svm in ((W, sv), (W3, sv3)):
        qa = {"apply_out_scales": False, "g_scale_override": 1.13, "shared_input_scales_key": key,
              "g_scale_into_sv": True}
        _, W_r, _, su_r, sv_r = _regularize_gpu(Wm, su, svm, qa)
        W_o, su_o, sv_o = oldlq.regularize(Wm.double().numpy(), su, svm, 1.13, g_into_sv=True,
                                           input_scales=shared_profile)
        errs = (_rel(W_r.cpu(), W_o), _rel(su_r.cpu(), su_o), _rel(sv_r.cpu(), sv_o))
        _say(f"[backend-oracle] shared profile: W_r {errs[0]:.2e}, su {errs[1]:.2e}, sv {errs[2]:.2e}")
        assert errs[0] <= 1e-13 and errs[1] <= 1e-14 and errs[2] <= 1e-15
    be._SHARED_INPUT_SCALES.pop(key, None)


@pytest.mark.parametrize("apply_out", [False, True])
def test_regularize_on_device_matches_oracle_with_output_scales_and_dead_channels(apply_out):
    """The device regularize (its divisions fused into the float64 rotation
    kernel) against ``oracle.ldlq.regularize``, whose output-scale branch
    is pinned by closed forms in ``test_ldlq_oracle.py``: with and without
    output scales, with an all-zero output channel (its sv zeroed) and an
    all-zero input row (its scale at 0.1)."""

    k, n = 512, 768
    _say(f"[backend-oracle] regularize [{k} x {n}], apply_out_scales={apply_out}, dead channels")
    gen = torch.Generator().manual_seed(72)
    W = bench.student_t_like((k, n), std=0.02, gen=gen) * torch.linspace(0.3, 3.0, n)[None, :]
    W[:, 5] = 0.0  # a dead output channel
    W[7, :] = 0.0  # a dead input channel
    su, sv = _signs(k, 8), _signs(n, 9)
    qa = {"apply_out_scales": apply_out, "g_scale_override": 0.9}
    applied, W_r, g, su_r, sv_r = _regularize_gpu(W, su, sv, qa)
    assert applied is apply_out and g == pytest.approx(0.9)
    W_o, su_o, sv_o = oldlq.regularize(W.double().numpy(), su, sv, 0.9, apply_out_scales=apply_out)
    errs = (_rel(W_r.cpu(), W_o), _rel(su_r.cpu(), su_o), _rel(sv_r.cpu(), sv_o))
    _say(f"[backend-oracle] W_r {errs[0]:.2e}, su {errs[1]:.2e}, sv {errs[2]:.2e} (max rel)")
    assert errs[0] <= 1e-13 and errs[1] <= 1e-14 and errs[2] <= 1e-15
    assert float(sv_r[0, 5]) == 0.0


def _problem(k: int, n: int, seed: int):
    H_sum = _hessian_sum(k, 4 * k, 0.8, seed)
    Hp = oenc.prepare_hessian(H_sum.double().numpy(), 4 * k, 0.01)
    L, _ = be.block_ldl(torch.from_numpy(Hp).float().to(DEV), 16, {"sigma_reg": 0.01}, False)
    L[torch.arange(k), torch.arange(k)] = 0
    W = torch.from_numpy(np.random.default_rng(seed).standard_normal((k, n)).astype(np.float32)).to(DEV)
    return W, L


def _qa(bits_map, axis):
    return {"K": 3, "seed": 7, "sv_seed": 8, "sigma_reg": 0.01, "devices": [str(DEV)], "apply_out_scales": False,
            "tailbite_context": 128, "sqg_e4m3_luts_by_bits": {b: sqg_xor_cheb_t12_bytes(b) for b in (2, 3, 4)},
            "mixed_rate_axis": axis, "mixed_tile_bits": tuple(bits_map)}


def _record(monkeypatch):
    calls = []
    real = be.quantize_tiles_multigpu

    def recording(tiles, quant_args):
        recon, states = real(tiles, quant_args)
        calls.append((tiles.cpu().numpy(), int(quant_args["K"]), recon.cpu().numpy(),
                      states.cpu().numpy().view(np.uint16)))
        return recon, states

    monkeypatch.setattr(be, "quantize_tiles_multigpu", recording)
    return calls


def _assert_rounded_once(targets: np.ndarray, want: np.ndarray) -> None:
    """GPU targets (the Viterbi's FP32 inputs) against the float64
    recursion: each the float64 value rounded once to FP32, except rare
    elements one ulp away (a float64 sum in another order on the other side
    of a rounding boundary)."""

    g = np.ascontiguousarray(targets, dtype=np.float32)
    c = np.ascontiguousarray(want).astype(np.float32)
    ulps = np.abs(g.view(np.int32).astype(np.int64) - c.view(np.int32).astype(np.int64))
    _say(f"[backend-oracle] targets: {int(np.count_nonzero(ulps))} of {g.size} one ulp from the float64 "
         f"recursion rounded once (max {int(ulps.max())})")
    assert int(ulps.max()) <= 1 and int(np.count_nonzero(ulps)) <= max(4, g.size // 100_000)


def _replay_and_targets(calls, members, tile_bits_of):
    """Replay every recorded call on the oracle and rebuild, per member, the
    row-major targets the GPU fed the Viterbi.  ``members``: list of
    ``(kt, nt)``; calls arrive per 16-row step (bottom first), one per
    distinct rate in ascending order, tiles member-major inside a rate."""

    lags = {2: 0, 3: 1, 4: 1}
    labels = {b: otables.t12_values(b) for b in (2, 3, 4)}
    for tiles, bits, recon, states in calls:
        o_recon, o_states = ov.encode(tiles, labels[bits], K=bits, boundary_lag=lags[bits])
        assert np.array_equal(states, o_states) and np.array_equal(recon, o_recon), f"K{bits} call differs"
    kt, nt = members[0]
    targets = [np.zeros((kt, nt, 256), dtype=np.float32) for _ in members]
    it = iter(calls)
    for step in range(kt):
        rb = kt - 1 - step
        keys = [(m, t, tile_bits_of(m, rb, t)) for m in range(len(members)) for t in range(nt)]
        for bits in sorted({b for _, _, b in keys}):
            tiles, kb, _, _ = next(it)
            assert kb == bits
            where = [(m, t) for m, t, b in keys if b == bits]
            assert tiles.shape[0] == len(where)
            for (m, t), tile in zip(where, tiles):
                targets[m][rb, t] = tile
    assert next(it, None) is None
    return [ofmt.tiles_to_matrix(t.astype(np.float64)) for t in targets]


def test_ldlq_mixed_teacher_forced_per_rate(monkeypatch):
    k, n = 256, 256
    _say(f"[backend-oracle] ldlq_mixed [{k} x {n}], rates along N (K2/K3/K4), teacher-forced")
    W, L = _problem(k, n, 81)
    nmap = [2, 3, 4, 3] * 4
    calls = _record(monkeypatch)
    Q, enc = be.ldlq_mixed(W, L, _qa(nmap, "n"))
    torch.cuda.synchronize()
    targets = _replay_and_targets(calls, [(k // 16, n // 16)], lambda m, rb, t: nmap[t])[0]
    want = oldlq.feedback_targets(W.cpu().double().numpy(), L.cpu().double().numpy(), Q.cpu().double().numpy())
    _say(f"[backend-oracle] {len(calls)} tile calls replayed bit-exactly")
    _assert_rounded_once(targets, want)

    calls.clear()
    kmap = [4, 3, 2, 3] * 4
    Q, enc = be.ldlq_mixed(W, L, _qa(kmap, "k"))
    torch.cuda.synchronize()
    targets = _replay_and_targets(calls, [(k // 16, n // 16)], lambda m, rb, t: kmap[rb])[0]
    want = oldlq.feedback_targets(W.cpu().double().numpy(), L.cpu().double().numpy(), Q.cpu().double().numpy())
    _assert_rounded_once(targets, want)


def test_ldlq_mixed_batched_teacher_forced_per_rate(monkeypatch):
    k, n = 256, 256
    _say(f"[backend-oracle] ldlq_mixed_batched, 2 members [{k} x {n}], teacher-forced")
    W0, L0 = _problem(k, n, 91)
    W1, L1 = _problem(k, n, 92)
    maps = [[3] * 14 + [4] * 2, [2, 3] * 8]
    calls = _record(monkeypatch)
    Q, enc = be.ldlq_mixed_batched(torch.stack([W0, W1]), torch.stack([L0, L1]), [_qa(m, "n") for m in maps])
    torch.cuda.synchronize()
    targets = _replay_and_targets(calls, [(k // 16, n // 16)] * 2, lambda m, rb, t: maps[m][t])
    for m, (W, L) in enumerate(((W0, L0), (W1, L1))):
        want = oldlq.feedback_targets(W.cpu().double().numpy(), L.cpu().double().numpy(), Q[m].cpu().double().numpy())
        _say(f"[backend-oracle] member {m}")
        _assert_rounded_once(targets[m], want)


def test_l4_stored_payload_decodes_through_the_oracle_container_reader():
    """``quantize_qsrt_matrix`` (R2 on a 512 x 256 geometry): the oracle reads
    the record-major payload itself, looks every tile's labels up at its
    record's rate and decodes in float64; the product's decode of the same
    payload (reference-form torch decode and the fused HIP kernel) agrees."""

    from qsrt_amd import qsrt_encoder as enc
    from qsrt_amd.decode import decode_packed
    from qsrt_amd.qsrt import Geometry, decode_qsrt_exl3_weight, record_bits

    geo = Geometry(512, 256)
    _say("[backend-oracle] quantize_qsrt_matrix w2 R2: payload through the oracle's reader")
    g = torch.Generator().manual_seed(101)
    ctx = torch.arange(geo.records).repeat_interleave(32)[torch.randperm(32 * geo.records, generator=g)]
    source = (0.02 * torch.randn((geo.latent_channels, geo.intermediate_channels), generator=g)).to(DEV)
    x = torch.randn(4 * 512, 512, generator=g)
    hessian = (x.T @ x / x.shape[0] + 0.01 * torch.eye(512)).to(DEV)
    out = enc.quantize_qsrt_matrix(source, ctx, matrix="w2", mode="R2", hessian=hessian, layer=7, device=DEV,
                                   shared_scale_scope=("backend-oracle", "w2"))
    d = out.packed.descriptor
    states, tile_bits = ofmt.unpack_records(out.packed.payload.cpu().numpy(), record_bits(d.mode), d.rate_axis,
                                            d.k_tiles, d.n_tiles)
    labels = np.zeros(states.shape, dtype=np.float64)
    for bits in np.unique(tile_bits):
        mask = tile_bits == bits
        labels[mask] = otables.t12_values(int(bits))[states[mask].astype(np.int64)]
    suh, svh = out.tensors["suh"], out.tensors["svh"]
    want = ofmt.decode_tile_values(labels, suh.float().cpu().numpy(), svh.float().cpu().numpy())
    ref = decode_qsrt_exl3_weight(out.packed, suh, svh).double().cpu().numpy()
    luts = {b: sqg_xor_cheb_t12_bytes(b).to(DEV) for b in (2, 3, 4)}
    hip = decode_packed(out.packed, suh.float(), svh.float(), luts, out_dtype=torch.float32).double().cpu().numpy()
    errs = (_rel(ref, want), _rel(hip, want))
    _say(f"[backend-oracle] records {record_bits(d.mode)}: torch decode {errs[0]:.2e}, HIP decode {errs[1]:.2e}")
    assert errs[0] <= 1e-6 and errs[1] <= 1e-6
