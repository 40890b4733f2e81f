"""GPU encoder backend parity against the oracle.

* teacher-forced BlockLDLQ: every tile-quantizer call made by the GPU
  recursion is replayed on the CPU oracle Viterbi (states and labels
  bit-exact), and the GPU's feedback targets equal the float64 recursion
  T = W + L0^T (W - Q) driven by the GPU's own Q (1e-5 relative);
* the global-scale search picks the same scale as the search driven by the
  oracle Viterbi on the same sample tiles;
* ``quantize_qsrt`` end to end: closed payload, decode of the stored
  payload equals the regularised reconstruction, sensible proxy error.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import ldlq as oldlq
from oracle import tables as otables
from oracle import viterbi as ov
from qsrt_amd import exl3_encoder_backend as be
from qsrt_amd import qsrt as Q
from qsrt_amd.exl3_reference import decode_regularized_weight, reconstruct_trellis_states
from qsrt_amd.ldlq import make_shared_h
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _ar1(n_rows, k, rho, seed):
    rng = np.random.default_rng(seed)
    x = np.empty((n_rows, k), dtype=np.float64)
    x[:, 0] = rng.standard_normal(n_rows)
    for j in range(1, k):
        x[:, j] = rho * x[:, j - 1] + np.sqrt(1 - rho * rho) * rng.standard_normal(n_rows)
    return x


def _qa(bits, **extra):
    qa = {
        "K": bits,
        "seed": 1_000_002,
        "sv_seed": 1_499_981,
        "sigma_reg": 0.01,
        "devices": ["cuda:0"],
        "apply_out_scales": False,
        "tailbite_context": 128,
        "sqg_e4m3_lut": sqg_xor_cheb_t12_bytes(bits),
    }
    qa.update(extra)
    return qa


@pytest.mark.parametrize("bits", [2, 3])
def test_ldlq_teacher_forced_parity(bits, monkeypatch):
    _say(f"[backend] teacher-forced LDLQ K{bits}")
    k, n = 256, 256
    x = _ar1(2048, k, 0.8, 11 + bits)
    H = torch.from_numpy(x.T @ x)
    shared = make_shared_h(k, torch.device("cuda:0"), H.float())
    shared["count"] = 2048
    qa = _qa(bits)
    _, _, L, _, _ = be.finalize_capture_H(shared, qa, False)
    rng = np.random.default_rng(bits)
    W = torch.from_numpy(rng.standard_normal((k, n)).astype(np.float32) * 0.9).cuda()

    calls = []
    real = be.quantize_tiles_multigpu

    def recording(tiles, quant_args):
        recon, states = real(tiles, quant_args)
        calls.append((tiles.cpu().numpy(), recon.cpu().numpy(), states.cpu().numpy().view(np.uint16), quant_args["K"]))
        return recon, states

    monkeypatch.setattr(be, "quantize_tiles_multigpu", recording)
    weight_q, encoded = be.ldlq(W, L, qa)
    torch.cuda.synchronize()
    assert len(calls) == k // 16

    lag = 0 if bits == 2 else 1
    labels = otables.t12_values(bits)
    for tiles, recon, states, kb in calls:
        o_recon, o_states = ov.encode(tiles, labels, K=kb, boundary_lag=lag)
        assert np.array_equal(states, o_states)
        assert np.array_equal(recon, o_recon)

    # feedback targets: GPU tiles (back in row-major) vs float64 recursion on the GPU's Q
    perm_i = be.tensor_core_perm_i("cpu").long().numpy()
    targets = np.zeros((k, n))
    for step, (tiles, _, _, _) in enumerate(calls):
        blk = k - 16 * (step + 1)
        rows = tiles[:, perm_i].reshape(n // 16, 16, 16).transpose(1, 0, 2).reshape(16, n)
        targets[blk:blk + 16] = rows
    want = oldlq.feedback_targets(W.cpu().double().numpy(), L.cpu().double().numpy(), weight_q.cpu().double().numpy())
    # each target is the float64 recursion's value rounded once to FP32 (rare one-ulp summation-order flips)
    g = np.ascontiguousarray(targets, dtype=np.float32)
    c = want.astype(np.float32)
    ulps = np.abs(g.view(np.int32).astype(np.int64) - c.view(np.int32).astype(np.int64))
    assert int(ulps.max()) <= 1 and int(np.count_nonzero(ulps)) <= 4
    # encoded states are the closed paths the kernel returned, and decode to Q
    enc = encoded.cpu()
    assert torch.equal(enc, reconstruct_trellis_states(enc.to(torch.int64) & ((1 << bits) - 1), bits))
    assert torch.equal(decode_regularized_weight(enc, bits=bits), weight_q.cpu())


def test_g_scale_search_matches_oracle_driven_search():
    _say("[backend] g-scale search K2")
    rng = np.random.default_rng(4)
    w = torch.from_numpy(rng.standard_normal((256, 512)).astype(np.float32) * 0.7).cuda()
    qa = _qa(2)
    samples = be.sample_scale_tiles(w)
    (g_gpu, _mse) = be.g_scale_search_batch([samples], qa)[0]

    labels = otables.t12_values(2)
    s = samples.cpu().numpy()

    def mse(tiles, scale):
        recon, _ = ov.encode(tiles * np.float32(scale), labels, K=2, boundary_lag=0)
        return float(((recon / np.float32(scale) - tiles) ** 2).mean())

    coarse = [0.1 + 0.2 * i for i in range(10)]
    sub = s[::3]
    c = coarse[int(np.argmin([mse(sub, sc) for sc in coarse]))]
    fine = [c + 0.075 * (i - 2) for i in range(5)]
    ys = [mse(s, sc) for sc in fine]
    best = int(np.argmin(ys))
    off = 0.0
    if 0 < best < 4:
        den = ys[best - 1] - 2 * ys[best] + ys[best + 1]
        off = max(-0.5, min(0.5, 0.5 * (ys[best - 1] - ys[best + 1]) / den if den > 0 else 0.0))
    g_ref = max(fine[best] + off * 0.075, 0.01)
    assert abs(g_gpu - g_ref) < 1e-4


@pytest.mark.parametrize("bits", [2, 3])
def test_quantize_qsrt_end_to_end_small(bits):
    _say(f"[backend] quantize_qsrt 256x512 K{bits}")
    k, n = 256, 512
    x = _ar1(4096, k, 0.8, 20 + bits)
    H = torch.from_numpy(x.T @ x).float()
    shared = make_shared_h(k, torch.device("cuda:0"), H)
    shared["count"] = 4096
    rng = np.random.default_rng(30 + bits)
    W = torch.from_numpy((rng.standard_t(5, size=(k, n)) * 0.02 / np.sqrt(5 / 3)).astype(np.float32)).cuda()
    qa = _qa(bits)
    w_in = W.clone()
    weight_q_reg, proxy, tensors = be.quantize_qsrt(w_in, shared, qa, False)
    torch.cuda.synchronize()
    trellis, suh, svh = tensors["trellis"], tensors["suh"], tensors["svh"]
    assert trellis.dtype == torch.int16 and tuple(trellis.shape) == (k // 16, n // 16, 16 * bits)
    assert suh.dtype == torch.float16 and suh.shape == (k,) and svh.shape == (n,)
    assert 0.0 < proxy < 0.2
    assert 0.1 < qa["g_scale"] < 2.0 and qa["q_fallback"] is False
    states = Q.unpack_trellis_states(trellis, bits)
    assert torch.equal(decode_regularized_weight(states.cpu(), bits=bits), weight_q_reg.cpu())
    # full decode reproduces the dequantised matrix returned with return_weight_q
    shared2 = make_shared_h(k, torch.device("cuda:0"), H)
    shared2["count"] = 4096
    qa2 = _qa(bits)
    weight_q, proxy2, tensors2 = be.quantize_qsrt(W.clone(), shared2, qa2, True)
    assert proxy2 == pytest.approx(proxy, rel=1e-6)
    assert torch.equal(tensors2["trellis"], trellis)
    from qsrt_amd.exl3_reference import decode_exl3_weight

    dec = decode_exl3_weight(states, suh, svh, bits=bits)
    rel = (dec - weight_q).norm() / weight_q.norm()
    assert rel < 2e-3  # fp16 storage of su/sv
    err = (weight_q - W).norm() / W.norm()
    assert err < (0.5 if bits == 2 else 0.3)


def test_factored_hessian_stays_on_the_device():
    """The conditioned Hessian and its block-LDL factor stay in HBM after
    finalisation (no host round trip); refactoring the kept Hessian gives the
    stored factor back, and a second matrix on the same Hessian reuses it."""

    _say("[backend] factored Hessian residency")
    k, n = 256, 256
    x = _ar1(2048, k, 0.8, 50)
    H = torch.from_numpy(x.T @ x).float()
    shared = make_shared_h(k, torch.device("cuda:0"), H)
    shared["count"] = 2048
    rng = np.random.default_rng(51)
    W = torch.from_numpy((rng.standard_normal((k, n)) * 0.02).astype(np.float32)).cuda()
    qa = _qa(3)
    _, proxy, _ = be.quantize_qsrt(W.clone(), shared, qa, False)
    assert shared["H"].is_cuda and shared["L"].is_cuda
    L_again, H_again = be.block_ldl(shared["H"].clone(), 16, qa, False)
    d = torch.arange(k)
    L_again[d, d] = 0
    assert torch.equal(H_again, shared["H"])
    assert torch.allclose(L_again, shared["L"].float(), rtol=0, atol=1e-6)
    L_obj = shared["L"]
    _, proxy2, _ = be.quantize_qsrt(W.clone(), shared, _qa(3), False)
    assert shared["L"] is L_obj and proxy2 == pytest.approx(proxy, rel=1e-6)


@pytest.mark.parametrize("shared_h", [True, False])
def test_quantize_uniform_batch_equals_single_encodes(shared_h):
    """The same-K batch API against one ``quantize_qsrt`` per tensor on
    fresh Hessian dicts: equal packed trellis, sign/scale vectors, global
    scale and output-scale decision, the proxy error to FP32 rounding, and
    the caller's weight left regularised the same way.  Shared Hessian: the
    members concatenated along N under one factor; distinct Hessians:
    stacked, one factor each, with one member whose Hessian is empty (the
    fallback encode)."""

    _say(f"[backend] quantize_uniform_batch vs single encodes, shared H {shared_h}")
    k, n, members = 256, 256, 3
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(77)
    Ws = [torch.from_numpy((rng.standard_normal((k, n)) * 0.02).astype(np.float32)).to(dev) for _ in range(members)]
    Hs = []
    for i in range(1 if shared_h else members):
        x = _ar1(1024, k, 0.8, 90 + i)
        Hs.append(torch.from_numpy(x.T @ x).float())

    def h_data(i):
        d = make_shared_h(k, dev, Hs[0 if shared_h else i])
        d["count"] = 0 if (not shared_h and i == members - 1) else 1024
        return d

    if shared_h:
        one = h_data(0)
        batch_h = [one] * members
    else:
        batch_h = [h_data(i) for i in range(members)]
    qas_b = [_qa(3, sv_seed=200 + i) for i in range(members)]
    batch_w = [w.clone() for w in Ws]
    out = be.quantize_uniform_batch(list(batch_w), batch_h, qas_b)
    for i in range(members):
        qa_s = _qa(3, sv_seed=200 + i)
        w_s = Ws[i].clone()
        _, proxy_s, tensors_s = be.quantize_qsrt(w_s, h_data(i), qa_s, False)
        proxy_b, tensors_b = out[i]
        assert torch.equal(tensors_b["trellis"], tensors_s["trellis"]), f"member {i}"
        assert torch.equal(tensors_b["suh"], tensors_s["suh"]) and torch.equal(tensors_b["svh"], tensors_s["svh"])
        for key in ("g_scale", "apply_out_scales", "q_fallback"):
            assert qas_b[i][key] == qa_s[key], (i, key)
        assert proxy_b == pytest.approx(proxy_s, rel=1e-6)
        assert torch.equal(batch_w[i], w_s)


def test_quantize_uniform_batch_shared_hessian_payloads_close():
    _say("[backend] quantize_uniform_batch shared H")
    k, n = 256, 256
    x = _ar1(2048, k, 0.85, 40)
    H = torch.from_numpy(x.T @ x).float()
    rng = np.random.default_rng(41)
    Ws = [torch.from_numpy((rng.standard_normal((k, n)) * 0.02).astype(np.float32)).cuda() for _ in range(2)]
    shared = make_shared_h(k, torch.device("cuda:0"), H)
    shared["count"] = 2048
    qas = [_qa(3, sv_seed=100 + i) for i in range(2)]
    out = be.quantize_uniform_batch([w.clone() for w in Ws], [shared, shared], qas)
    for (proxy, tensors), qa in zip(out, qas):
        assert 0.0 < proxy < 0.2
        assert tensors["trellis"].shape == (k // 16, n // 16, 48)
        assert qa["q_fallback"] is False
        states = Q.unpack_trellis_states(tensors["trellis"], 3)
        assert torch.equal(states, reconstruct_trellis_states(states.to(torch.int64) & 7, 3))
