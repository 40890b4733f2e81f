"""Two-sided curvature on the GPU.

* ``ldlq_two_sided`` teacher-forced: every tile-quantizer call is replayed on
  the CPU oracle Viterbi (bit-exact), and each target equals the float64
  three-term update ``W + L_out^T E L_in + L_out^T E + E L_in`` driven by the
  GPU's own committed reconstruction (a block's own error never enters its
  target, so the final reconstruction gives every target exactly);
* an all-zero output factor is bit-identical to ``ldlq``;
* ``quantize_qsrt`` with an identity output Hessian equals the one-sided
  encode and with a correlated one lowers the Kronecker loss; every payload
  decodes to the returned reconstruction.  Dense-H path refinement sweeps are
  a research control outside the hot path and raise.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import tables as otables
from oracle import viterbi as ov
from qsrt_amd import exl3_encoder_backend as be
from qsrt_amd import qsrt as Q
from qsrt_amd.exl3_reference import decode_regularized_weight
from qsrt_amd.ldlq import make_shared_h
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _qa(bits, **extra):
    qa = {"K": bits, "seed": 1_000_002, "sv_seed": 1_499_981, "sigma_reg": 0.01, "devices": ["cuda:0"],
          "apply_out_scales": False, "tailbite_context": 128, "sqg_e4m3_lut": sqg_xor_cheb_t12_bytes(bits)}
    qa.update(extra)
    return qa


def _strict(g, n, scale):
    f = torch.tril(scale * torch.randn(n, n, generator=g), diagonal=-1)
    for b in range(0, n, 16):
        f[b:b + 16, b:b + 16] = 0
    return f


def _ar1_gram(n, rho, rows, seed):
    rng = np.random.default_rng(seed)
    x = np.empty((rows, n))
    x[:, 0] = rng.standard_normal(rows)
    for j in range(1, n):
        x[:, j] = rho * x[:, j - 1] + np.sqrt(1 - rho * rho) * rng.standard_normal(rows)
    return torch.from_numpy(x.T @ x / rows).float()


def test_two_sided_ldlq_teacher_forced(monkeypatch):
    k, n, bits = 128, 96, 3
    _say(f"[two-sided] ldlq_two_sided {k}x{n} K{bits}")
    g = torch.Generator().manual_seed(7)
    weight = (0.8 * torch.randn(k, n, generator=g)).to(DEV)
    l_in, l_out = _strict(g, k, 0.3).to(DEV), _strict(g, n, 0.3).to(DEV)
    calls = []
    original = be.quantize_tiles_multigpu

    def recording(tiles, qa):
        recon, states = original(tiles, qa)
        calls.append((tiles.detach().cpu().clone(), recon.detach().cpu().clone(), states.detach().cpu().clone()))
        return recon, states

    monkeypatch.setattr(be, "quantize_tiles_multigpu", recording)
    qa = _qa(bits)
    weight_q, encoded = be.ldlq_two_sided(weight, l_in, l_out, qa)
    torch.cuda.synchronize()
    ob, ib = n // 16, k // 16  # source orientation: [output n, input k]
    assert len(calls) == ob + ib - 1
    labels = otables.t12_values(bits)
    lag = 1
    for tiles, recon, states in calls:
        o_recon, o_states = ov.encode(tiles.numpy(), labels, K=bits, context=128, boundary_lag=lag)
        assert np.array_equal(states.numpy().view(np.uint16), o_states)
        assert np.array_equal(recon.numpy(), o_recon)
    # float64 teacher-forced targets from the GPU's own reconstruction
    src = weight.T.double().cpu()
    rec = weight_q.T.double().cpu()
    lo, li = l_out.double().cpu(), l_in.double().cpu()
    perm = be.tensor_core_perm("cpu").long()
    worst = 0.0
    for call, d in zip(calls, range(ob + ib - 2, -1, -1)):
        coords = [(o, d - o) for o in range(ob) if 0 <= d - o < ib]
        assert call[0].shape[0] == len(coords)
        for t, (o, i) in enumerate(coords):
            r0, c0 = 16 * o, 16 * i
            tail = src[r0:, c0:] - rec[r0:, c0:]
            fb = lo[r0:, r0:r0 + 16].T @ tail @ li[c0:, c0:c0 + 16]
            fb += lo[r0:, r0:r0 + 16].T @ tail[:, :16] + tail[:16] @ li[c0:, c0:c0 + 16]
            target = (src[r0:r0 + 16, c0:c0 + 16] + fb).T.reshape(256)[perm]  # encoder tile, tensor-core order
            got = call[0][t].double()
            worst = max(worst, float((got - target).abs().max() / target.abs().max()))
    assert worst < 1e-5, worst
    # codes are the recorded states in the encoder's tile grid
    grid = torch.zeros((ib, ob, 256), dtype=torch.int16)
    for call, d in zip(calls, range(ob + ib - 2, -1, -1)):
        for t, o in enumerate(o for o in range(ob) if 0 <= d - o < ib):
            grid[d - o, o] = call[2][t]
    assert torch.equal(encoded.cpu(), grid)


def test_zero_output_factor_is_ldlq():
    k, n = 128, 128  # ldlq takes whole 128-column spans
    _say("[two-sided] zero output factor == ldlq")
    g = torch.Generator().manual_seed(3)
    weight = torch.randn(k, n, generator=g).to(DEV)
    l_in = _strict(g, k, 0.3).to(DEV)
    a = be.ldlq_two_sided(weight, l_in, torch.zeros(n, n, device=DEV), _qa(3))
    b = be.ldlq(weight, l_in, _qa(3))
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def _encode(W, H, qa, return_weight_q):
    shared = make_shared_h(W.shape[0], DEV, H)
    shared["count"] = 4096
    return be.quantize_qsrt(W.clone(), shared, qa, return_weight_q)


def _kron_loss(E, h_in, h_out):
    E = E.double()
    return float(torch.sum((h_in.double() @ E) * (E @ h_out.double())))


def test_quantize_qsrt_output_hessian():
    k, n, bits = 256, 256, 3
    _say(f"[two-sided] quantize_qsrt output_hessian {k}x{n} K{bits}")
    H = _ar1_gram(k, 0.8, 4096, 11) * 4096
    rng = np.random.default_rng(12)
    W = torch.from_numpy((rng.standard_normal((k, n)) * 0.02).astype(np.float32)).to(DEV)
    base_q, base_proxy, base_t = _encode(W, H, _qa(bits), True)
    ident_q, _, ident_t = _encode(W, H, _qa(bits, output_hessian=torch.eye(n)), True)
    assert torch.equal(ident_t["trellis"], base_t["trellis"])
    h_out = _ar1_gram(n, 0.9, 4096, 13)
    qa = _qa(bits, output_hessian=h_out)
    two_q, _, two_t = _encode(W, H, qa, True)
    assert qa["output_hessian_record"]["strict_factor_nonzero_count"] > 0
    assert qa["h2_viterbi_refine_receipt"]["reason"] == "two_sided_curvature"
    h_in = H / 4096
    base_loss = _kron_loss(W - base_q, h_in.to(DEV), h_out.to(DEV))
    two_loss = _kron_loss(W - two_q, h_in.to(DEV), h_out.to(DEV))
    _say(f"[two-sided] Kronecker loss one-sided {base_loss:.4e} two-sided {two_loss:.4e}")
    assert two_loss < base_loss
    # the stored payload decodes to the regularised reconstruction
    reg_q, _, reg_t = _encode(W, H, _qa(bits, output_hessian=h_out), False)
    states = Q.unpack_trellis_states(reg_t["trellis"], bits)
    assert torch.equal(decode_regularized_weight(states.cpu(), bits=bits), reg_q.cpu())
    with pytest.raises(ValueError, match="cannot be combined"):
        _encode(W, H, _qa(bits, output_hessian=h_out, h2_viterbi_refine_sweeps=1), False)


def test_dense_h_refinement_sweeps_run_one_sided():
    """Refinement sweeps run on the one-sided encode (the two-sided
    combination is rejected above) and report an enabled receipt whose
    objective never rises."""

    k, n, bits = 256, 128, 2
    H = _ar1_gram(k, 0.9, 4096, 21) * 4096
    W = torch.from_numpy((np.random.default_rng(22).standard_normal((k, n)) * 0.02).astype(np.float32)).to(DEV)
    qa = _qa(bits, h2_viterbi_refine_sweeps=2)
    _encode(W, H, qa, False)
    receipt = qa["h2_viterbi_refine_receipt"]
    assert receipt["enabled"] and receipt["rate_bits"] == bits
    for sweep in receipt["sweeps"]:
        assert sweep["objective_after"] <= sweep["objective_before"] * (1 + 1e-9)
