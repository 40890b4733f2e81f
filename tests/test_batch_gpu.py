"""Batched mixed-rate LDLQ and the candidate-batch encoder on the GPU.

* ``ldlq_mixed_batched`` is the per-member ``ldlq_mixed`` recursion: the
  same feedback products and tile calls, so results are bit-identical;
* an upper-interval call plus a lower-interval continuation equals one full
  traversal; members mapped onto shared sources equal separate sources;
* ``quantize_qsrt_batch`` returns closed trellis paths whose payload decodes
  to its reconstruction, and updates every candidate's ``quant_args``.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from qsrt_amd import exl3_encoder_backend as be
from qsrt_amd.decode import decode_words
from qsrt_amd import qsrt as Q
from qsrt_amd.exl3_reference import reconstruct_trellis_states
from qsrt_amd.ldlq import make_shared_h
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

pytestmark = pytest.mark.gpu


def _qa(bits_map, axis="n", **extra):
    qa = {"K": 3, "seed": 7, "sv_seed": 8, "sigma_reg": 0.01, "devices": ["cuda:0"], "apply_out_scales": False,
          "tailbite_context": 128, "sqg_e4m3_luts_by_bits": {b: sqg_xor_cheb_t12_bytes(b) for b in (2, 3, 4)},
          "mixed_rate_axis": axis, "mixed_tile_bits": tuple(bits_map)}
    qa.update(extra)
    return qa


def _problem(k, n, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((4 * k, k))
    for j in range(1, k):
        x[:, j] = 0.8 * x[:, j - 1] + 0.6 * x[:, j]
    H = torch.from_numpy(x.T @ x / (4 * k) + 0.01 * np.eye(k)).float()
    L, _ = be.block_ldl(H.clone().cuda(), 16, {"sigma_reg": 0.01}, False)
    L[torch.arange(k), torch.arange(k)] = 0
    W = torch.from_numpy(rng.standard_normal((k, n)).astype(np.float32)).cuda()
    return W, L.cuda(), H


def test_mixed_batched_equals_per_member_mixed():
    print("[batch] ldlq_mixed_batched vs ldlq_mixed", file=sys.stderr, flush=True)
    k, n = 256, 256
    W0, L0, _ = _problem(k, n, 1)
    W1, L1, _ = _problem(k, n, 2)
    maps = [[2, 3] * 8, [3] * 12 + [4] * 4]
    qas = [_qa(m) for m in maps]
    wq, enc = be.ldlq_mixed_batched(torch.stack([W0, W1]), torch.stack([L0, L1]), qas)
    for i, (W, L) in enumerate(((W0, L0), (W1, L1))):
        q1, e1 = be.ldlq_mixed(W, L, qas[i])
        assert torch.equal(wq[i], q1) and torch.equal(enc[i], e1)
    # k-axis maps
    kmaps = [[2] * 8 + [3] * 8, [4] * 16]
    wq, enc = be.ldlq_mixed_batched(torch.stack([W0, W1]), torch.stack([L0, L1]), [_qa(m, "k") for m in kmaps])
    q1, e1 = be.ldlq_mixed(W1, L1, _qa(kmaps[1], "k"))
    assert torch.equal(wq[1], q1) and torch.equal(enc[1], e1)


def test_mixed_batched_continuation_and_shared_sources():
    print("[batch] continuation + source_indices", file=sys.stderr, flush=True)
    k, n = 512, 128
    W0, L0, _ = _problem(k, n, 3)
    qas = [_qa([3] * 8), _qa([2, 4] * 4)]
    Ws, Ls = W0[None], L0[None]
    idx = torch.zeros(2, dtype=torch.int64, device="cuda")
    full_q, full_e = be.ldlq_mixed_batched(Ws, Ls, qas, source_indices=idx)
    up_q, up_e, up_p = be.ldlq_mixed_batched(Ws, Ls, qas, source_indices=idx, process_begin=256,
                                             return_product_cache=True)
    lo_q, lo_e = be.ldlq_mixed_batched(Ws, Ls, qas, source_indices=idx, process_begin=0, process_end=256,
                                       initial_weights_q=up_q, initial_encoded_q=up_e, initial_product_cache=up_p)
    assert torch.equal(lo_q, full_q) and torch.equal(lo_e, full_e)
    sep_q, sep_e = be.ldlq_mixed_batched(torch.stack([W0, W0]), torch.stack([L0, L0]), qas)
    assert torch.equal(sep_q, full_q) and torch.equal(sep_e, full_e)
    with pytest.raises(ValueError):
        be.ldlq_mixed_batched(Ws, Ls, qas, source_indices=idx, process_end=256)


def test_quantize_qsrt_batch_candidates_close_and_decode():
    print("[batch] quantize_qsrt_batch 2 sources x 2 candidates", file=sys.stderr, flush=True)
    k, n = 256, 256
    rng = np.random.default_rng(9)
    weights, H_datas, groups = [], [], []
    for s in range(2):
        x = rng.standard_normal((2048, k))
        H = torch.from_numpy(x.T @ x).float()
        hd = make_shared_h(k, torch.device("cuda:0"), H)
        hd["count"] = 2048
        H_datas.append(hd)
        weights.append(torch.from_numpy((rng.standard_t(5, size=(k, n)) * 0.02).astype(np.float32)).cuda())
        groups.append([_qa([3] * 16, seed=10 + s, sv_seed=20 + s), _qa([2, 4] * 8, seed=10 + s, sv_seed=20 + s)])
    out = be.quantize_qsrt_batch(weights, H_datas, groups)
    assert len(out) == 2 and all(len(r) == 2 for r in out)
    for s in range(2):
        for c, res in enumerate(out[s]):
            qa = groups[s][c]
            assert 0.0 < res["proxy"] < 0.2 and qa["g_scale"] == res["g_scale"] and qa["q_fallback"] is False
            bits_map = qa["mixed_tile_bits"]
            enc = res["encoded"]
            # closed paths at each column's rate
            for t, b in enumerate(bits_map):
                col = enc[:, t].to(torch.int64)
                assert torch.equal(col.to(torch.int16), reconstruct_trellis_states(col & ((1 << b) - 1), b))
            # the uniform K3 candidate's payload decodes to the reconstruction
            if c == 0:
                words = Q.pack_trellis_edges(enc, 3)
                dec = decode_words(words, res["suh"], res["svh"], 3, sqg_xor_cheb_t12_bytes(3), out_dtype=torch.float32)
                assert float((dec - res["weight_q"]).abs().max()) <= 1e-5 * float(res["weight_q"].abs().max())
    with pytest.raises(ValueError):
        be.quantize_qsrt_batch(weights, H_datas, [groups[0], []])


def _direct(W, L, qas_by_source):
    """Every (source, candidate) encoded on its own, source-major."""

    out_q, out_e = [], []
    for s, qas in enumerate(qas_by_source):
        for qa in qas:
            q, e = be.ldlq_mixed(W[s], L[s], qa)
            out_q.append(q)
            out_e.append(e)
    return torch.stack(out_q), torch.stack(out_e)


def test_output_axis_candidate_reuse_is_bit_identical():
    """R0/R1/R2-style ladders along N: one all-K3 encode plus the union of
    replacement tiles per width reproduces every candidate exactly."""

    print("[batch] ldlq_mixed_n_candidates_reuse", file=sys.stderr, flush=True)
    k, n = 256, 512
    W0, L0, _ = _problem(k, n, 11)
    W1, L1, _ = _problem(k, n, 12)
    t = n // 16
    r1 = [2] * 8 + [3] * (t - 16) + [4] * 8
    r2 = [2] * 16 + [3] * (t - 32) + [4] * 16
    groups = [[_qa([3] * t), _qa(r1), _qa(r2)], [_qa([3] * t), _qa(r2)]]
    W, L = torch.stack([W0, W1]), torch.stack([L0, L1])
    q, e = be.ldlq_mixed_n_candidates_reuse(W, L, groups)
    dq, de = _direct(W, L, groups)
    assert torch.equal(q, dq) and torch.equal(e, de)
    with pytest.raises(ValueError, match="all-K3"):
        be.ldlq_mixed_n_candidates_reuse(W, L, [[_qa(r1)], [_qa(r2)]])
    with pytest.raises(ValueError, match="multiple non-K3"):
        be.ldlq_mixed_n_candidates_reuse(W[:1], L[:1], [[_qa([3] * t), _qa([2] * t), _qa([4] * t)]])


def test_input_axis_prefix_reuse_is_bit_identical():
    """Candidates along K that agree on the last records: the shared suffix is
    encoded once and the trie continues only where the maps differ."""

    print("[batch] ldlq_mixed_k_candidates_prefix_reuse", file=sys.stderr, flush=True)
    k, n = 512, 256
    W0, L0, _ = _problem(k, n, 21)
    W1, L1, _ = _problem(k, n, 22)
    t = k // 16
    base = [3] * t
    a = [2] * 8 + [4] * 8 + [3] * (t - 16)          # differs in the first two 128-row spans
    b = [2] * 8 + [3] * 8 + [4] * 8 + [3] * (t - 24)  # shares span 0 with a, differs in span 1 and 2
    groups = [[_qa(base, "k"), _qa(a, "k"), _qa(b, "k")], [_qa(a, "k"), _qa(b, "k")]]
    W, L = torch.stack([W0, W1]), torch.stack([L0, L1])
    q, e = be.ldlq_mixed_k_candidates_prefix_reuse(W, L, groups)
    dq, de = _direct(W, L, groups)
    assert torch.equal(q, dq) and torch.equal(e, de)
    # no shared suffix at all: the flat batch
    c = [4] * 8 + [3] * (t - 16) + [2] * 8
    q, e = be.ldlq_mixed_k_candidates_prefix_reuse(W[:1], L[:1], [[_qa(base, "k"), _qa(c, "k")]])
    dq, de = _direct(W[:1], L[:1], [[_qa(base, "k"), _qa(c, "k")]])
    assert torch.equal(q, dq) and torch.equal(e, de)
