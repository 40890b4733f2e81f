"""BaKron two-sided rounding on the GPU: the lockstep batch against
independent encodes, and the recursion driven by the HIP tile Viterbi (payload
decodes to the reconstruction; lower Kronecker loss than per-tile encoding)."""

from __future__ import annotations

import sys

import pytest
import torch

from qsrt_amd.exl3_reference import tensor_core_permutation
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes
from qsrt_amd.sqg_quantizer import viterbi_tiles
from qsrt_amd.two_sided_rounding import (bakron_block_round_encoder, bakron_block_round_encoder_batch,
                                         bakron_block_round_encoder_prepared_batch, factor_bakron_hessian)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _spd(n, seed):
    g = torch.Generator().manual_seed(seed)
    root = torch.randn((3 * n, n), generator=g)
    return root.T @ root / (3 * n) + 0.3 * torch.eye(n)


def _round_tiles(tiles):
    code = torch.round(tiles * 4).to(torch.int16)
    return code.to(tiles.dtype) / 4, code


def test_lockstep_batch_matches_independent_encodes():
    _say("[bakron] batch of 2 x 32x48 vs independent")
    g = torch.Generator().manual_seed(8100)
    w = torch.randn((2, 32, 48), generator=g).to(DEV)
    h_in = torch.stack((_spd(32, 8101), _spd(32, 8102))).to(DEV)
    h_out = torch.stack((_spd(48, 8103), _spd(48, 8104))).to(DEV)
    batched = bakron_block_round_encoder_batch(w, h_in, h_out, _round_tiles)
    for j in range(2):  # both run the HIP band kernel ("auto" on a GPU FP32 problem): the same sums
        one = bakron_block_round_encoder(w[j], h_in[j], h_out[j], _round_tiles, work_dtype=torch.float32)
        assert torch.equal(one.payload, batched.payload[j])
    f_in, r_in = factor_bakron_hessian(h_in[0])
    f_out, r_out = factor_bakron_hessian(h_out[0])
    shared = bakron_block_round_encoder_prepared_batch(w, f_in, f_out, r_in, r_out, _round_tiles)
    one = bakron_block_round_encoder(w[1], h_in[0], h_out[0], _round_tiles, work_dtype=torch.float32)
    assert torch.equal(one.payload, shared.payload[1])


def test_bakron_with_the_tile_viterbi():
    k, n, bits = 128, 256, 3
    _say(f"[bakron] tile Viterbi K{bits} {k}x{n}")
    lut = sqg_xor_cheb_t12_bytes(bits).to(DEV)
    labels = lut.view(torch.float8_e4m3fn).float()
    perm = tensor_core_permutation(DEV)
    inv = torch.argsort(perm)

    def tiles_viterbi(tiles):  # encoder-orientation [b, b] tiles -> tensor-core order -> Viterbi
        flat = tiles.float().reshape(-1, 256)[:, perm].contiguous()
        recon, states = viterbi_tiles(flat, lut, bits, tailbite_context=128, lag=1)
        return recon[:, inv].reshape(-1, 16, 16).to(tiles.dtype), states

    g = torch.Generator().manual_seed(5)
    w = (0.7 * torch.randn((k, n), generator=g)).to(DEV)
    h_in, h_out = _spd(k, 6).to(DEV), _spd(n, 7).to(DEV)
    res = bakron_block_round_encoder(w, h_in, h_out, tiles_viterbi, work_dtype=torch.float32)
    assert res.payload.shape == (k // 16, n // 16, 256)
    decoded = labels[res.payload.long() & 0xFFFF][..., inv].reshape(k // 16, n // 16, 16, 16)
    decoded = decoded.permute(0, 2, 1, 3).reshape(k, n)
    assert torch.equal(decoded, res.reconstruction)
    independent = tiles_viterbi(w.reshape(k // 16, 16, n // 16, 16).permute(0, 2, 1, 3).reshape(-1, 16, 16))[0]
    independent = independent.reshape(k // 16, n // 16, 16, 16).permute(0, 2, 1, 3).reshape(k, n)
    loss = lambda q: float(torch.sum((h_in.double() @ (w - q).double()) * ((w - q).double() @ h_out.double())))
    _say(f"[bakron] Kronecker loss independent {loss(independent):.4e} two-sided {loss(res.reconstruction):.4e}")
    assert loss(res.reconstruction) < loss(independent)
