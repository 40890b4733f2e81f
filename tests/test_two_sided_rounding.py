"""Two-sided adaptive rounding (reference tests/test_two_sided_rounding.py):
the YAQA three-term recurrence, BaKron's inverse-Cholesky anti-diagonal form
and its divide-and-conquer schedule must choose identical rounding paths;
identity metrics reduce to independent and one-sided rounding; the output
metric transform preserves the quadratic form."""

from __future__ import annotations

import pytest
import torch

from qsrt_amd.qsrt_coupled import block_hadamard
from qsrt_amd.two_sided_rounding import (bakron_block_antidiagonal_encoder, bakron_block_round_encoder,
                                         factor_bakron_hessian, transform_output_hessian_blocks_for_regularization,
                                         transform_output_hessian_for_regularization, yaqa_block_round_encoder)


def _spd(n, seed):
    g = torch.Generator().manual_seed(seed)
    root = torch.randn((3 * n, n), generator=g)
    return root.T @ root + 0.3 * torch.eye(n)


def _round_tiles(tiles):
    code = torch.round(tiles * 4).to(torch.int16)
    return code.to(tiles.dtype) / 4, code


def _one_sided(weight, h_in, bs):
    """Row-block BlockLDLQ written from its definition (strict block factor
    of the Cholesky factor)."""

    k = weight.shape[0]
    c = torch.linalg.cholesky(h_in.double())
    f = c.clone()
    for s in range(0, k, bs):
        f[:, s:s + bs] = c[:, s:s + bs] @ torch.linalg.inv(c[s:s + bs, s:s + bs])
        f[s:s + bs, s:s + bs] = 0
    q = torch.zeros_like(weight, dtype=torch.float64)
    code = torch.empty_like(weight, dtype=torch.int16)
    for end in range(k, 0, -bs):
        s = end - bs
        target = weight[s:end].double() + f[s:, s:end].T @ (weight.double() - q)[s:]
        r, cd = _round_tiles(target)
        q[s:end], code[s:end] = r, cd
    return q.to(weight.dtype), code


def test_identity_metrics_reduce_to_independent_rounding():
    w = torch.randn((8, 12), generator=torch.Generator().manual_seed(1))
    res = yaqa_block_round_encoder(w, torch.eye(8), torch.eye(12), _round_tiles, block_size=4)
    code = torch.round(w * 4).to(torch.int16)
    torch.testing.assert_close(res.reconstruction, code.float() / 4, rtol=0, atol=0)
    torch.testing.assert_close(res.payload.permute(0, 2, 1, 3).reshape_as(w), code, rtol=0, atol=0)


def test_identity_output_metric_is_one_sided_blockldlq():
    w = torch.randn((12, 8), generator=torch.Generator().manual_seed(2))
    h = _spd(12, 3)
    expected, code = _one_sided(w, h, 4)
    res = yaqa_block_round_encoder(w, h, torch.eye(8), _round_tiles, block_size=4)
    torch.testing.assert_close(res.reconstruction, expected, rtol=0, atol=0)
    torch.testing.assert_close(res.payload.permute(0, 2, 1, 3).reshape_as(w), code, rtol=0, atol=0)


def test_non_scalar_payload():
    def quantizer(tiles):
        r = torch.where(tiles.mean(dim=(1, 2))[:, None, None] >= 0, 0.5, -0.5).expand_as(tiles).contiguous()
        return r, torch.stack((r[:, 0, 0] > 0, tiles.square().mean(dim=(1, 2)) > 1), dim=1).to(torch.uint8)

    w = torch.randn((8, 8), generator=torch.Generator().manual_seed(4))
    res = yaqa_block_round_encoder(w, _spd(8, 5), _spd(8, 6), quantizer, block_size=4)
    assert res.reconstruction.shape == w.shape and res.payload.shape == (2, 2, 2)
    assert set(res.reconstruction.unique().tolist()) <= {-0.5, 0.5}


@pytest.mark.parametrize("bs,shape", [(1, (4, 4)), (2, (8, 12)), (4, (12, 8)), (4, (20, 28)), (2, (6, 16))])
def test_three_formulations_choose_identical_paths(bs, shape):
    g = torch.Generator().manual_seed(1000 + bs + shape[0])
    w = torch.randn(shape, generator=g)
    h_in, h_out = _spd(shape[0], 2000 + bs), _spd(shape[1], 3000 + bs)
    yaqa = yaqa_block_round_encoder(w, h_in, h_out, _round_tiles, block_size=bs)
    anti = bakron_block_antidiagonal_encoder(w, h_in, h_out, _round_tiles, block_size=bs)
    rec = bakron_block_round_encoder(w, h_in, h_out, _round_tiles, block_size=bs, update_chunk_blocks=2)
    for other in (anti, rec):
        torch.testing.assert_close(other.reconstruction, yaqa.reconstruction, rtol=0, atol=0)
        torch.testing.assert_close(other.payload, yaqa.payload, rtol=0, atol=0)


def test_two_sided_rounding_lowers_the_kronecker_loss():
    g = torch.Generator().manual_seed(77)
    w = torch.randn((32, 48), generator=g)
    h_in, h_out = _spd(32, 78), _spd(48, 79)
    loss = lambda q: float(torch.sum((h_in.double() @ (w - q).double()) * ((w - q).double() @ h_out.double())))
    independent = torch.round(w * 4) / 4
    rounded = bakron_block_round_encoder(w, h_in, h_out, _round_tiles, block_size=4).reconstruction
    assert loss(rounded) < loss(independent)


def test_factor_bakron_hessian_is_unit_block_inverse_cholesky():
    h = _spd(12, 9).double()
    f, rev = factor_bakron_hessian(h, block_size=4, dtype=torch.float64)
    hr = h[rev][:, rev]
    for s in range(0, 12, 4):
        torch.testing.assert_close(f[s:s + 4, s:s + 4], torch.eye(4, dtype=torch.float64))
    assert torch.all(torch.triu(f, 1).reshape(3, 4, 3, 4)[[0, 0, 1], :, [1, 2, 2]] == 0)
    # f D f^T = H_rev^-1 for the block-diagonal D of the factorisation
    inv = torch.linalg.inv(hr)
    finv = torch.linalg.inv(f)
    d = finv @ inv @ finv.T
    off = d.clone()
    for s in range(0, 12, 4):
        off[s:s + 4, s:s + 4] = 0
    assert float(off.abs().max()) < 1e-10


def test_output_metric_transform_preserves_the_quadratic_form():
    g = torch.Generator().manual_seed(7001)
    e = torch.randn((12, 8), generator=g)
    root = torch.randn((13, 8), generator=g)
    h = root.T @ root + 0.2 * torch.eye(8)
    s = torch.rand(8, generator=g) + 0.5
    reg = transform_output_hessian_for_regularization(h, s, block_size=4)
    dec = block_hadamard(e, block_size=4, dim=1) * s
    torch.testing.assert_close(torch.sum(e * (e @ reg)), torch.sum(dec * (dec @ h)), rtol=2e-5, atol=2e-5)
    roots = torch.randn((3, 8, 8), generator=g)
    blocks = roots.transpose(1, 2) @ roots + 0.2 * torch.eye(8)
    scales = torch.rand(24, generator=g) + 0.5
    got = transform_output_hessian_blocks_for_regularization(blocks, scales, block_size=8)
    dense = transform_output_hessian_for_regularization(torch.block_diag(*blocks), scales, block_size=8).reshape(3, 8, 3, 8)
    torch.testing.assert_close(got, dense[torch.arange(3), :, torch.arange(3)], rtol=0, atol=0)
    off = dense.clone()
    off[torch.arange(3), :, torch.arange(3)] = 0
    assert torch.count_nonzero(off) == 0
