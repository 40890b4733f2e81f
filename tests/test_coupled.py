"""Coupled expert basis (qsrt_amd.qsrt_coupled) on CPU tensors: the
butterfly against the float64 Sylvester matrix, exact closure, the coupled
forward equal to the ordinary expert forward, and Hessian transforms that
preserve quadratic forms (the reference's own invariants,
tests/test_qsrt_coupled.py:24-125)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fmt as ofmt
from qsrt_amd.qsrt_coupled import (
    CoupledHadamardSpec,
    block_hadamard,
    coupled_execution,
    decode_coupled_weights,
    encode_coupled_down_weight,
    encode_coupled_upstream_weights,
    encode_coupled_weights,
    rotation_signs,
    signed_block_hadamard,
    situ,
)


def _blockdiag_apply(x: np.ndarray, block: int, axis: int) -> np.ndarray:
    h = ofmt.hadamard(block)
    x = np.moveaxis(x, axis, -1)
    shape = x.shape
    y = (x.reshape(*shape[:-1], shape[-1] // block, block) @ h.T).reshape(shape)
    return np.moveaxis(y, -1, axis)


def test_empty_batch_keeps_shape_and_widens():
    values = torch.empty((0, 7, 16), dtype=torch.float16)
    out = block_hadamard(values, block_size=8, dim=2)
    assert out.shape == values.shape and out.dtype == torch.float32 and out.numel() == 0


@pytest.mark.parametrize("block", [2, 8, 64, 512])
@pytest.mark.parametrize("dim", [0, 1])
def test_butterfly_matches_sylvester_matrix(block, dim):
    g = torch.Generator().manual_seed(block + dim)
    x = torch.randn(1024, 512, generator=g)
    got = block_hadamard(x, block_size=block, dim=dim).double().numpy()
    want = _blockdiag_apply(x.double().numpy(), block, dim)
    assert np.max(np.abs(got - want)) < 1e-5 * np.abs(want).max()


def test_signed_transform_and_inverse_close():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(64, 256, generator=g)
    s = rotation_signs(256, draw=3, axis=1, device="cpu")
    y = signed_block_hadamard(x, block_size=128, signs=s, dim=1)
    want = _blockdiag_apply(x.double().numpy() * s.double().numpy(), 128, 1)
    assert np.allclose(y.double().numpy(), want, atol=1e-5)
    back = signed_block_hadamard(y, block_size=128, signs=s, dim=1, inverse=True)
    assert torch.allclose(back, x, atol=1e-5)


def test_rotation_signs_family():
    assert torch.equal(rotation_signs(10, draw=0, axis=2, device="cpu"), torch.ones(10))
    a = rotation_signs(4096, draw=3, axis=1, device="cpu")
    b = rotation_signs(4096, draw=3, axis=2, device="cpu")
    assert set(a.unique().tolist()) == {-1.0, 1.0}
    assert abs(float(a.mean())) < 0.1 and not torch.equal(a, b)
    assert torch.equal(a, rotation_signs(4096, draw=3, axis=1, device="cpu"))
    with pytest.raises(ValueError):
        rotation_signs(0, draw=1, axis=0, device="cpu")


def _expert(seed, hidden=16, intermediate=12):
    g = torch.Generator().manual_seed(seed)
    return (
        torch.randn(intermediate, hidden, generator=g),
        torch.randn(intermediate, hidden, generator=g),
        torch.randn(hidden, intermediate, generator=g),
    ), g


def test_coupled_transform_closes_and_preserves_the_forward():
    weights, g = _expert(871)
    inputs = torch.randn(9, 16, generator=g)
    spec = CoupledHadamardSpec(residual_block_size=8, preactivation_block_size=8, postactivation_block_size=4,
                               intermediate_draw=3)
    enc = encode_coupled_weights(weights, spec)
    up = encode_coupled_upstream_weights(weights[0], weights[1], spec)
    assert torch.equal(up[0], enc[0]) and torch.equal(up[1], enc[1])
    assert torch.equal(encode_coupled_down_weight(weights[2], spec), enc[2])
    for a, b in zip(decode_coupled_weights(enc, spec), weights):
        assert torch.allclose(a, b, rtol=2e-5, atol=2e-5)
    out = coupled_execution(enc, spec).execute(inputs, enc)
    ref = torch.nn.functional.linear(
        situ(torch.nn.functional.linear(inputs, weights[0]), torch.nn.functional.linear(inputs, weights[1])),
        weights[2])
    assert torch.allclose(out, ref, rtol=2e-5, atol=2e-5)
    # a planted mistake (gate/up swapped in the interleave) breaks the forward
    bad = coupled_execution(enc, spec).execute(inputs, (enc[1], enc[0], enc[2]))
    assert not torch.allclose(bad, ref, rtol=1e-2, atol=1e-2)


def test_coupled_hessian_transforms_preserve_quadratic_forms():
    weights, g = _expert(91)
    spec = CoupledHadamardSpec(residual_block_size=8, preactivation_block_size=8, postactivation_block_size=4,
                               intermediate_draw=5)
    ex = coupled_execution(encode_coupled_weights(weights, spec), spec)
    rows = torch.randn(11, 16, generator=g)
    hidden_rows = torch.randn(11, 12, generator=g)
    tr = ex.transform_inputs(rows)
    assert torch.allclose(ex.transform_h13(rows.T @ rows), tr.T @ tr, rtol=2e-5, atol=2e-5)
    th = ex.transform_postactivation_rows(hidden_rows)
    assert torch.allclose(ex.transform_h2(hidden_rows.T @ hidden_rows), th.T @ th, rtol=2e-5, atol=2e-5)
    outs = torch.randn(11, 16, generator=g)
    root = torch.randn(19, 16, generator=g)
    oh = root.T @ root
    ordinary = ex.decode_output(outs)
    lhs = torch.einsum("bi,ij,bj->", outs, ex.transform_output_hessian(oh), outs)
    rhs = torch.einsum("bi,ij,bj->", ordinary, oh, ordinary)
    assert torch.allclose(lhs, rhs, rtol=3e-5, atol=3e-5)


def test_spec_validation():
    with pytest.raises(ValueError):
        CoupledHadamardSpec(residual_block_size=96)
    with pytest.raises(ValueError):
        CoupledHadamardSpec(residual_draw=1)
    with pytest.raises(ValueError):
        CoupledHadamardSpec(intermediate_draw=8)
