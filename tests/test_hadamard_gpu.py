"""HIP blockwise Hadamard kernel (qsrt_hadamard) against the float64
Sylvester matrix: every block size, both sides, partial tiles, strided
rows, fused pre/post scales; the coupled expert basis on the device against
the CPU path."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import fmt as ofmt
from qsrt_amd import hadamard
from qsrt_amd.qsrt_coupled import CoupledHadamardSpec, coupled_execution, decode_coupled_weights, encode_coupled_weights

pytestmark = pytest.mark.gpu


def _want(x, block, side, pre_mul=None, pre_div=None, post_mul=None):
    x = x.astype(np.float64)
    axis = 0 if side == "left" else 1
    shape = (-1, 1) if axis == 0 else (1, -1)
    if pre_mul is not None:
        x = x * pre_mul.reshape(shape)
    if pre_div is not None:
        x = x / pre_div.reshape(shape)
    h = ofmt.hadamard(block)
    xm = np.moveaxis(x, axis, -1)
    s = xm.shape
    y = np.moveaxis((xm.reshape(*s[:-1], s[-1] // block, block) @ h.T).reshape(s), -1, axis)
    if post_mul is not None:
        y = y * post_mul.reshape(shape)
    return y


CASES = [
    (block, side, shape)
    for block in (64, 128, 256, 512)
    for side in ("left", "right")
    for shape in ((1024, 1024), (512, 516) if side == "left" else (516, 512))
]


@pytest.mark.parametrize("block,side,shape", CASES)
def test_hadamard_matches_float64(block, side, shape):
    print(f"[hadamard] block {block} {side} {shape}", file=sys.stderr, flush=True)
    rows, cols = shape
    g = torch.Generator().manual_seed(block * 7 + rows)
    x = torch.randn(rows, cols, generator=g)
    got = x.cuda()
    hadamard.rotate_(got, block, side=side)
    want = _want(x.numpy(), block, side)
    err = np.max(np.abs(got.cpu().double().numpy() - want))
    assert err <= 1e-5 * np.abs(want).max()


@pytest.mark.parametrize("side", ["left", "right"])
def test_hadamard_fused_scales_and_strided_rows(side):
    g = torch.Generator().manual_seed(9)
    big = torch.randn(640, 776, generator=g)
    x = big[:, 8:520]  # ld 776 > cols 512, 32-byte offset
    ext = 640 if side == "left" else 512
    pre_mul = torch.randn(ext, generator=g)
    pre_div = torch.rand(ext, generator=g) + 0.5
    post_mul = torch.randn(ext, generator=g)
    dev = big.cuda()
    view = dev[:, 8:520]
    hadamard.rotate_(view, 128, side=side, pre_mul=pre_mul.cuda(), pre_div=pre_div.cuda(), post_mul=post_mul.cuda())
    want = _want(x.numpy(), 128, side, pre_mul.numpy(), pre_div.numpy(), post_mul.numpy())
    got = dev.cpu()
    assert np.max(np.abs(got[:, 8:520].double().numpy() - want)) <= 1e-5 * np.abs(want).max()
    # columns outside the view are untouched
    assert torch.equal(got[:, :8], big[:, :8]) and torch.equal(got[:, 520:], big[:, 520:])


def test_hadamard_rejects_bad_shapes():
    x = torch.zeros(100, 128, device="cuda")
    with pytest.raises(ValueError):
        hadamard.rotate_(x, 128, side="left")
    with pytest.raises(ValueError):
        hadamard.rotate_(torch.zeros(128, 128, device="cuda"), 32, side="left")
    y = torch.zeros(0, 128, device="cuda")
    hadamard.rotate_(y, 128, side="right")


def test_coupled_basis_on_device_matches_cpu_path():
    print("[hadamard] coupled expert 2048x512", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(33)
    hidden, inter = 2048, 512
    w = (torch.randn(inter, hidden, generator=g), torch.randn(inter, hidden, generator=g),
         torch.randn(hidden, inter, generator=g))
    spec = CoupledHadamardSpec(intermediate_draw=3)
    cpu = encode_coupled_weights(w, spec)
    gpu = encode_coupled_weights(tuple(t.cuda() for t in w), spec)
    for a, b in zip(gpu, cpu):
        assert torch.allclose(a.cpu(), b, rtol=1e-5, atol=1e-5)
    back = decode_coupled_weights(gpu, spec)
    for a, b in zip(back, w):
        assert torch.allclose(a.cpu(), b, rtol=1e-5, atol=1e-5)
    ex = coupled_execution(gpu, spec)
    rows = torch.randn(64, hidden, generator=g)
    h13 = rows.T @ rows
    tr = ex.transform_inputs(rows.cuda())
    assert torch.allclose(ex.transform_h13(h13.cuda()).cpu(), (tr.T @ tr).cpu(), rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("block,side", [(b, s) for b in (64, 128, 256, 512) for s in ("left", "right")])
def test_float64_hadamard_matches_float64(block, side):
    """qsrt_hadamard_f64 (the regularisation's rotation) against the float64
    Sylvester product, with fused pre-division and post-scale: float64 on
    both sides, so they agree to float64 rounding."""

    print(f"[hadamard] f64 block {block} {side}", file=sys.stderr, flush=True)
    rows, cols = (1024, 516) if side == "left" else (516, 1024)
    g = torch.Generator().manual_seed(block * 11 + rows)
    x = torch.randn(rows, cols, generator=g, dtype=torch.float64)
    ext = rows if side == "left" else cols
    div = torch.rand(ext, generator=g, dtype=torch.float64) + 0.5
    post = torch.randn(ext, generator=g, dtype=torch.float64)
    got = x.cuda()
    hadamard.rotate_(got, block, side=side, pre_div=div.cuda(), post_mul=post.cuda())
    want = _want(x.numpy(), block, side, pre_div=div.numpy(), post_mul=post.numpy())
    assert got.dtype == torch.float64
    assert np.max(np.abs(got.cpu().numpy() - want)) <= 1e-14 * np.abs(want).max()
