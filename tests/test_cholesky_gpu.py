"""The blocked float64 Cholesky (``qsrt_amd/cholesky.py`` over
``qsrt_chol_diag_block_f64``) against float64 references.

* the factor reproduces the matrix (``L L^T == A`` to float64 rounding) and
  equals rocsolver's factor of the same matrix to 1e-12 relative (the
  Cholesky factor is unique, so any two float64 factorisations agree to
  rounding times the condition number);
* sizes that are not multiples of the 128-row block (a short last block)
  and one block alone;
* the diagonal-block entry point's own contract: the block's factor and its
  inverse (``L11 X == I``), zeros above both diagonals;
* ``info`` follows LAPACK: the order of the first leading minor that is not
  positive definite (a matrix made indefinite at a chosen row), and the
  retry-with-damping path of ``_block_ldl_f64`` recovers from it.
"""

from __future__ import annotations

import sys

import pytest
import torch

from qsrt_amd import _native
from qsrt_amd.cholesky import cholesky_f64

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _spd(n: int, seed: int, rows: int | None = None, damp: float = 0.01) -> torch.Tensor:
    g = torch.Generator(device="cuda").manual_seed(seed)
    X = torch.randn(rows or 2 * n, n, device=DEV, generator=g, dtype=torch.float64)
    A = X.T @ X / X.shape[0]
    A.diagonal().add_(damp * A.diagonal().mean())
    return A


@pytest.mark.parametrize("n", [1, 77, 128, 200, 256, 1000, 2048])
def test_blocked_factor_matches_rocsolver(n):
    print(f"[cholesky] n {n}", file=sys.stderr, flush=True)
    A = _spd(n, n)
    L, info = cholesky_f64(A)
    ref, ref_info = torch.linalg.cholesky_ex(A)
    torch.cuda.synchronize()
    assert int(info) == 0 and int(ref_info) == 0
    assert torch.equal(L, torch.tril(L))
    scale = ref.abs().max().item()
    assert (L - ref).abs().max().item() <= 1e-12 * scale
    assert (L @ L.T - A).abs().max().item() <= 1e-13 * A.abs().max().item()


def test_ill_conditioned_few_row_hessian():
    """A 7168-channel Hessian from 35 rows plus 1% damping (condition number
    ~1e4): the blocked factor still equals rocsolver's to rounding times the
    condition number."""

    A = _spd(7168, 35, rows=35)
    L, info = cholesky_f64(A)
    ref, _ = torch.linalg.cholesky_ex(A)
    assert int(info) == 0
    assert (L - ref).abs().max().item() <= 1e-9 * ref.abs().max().item()
    assert (L @ L.T - A).abs().max().item() <= 1e-13 * A.abs().max().item()


@pytest.mark.parametrize("nb", [1, 5, 64, 128])
def test_diagonal_block_and_its_inverse(nb):
    n, j0 = 300, 100
    A = _spd(n, nb + 1)
    M = A.clone()
    inv = torch.full((nb, nb), float("nan"), dtype=torch.float64, device=DEV)
    info = torch.zeros(1, dtype=torch.int32, device=DEV)
    lib = _native.lib()
    _native.check(lib.qsrt_chol_diag_block_f64(M.data_ptr(), n, 1, n * n, j0, nb, inv.data_ptr(), info.data_ptr(),
                                                _native.stream_handle(DEV)), "chol")
    torch.cuda.synchronize()
    assert int(info[0]) == 0
    blk = M[j0:j0 + nb, j0:j0 + nb]
    ref = torch.linalg.cholesky(A[j0:j0 + nb, j0:j0 + nb])
    assert torch.equal(blk, torch.tril(blk)) and torch.equal(inv, torch.tril(inv))
    assert (blk - ref).abs().max().item() <= 1e-13 * ref.abs().max().item()
    eye = torch.eye(nb, dtype=torch.float64, device=DEV)
    assert (blk @ inv - eye).abs().max().item() <= 1e-12
    # everything outside the block is untouched
    outside = torch.ones(n, n, dtype=torch.bool, device=DEV)
    outside[j0:j0 + nb, j0:j0 + nb] = False
    assert torch.equal(M[outside], A[outside])


@pytest.mark.parametrize("bad_row", [0, 127, 128, 300])
def test_info_reports_the_first_indefinite_leading_minor(bad_row):
    n = 400
    A = _spd(n, 9)
    A[bad_row, bad_row] = -1.0
    _, info = cholesky_f64(A)
    _, ref_info = torch.linalg.cholesky_ex(A)
    assert int(info) == int(ref_info) == bad_row + 1


def test_block_ldl_retries_an_indefinite_matrix():
    from qsrt_amd.exl3_encoder_backend import _block_ldl_f64

    n = 256
    A = _spd(n, 10, rows=8, damp=0.0)
    A.diagonal().sub_(0.5 * A.diagonal().mean() * 1e-3)  # slightly indefinite: rank 8 minus a shift
    H = A.clone()
    L = _block_ldl_f64(H, 16, {"sigma_reg": 0.01})
    assert torch.isfinite(L).all()
    assert not torch.equal(H, A)  # the retry damped it
    assert torch.equal(L.tril(), L)
    assert int(torch.linalg.cholesky_ex(H)[1]) == 0


def test_diagonal_block_batched_with_an_indefinite_member():
    """Three matrices in one launch (batch stride n * n): each member's block
    is its own factor and inverse, and a member made indefinite reports its
    own info without touching the others'."""

    n, j0, nb, batch = 256, 128, 128, 3
    A = torch.stack([_spd(n, 40 + b) for b in range(batch)])
    A[1, j0 + 7, j0 + 7] = -1.0
    M = A.clone()
    inv = torch.zeros(batch, nb, nb, dtype=torch.float64, device=DEV)
    info = torch.zeros(batch, dtype=torch.int32, device=DEV)
    lib = _native.lib()
    _native.check(lib.qsrt_chol_diag_block_f64(M.data_ptr(), n, batch, n * n, j0, nb, inv.data_ptr(),
                                                info.data_ptr(), _native.stream_handle(DEV)), "chol")
    torch.cuda.synchronize()
    assert info.tolist() == [0, j0 + 8, 0]
    eye = torch.eye(nb, dtype=torch.float64, device=DEV)
    for b in (0, 2):
        blk = M[b, j0:j0 + nb, j0:j0 + nb]
        ref = torch.linalg.cholesky(A[b, j0:j0 + nb, j0:j0 + nb])
        assert (blk - ref).abs().max().item() <= 1e-13 * ref.abs().max().item()
        assert (blk @ inv[b] - eye).abs().max().item() <= 1e-12


def test_bad_arguments_are_rejected():
    lib = _native.lib()
    A = torch.zeros(4, 4, dtype=torch.float64, device=DEV)
    inv = torch.zeros(4, 4, dtype=torch.float64, device=DEV)
    info = torch.zeros(1, dtype=torch.int32, device=DEV)
    s = _native.stream_handle(DEV)
    for args in ((4, 1, 16, 0, 129), (4, 1, 16, 2, 3), (4, 1, 16, -1, 2), (4, 2, 8, 0, 2), (0, 1, 0, 0, 1)):
        n, batch, stride, j0, nb = args
        with pytest.raises(ValueError):
            _native.check(lib.qsrt_chol_diag_block_f64(A.data_ptr(), n, batch, stride, j0, nb, inv.data_ptr(),
                                                        info.data_ptr(), s), "chol")


def _block_diag_of(C: torch.Tensor, b: int = 16) -> torch.Tensor:
    n = C.shape[-1]
    m = n // b
    return torch.diagonal(C.view(-1, m, b, m, b), dim1=1, dim2=3).permute(0, 3, 1, 2)


@pytest.mark.parametrize("n,batch,layout", [(16, 1, "row"), (1024, 1, "row"), (1024, 3, "row"), (784, 2, "col"),
                                            (16, 2, "col")])
def test_block_unit_lower_matches_the_column_block_products(n, batch, layout):
    """``qsrt_block_unit_lower_f64`` on row-major factors (the blocked
    Cholesky's) and column-major ones (torch's batched Cholesky's): equal to
    the torch column-block products within float64 rounding, exact identity
    diagonal blocks, the zeros above left alone, and ``L D L^T`` gives the
    matrix back (``D`` the blocks ``C_jj C_jj^T``)."""

    from qsrt_amd.cholesky import block_unit_lower_f64_

    print(f"[block_unit_lower] n {n} batch {batch} {layout}", file=sys.stderr, flush=True)
    A = torch.stack([_spd(n, 60 + b) for b in range(batch)])
    C = torch.linalg.cholesky(A)
    if layout == "row":
        C = C.contiguous()
    else:
        C = C.mT.contiguous().mT
    assert (C.stride(2) == 1) == (layout == "row")
    inv = torch.linalg.inv(_block_diag_of(C))
    D = _block_diag_of(C) @ _block_diag_of(C).mT
    ref = block_unit_lower_f64_(C.cpu().clone(), inv.cpu())
    out = block_unit_lower_f64_(C, inv)
    torch.cuda.synchronize()
    assert out.data_ptr() == C.data_ptr()
    assert (out.cpu() - ref).abs().max().item() <= 1e-13 * ref.abs().max().item()
    m = n // 16
    blocks = out.view(batch, m, 16, m, 16).permute(0, 1, 3, 2, 4)
    idx = torch.arange(m, device=DEV)
    assert torch.equal(blocks[:, idx, idx], torch.eye(16, dtype=torch.float64, device=DEV).expand(batch, m, 16, 16))
    assert torch.equal(out, out.tril())
    Dfull = torch.block_diag(*D.reshape(-1, 16, 16)).view(batch, m * 16, batch, m * 16)
    Dfull = torch.stack([Dfull[b, :, b] for b in range(batch)])
    assert (out @ Dfull @ out.mT - A).abs().max().item() <= 1e-12 * A.abs().max().item()


def test_block_unit_lower_rejects_bad_arguments():
    lib = _native.lib()
    C = torch.zeros(2, 32, 32, dtype=torch.float64, device=DEV)
    inv = torch.zeros(2, 2, 16, 16, dtype=torch.float64, device=DEV)
    s = _native.stream_handle(DEV)
    # n not a multiple of 16, no unit stride, leading dimension < n, overlapping members, odd row stride
    for n, rs, cs, bs, batch in ((24, 32, 1, 1024, 2), (32, 32, 2, 1024, 2), (32, 16, 1, 1024, 2),
                                 (32, 32, 1, 512, 2), (32, 33, 1, 1056, 1), (0, 32, 1, 1024, 2)):
        with pytest.raises(ValueError):
            _native.check(lib.qsrt_block_unit_lower_f64(C.data_ptr(), inv.data_ptr(), batch, n, rs, cs, bs, s),
                          "unit")
