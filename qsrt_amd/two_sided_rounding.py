"""Two-sided adaptive rounding for block trellis quantizers (mirrors
``qsrt/two_sided_rounding.py``).

Weights are in the encoder orientation ``[input, output]``; the tile
quantizer receives whole ``[b, b]`` tiles in that orientation, so a trellis
quantizer keeps one legal path per tile.  Three equivalent recurrences:

* ``yaqa_block_round_encoder``: the three-term YAQA update over reverse
  anti-diagonals (the batched recurrence of ``qsrt_amd.two_sided_ldlq``);
* ``bakron_block_antidiagonal_encoder``: BaKron's inverse-Cholesky form in
  reversed block order — after each anti-diagonal the running target gains
  ``L_out (Q - T)_d L_in^T``;
* ``bakron_block_round_encoder``: the same update scheduled by BaKron's
  divide and conquer: a finished band of anti-diagonals ``[first, middle)``
  is propagated into the next band ``[middle, last)`` once, as two products
  restricted to the blocks the bands can reach.

On the GPU in FP32 with 16 x 16 blocks, every band propagation of the
divide and conquer (and of the lockstep batches) is the fused HIP band
kernel (``qsrt_amd.sqg_quantizer.apply_bakron_block_update``, two launches
per band on the FP32 matrix cores; with the factors computed here, which are
unit-block-lower, the left launch skips their zero blocks); otherwise,
and for the anti-diagonal recurrence, the update is two dense tensor
products on the bands' bounding boxes.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass

import torch

from .qsrt_coupled import block_hadamard
from .sqg_quantizer import apply_bakron_block_update as _hip_apply_update
from .two_sided_ldlq import two_sided_block_ldlq

TileQuantizer = Callable[[torch.Tensor], tuple[torch.Tensor, torch.Tensor]]


@dataclass(frozen=True)
class TwoSidedRoundingResult:
    """Decoded weights and one payload item per (input, output) tile."""

    reconstruction: torch.Tensor
    payload: torch.Tensor


def _finite_matrix(value: torch.Tensor, name: str) -> None:
    if value.ndim != 2 or not value.numel():
        raise ValueError(f"{name} must be a nonempty matrix")
    if not bool(torch.all(torch.isfinite(value))):
        raise ValueError(f"{name} must be finite")


def transform_output_hessian_for_regularization(hessian: torch.Tensor, output_scales: torch.Tensor, *,
                                                block_size: int = 128) -> torch.Tensor:
    """``H D hessian D H`` for decoded error ``E_work H D`` (reference
    two_sided_rounding.py:29-55), symmetrised."""

    _finite_matrix(hessian, "output Hessian")
    if hessian.shape[0] != hessian.shape[1]:
        raise ValueError("output Hessian must be square")
    scales = output_scales.flatten()
    if scales.numel() != hessian.shape[0]:
        raise ValueError("output scales do not match the Hessian dimension")
    if not bool(torch.all(torch.isfinite(scales))):
        raise ValueError("output scales must be finite")
    s = scales.to(device=hessian.device, dtype=hessian.dtype)
    out = hessian * s[None, :] * s[:, None]
    out = block_hadamard(block_hadamard(out, block_size=block_size, dim=1), block_size=block_size, dim=0)
    return ((out + out.T) * 0.5).contiguous()


def transform_output_hessian_blocks_for_regularization(hessian_blocks: torch.Tensor, output_scales: torch.Tensor, *,
                                                       block_size: int = 128) -> torch.Tensor:
    """The same transform of a block-diagonal metric given as its diagonal
    blocks ``[..., blocks, b, b]`` (reference :58-94)."""

    if hessian_blocks.ndim < 3 or hessian_blocks.shape[-2:] != (block_size, block_size):
        raise ValueError("output Hessian blocks have incompatible geometry")
    blocks = int(hessian_blocks.shape[-3])
    if output_scales.shape != (*hessian_blocks.shape[:-3], blocks * block_size):
        raise ValueError("output scales do not match the block Hessian geometry")
    if hessian_blocks.device != output_scales.device:
        raise ValueError("output Hessian blocks and scales must share one device")
    if not bool(torch.all(torch.isfinite(hessian_blocks))) or not bool(torch.all(torch.isfinite(output_scales))):
        raise ValueError("output Hessian blocks and scales must be finite")
    s = output_scales.to(hessian_blocks.dtype).reshape(*hessian_blocks.shape[:-3], blocks, block_size)
    out = hessian_blocks * s.unsqueeze(-2) * s.unsqueeze(-1)
    out = block_hadamard(block_hadamard(out, block_size=block_size, dim=-1), block_size=block_size, dim=-2)
    return ((out + out.transpose(-1, -2)) * 0.5).contiguous()


def _normalise_columns(lower: torch.Tensor, block_size: int) -> torch.Tensor:
    """``lower[:, blk] <- lower[:, blk] lower[blk, blk]^-1`` for every column
    block (batched over leading dimensions)."""

    n = lower.shape[-1]
    m = n // block_size
    lead = lower.shape[:-2]
    cols = lower.reshape(*lead, n, m, block_size).movedim(-2, -3)            # [..., m, n, b]
    diag = torch.diagonal(lower.reshape(*lead, m, block_size, m, block_size), dim1=-4, dim2=-2)
    diag = diag.movedim(-1, -3)                                               # [..., m, b, b]
    solved = torch.linalg.solve_triangular(diag.transpose(-1, -2), cols.transpose(-1, -2), upper=True)
    return solved.transpose(-1, -2).movedim(-3, -2).reshape(*lead, n, n).contiguous()


def _check_square(hessian: torch.Tensor, block_size: int) -> int:
    if hessian.shape[-1] != hessian.shape[-2]:
        raise ValueError("Hessian must be square")
    n = int(hessian.shape[-1])
    if block_size <= 0 or n % block_size:
        raise ValueError("block size must divide the Hessian dimension")
    return n


def _strict_block_ldl_factor(hessian: torch.Tensor, block_size: int, *, dtype, device) -> torch.Tensor:
    """``C blockdiag(C_bb)^-1`` with zero diagonal blocks, ``C`` the Cholesky
    factor (reference :104-131)."""

    _finite_matrix(hessian, "Hessian")
    n = _check_square(hessian, block_size)
    h = hessian.to(device=device, dtype=dtype)
    lower = _normalise_columns(torch.linalg.cholesky((h + h.T) * 0.5), block_size)
    m = n // block_size
    blocks = lower.view(m, block_size, m, block_size)
    idx = torch.arange(m, device=lower.device)
    blocks[idx, :, idx] = 0
    return lower


def _reverse_block_indices(dimension: int, block_size: int, *, device) -> torch.Tensor:
    return torch.arange(dimension, device=device).reshape(dimension // block_size, block_size).flip(0).reshape(-1)


def _unit_block_inverse_cholesky_factor(hessian: torch.Tensor, block_size: int, *, dtype, device):
    """Unit-block-lower Cholesky factor of ``H^-1`` in reversed block order,
    and that order (reference :144-174)."""

    _finite_matrix(hessian, "Hessian")
    n = _check_square(hessian, block_size)
    reverse = _reverse_block_indices(n, block_size, device=device)
    h = hessian.to(device=device, dtype=dtype).index_select(0, reverse).index_select(1, reverse)
    inverse = torch.cholesky_inverse(torch.linalg.cholesky((h + h.T) * 0.5))
    return _normalise_columns(torch.linalg.cholesky((inverse + inverse.T) * 0.5), block_size), reverse


def factor_bakron_hessian(hessian: torch.Tensor, *, block_size: int = 16, dtype: torch.dtype = torch.float32):
    """Factor one Hessian for reuse by prepared BaKron recurrences."""

    return _unit_block_inverse_cholesky_factor(hessian, block_size, dtype=dtype, device=hessian.device)


def _unit_block_inverse_cholesky_factor_batch(hessians: torch.Tensor, block_size: int, *, dtype, device):
    if hessians.ndim != 3 or not hessians.shape[0]:
        raise ValueError("Hessians must be a nonempty matrix batch")
    n = _check_square(hessians, block_size)
    if not bool(torch.all(torch.isfinite(hessians))):
        raise ValueError("Hessians must be finite")
    reverse = _reverse_block_indices(n, block_size, device=device)
    h = hessians.to(device=device, dtype=dtype).index_select(1, reverse).index_select(2, reverse)
    inverse = torch.cholesky_inverse(torch.linalg.cholesky((h + h.transpose(1, 2)) * 0.5))
    lower = torch.linalg.cholesky((inverse + inverse.transpose(1, 2)) * 0.5)
    return _normalise_columns(lower, block_size), reverse


def _check_weight_and_hessians(weight, input_hessian, output_hessian, block_size, work_dtype):
    _finite_matrix(weight, "weight")
    if work_dtype not in (torch.float32, torch.float64):
        raise ValueError("work_dtype must be float32 or float64")
    k, n = map(int, weight.shape)
    if k % block_size or n % block_size:
        raise ValueError("block size must divide both weight dimensions")
    if tuple(input_hessian.shape) != (k, k):
        raise ValueError("input Hessian has the wrong shape")
    if tuple(output_hessian.shape) != (n, n):
        raise ValueError("output Hessian has the wrong shape")
    return k, n


def _check_tiles(recon: torch.Tensor, payload: torch.Tensor, tiles: torch.Tensor) -> None:
    if recon.shape != tiles.shape:
        raise ValueError("tile quantizer returned the wrong reconstruction shape")
    if payload.ndim < 1 or payload.shape[0] != tiles.shape[0]:
        raise ValueError("tile quantizer payload must have one leading item per tile")
    if not bool(torch.all(torch.isfinite(recon))):
        raise ValueError("tile quantizer returned a nonfinite reconstruction")


def yaqa_block_round_encoder(weight: torch.Tensor, input_hessian: torch.Tensor, output_hessian: torch.Tensor,
                             quantize_tiles: TileQuantizer, *, block_size: int = 16,
                             work_dtype: torch.dtype = torch.float64) -> TwoSidedRoundingResult:
    """YAQA's reverse anti-diagonal block update with strict block-LDL factors
    of both metrics, the quantizer kept as the legal set (reference :423-543)."""

    k, n = _check_weight_and_hessians(weight, input_hessian, output_hessian, block_size, work_dtype)
    device = weight.device
    l_in = _strict_block_ldl_factor(input_hessian, block_size, dtype=work_dtype, device=device)
    l_out = _strict_block_ldl_factor(output_hessian, block_size, dtype=work_dtype, device=device)

    def source_tiles(tiles):  # [output, input] tiles -> encoder orientation and back
        recon, payload = quantize_tiles(tiles.transpose(1, 2).contiguous())
        _check_tiles(recon, payload, tiles)
        return recon.to(device=device, dtype=work_dtype).transpose(1, 2).contiguous(), payload

    recon, payload = two_sided_block_ldlq(weight.to(work_dtype).T.contiguous(), l_in, l_out, source_tiles,
                                          block_size=block_size)
    return TwoSidedRoundingResult(recon.T.to(dtype=weight.dtype).contiguous(),
                                  payload.transpose(0, 1).contiguous())


def _diagonal_blocks(ob: int, ib: int, first: int, last: int, device):
    """Block coordinates (output, input) of anti-diagonals [first, last),
    output ascending within a diagonal."""

    o, i = [], []
    for d in range(first, last):
        lo, hi = max(0, d - ib + 1), min(ob, d + 1)
        o.extend(range(lo, hi))
        i.extend(d - x for x in range(lo, hi))
    return torch.tensor(o, dtype=torch.long, device=device), torch.tensor(i, dtype=torch.long, device=device)


def _band_box(ob: int, ib: int, first: int, last: int):
    """Row and column block ranges of the anti-diagonal band [first, last)."""

    return (max(0, first - ib + 1), min(ob, last)), (max(0, first - ob + 1), min(ib, last))


def _propagate_band(workspace, quantized, output_factor, input_factor, *, first: int, middle: int, last: int,
                    block_size: int) -> None:
    """``T[band2] += (L_out (Q - T)[band1] L_in^T)[band2]`` for the finished
    band ``[first, middle)`` and the next band ``[middle, last)``; leading
    dimensions are a batch.  Both products run on the bounding boxes of the
    bands (a block-lower factor maps rows and columns only forward)."""

    b = block_size
    ob, ib = workspace.shape[-2] // b, workspace.shape[-1] // b
    (sr0, sr1), (sc0, sc1) = _band_box(ob, ib, first, middle)
    (tr0, tr1), (tc0, tc1) = _band_box(ob, ib, middle, last)
    if sr0 >= sr1 or sc0 >= sc1 or tr0 >= tr1 or tc0 >= tc1:
        return
    rows = torch.arange(sr0, sr1, device=workspace.device)
    cols = torch.arange(sc0, sc1, device=workspace.device)
    in_source = ((rows[:, None] + cols[None, :]) >= first) & ((rows[:, None] + cols[None, :]) < middle)
    mask = in_source.repeat_interleave(b, 0).repeat_interleave(b, 1).to(workspace.dtype)
    delta = (quantized[..., sr0 * b:sr1 * b, sc0 * b:sc1 * b] - workspace[..., sr0 * b:sr1 * b, sc0 * b:sc1 * b]) * mask
    left = torch.matmul(output_factor[..., tr0 * b:tr1 * b, sr0 * b:sr1 * b], delta)
    update = torch.matmul(left, input_factor[..., tc0 * b:tc1 * b, sc0 * b:sc1 * b].transpose(-1, -2))
    trows = torch.arange(tr0, tr1, device=workspace.device)
    tcols = torch.arange(tc0, tc1, device=workspace.device)
    in_target = ((trows[:, None] + tcols[None, :]) >= middle) & ((trows[:, None] + tcols[None, :]) < last)
    tmask = in_target.repeat_interleave(b, 0).repeat_interleave(b, 1).to(workspace.dtype)
    workspace[..., tr0 * b:tr1 * b, tc0 * b:tc1 * b] += update * tmask


def _hip_update_applies(workspace: torch.Tensor, work_dtype, block_size: int) -> bool:
    return workspace.is_cuda and work_dtype == torch.float32 and block_size == 16


def apply_bakron_block_update(workspace, quantized, output_factor, input_factor, intermediate=None, *,
                              first_diagonal: int, middle_diagonal: int, last_diagonal: int,
                              block_size: int = 16) -> None:
    """One band propagation of the recursive BaKron recurrence (the operation
    the reference binds as ``qsrt.sqg_quantizer.apply_bakron_block_update``).
    GPU FP32 problems with 16 x 16 blocks run the fused HIP band kernel
    (``intermediate`` is then the kernel's [.., n_out, n_in] buffer,
    allocated here when None); others run the two bounding-box products."""

    if not first_diagonal < middle_diagonal < last_diagonal:
        raise ValueError("band diagonals must satisfy first < middle < last")
    if _hip_update_applies(workspace, workspace.dtype, block_size):
        if intermediate is None:
            intermediate = torch.empty_like(workspace)
        _hip_apply_update(workspace, quantized, output_factor, input_factor, intermediate,
                          first_diagonal=first_diagonal, middle_diagonal=middle_diagonal,
                          last_diagonal=last_diagonal, block_size=block_size)
        return
    _propagate_band(workspace, quantized, output_factor, input_factor, first=first_diagonal, middle=middle_diagonal,
                    last=last_diagonal, block_size=block_size)


class _BakronState:
    """Reversed-order running targets, reconstructions and payload grid of
    one or a batch of matrices."""

    def __init__(self, weights, input_factor, output_factor, input_reverse, output_reverse, block_size, work_dtype,
                 hip_update=False, own_factors=True):
        self.b = block_size
        self.batched = weights.ndim == 3
        w = weights if self.batched else weights.unsqueeze(0)
        self.batch, k, n = map(int, w.shape)
        self.ob, self.ib = n // block_size, k // block_size
        source = w.to(dtype=work_dtype).transpose(1, 2)
        self.workspace = source.index_select(1, output_reverse).index_select(2, input_reverse).contiguous()
        self.quantized = torch.zeros_like(self.workspace)
        self.l_in, self.l_out = input_factor, output_factor
        self.in_rev, self.out_rev = input_reverse, output_reverse
        self.payload = None
        self.dtype = work_dtype
        self.intermediate = torch.empty_like(self.workspace) if hip_update else None
        # factors computed here are unit-block-lower; supplied ones are taken as they come
        self.block_lower = own_factors

    def propagate(self, first: int, middle: int, last: int) -> None:
        """Band [first, middle) into [middle, last): the fused HIP kernel when
        the state was built for it, the bounding-box products otherwise."""

        if self.intermediate is not None:
            l_out = self.l_out[0] if self.l_out.ndim == 3 and self.l_out.shape[0] == 1 else self.l_out
            l_in = self.l_in[0] if self.l_in.ndim == 3 and self.l_in.shape[0] == 1 else self.l_in
            _hip_apply_update(self.workspace, self.quantized, l_out.contiguous(), l_in.contiguous(),
                              self.intermediate, first_diagonal=first, middle_diagonal=middle,
                              last_diagonal=last, block_size=self.b, block_lower=self.block_lower)
        else:
            _propagate_band(self.workspace, self.quantized, self.l_out, self.l_in, first=first, middle=middle,
                            last=last, block_size=self.b)

    def _blocks(self, x):
        return x.view(self.batch, self.ob, self.b, self.ib, self.b).permute(0, 1, 3, 2, 4)

    def quantize_diagonal(self, d: int, quantize_tiles) -> torch.Tensor:
        o, i = _diagonal_blocks(self.ob, self.ib, d, d + 1, self.workspace.device)
        tiles = self._blocks(self.workspace)[:, o, i].transpose(-1, -2).reshape(-1, self.b, self.b).contiguous()
        recon, payload = quantize_tiles(tiles)
        _check_tiles(recon, payload, tiles)
        count = o.numel()
        if self.payload is None:
            self.payload = torch.empty((self.batch, self.ib, self.ob, *payload.shape[1:]), dtype=payload.dtype,
                                       device=payload.device)
        elif self.payload.shape[3:] != payload.shape[1:]:
            raise ValueError("tile quantizer payload shape changed between calls")
        recon = recon.to(device=self.workspace.device, dtype=self.dtype).reshape(self.batch, count, self.b, self.b)
        self._blocks(self.quantized)[:, o, i] = recon.transpose(-1, -2)
        dev = self.payload.device
        self.payload[:, (self.ib - 1 - i).to(dev), (self.ob - 1 - o).to(dev)] = payload.reshape(
            self.batch, count, *payload.shape[1:])
        return recon

    def result(self, dtype) -> TwoSidedRoundingResult:
        if not bool(torch.all(torch.isfinite(self.quantized))):
            raise ValueError("tile quantizer returned a nonfinite reconstruction")
        recon = self.quantized.index_select(1, self.out_rev).index_select(2, self.in_rev).transpose(1, 2)
        recon = recon.to(dtype=dtype).contiguous()
        payload = self.payload
        if not self.batched:
            recon, payload = recon[0], payload[0]
        return TwoSidedRoundingResult(recon, payload)


def bakron_block_antidiagonal_encoder(weight: torch.Tensor, input_hessian: torch.Tensor, output_hessian: torch.Tensor,
                                      quantize_tiles: TileQuantizer, *, block_size: int = 16,
                                      work_dtype: torch.dtype = torch.float64) -> TwoSidedRoundingResult:
    """BaKron's anti-diagonal recurrence, one update after every anti-diagonal
    (reference :546-652): the correctness oracle of the recursive scheduler."""

    _check_weight_and_hessians(weight, input_hessian, output_hessian, block_size, work_dtype)
    device = weight.device
    l_in, in_rev = _unit_block_inverse_cholesky_factor(input_hessian, block_size, dtype=work_dtype, device=device)
    l_out, out_rev = _unit_block_inverse_cholesky_factor(output_hessian, block_size, dtype=work_dtype, device=device)
    st = _BakronState(weight, l_in, l_out, in_rev, out_rev, block_size, work_dtype)
    diagonals = st.ob + st.ib - 1
    for d in range(diagonals):
        st.quantize_diagonal(d, quantize_tiles)
        _propagate_band(st.workspace, st.quantized, l_out, l_in, first=d, middle=d + 1, last=diagonals,
                        block_size=block_size)
    return st.result(weight.dtype)


def _recurse(st: _BakronState, quantize_tiles, first: int, last: int) -> None:
    if last == first + 1:
        st.quantize_diagonal(first, quantize_tiles)
        return
    middle = (first + last) // 2
    _recurse(st, quantize_tiles, first, middle)
    st.propagate(first, middle, last)
    _recurse(st, quantize_tiles, middle, last)


def bakron_block_round_encoder(weight: torch.Tensor, input_hessian: torch.Tensor, output_hessian: torch.Tensor,
                               quantize_tiles: TileQuantizer, *, block_size: int = 16,
                               work_dtype: torch.dtype = torch.float64, update_chunk_blocks: int = 16,
                               update_backend: str = "auto") -> TwoSidedRoundingResult:
    """Two-sided adaptive rounding by BaKron's divide and conquer over
    anti-diagonals: one quantizer call per anti-diagonal, every band pair
    propagated once (reference :655-820).  ``update_chunk_blocks`` is
    validated for interface parity (the band products are not chunked).
    ``update_backend`` as the reference's (:707-715): ``"auto"`` runs the
    fused HIP band kernel for a GPU FP32 problem with 16x16 blocks and the
    bounding-box products otherwise, ``"torch"`` always the products,
    ``"cuda"`` requires the kernel's conditions."""

    _check_weight_and_hessians(weight, input_hessian, output_hessian, block_size, work_dtype)
    if update_chunk_blocks <= 0:
        raise ValueError("update_chunk_blocks must be positive")
    if update_backend not in ("auto", "torch", "cuda"):
        raise ValueError("update_backend must be 'auto', 'torch', or 'cuda'")
    hip_update = update_backend == "cuda" or (update_backend == "auto"
                                              and _hip_update_applies(weight, work_dtype, block_size))
    if update_backend == "cuda" and not _hip_update_applies(weight, work_dtype, block_size):
        raise ValueError("GPU BaKron updates require a GPU FP32 problem with 16x16 blocks")
    device = weight.device
    l_in, in_rev = _unit_block_inverse_cholesky_factor(input_hessian, block_size, dtype=work_dtype, device=device)
    l_out, out_rev = _unit_block_inverse_cholesky_factor(output_hessian, block_size, dtype=work_dtype, device=device)
    st = _BakronState(weight, l_in, l_out, in_rev, out_rev, block_size, work_dtype, hip_update)
    _recurse(st, quantize_tiles, 0, st.ob + st.ib - 1)
    return st.result(weight.dtype)


def _check_batch(weights, block_size, work_dtype, what):
    if weights.ndim != 3 or not weights.shape[0] or not weights.is_floating_point():
        raise ValueError("weights must be a nonempty floating-point matrix batch")
    if not weights.is_cuda:
        raise ValueError(f"{what} requires a GPU")
    if work_dtype != torch.float32 or block_size != 16:
        raise ValueError(f"{what} requires FP32 and 16x16 blocks")
    batch, k, n = map(int, weights.shape)
    if k % block_size or n % block_size:
        raise ValueError("block size must divide both weight dimensions")
    if not bool(torch.all(torch.isfinite(weights))):
        raise ValueError("weights must be finite")
    return batch, k, n


def bakron_block_round_encoder_batch(weights: torch.Tensor, input_hessians: torch.Tensor,
                                     output_hessians: torch.Tensor, quantize_tiles: TileQuantizer, *,
                                     block_size: int = 16,
                                     work_dtype: torch.dtype = torch.float32) -> TwoSidedRoundingResult:
    """Independent matrices in lockstep: one quantizer call per anti-diagonal
    holds every member's tiles (member-major), and each band propagation is
    one batched product (reference :823-985).  Factors are computed one matrix
    at a time, as a batched factorisation rounds differently."""

    batch, k, n = _check_batch(weights, block_size, work_dtype, "batched BaKron rounding")
    if tuple(input_hessians.shape) != (batch, k, k):
        raise ValueError("input Hessians have the wrong shape")
    if tuple(output_hessians.shape) != (batch, n, n):
        raise ValueError("output Hessians have the wrong shape")
    if input_hessians.device != weights.device or output_hessians.device != weights.device:
        raise ValueError("weights and Hessians must share one GPU")
    device = weights.device
    ins = [_unit_block_inverse_cholesky_factor(input_hessians[j], block_size, dtype=work_dtype, device=device)
           for j in range(batch)]
    outs = [_unit_block_inverse_cholesky_factor(output_hessians[j], block_size, dtype=work_dtype, device=device)
            for j in range(batch)]
    st = _BakronState(weights, torch.stack([f for f, _ in ins]), torch.stack([f for f, _ in outs]), ins[0][1],
                      outs[0][1], block_size, work_dtype, hip_update=True)
    _recurse(st, quantize_tiles, 0, st.ob + st.ib - 1)
    return st.result(weights.dtype)


def bakron_block_round_encoder_prepared_batch(weights: torch.Tensor, input_factors: torch.Tensor,
                                              output_factors: torch.Tensor, input_reverse: torch.Tensor,
                                              output_reverse: torch.Tensor, quantize_tiles: TileQuantizer, *,
                                              block_size: int = 16,
                                              work_dtype: torch.dtype = torch.float32) -> TwoSidedRoundingResult:
    """Lockstep batch with supplied BaKron factors: a rank-2 factor is shared
    by every member, a rank-3 factor gives one per member (reference :988-1155)."""

    batch, k, n = _check_batch(weights, block_size, work_dtype, "prepared batched BaKron rounding")
    for factor, dim, name in ((input_factors, k, "input factors"), (output_factors, n, "output factors")):
        if tuple(factor.shape) not in ((dim, dim), (batch, dim, dim)):
            raise ValueError(f"{name} has the wrong shape")
        if factor.device != weights.device or factor.dtype != work_dtype or not factor.is_contiguous():
            raise ValueError(f"{name} must be contiguous GPU FP32")
        if not bool(torch.all(torch.isfinite(factor))):
            raise ValueError(f"{name} must be finite")
    for reverse, dim, name in ((input_reverse, k, "input reverse order"), (output_reverse, n, "output reverse order")):
        if tuple(reverse.shape) != (dim,) or reverse.device != weights.device or reverse.dtype != torch.long:
            raise ValueError(f"{name} has incompatible geometry")
    st = _BakronState(weights, input_factors, output_factors, input_reverse, output_reverse, block_size, work_dtype,
                      hip_update=True, own_factors=False)
    _recurse(st, quantize_tiles, 0, st.ob + st.ib - 1)
    return st.result(weights.dtype)


__all__ = [
    "TileQuantizer",
    "TwoSidedRoundingResult",
    "apply_bakron_block_update",
    "bakron_block_antidiagonal_encoder",
    "bakron_block_round_encoder",
    "bakron_block_round_encoder_batch",
    "bakron_block_round_encoder_prepared_batch",
    "factor_bakron_hessian",
    "transform_output_hessian_for_regularization",
    "transform_output_hessian_blocks_for_regularization",
    "yaqa_block_round_encoder",
]
