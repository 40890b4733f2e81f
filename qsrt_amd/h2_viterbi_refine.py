"""Dense-H coordinate refinement of legal QSRT trellis paths (mirrors
``qsrt/h2_viterbi_refine.py``).

BlockLDLQ commits each 16-row block once.  A refinement sweep revisits the
blocks with every other block's error known: the exact conditional target of
a block under the dense Hessian, ``W_b + H_bb^-1 (H E - H_bb E_b)_b``, is
encoded by the ordinary tile Viterbi (plus optional H-whitened dithers), and a
tile takes a proposed path only when it strictly lowers the block's quadratic
score.  The running ``H E`` is updated with a rank-16 product per changed
block, which runs on the FP32 matrix-core GEMM for device FP32 scores.

Tensors are in the regularised encoder coordinates; the quantizer callback
takes and returns flattened 16x16 tiles in the EXL tensor-core order.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Callable, Iterable

import torch

from . import gemm
from .exl3_reference import tensor_core_permutation
from .gradient_guided_viterbi import LowRankViterbiGradientGuidance, ViterbiGradientGuidance

QuantizeTiles = Callable[[torch.Tensor], tuple[torch.Tensor, torch.Tensor]]
GradientGuidance = ViterbiGradientGuidance | LowRankViterbiGradientGuidance


@dataclass(frozen=True)
class H2ViterbiRefineConfig:
    """Search controls (reference h2_viterbi_refine.py:31-45)."""

    sweeps: int = 1
    alternate_sweep_order: bool = True
    dither_scales: tuple[float, ...] = ()
    num_dither_patterns: int = 0
    seed: int = 0x48325643
    max_quantizer_batch: int = 256
    acceptance_abs_tol: float = 1.0e-8
    acceptance_rel_tol: float = 1.0e-8
    score_dtype: torch.dtype = torch.float32
    stop_on_no_change: bool = True


@dataclass(frozen=True)
class H2ViterbiSweepStats:
    sweep: int
    objective_before: float
    objective_after: float
    quadratic_before: float
    quadratic_after: float
    linear_before: float
    linear_after: float
    relative_improvement: float
    accepted_tiles: int
    proposed_tiles: int
    unique_candidate_paths: int


@dataclass
class H2ViterbiRefineResult:
    weight_q: torch.Tensor
    encoded: torch.Tensor
    sweep_stats: list[H2ViterbiSweepStats]

    def stats_dict(self) -> dict[str, object]:
        return {"sweeps": [asdict(s) for s in self.sweep_stats]}


def _column_weights(column_weights, columns: int, device, dtype) -> torch.Tensor:
    if column_weights is None:
        return torch.ones(columns, dtype=dtype, device=device)
    if column_weights.numel() != columns:
        raise ValueError("column weights do not match the output dimension")
    weights = column_weights.reshape(-1).to(device=device, dtype=dtype)
    if bool(torch.any(weights < 0)):
        raise ValueError("column weights must be nonnegative")
    return weights


def dense_h_objective(weight: torch.Tensor, weight_q: torch.Tensor, hessian: torch.Tensor, *,
                      column_weights: torch.Tensor | None = None, chunk_columns: int = 512,
                      dtype: torch.dtype = torch.float64) -> float:
    """``sum_c a_c (W - Q)[:, c]^T H (W - Q)[:, c]`` (reference :72-105)."""

    if weight.shape != weight_q.shape or weight.ndim != 2:
        raise ValueError("weight and reconstruction must have one rank-2 shape")
    if hessian.shape != (weight.shape[0], weight.shape[0]):
        raise ValueError("Hessian shape does not match the input dimension")
    if chunk_columns <= 0:
        raise ValueError("chunk_columns must be positive")
    weights = _column_weights(column_weights, weight.shape[1], weight.device, dtype)
    h = hessian.to(device=weight.device, dtype=dtype)
    total = torch.zeros((), dtype=dtype, device=weight.device)
    for start in range(0, weight.shape[1], chunk_columns):
        stop = min(start + chunk_columns, weight.shape[1])
        error = (weight[:, start:stop] - weight_q[:, start:stop]).to(dtype)
        total += torch.sum(error * (h @ error) * weights[start:stop].unsqueeze(0))
    return float(total.item())


def _linear_term(guidance, reconstruction, dense_gradient, anchor, dtype) -> float:
    if guidance is None:
        return 0.0
    if isinstance(guidance, LowRankViterbiGradientGuidance):
        return guidance.linear_term(reconstruction, dtype=dtype)
    return float(float(guidance.strength) * torch.sum(dense_gradient * (reconstruction.to(dtype) - anchor)).item())


def dense_h_guided_objective(weight, weight_q, hessian, guidance: GradientGuidance, *, column_weights=None,
                             chunk_columns: int = 512, dtype: torch.dtype = torch.float64):
    """(quadratic, anchor-relative linear, sum) (reference :108-139)."""

    guidance.validate(weight.shape)
    quadratic = dense_h_objective(weight, weight_q, hessian, column_weights=column_weights,
                                  chunk_columns=chunk_columns, dtype=dtype)
    dense = None
    anchor = guidance.anchor.to(device=weight.device, dtype=dtype)
    if not isinstance(guidance, LowRankViterbiGradientGuidance):
        dense = guidance.gradient.to(device=weight.device, dtype=dtype)
    linear = _linear_term(guidance, weight_q, dense, anchor, dtype)
    return quadratic, linear, quadratic + linear


def _quantize_in_chunks(inputs: torch.Tensor, quantize_tiles: QuantizeTiles, max_batch: int):
    if max_batch <= 0:
        raise ValueError("max_quantizer_batch must be positive")
    recon, payloads = [], []
    for start in range(0, inputs.shape[0], max_batch):
        source = inputs[start:start + max_batch].contiguous()
        r, p = quantize_tiles(source)
        if r.shape != source.shape:
            raise ValueError("tile quantizer returned the wrong reconstruction shape")
        if p.ndim < 1 or p.shape[0] != source.shape[0]:
            raise ValueError("tile quantizer returned the wrong payload batch")
        recon.append(r)
        payloads.append(p)
    return torch.cat(recon), torch.cat(payloads)


def _h_whitened_patterns(hessian_block: torch.Tensor, *, count: int, seed: int, dtype: torch.dtype) -> torch.Tensor:
    """``count`` Rademacher probes mapped through ``L^-T`` (``H_bb = L L^T``)
    and rescaled to H-energy ``b^2`` (reference :183-219)."""

    b = hessian_block.shape[0]
    if count <= 0:
        return torch.empty((0, b, b), dtype=dtype, device=hessian_block.device)
    generator = torch.Generator(device=hessian_block.device)
    generator.manual_seed(seed)
    probes = torch.randint(0, 2, (count, b, b), generator=generator, device=hessian_block.device, dtype=torch.int64)
    probes = (probes * 2 - 1).to(dtype)
    h = hessian_block.to(dtype)
    chol = torch.linalg.cholesky(h)
    cols = torch.linalg.solve_triangular(chol.T, probes.permute(1, 0, 2).reshape(b, count * b), upper=True)
    patterns = cols.reshape(b, count, b).permute(1, 0, 2)
    energy = torch.sum(patterns * torch.matmul(h, patterns), dim=(1, 2), keepdim=True).clamp_min(1.0e-20)
    return patterns * torch.sqrt(torch.tensor(float(b * b), dtype=dtype, device=h.device) / energy)


def _conditional_target(weight_block, error_block, hessian_error_block, hessian_block, *, gradient_block=None,
                        gradient_strength: float = 0.0, column_weights=None):
    """``W_b + H_bb^-1 (H E)_b - E_b``-style exact conditional minimiser, with
    the completed-square gradient shift (reference :222-245)."""

    target = weight_block + torch.linalg.solve(hessian_block, hessian_error_block - hessian_block @ error_block)
    if gradient_block is None or gradient_strength == 0.0:
        return target
    if column_weights is None:
        scaled = gradient_block
    else:
        if bool(torch.any(column_weights <= 0)):
            raise ValueError("gradient-guided refinement requires positive column weights")
        scaled = gradient_block / column_weights.unsqueeze(0)
    return target - 0.5 * float(gradient_strength) * torch.linalg.solve(hessian_block, scaled)


def _conditional_scores(target_tiles, candidates, hessian_block, column_weight_tiles, dtype):
    """``sum a_c d^T H_bb d`` per tile and candidate, ``d = target - candidate``."""

    diff = (target_tiles[:, None] - candidates).to(dtype)
    weighted = torch.matmul(hessian_block.to(dtype), diff)
    return torch.sum(diff * weighted * column_weight_tiles[:, None, None, :].to(dtype), dim=(-2, -1))


def _candidate_paths(target_tiles, current_tiles, current_payload, hessian_block, permutation, inverse_permutation,
                     quantize_tiles, config: H2ViterbiRefineConfig, *, sweep: int, row_block: int):
    patterns = _h_whitened_patterns(hessian_block, count=config.num_dither_patterns,
                                    seed=config.seed + 1009 * sweep + 9176 * row_block, dtype=target_tiles.dtype)
    variants = [target_tiles]
    if patterns.numel() and config.dither_scales:
        rms = target_tiles.square().mean(dim=(-2, -1), keepdim=True).sqrt().clamp_min(1.0e-8)
        for scale in config.dither_scales:
            for pattern in patterns:
                shift = float(scale) * rms * pattern.unsqueeze(0)
                variants.extend((target_tiles + shift, target_tiles - shift))
    stacked = torch.stack(variants)
    n_var, n_tiles = stacked.shape[:2]
    recon, payload = _quantize_in_chunks(stacked.reshape(n_var * n_tiles, 256)[:, permutation], quantize_tiles,
                                         config.max_quantizer_batch)
    recon = recon[:, inverse_permutation].reshape(n_var, n_tiles, 16, 16).permute(1, 0, 2, 3).contiguous()
    payload_shape = payload.shape[1:]
    payload = payload.reshape(n_var, n_tiles, *payload_shape)
    payload = payload.permute(1, 0, *range(2, payload.ndim)).contiguous()
    if current_payload.shape[1:] != payload_shape:
        raise ValueError("stored and proposed trellis payload shapes differ")
    candidates = torch.cat((current_tiles[:, None], recon), dim=1)
    payloads = torch.cat((current_payload[:, None], payload), dim=1)
    flat = payloads.reshape(n_tiles, payloads.shape[1], -1)
    unique = torch.ones(n_tiles, dtype=torch.int64, device=payloads.device)
    for k in range(1, flat.shape[1]):
        unique.add_(~torch.any(torch.all(flat[:, k:k + 1] == flat[:, :k], dim=-1), dim=1))
    return candidates, payloads, int(unique.sum().item())


def _add_rank16(hessian_error: torch.Tensor, hessian: torch.Tensor, rows: slice, delta: torch.Tensor) -> None:
    """``H E += H[:, rows] delta``: on the FP32 matrix cores for device FP32."""

    if hessian_error.is_cuda and hessian_error.dtype == torch.float32:
        gemm.addmm_tn_(hessian_error, hessian[:, rows].T.contiguous(), delta.contiguous())
    else:
        hessian_error.addmm_(hessian[:, rows], delta)


@torch.no_grad()
def refine_h2_viterbi_paths(weight: torch.Tensor, hessian: torch.Tensor, initial_weight_q: torch.Tensor,
                            initial_encoded: torch.Tensor, quantize_tiles: QuantizeTiles,
                            config: H2ViterbiRefineConfig = H2ViterbiRefineConfig(), *,
                            column_weights: torch.Tensor | None = None,
                            guidance: GradientGuidance | None = None) -> H2ViterbiRefineResult:
    """Refine legal paths under dense H plus an optional linear objective
    (reference :334-560).  Sweeps alternate their row-block order; the
    objective may not rise beyond roundoff."""

    if weight.ndim != 2 or initial_weight_q.shape != weight.shape:
        raise ValueError("weight and reconstruction must have one rank-2 shape")
    rows, columns = weight.shape
    if rows % 16 or columns % 16:
        raise ValueError("weight dimensions must be multiples of 16")
    if hessian.shape != (rows, rows):
        raise ValueError("Hessian shape does not match the input dimension")
    if initial_encoded.ndim < 3 or initial_encoded.shape[:2] != (rows // 16, columns // 16):
        raise ValueError("stored trellis payload has the wrong tile grid")
    if config.sweeps <= 0:
        raise ValueError("sweeps must be positive")
    if guidance is not None:
        guidance.validate(weight.shape)
    device, dtype = weight.device, config.score_dtype
    h = hessian.to(device=device, dtype=dtype).contiguous()
    colw = _column_weights(column_weights, columns, device, dtype)
    w = weight.to(device)
    recon = initial_weight_q.to(device).clone()
    encoded = initial_encoded.to(device).clone()
    dense_gradient = None
    if guidance is not None and not isinstance(guidance, LowRankViterbiGradientGuidance):
        dense_gradient = guidance.gradient.to(device=device, dtype=dtype)
    anchor = None if guidance is None else guidance.anchor.to(device=device, dtype=dtype)
    strength = 0.0 if guidance is None else float(guidance.strength)
    error = (w - recon).to(dtype)
    herr = h @ error
    quadratic = float(torch.sum(error * herr * colw.unsqueeze(0)).item())
    linear = _linear_term(guidance, recon, dense_gradient, anchor, dtype)
    objective = quadratic + linear
    stats: list[H2ViterbiSweepStats] = []
    row_blocks, col_blocks = rows // 16, columns // 16
    permutation = tensor_core_permutation(device)
    inverse = torch.argsort(permutation)

    for sweep in range(config.sweeps):
        before, q_before, l_before = objective, quadratic, linear
        accepted = unique_paths = 0
        reverse = not config.alternate_sweep_order or sweep % 2 == 0
        order: Iterable[int] = range(row_blocks - 1, -1, -1) if reverse else range(row_blocks)
        for rb in order:
            sl = slice(rb * 16, rb * 16 + 16)
            h_bb = h[sl, sl]
            gradient_block = None
            if guidance is not None:
                gradient_block = (guidance.rows(sl, device=device, dtype=dtype)
                                  if isinstance(guidance, LowRankViterbiGradientGuidance) else dense_gradient[sl])
            target = _conditional_target(w[sl].to(dtype), error[sl], herr[sl], h_bb, gradient_block=gradient_block,
                                         gradient_strength=strength, column_weights=colw).to(w.dtype)
            target_tiles = target.reshape(16, col_blocks, 16).permute(1, 0, 2)
            current_tiles = recon[sl].reshape(16, col_blocks, 16).permute(1, 0, 2).contiguous()
            current_payload = encoded[rb]
            candidates, payloads, unique = _candidate_paths(target_tiles.contiguous(), current_tiles, current_payload,
                                                            h_bb, permutation, inverse, quantize_tiles, config,
                                                            sweep=sweep, row_block=rb)
            unique_paths += unique
            scores = _conditional_scores(target_tiles, candidates, h_bb, colw.reshape(col_blocks, 16), dtype)
            current = scores[:, 0]
            best, best_index = torch.min(scores, dim=1)
            accept = best + (config.acceptance_abs_tol + config.acceptance_rel_tol * current.abs()) < current
            accepted += int(torch.count_nonzero(accept))
            if not bool(torch.any(accept)):
                continue
            idx = torch.arange(col_blocks, device=device)
            chosen = torch.where(accept[:, None, None], candidates[idx, best_index], current_tiles)
            mask = accept.reshape(accept.shape[0], *([1] * (payloads.ndim - 2)))
            encoded[rb] = torch.where(mask, payloads[idx, best_index], current_payload)
            new_block = chosen.permute(1, 0, 2).reshape(16, columns)
            new_error = (w[sl] - new_block).to(dtype)
            delta = new_error - error[sl]
            recon[sl] = new_block
            error[sl] = new_error
            _add_rank16(herr, h, sl, delta)

        herr = h @ error
        quadratic = float(torch.sum(error * herr * colw.unsqueeze(0)).item())
        linear = _linear_term(guidance, recon, dense_gradient, anchor, dtype)
        objective = quadratic + linear
        if objective > before + max(1.0e-5, 1.0e-6 * abs(before)):
            raise RuntimeError("dense-H objective increased; quantizer coordinates are inconsistent")
        stats.append(H2ViterbiSweepStats(
            sweep=sweep, objective_before=before, objective_after=objective, quadratic_before=q_before,
            quadratic_after=quadratic, linear_before=l_before, linear_after=linear,
            relative_improvement=(before - objective) / max(abs(before), 1.0e-30), accepted_tiles=accepted,
            proposed_tiles=row_blocks * col_blocks, unique_candidate_paths=unique_paths))
        if config.stop_on_no_change and accepted == 0:
            break
    return H2ViterbiRefineResult(recon, encoded, stats)


def config_from_quant_args(quant_args: dict) -> H2ViterbiRefineConfig:
    """Refinement controls from ``quant_args["h2_viterbi_refine_*"]`` (reference :563-587)."""

    return H2ViterbiRefineConfig(
        sweeps=int(quant_args.get("h2_viterbi_refine_sweeps", 1)),
        alternate_sweep_order=bool(quant_args.get("h2_viterbi_refine_alternate_order", True)),
        dither_scales=tuple(float(v) for v in quant_args.get("h2_viterbi_refine_dither_scales", ())),
        num_dither_patterns=int(quant_args.get("h2_viterbi_refine_patterns", 0)),
        seed=int(quant_args.get("h2_viterbi_refine_seed", 0x48325643)),
        max_quantizer_batch=int(quant_args.get("h2_viterbi_refine_max_batch", 256)),
        score_dtype=torch.float64 if quant_args.get("h2_viterbi_refine_fp64_score", False) else torch.float32,
    )


__all__ = [
    "H2ViterbiRefineConfig",
    "H2ViterbiRefineResult",
    "H2ViterbiSweepStats",
    "config_from_quant_args",
    "dense_h_guided_objective",
    "dense_h_objective",
    "refine_h2_viterbi_paths",
]
