"""Dense-H block-coordinate refinement of legal trellis paths
(reference ``qsrt/h2_viterbi_refine.py:1-587``; driven by
``refine_uniform_h2_candidate``, ``qsrt/exl3_encoder_backend.py:840-895``).

BlockLDLQ commits each 16-row block once, seeing only the error of the
blocks below it.  Once every block's error ``E = W - Q`` is known, the
dense-H objective ``f(Q) = sum_c a_c e_c^T H e_c`` is, with every other
block held fixed, a quadratic in one block's rows alone:

    f = sum_c a_c (t_b - q_b')_c^T H_bb (t_b - q_b')_c + const,
    t_b = q_b + H_bb^-1 (H E)_b                      (conditional target)

(expand ``f`` around the current ``q_b``: the part linear in the change is
``-2 (H E)_b``).  A linear objective ``s <g, Q - anchor>`` moves the target
to ``t_b - s/2 H_bb^-1 g_b / a`` by completing the square.  A sweep visits
the row blocks in turn, asks the tile Viterbi for legal paths near ``t_b``
(the target itself and, optionally, H-whitened dithers of it), scores each
proposal and the current tile exactly under ``H_bb``, and keeps a proposal
only when it lowers the objective by more than the tolerance.  The
objective therefore never rises; each sweep checks that against a full
recomputation.

On the device everything is float64 and the Viterbi sees each target
rounded once to FP32 (the encoder's contract).  ``H E`` is one product on
the FP64 matrix cores per sweep (``qsrt_gemm_tn_f64``), kept current by a
rank-16 product for each block, whose non-accepted columns contribute
exactly zero; the targets are a 16 x 16 by 16 x N product on the same
kernel; the scores are a batched float64 product over (tile, candidate).
Acceptance, selection and the counters stay on the device, so a sweep runs
without a host synchronisation until its end.

The dither probes are drawn from a seeded CPU generator (the reference draws
them on the device, whose random stream is not reproducible elsewhere), and
the blocks' Cholesky factors and inverses are formed once, on the CPU, in
float64.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Callable

import torch

from . import gemm
from .exl3_reference import tensor_core_permutation
from .gradient_guided_viterbi import LowRankViterbiGradientGuidance, ViterbiGradientGuidance

QuantizeTiles = Callable[[torch.Tensor], tuple[torch.Tensor, torch.Tensor]]
GradientGuidance = ViterbiGradientGuidance | LowRankViterbiGradientGuidance

BLOCK = 16


@dataclass(frozen=True)
class H2ViterbiRefineConfig:
    """Search controls (reference :31-44, same fields and defaults).
    ``score_dtype`` is accepted for the reference's interface; this build
    scores in float64 whatever it names."""

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
    """Per-sweep receipt (reference :47-59)."""

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
    sweep_stats: list

    def stats_dict(self) -> dict:
        return {"sweeps": [asdict(s) for s in self.sweep_stats]}


def _column_weights(column_weights, columns: int, device) -> torch.Tensor:
    if column_weights is None:
        return torch.ones(columns, dtype=torch.float64, device=device)
    if column_weights.numel() != columns:
        raise ValueError("column weights do not match the output dimension")
    a = column_weights.reshape(-1).to(device=device, dtype=torch.float64)
    if bool(torch.any(a < 0)):
        raise ValueError("column weights must be nonnegative")
    return a


def _hessian_times_error(hessian64: torch.Tensor, weight64: torch.Tensor, weight_q: torch.Tensor) -> torch.Tensor:
    """``H (W - Q)`` with float64 ``H`` (symmetric) and ``W``, FP32 ``Q``."""

    he = torch.zeros(weight64.shape, dtype=torch.float64, device=weight64.device)
    return gemm.addmm_sub_tn_(he, hessian64, weight64, weight_q.float().contiguous())


def _quadratic(weight64: torch.Tensor, weight_q: torch.Tensor, he: torch.Tensor, a: torch.Tensor) -> torch.Tensor:
    """``sum_c a_c e_c^T (H E)_c`` as a device scalar."""

    return torch.sum((weight64 - weight_q.double()) * he * a.unsqueeze(0))


def _linear(guidance, weight_q: torch.Tensor) -> float:
    if guidance is None:
        return 0.0
    return float(guidance.linear_term(weight_q, dtype=torch.float64))


def dense_h_objective(weight: torch.Tensor, weight_q: torch.Tensor, hessian: torch.Tensor, *,
                      column_weights: torch.Tensor | None = None, chunk_columns: int = 512,
                      dtype: torch.dtype = torch.float64) -> float:
    """``sum_c a[c] (W - Q)[:, c]^T H (W - Q)[:, c]`` (reference :62-98),
    ``chunk_columns`` columns at a time."""

    if weight.shape != weight_q.shape or weight.ndim != 2:
        raise ValueError("weight and reconstruction must have one rank-2 shape")
    if hessian.shape != (weight.shape[0], weight.shape[0]):
        raise ValueError("Hessian shape does not match the input dimension")
    if chunk_columns <= 0:
        raise ValueError("chunk_columns must be positive")
    a = _column_weights(column_weights, weight.shape[1], weight.device).to(dtype)
    h = hessian.to(device=weight.device, dtype=dtype)
    total = torch.zeros((), dtype=dtype, device=weight.device)
    for c0 in range(0, weight.shape[1], chunk_columns):
        c1 = min(c0 + chunk_columns, weight.shape[1])
        e = (weight[:, c0:c1].to(dtype) - weight_q[:, c0:c1].to(dtype))
        total += torch.sum(e * (h @ e) * a[c0:c1].unsqueeze(0))
    return float(total)


def dense_h_guided_objective(weight: torch.Tensor, weight_q: torch.Tensor, hessian: torch.Tensor,
                             guidance: GradientGuidance, *, column_weights: torch.Tensor | None = None,
                             chunk_columns: int = 512, dtype: torch.dtype = torch.float64):
    """``(quadratic, linear, quadratic + linear)`` with the linear term
    ``strength <g, Q - anchor>`` (reference :101-139)."""

    guidance.validate(weight.shape)
    quadratic = dense_h_objective(weight, weight_q, hessian, column_weights=column_weights,
                                  chunk_columns=chunk_columns, dtype=dtype)
    linear = float(guidance.linear_term(weight_q, dtype=dtype))
    return quadratic, linear, quadratic + linear


class _BlockMetric:
    """Per 16-row block of ``H``: the diagonal block, its inverse (target
    solves) and its Cholesky factor (dither whitening), all float64, formed
    once on the CPU."""

    def __init__(self, hessian64: torch.Tensor):
        k = hessian64.shape[0]
        nb = k // BLOCK
        idx = torch.arange(nb, device=hessian64.device) * BLOCK
        rows = idx[:, None, None] + torch.arange(BLOCK, device=hessian64.device)[None, :, None]
        cols = idx[:, None, None] + torch.arange(BLOCK, device=hessian64.device)[None, None, :]
        diag = hessian64[rows, cols].cpu()
        chol, info = torch.linalg.cholesky_ex(diag)
        if bool(torch.any(info != 0)):
            bad = int(torch.nonzero(info)[0, 0])
            raise ValueError(f"diagonal block {bad} of the Hessian is not positive definite")
        inv = torch.cholesky_inverse(chol)
        inv = 0.5 * (inv + inv.transpose(-1, -2))  # exactly symmetric: the product kernel takes it transposed
        self.diag = diag.to(hessian64.device)
        self.inv = inv.to(hessian64.device).contiguous()
        self.chol = chol  # CPU

    def patterns(self, b: int, count: int, seed: int) -> torch.Tensor | None:
        """``count`` H_bb-whitened sign patterns ``L^-T p`` of energy
        ``p^T H_bb p = 256`` (reference :187-222)."""

        if count <= 0:
            return None
        g = torch.Generator().manual_seed(int(seed))
        probes = (torch.randint(0, 2, (count, BLOCK, BLOCK), generator=g, dtype=torch.int64) * 2 - 1).double()
        chol = self.chol[b]
        cols = probes.permute(1, 0, 2).reshape(BLOCK, count * BLOCK)
        x = torch.linalg.solve_triangular(chol.T, cols, upper=True).reshape(BLOCK, count, BLOCK).permute(1, 0, 2)
        hb = self.diag[b].cpu()
        energy = torch.sum(x * torch.matmul(hb, x), dim=(1, 2), keepdim=True).clamp_min(1e-20)
        return (x * torch.sqrt(float(BLOCK * BLOCK) / energy)).to(self.diag.device)


def _unique_paths(payloads: torch.Tensor) -> torch.Tensor:
    """Distinct payloads among each tile's candidates (device scalar)."""

    t, m = payloads.shape[:2]
    flat = payloads.reshape(t, m, -1)
    eq = (flat[:, :, None, :] == flat[:, None, :, :]).all(dim=-1)  # [t, m, m]
    earlier = torch.tril(torch.ones(m, m, dtype=torch.bool, device=payloads.device), diagonal=-1)
    duplicate = (eq & earlier).any(dim=-1)
    return (~duplicate).sum()


@torch.no_grad()
def refine_h2_viterbi_paths(weight: torch.Tensor, hessian: torch.Tensor, initial_weight_q: torch.Tensor,
                            initial_encoded: torch.Tensor, quantize_tiles: QuantizeTiles,
                            config: H2ViterbiRefineConfig = H2ViterbiRefineConfig(), *,
                            column_weights: torch.Tensor | None = None,
                            guidance: GradientGuidance | None = None) -> H2ViterbiRefineResult:
    """Refine the legal paths of ``initial_encoded`` under the dense-H
    objective plus an optional linear term (reference :330-563).

    ``weight`` (the regularised source), ``hessian`` and ``initial_weight_q``
    are in the encoder's regularised coordinates; ``initial_encoded`` holds
    the states ``[K/16, N/16, 256]`` in tensor-core order;
    ``quantize_tiles(tiles f32 [T, 256]) -> (recon [T, 256], payload [T, ...])``
    is the tile quantizer that made them.  Returns the refined FP32
    reconstruction and payload, and one receipt per sweep."""

    if weight.ndim != 2 or initial_weight_q.shape != weight.shape:
        raise ValueError("weight and reconstruction must have one rank-2 shape")
    rows, columns = weight.shape
    if rows % BLOCK or columns % BLOCK:
        raise ValueError("weight dimensions must be multiples of 16")
    if hessian.shape != (rows, rows):
        raise ValueError("Hessian shape does not match the input dimension")
    grid = (rows // BLOCK, columns // BLOCK)
    if initial_encoded.ndim < 3 or tuple(initial_encoded.shape[:2]) != grid:
        raise ValueError("stored trellis payload has the wrong tile grid")
    if config.sweeps <= 0:
        raise ValueError("sweeps must be positive")
    if config.max_quantizer_batch <= 0:
        raise ValueError("max_quantizer_batch must be positive")
    if guidance is not None:
        guidance.validate(weight.shape)

    device = weight.device
    rb_n, cb_n = grid
    h64 = hessian.to(device=device, dtype=torch.float64)
    h64 = (0.5 * (h64 + h64.T)).contiguous()  # the symmetric part (H itself when it is symmetric)
    w64 = weight.to(device=device, dtype=torch.float64).contiguous()
    q = initial_weight_q.to(device=device, dtype=torch.float32).contiguous().clone()
    encoded = initial_encoded.to(device).contiguous().clone()
    a = _column_weights(column_weights, columns, device)
    a_tiles = a.reshape(cb_n, BLOCK)
    guided = guidance is not None and float(guidance.strength) != 0.0
    if guided:
        if bool(torch.any(a <= 0)):
            raise ValueError("gradient-guided refinement requires positive column weights")
        dense_grad = (guidance.gradient.to(device=device, dtype=torch.float64)
                      if isinstance(guidance, ViterbiGradientGuidance) else None)
        strength = float(guidance.strength)
    metric = _BlockMetric(h64)
    perm = tensor_core_permutation(device).long()
    perm_i = torch.argsort(perm)

    he = _hessian_times_error(h64, w64, q)
    quadratic = float(_quadratic(w64, q, he, a))
    linear = _linear(guidance, q)
    objective = quadratic + linear
    stats = []
    for sweep in range(config.sweeps):
        before, quadratic_before, linear_before = objective, quadratic, linear
        accepted = torch.zeros((), dtype=torch.int64, device=device)
        unique = torch.zeros((), dtype=torch.int64, device=device)
        backward = not config.alternate_sweep_order or sweep % 2 == 0
        order = range(rb_n - 1, -1, -1) if backward else range(rb_n)
        for b in order:
            r0, r1 = b * BLOCK, (b + 1) * BLOCK
            # conditional target t = q_b + H_bb^-1 (H E)_b  [- s/2 H_bb^-1 g_b / a]
            target = q[r0:r1].double()
            gemm.addmm_sub_tn_(target, metric.inv[b], he[r0:r1].contiguous())
            if guided:
                g_b = dense_grad[r0:r1] if dense_grad is not None else guidance.rows(
                    slice(r0, r1), device=device, dtype=torch.float64)
                gemm.addmm_sub_tn_(target, metric.inv[b], (g_b / a.unsqueeze(0)).contiguous(), alpha=-0.5 * strength)
            t_tiles = target.reshape(BLOCK, cb_n, BLOCK).permute(1, 0, 2)  # [tile, row, col] float64
            variants = [t_tiles]
            pats = metric.patterns(b, config.num_dither_patterns, config.seed + 1009 * sweep + 9176 * b)
            if pats is not None and config.dither_scales:
                rms = t_tiles.square().mean(dim=(1, 2), keepdim=True).sqrt().clamp_min(1e-8)
                for scale in config.dither_scales:
                    for p in pats:
                        shift = float(scale) * rms * p.unsqueeze(0)
                        variants.extend((t_tiles + shift, t_tiles - shift))
            stacked = torch.stack(variants)  # [v, tile, 16, 16]
            v_n = stacked.shape[0]
            inputs = stacked.reshape(v_n * cb_n, 256).float()[:, perm].contiguous()  # rounded once
            recons, pays = [], []
            for c0 in range(0, inputs.shape[0], config.max_quantizer_batch):
                chunk = inputs[c0:c0 + config.max_quantizer_batch].contiguous()
                rc, py = quantize_tiles(chunk)
                if rc.shape != chunk.shape:
                    raise ValueError("tile quantizer returned the wrong reconstruction shape")
                if py.ndim < 1 or py.shape[0] != chunk.shape[0]:
                    raise ValueError("tile quantizer returned the wrong payload batch")
                recons.append(rc)
                pays.append(py)
            recon = torch.cat(recons)[:, perm_i].reshape(v_n, cb_n, BLOCK, BLOCK).transpose(0, 1)
            payload = torch.cat(pays)
            payload = payload.reshape(v_n, cb_n, *payload.shape[1:]).transpose(0, 1)
            current_payload = encoded[b]
            if tuple(current_payload.shape[1:]) != tuple(payload.shape[2:]):
                raise ValueError("stored and proposed trellis payload shapes differ")
            current = q[r0:r1].reshape(BLOCK, cb_n, BLOCK).permute(1, 0, 2)
            cands = torch.cat((current.unsqueeze(1), recon.float()), dim=1)  # [tile, 1 + v, 16, 16]
            pays_all = torch.cat((current_payload.unsqueeze(1), payload.to(current_payload.dtype)), dim=1)
            unique += _unique_paths(pays_all)
            # exact conditional scores under H_bb, column-weighted
            d = t_tiles.unsqueeze(1) - cands.double()
            hd = torch.matmul(metric.diag[b], d)
            scores = torch.sum(d * hd * a_tiles[:, None, None, :], dim=(2, 3))  # [tile, 1 + v]
            cur = scores[:, 0]
            best_score, best = torch.min(scores, dim=1)
            # lowest index among exact ties (torch.min does not promise which)
            best = torch.where(scores == best_score.unsqueeze(1),
                               torch.arange(scores.shape[1], device=device).unsqueeze(0),
                               scores.shape[1]).min(dim=1).values
            accept = best_score + (config.acceptance_abs_tol + config.acceptance_rel_tol * cur.abs()) < cur
            choice = torch.where(accept, best, torch.zeros_like(best))
            accepted += accept.sum()
            tiles_ix = torch.arange(cb_n, device=device)
            new_block = cands[tiles_ix, choice].permute(1, 0, 2).reshape(BLOCK, columns)
            encoded[b] = pays_all[tiles_ix, choice]
            # H E += H[:, b] (Q_old - Q_new)_b; unchanged columns add exact zeros
            old_block = q[r0:r1].double()
            q[r0:r1] = new_block
            gemm.addmm_sub_tn_(he, h64[r0:r1], old_block.contiguous(), q[r0:r1].contiguous())
        he = _hessian_times_error(h64, w64, q)
        quadratic = float(_quadratic(w64, q, he, a))
        linear = _linear(guidance, q)
        objective = quadratic + linear
        if objective > before + max(1.0e-5, 1.0e-6 * abs(before)):
            raise RuntimeError("dense-H objective increased; quantizer coordinates are inconsistent")
        n_accepted = int(accepted)
        stats.append(H2ViterbiSweepStats(
            sweep=sweep, objective_before=before, objective_after=objective, quadratic_before=quadratic_before,
            quadratic_after=quadratic, linear_before=linear_before, linear_after=linear,
            relative_improvement=(before - objective) / max(abs(before), 1.0e-30), accepted_tiles=n_accepted,
            proposed_tiles=rb_n * cb_n, unique_candidate_paths=int(unique)))
        if config.stop_on_no_change and n_accepted == 0:
            break
    return H2ViterbiRefineResult(q, encoded, stats)


def config_from_quant_args(quant_args: dict) -> H2ViterbiRefineConfig:
    """The refinement controls from the encoder's private keys
    (reference :566-587)."""

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
