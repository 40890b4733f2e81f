"""Pooled sufficient statistics for routed expert calibration (reference
``qsrt/pooled_calibration.py:25-927``).

A decoded gate/up candidate of an expert changes the expert's post-activation
rows from the source's ``S`` to the candidate's ``C``.  Everything the
calibration needs from the routed rows -- the candidate-local H2, the exact
routed-output SSE of any down projection, the ridge refit of the down
projection -- is a quadratic form in those rows, so it is kept as weighted
cross-products instead of the rows themselves.  Route weights enter squared,
once, as in the routed output's squared error.

Design on the matrix cores: each row chunk's candidate rows and residual rows
``R = C - S`` are stacked side by side, ``X = [C | R]`` (rows x 2w), and one
weighted Gram ``X^T diag(w) X`` is accumulated per chunk
(``qsrt_amd.gemm``: the FP32 matrix-core product, or the float64 one for
float64 statistics).  Its blocks are the five statistics the reference keeps
as separate accumulators:

* ``C^T W C`` -- ``candidate_gram`` (top-left block);
* ``C^T W R`` -- ``candidate_residual_cross`` (top-right block);
* ``R^T W R`` -- ``hidden_residual_gram`` (bottom-right block);
* ``C^T W S = C^T W C - C^T W R`` -- ``candidate_source_cross``;
* ``S^T W S = C^T W C - C^T W R - R^T W C + R^T W R`` -- ``source_gram``.

The residual blocks come from ``R`` itself, so they carry relative precision
at the error scale even when the candidate is close to the source; one pass
over the rows replaces five products.  Forward passes through the expert are
plain library GEMMs (torch); the scoring reference is the ordinary-coordinate
expert, as in the reference.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Iterable, Iterator, Mapping

import torch
import torch.nn.functional as F

from . import gemm
from .qsrt_coupled import CoupledHadamardExecution, encode_coupled_weights, situ, situ_derivatives


@dataclass(frozen=True)
class CoupledTriplet:
    """One gated expert in the framework's ``[out, in]`` orientation
    (reference ``qsrt/coupled_expert_study.py:26-62``): gate and up
    ``[intermediate, hidden]``, down ``[hidden, intermediate]``."""

    gate: torch.Tensor
    up: torch.Tensor
    down: torch.Tensor

    def __post_init__(self) -> None:
        if any(t.ndim != 2 for t in self.tensors()):
            raise ValueError("coupled expert weights must be rank-two tensors")
        if self.gate.shape != self.up.shape:
            raise ValueError("gate and up projections must have identical shapes")
        if tuple(self.down.shape) != (self.hidden, self.intermediate):
            raise ValueError("down must have shape [hidden, intermediate]")
        if not all(torch.is_floating_point(t) for t in self.tensors()):
            raise TypeError("coupled expert weights must be floating point")

    @property
    def intermediate(self) -> int:
        return int(self.gate.shape[0])

    @property
    def hidden(self) -> int:
        return int(self.gate.shape[1])

    def tensors(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        return self.gate, self.up, self.down

    def to(self, *args, **kwargs) -> "CoupledTriplet":
        return CoupledTriplet(*(t.to(*args, **kwargs) for t in self.tensors()))


def _check_dtype(dtype: torch.dtype) -> None:
    if dtype not in (torch.float32, torch.float64):
        raise TypeError("sufficient statistics require FP32 or FP64")


def _weighted_gram_(acc: torch.Tensor, rows: torch.Tensor, weights: torch.Tensor) -> None:
    """``acc += rows^T diag(weights) rows`` on the matrix cores (float32 or
    float64 by ``acc``'s dtype; torch on CPU tensors)."""

    rows = rows.to(dtype=acc.dtype).contiguous()
    gemm.addmm_sub_tn_(acc, rows, (rows * weights.to(acc.dtype)[:, None]).contiguous())


@dataclass
class CandidateHiddenStatistics:
    """Weighted source/candidate post-activation cross-products, held as the
    stacked Gram ``[C | C - S]^T W [C | C - S]`` (``stacked``, 2w x 2w)
    plus the weight support.  The reference's five statistics are views or
    sums of its blocks; with ``retain_source_gram`` False the two that need
    the source side as a whole (``source_gram``, ``hidden_residual_gram``)
    report None, as the reference's do."""

    stacked: torch.Tensor
    weight_sum: float
    weight_square_sum: float
    rows: int
    retain_source_gram: bool = True

    @classmethod
    def zeros(cls, width: int, *, device="cpu", dtype: torch.dtype = torch.float64,
              retain_source_gram: bool = True) -> "CandidateHiddenStatistics":
        if width <= 0:
            raise ValueError("hidden width must be positive")
        _check_dtype(dtype)
        return cls(torch.zeros((2 * width, 2 * width), device=device, dtype=dtype), 0.0, 0.0, 0,
                   bool(retain_source_gram))

    @property
    def width(self) -> int:
        return int(self.stacked.shape[0]) // 2

    @property
    def effective_sample_size(self) -> float:
        if self.weight_sum <= 0 or self.weight_square_sum <= 0:
            return 0.0
        return self.weight_sum ** 2 / self.weight_square_sum

    # ---- the reference's statistics, from the blocks of the stacked Gram
    @property
    def candidate_gram(self) -> torch.Tensor:
        w = self.width
        return self.stacked[:w, :w]

    @property
    def candidate_residual_cross(self) -> torch.Tensor:
        w = self.width
        return self.stacked[:w, w:]

    @property
    def candidate_source_cross(self) -> torch.Tensor:
        return self.candidate_gram - self.candidate_residual_cross

    @property
    def hidden_residual_gram(self) -> torch.Tensor | None:
        if not self.retain_source_gram:
            return None
        w = self.width
        return self.stacked[w:, w:]

    @property
    def source_gram(self) -> torch.Tensor | None:
        if not self.retain_source_gram:
            return None
        w = self.width
        g = self.stacked
        return g[:w, :w] - g[:w, w:] - g[w:, :w] + g[w:, w:]

    def _validate(self) -> None:
        g = self.stacked
        if g.ndim != 2 or g.shape[0] != g.shape[1] or g.shape[0] % 2 or g.shape[0] == 0:
            raise ValueError("candidate statistics must be one even-size square")
        if not bool(torch.all(torch.isfinite(g))):
            raise ValueError("candidate statistics must be finite")
        if (not math.isfinite(self.weight_sum) or not math.isfinite(self.weight_square_sum) or self.weight_sum < 0
                or self.weight_square_sum < 0 or self.rows < 0):
            raise ValueError("candidate statistics have invalid support")

    def update(self, candidate_hidden: torch.Tensor, source_hidden: torch.Tensor,
               route_weights: torch.Tensor) -> None:
        """Accumulate one row chunk, weighting each row by its route weight
        squared."""

        self._validate()
        if (candidate_hidden.ndim != 2 or source_hidden.shape != candidate_hidden.shape
                or candidate_hidden.shape[1] != self.width):
            raise ValueError("source and candidate hidden rows do not align")
        if route_weights.ndim != 1 or route_weights.numel() != candidate_hidden.shape[0]:
            raise ValueError("route weights must contain one value per hidden row")
        if not all(bool(torch.all(torch.isfinite(t))) for t in (candidate_hidden, source_hidden, route_weights)):
            raise ValueError("candidate rows and route weights must be finite")
        dtype, device = self.stacked.dtype, self.stacked.device
        candidate = candidate_hidden.to(device=device, dtype=dtype)
        source = source_hidden.to(device=device, dtype=dtype)
        weights = route_weights.to(device=device, dtype=dtype).square()
        _weighted_gram_(self.stacked, torch.cat((candidate, candidate - source), dim=1), weights)
        w64 = weights.double()
        self.weight_sum += float(w64.sum())
        self.weight_square_sum += float(w64.square().sum())
        self.rows += int(candidate.shape[0])

    def merge_(self, other: "CandidateHiddenStatistics") -> None:
        """Merge the statistics of a disjoint row partition."""

        self._validate()
        other._validate()
        if other.width != self.width:
            raise ValueError("candidate statistics widths differ")
        if other.retain_source_gram != self.retain_source_gram:
            raise ValueError("candidate statistics disagree on source-Gram retention")
        self.stacked.add_(other.stacked.to(self.stacked))
        self.weight_sum += other.weight_sum
        self.weight_square_sum += other.weight_square_sum
        self.rows += other.rows

    def to(self, *, device, dtype: torch.dtype | None = None) -> "CandidateHiddenStatistics":
        """A copy on ``device`` (and ``dtype``), with the same support."""

        target = self.stacked.dtype if dtype is None else dtype
        _check_dtype(target)
        return CandidateHiddenStatistics(self.stacked.to(device=device, dtype=target, copy=True), self.weight_sum,
                                         self.weight_square_sum, self.rows, self.retain_source_gram)


@dataclass(frozen=True)
class PooledExpertEvaluation:
    """Exact routed-function score and down-projection statistics of one
    candidate."""

    statistics: CandidateHiddenStatistics
    sse: float
    source_energy: float
    routed_occurrences: int
    prefix_scores: Mapping[int, tuple[float, float, int]]

    @property
    def nmse(self) -> float:
        if self.source_energy <= 0:
            raise ValueError("pooled expert evaluation has no source energy")
        return self.sse / self.source_energy


@dataclass(frozen=True)
class PooledPortfolioEvaluation:
    """Exact routed-function scores of candidates sharing one source expert."""

    candidate_sse: Mapping[str, float]
    source_energy: float
    routed_occurrences: int

    def __post_init__(self) -> None:
        if (not self.candidate_sse or any(not math.isfinite(v) or v < 0 for v in self.candidate_sse.values())
                or not math.isfinite(self.source_energy) or self.source_energy <= 0 or self.routed_occurrences <= 0):
            raise ValueError("pooled portfolio evaluation is invalid")


@dataclass
class UpstreamFunctionalStatistics:
    """Per-neuron post-activation energy and 2 x 2 gate/up sensitivity
    metric over routed rows."""

    hidden_energy: torch.Tensor
    derivative_metric: torch.Tensor
    weight_sum: float
    weight_square_sum: float
    rows: int

    @property
    def effective_sample_size(self) -> float:
        if self.weight_sum <= 0 or self.weight_square_sum <= 0:
            return 0.0
        return self.weight_sum ** 2 / self.weight_square_sum


def _routed_batches(batches: Iterable[Mapping[str, torch.Tensor]], hidden: int, device,
                    what: str) -> Iterator[tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
    """Validated ``(input rows f32, route weights f32, global row indices)``
    of each non-empty batch, on ``device``.  Batches hold ``input``,
    ``route_weight`` and ``row_index``; row indices are int64 and strictly
    increasing across all batches."""

    previous = -1
    for batch in batches:
        if not {"input", "route_weight", "row_index"}.issubset(batch):
            raise ValueError(f"{what} batch lacks input, route weight, or row index")
        rows, weights, index = batch["input"], batch["route_weight"], batch["row_index"]
        if (rows.ndim != 2 or rows.shape[1] != hidden or weights.ndim != 1 or index.ndim != 1
                or weights.numel() != rows.shape[0] or index.numel() != rows.shape[0]):
            raise ValueError(f"{what} batch tensors do not align")
        if rows.shape[0] == 0:
            continue
        if index.dtype != torch.int64:
            raise TypeError("global row indices must be int64")
        if int(index[0]) <= previous or bool(torch.any(index[1:] <= index[:-1])):
            raise ValueError(f"{what} rows must be globally increasing")
        previous = int(index[-1])
        yield (rows.to(device=device, dtype=torch.float32), weights.to(device=device, dtype=torch.float32), index)


def collect_upstream_functional_statistics(batches: Iterable[Mapping[str, torch.Tensor]], *, source: CoupledTriplet,
                                           device) -> UpstreamFunctionalStatistics:
    """Per neuron n: post-activation energy ``sum_r w_r h_rn^2`` and the PSD
    metric ``e_n sum_r w_r d_rn d_rn^T`` with ``d = (dh/dgate, dh/dup)`` and
    ``e_n`` the squared norm of the down projection's column n, ``w`` the
    squared route weights (reference :363-430): the first-order routed-output
    sensitivity to a per-neuron change of the gate and up pre-activations."""

    target = torch.device(device)
    source = source.to(device=target, dtype=torch.float32)
    n = source.intermediate
    energy = torch.zeros(n, device=target, dtype=torch.float64)
    metric = torch.zeros(n, 2, 2, device=target, dtype=torch.float64)
    down_energy = source.down.double().square().sum(dim=0)
    w_sum = w_sq = 0.0
    rows = 0
    for x, route, _ in _routed_batches(batches, source.hidden, target, "functional-statistics"):
        w = route.double().square()
        gate, up = F.linear(x, source.gate), F.linear(x, source.up)
        hidden = situ(gate, up).double()
        d_gate, d_up = (d.double() for d in situ_derivatives(gate, up))
        energy += (hidden.square() * w[:, None]).sum(dim=0)
        wg, wu = d_gate * w[:, None], d_up * w[:, None]
        m11, m13, m33 = (wg * d_gate).sum(dim=0), (wg * d_up).sum(dim=0), (wu * d_up).sum(dim=0)
        metric += torch.stack((torch.stack((m11, m13), dim=1), torch.stack((m13, m33), dim=1)), dim=1) \
            * down_energy[:, None, None]
        w_sum += float(w.sum())
        w_sq += float(w.square().sum())
        rows += int(x.shape[0])
    if rows == 0 or w_sum <= 0:
        raise ValueError("functional statistics require routed support")
    return UpstreamFunctionalStatistics(energy, metric, w_sum, w_sq, rows)


def blockwise_upstream_conditioning_coefficients(derivative_metric: torch.Tensor, *, block_size: int):
    """Conditional gate/up target coefficients from per-neuron 2 x 2 PSD
    metrics (reference :295-360): the metrics are summed over contiguous
    blocks of ``block_size`` neurons, and each block's ``m13 / m11`` (gate
    from up) and ``m13 / m33`` (up from gate) is repeated over its neurons;
    a diagonal below ``1e-12`` of the largest block diagonal is floored.
    Returns ``(gate_from_up, up_from_gate, evidence)``."""

    if (derivative_metric.ndim != 3 or tuple(derivative_metric.shape[1:]) != (2, 2)
            or not torch.is_floating_point(derivative_metric)):
        raise ValueError("derivative metric must have shape [neurons, 2, 2]")
    neurons = int(derivative_metric.shape[0])
    if block_size <= 0 or neurons % block_size:
        raise ValueError("block size must divide the intermediate width")
    if not bool(torch.all(torch.isfinite(derivative_metric))):
        raise ValueError("derivative metric must be finite")
    m = derivative_metric.double()
    m = (m + m.transpose(1, 2)) * 0.5
    tol = 256 * torch.finfo(torch.float64).eps * max(float(m.abs().max()), 1.0)
    # a symmetric 2 x 2 matrix is PSD iff its smaller eigenvalue is; closed form instead of a batched eigensolver
    a, b, c = m[:, 0, 0], m[:, 0, 1], m[:, 1, 1]
    smallest = 0.5 * (a + c) - torch.sqrt((0.5 * (a - c)).square() + b.square())
    if float(smallest.min()) < -tol:
        raise ValueError("derivative metric must be positive semidefinite")
    blocks = m.reshape(neurons // block_size, block_size, 2, 2).sum(dim=1)
    floor = max(float(blocks.diagonal(dim1=1, dim2=2).max().clamp_min(0)) * 1e-12, torch.finfo(torch.float64).tiny)
    gate_from_up_blocks = blocks[:, 0, 1] / blocks[:, 0, 0].clamp_min(floor)
    up_from_gate_blocks = blocks[:, 0, 1] / blocks[:, 1, 1].clamp_min(floor)
    q = torch.tensor((0.05, 0.5, 0.95), dtype=torch.float64, device=m.device)

    def summary(prefix: str, v: torch.Tensor) -> dict:
        p = torch.quantile(v, q)
        return {f"{prefix}_minimum": float(v.min()), f"{prefix}_p05": float(p[0]), f"{prefix}_median": float(p[1]),
                f"{prefix}_p95": float(p[2]), f"{prefix}_maximum": float(v.max())}

    return (gate_from_up_blocks.repeat_interleave(block_size), up_from_gate_blocks.repeat_interleave(block_size),
            {"block_size": float(block_size), "blocks": float(blocks.shape[0]), "diagonal_floor": floor,
             **summary("gate_from_up", gate_from_up_blocks), **summary("up_from_gate", up_from_gate_blocks)})


def _single_device(triplet: CoupledTriplet, what: str) -> torch.device:
    devices = {t.device for t in triplet.tensors()}
    if len(devices) != 1:
        raise ValueError(f"{what} tensors must share one device")
    return devices.pop()


def _check_geometry(source: CoupledTriplet, candidate: CoupledTriplet, execution: CoupledHadamardExecution) -> None:
    if source.hidden != candidate.hidden or source.intermediate != candidate.intermediate:
        raise ValueError("source and candidate expert geometry differ")
    if execution.hidden != source.hidden or execution.intermediate != source.intermediate:
        raise ValueError("coupled execution geometry differs from the expert")


def collect_coupled_hidden_statistics(batches: Iterable[Mapping[str, torch.Tensor]], *, source: CoupledTriplet,
                                      candidate_coordinates: CoupledTriplet, execution: CoupledHadamardExecution,
                                      statistics_dtype: torch.dtype = torch.float32,
                                      retain_source_gram: bool = False) -> CandidateHiddenStatistics:
    """Post-activation statistics of a decoded gate/up candidate (in the
    coupled basis) against the source, over routed row batches, without
    evaluating the down projection (reference :433-515).  One decoded
    candidate then gives its local H2, the refit target of the down
    projection and the exact score of any down candidate."""

    _check_geometry(source, candidate_coordinates, execution)
    _check_dtype(statistics_dtype)
    device = _single_device(candidate_coordinates, "candidate coordinate")
    source = source.to(device=device, dtype=torch.float32)
    cand = candidate_coordinates.to(device=device, dtype=torch.float32)
    src = CoupledTriplet(*encode_coupled_weights(source.tensors(), execution.spec))
    stats = CandidateHiddenStatistics.zeros(source.intermediate, device=device, dtype=statistics_dtype,
                                            retain_source_gram=retain_source_gram)
    for x, route, _ in _routed_batches(batches, source.hidden, device, "pooled expert"):
        xt = execution.transform_inputs(x)
        stats.update(execution.decode_middle(xt, cand.gate, cand.up), execution.decode_middle(xt, src.gate, src.up),
                     route)
    if stats.rows == 0:
        raise ValueError("pooled hidden statistics require routed support")
    return stats


def evaluate_coupled_expert_batches(batches: Iterable[Mapping[str, torch.Tensor]], *, source: CoupledTriplet,
                                    teacher_source: CoupledTriplet | None = None,
                                    candidate_coordinates: CoupledTriplet, execution: CoupledHadamardExecution,
                                    prefix_row_limits: Iterable[int] = (),
                                    statistics_dtype: torch.dtype = torch.float32,
                                    retain_source_gram: bool = False) -> PooledExpertEvaluation:
    """Score a whole candidate (coupled-basis gate, up and down) over routed
    row batches (reference :518-658): the routed-output SSE against the
    ordinary-coordinate teacher (``teacher_source``, default ``source``),
    the source energy, per-prefix scores for the global row limits in
    ``prefix_row_limits``, and the candidate's post-activation statistics."""

    _check_geometry(source, candidate_coordinates, execution)
    reference = source if teacher_source is None else teacher_source
    if reference.hidden != source.hidden or reference.intermediate != source.intermediate:
        raise ValueError("teacher and coordinate-source expert geometry differ")
    _check_dtype(statistics_dtype)
    limits = tuple(sorted({int(v) for v in prefix_row_limits}))
    if any(v <= 0 for v in limits):
        raise ValueError("prefix row limits must be positive")
    device = _single_device(candidate_coordinates, "candidate coordinate")
    source = source.to(device=device, dtype=torch.float32)
    reference = reference.to(device=device, dtype=torch.float32)
    cand = candidate_coordinates.to(device=device, dtype=torch.float32)
    src = CoupledTriplet(*encode_coupled_weights(source.tensors(), execution.spec))
    stats = CandidateHiddenStatistics.zeros(source.intermediate, device=device, dtype=statistics_dtype,
                                            retain_source_gram=retain_source_gram)
    sse = energy = 0.0
    count = 0
    prefix = {limit: [0.0, 0.0, 0] for limit in limits}
    for x, route, index in _routed_batches(batches, source.hidden, device, "pooled expert"):
        xt = execution.transform_inputs(x)
        src_hidden = execution.decode_middle(xt, src.gate, src.up)
        cand_hidden = execution.decode_middle(xt, cand.gate, cand.up)
        # the teacher output is the ordinary-coordinate expert's, so the change of basis's rounding never
        # redefines it; the transformed source rows only feed the statistics
        teacher = F.linear(situ(F.linear(x, reference.gate), F.linear(x, reference.up)), reference.down)
        output = execution.decode_output(cand_hidden @ cand.down.T)
        stats.update(cand_hidden, src_hidden, route)
        row_sse = ((output - teacher) * route[:, None]).square().sum(dim=1, dtype=torch.float64).cpu()
        row_energy = (teacher * route[:, None]).square().sum(dim=1, dtype=torch.float64).cpu()
        sse += float(row_sse.sum())
        energy += float(row_energy.sum())
        count += int(x.shape[0])
        cpu_index = index.cpu()
        for limit, acc in prefix.items():
            k = int(torch.searchsorted(cpu_index, limit, right=False))
            if k:
                acc[0] += float(row_sse[:k].sum())
                acc[1] += float(row_energy[:k].sum())
                acc[2] += k
    if count == 0 or energy <= 0:
        raise ValueError("pooled expert evaluation requires routed support")
    return PooledExpertEvaluation(stats, sse, energy, count,
                                  {limit: (float(a[0]), float(a[1]), int(a[2])) for limit, a in prefix.items()})


def evaluate_coupled_candidate_portfolio_batches(batches: Iterable[Mapping[str, torch.Tensor]], *,
                                                 source: CoupledTriplet,
                                                 candidate_coordinates: Mapping[str, CoupledTriplet],
                                                 executions: Mapping[str, CoupledHadamardExecution]
                                                 ) -> PooledPortfolioEvaluation:
    """Score several coupled candidates of one source expert with one shared
    source forward per batch (reference :661-771).  Candidates may use their
    own intermediate transform draws but must share the residual-side one,
    so the transformed inputs and the output inverse are shared."""

    names = tuple(candidate_coordinates)
    if not names or set(executions) != set(names):
        raise ValueError("candidate coordinates and executions must share identities")
    devices = {t.device for c in candidate_coordinates.values() for t in c.tensors()}
    if len(devices) != 1:
        raise ValueError("pooled portfolio candidates must share one device")
    device = devices.pop()
    source = source.to(device=device, dtype=torch.float32)
    cands = {name: c.to(device=device, dtype=torch.float32) for name, c in candidate_coordinates.items()}
    first = executions[names[0]]
    residual = (first.spec.residual_block_size, first.spec.residual_draw)
    for name in names:
        c, ex = cands[name], executions[name]
        if (c.hidden != source.hidden or c.intermediate != source.intermediate or ex.hidden != source.hidden
                or ex.intermediate != source.intermediate
                or (ex.spec.residual_block_size, ex.spec.residual_draw) != residual):
            raise ValueError("pooled portfolio candidates do not share residual geometry")
    sse = {name: 0.0 for name in names}
    energy = 0.0
    count = 0
    for x, route, _ in _routed_batches(batches, source.hidden, device, "pooled portfolio"):
        teacher = F.linear(situ(F.linear(x, source.gate), F.linear(x, source.up)), source.down)
        energy += float((teacher * route[:, None]).square().sum(dtype=torch.float64).cpu())
        xt = first.transform_inputs(x)
        for name in names:
            c, ex = cands[name], executions[name]
            output = ex.decode_output(ex.decode_middle(xt, c.gate, c.up) @ c.down.T)
            sse[name] += float(((output - teacher) * route[:, None]).square().sum(dtype=torch.float64).cpu())
        count += int(x.shape[0])
    return PooledPortfolioEvaluation(sse, energy, count)


def _down_operands(statistics: CandidateHiddenStatistics, *downs: torch.Tensor):
    statistics._validate()
    first = downs[0]
    if first.ndim != 2 or first.shape[0] != statistics.width:
        raise ValueError("down projections must be [intermediate, output] matching the statistics width")
    if any(d.shape != first.shape for d in downs):
        raise ValueError("down projections do not share the expected shape")
    return [d.to(device=statistics.stacked.device, dtype=statistics.stacked.dtype) for d in downs]


def decoded_down_sse(statistics: CandidateHiddenStatistics, candidate_down_t: torch.Tensor,
                     source_down_t: torch.Tensor) -> torch.Tensor:
    """Routed-output SSE of a down projection on the statistics' rows
    (reference :774-827), ``[intermediate, output]`` orientation.  With
    ``D = candidate - source`` the output error of a row is ``c D + r
    source`` (``c`` its candidate row, ``r`` its residual row), so the SSE is
    ``<D, G_cc D> + 2 <D, G_cr source> + <source, G_rr source>``: every term is
    at the error scale, none the difference of two output energies."""

    if statistics.hidden_residual_gram is None:
        raise ValueError("decoded down SSE requires retained source Gram statistics")
    cand, src = _down_operands(statistics, candidate_down_t, source_down_t)
    delta = cand - src
    quadratic = torch.sum(delta * (statistics.candidate_gram @ delta))
    cross = torch.sum(delta * (statistics.candidate_residual_cross @ src))
    residual = torch.sum(src * (statistics.hidden_residual_gram @ src))
    value = quadratic + 2.0 * cross + residual
    tol = 64 * torch.finfo(value.dtype).eps * max(float(quadratic.abs()), float((2.0 * cross).abs()),
                                                  float(residual.abs()), 1.0)
    if float(value) < -tol:
        raise ArithmeticError(f"pooled SSE is negative beyond roundoff: {float(value):.9g}")
    return value.clamp_min(0)


def decoded_down_sse_difference(statistics: CandidateHiddenStatistics, candidate_down_t: torch.Tensor,
                                baseline_down_t: torch.Tensor, source_down_t: torch.Tensor) -> torch.Tensor:
    """``SSE(candidate) - SSE(baseline)`` without the source-side Grams
    (reference :830-861): with ``D = candidate - baseline``, ``2 <D, g> + <D,
    G_cc D>`` where ``g = G_cc (baseline - source) + G_cr source`` is half the
    SSE's gradient at the baseline."""

    cand, base, src = _down_operands(statistics, candidate_down_t, baseline_down_t, source_down_t)
    delta = cand - base
    gradient = statistics.candidate_gram @ (base - src) + statistics.candidate_residual_cross @ src
    return 2.0 * torch.sum(delta * gradient) + torch.sum(delta * (statistics.candidate_gram @ delta))


def candidate_h2(statistics: CandidateHiddenStatistics, *, max_local_alpha: float = 0.75):
    """Candidate-local H2: the weighted covariance ``S = G_cc / sum w``
    shrunk toward ``tr(S)/p I`` (reference :864-924), with local weight
    ``min(max_local_alpha, 1 - rho)`` and ``rho`` the Oracle Approximating
    Shrinkage intensity in Chen, Wiesel, Eldar and Hero's original form
    (IEEE TSP 58(10), 2010, eq. 23), ``rho = ((1 - 2/p) tr(S^2) + tr(S)^2) /
    ((n + 1 - 2/p) (tr(S^2) - tr(S)^2 / p))`` clipped to [0, 1], ``n`` the
    Kish effective sample size.  No pooled post-activation covariance enters:
    intermediate coordinates are expert-local."""

    statistics._validate()
    cap = float(max_local_alpha)
    if not math.isfinite(cap) or not 0 <= cap <= 1:
        raise ValueError("max_local_alpha must be finite and in [0, 1]")
    if statistics.weight_sum <= 0 or statistics.effective_sample_size <= 0:
        raise ValueError("candidate H2 requires positive weighted support")
    S = statistics.candidate_gram / statistics.weight_sum
    S = (S + S.T) * 0.5
    p = statistics.width
    tr = torch.trace(S)
    if float(tr) <= 0:
        raise ValueError("candidate covariance must have positive trace")
    tr2 = tr.square()
    fro2 = S.square().sum()
    den = (statistics.effective_sample_size + 1.0 - 2.0 / p) * (fro2 - tr2 / p)
    rho = 1.0 if float(den) <= 0 else min(1.0, max(0.0, float(((1.0 - 2.0 / p) * fro2 + tr2) / den)))
    alpha = min(cap, 1.0 - rho)
    identity = torch.eye(p, dtype=S.dtype, device=S.device) * (tr / p)
    return torch.lerp(identity, S, alpha).contiguous(), {
        "rows": float(statistics.rows), "weight_sum": statistics.weight_sum,
        "effective_sample_size": statistics.effective_sample_size, "oas_shrinkage": rho, "local_alpha": alpha,
        "max_local_alpha": cap, "identity_scale": float(tr / p)}


def ridge_refit_down_from_statistics(statistics: CandidateHiddenStatistics, source_down_t: torch.Tensor, *,
                                     regularization_ratio: float):
    """The down projection ``X`` minimising the routed-output SSE on the
    candidate rows plus ``lambda ||X - source||^2`` (reference :927-960):
    ``(G_cc + lambda I) X = G_cs source + lambda source`` with ``lambda`` =
    ratio x ``tr(G_cc) / p``; solved by Cholesky (the system is SPD)."""

    statistics._validate()
    ratio = float(regularization_ratio)
    if not math.isfinite(ratio) or ratio <= 0:
        raise ValueError("regularization_ratio must be finite and positive")
    (src,) = _down_operands(statistics, source_down_t)
    scale = float(torch.trace(statistics.candidate_gram)) / statistics.width
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("candidate Gram matrix must have positive trace")
    lam = ratio * scale
    system = statistics.candidate_gram.clone()
    system = (system + system.T) * 0.5
    system.diagonal().add_(lam)
    rhs = statistics.candidate_source_cross @ src + lam * src
    factor, info = torch.linalg.cholesky_ex(system)
    refit = torch.cholesky_solve(rhs, factor) if int(info) == 0 else torch.linalg.solve(system, rhs)
    return refit.contiguous(), {"regularization_ratio": ratio, "regularization": lam,
                                "gram_trace_per_dimension": scale}


__all__ = [
    "CandidateHiddenStatistics",
    "CoupledTriplet",
    "PooledExpertEvaluation",
    "PooledPortfolioEvaluation",
    "UpstreamFunctionalStatistics",
    "blockwise_upstream_conditioning_coefficients",
    "candidate_h2",
    "collect_coupled_hidden_statistics",
    "collect_upstream_functional_statistics",
    "decoded_down_sse",
    "decoded_down_sse_difference",
    "evaluate_coupled_candidate_portfolio_batches",
    "evaluate_coupled_expert_batches",
    "ridge_refit_down_from_statistics",
]
