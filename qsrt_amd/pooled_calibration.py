"""Pooled sufficient statistics of routed expert calibration (mirrors
``qsrt/pooled_calibration.py``).

One decoded gate/up candidate determines the post-SiTU rows ``c`` of every
routed token; with the source rows ``s`` and route weight ``r``, the five
weighted cross-products

    G_cc = sum r^2 c c^T      G_cs = sum r^2 c s^T      G_ss = sum r^2 s s^T
    G_cr = sum r^2 c (c-s)^T  G_rr = sum r^2 (c-s)(c-s)^T

give the exact routed-output squared error of any down projection, the
candidate-local H2 and the ridge refit target, without keeping the rows.
FP32 statistics of device rows are accumulated on the FP32 matrix cores
(``qsrt_gemm_tn``: exact FP32 products, FP32 accumulation) over rows
pre-scaled by ``|r|``, with ``c - s`` formed before the scaling so the
residual products stay at the error's scale; FP64 statistics and CPU rows
use torch.
"""

from __future__ import annotations

import math
from collections.abc import Iterable, Mapping
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import gemm
from .qsrt_coupled import CoupledHadamardExecution, encode_coupled_weights, situ, situ_derivatives

Tensor = torch.Tensor


@dataclass
class CoupledTriplet:
    """One gated expert in ``[out, in]`` orientation: gate and up
    ``[intermediate, hidden]``, down ``[hidden, intermediate]`` (reference
    ``qsrt/coupled_expert_study.py:26-62``)."""

    gate: Tensor
    up: Tensor
    down: Tensor

    def __post_init__(self) -> None:
        if any(t.ndim != 2 for t in self.tensors()):
            raise ValueError("coupled expert weights must be rank-two tensors")
        if self.gate.shape != self.up.shape:
            raise ValueError("gate and up projections must have identical shapes")
        intermediate, hidden = self.gate.shape
        if tuple(self.down.shape) != (hidden, intermediate):
            raise ValueError("down must have shape [hidden, intermediate]")
        if not all(torch.is_floating_point(t) for t in self.tensors()):
            raise TypeError("coupled expert weights must be floating point")

    @property
    def intermediate(self) -> int:
        return int(self.gate.shape[0])

    @property
    def hidden(self) -> int:
        return int(self.gate.shape[1])

    @property
    def numel(self) -> int:
        return sum(t.numel() for t in self.tensors())

    def tensors(self) -> tuple[Tensor, Tensor, Tensor]:
        return self.gate, self.up, self.down

    def to(self, *args, **kwargs) -> "CoupledTriplet":
        return CoupledTriplet(*(t.to(*args, **kwargs) for t in self.tensors()))


def _all_finite(*tensors: Tensor) -> bool:
    return all(bool(torch.all(torch.isfinite(t))) for t in tensors)


@dataclass
class CandidateHiddenStatistics:
    """Weighted source/candidate post-activation cross-products (reference
    pooled_calibration.py:25-240).  ``source_gram`` and
    ``hidden_residual_gram`` are kept together or dropped together."""

    candidate_gram: Tensor
    candidate_source_cross: Tensor
    source_gram: Tensor | None
    candidate_residual_cross: Tensor
    hidden_residual_gram: Tensor | None
    weight_sum: float
    weight_square_sum: float
    rows: int

    @classmethod
    def zeros(cls, width: int, *, device="cpu", dtype: torch.dtype = torch.float64,
              retain_source_gram: bool = True) -> "CandidateHiddenStatistics":
        if width <= 0:
            raise ValueError("hidden width must be positive")
        if dtype not in (torch.float32, torch.float64):
            raise TypeError("sufficient statistics require FP32 or FP64")

        def z():
            return torch.zeros((width, width), device=device, dtype=dtype)

        return cls(z(), z(), z() if retain_source_gram else None, z(), z() if retain_source_gram else None,
                   0.0, 0.0, 0)

    @property
    def width(self) -> int:
        return int(self.candidate_gram.shape[0])

    @property
    def effective_sample_size(self) -> float:
        if self.weight_sum <= 0 or self.weight_square_sum <= 0:
            return 0.0
        return self.weight_sum ** 2 / self.weight_square_sum

    def _matrices(self) -> tuple[Tensor, ...]:
        kept = (self.source_gram, self.hidden_residual_gram) if self.source_gram is not None else ()
        return (self.candidate_gram, self.candidate_source_cross, self.candidate_residual_cross, *kept)

    def _validate(self) -> None:
        shape = self.candidate_gram.shape
        if (self.candidate_gram.ndim != 2 or shape[0] != shape[1]
                or (self.source_gram is None) != (self.hidden_residual_gram is None)
                or any(m.shape != shape for m in self._matrices())):
            raise ValueError("candidate statistics must contain equal-size squares")
        if not _all_finite(*self._matrices()):
            raise ValueError("candidate statistics must be finite")
        if (not math.isfinite(self.weight_sum) or not math.isfinite(self.weight_square_sum) or self.weight_sum < 0
                or self.weight_square_sum < 0 or self.rows < 0):
            raise ValueError("candidate statistics have invalid support")

    def update(self, candidate_hidden: Tensor, source_hidden: Tensor, route_weights: Tensor) -> None:
        """Accumulate one row chunk with weights ``route_weights ** 2``."""

        self._validate()
        if (candidate_hidden.ndim != 2 or source_hidden.shape != candidate_hidden.shape
                or candidate_hidden.shape[1] != self.width):
            raise ValueError("source and candidate hidden rows do not align")
        if route_weights.ndim != 1 or route_weights.numel() != candidate_hidden.shape[0]:
            raise ValueError("route weights must contain one value per hidden row")
        if not _all_finite(candidate_hidden, source_hidden, route_weights):
            raise ValueError("candidate rows and route weights must be finite")
        device, dtype = self.candidate_gram.device, self.candidate_gram.dtype
        c = candidate_hidden.to(device=device, dtype=dtype)
        s = source_hidden.to(device=device, dtype=dtype)
        r = route_weights.to(device=device, dtype=dtype)
        w = r.square()
        if c.shape[0]:
            if device.type == "cuda" and dtype == torch.float32:
                self._update_matrix_cores(c, s, r)
            else:
                wc = c * w[:, None]
                residual = c - s
                wr = residual * w[:, None]
                self.candidate_gram.add_(c.T @ wc)
                self.candidate_source_cross.add_(c.T @ (s * w[:, None]))
                self.candidate_residual_cross.add_(c.T @ wr)
                if self.source_gram is not None:
                    self.source_gram.add_(s.T @ (s * w[:, None]))
                    self.hidden_residual_gram.add_(residual.T @ wr)
        w64 = w.double()
        self.weight_sum += float(w64.sum())
        self.weight_square_sum += float(w64.square().sum())
        self.rows += int(c.shape[0])

    def _update_matrix_cores(self, c: Tensor, s: Tensor, r: Tensor) -> None:
        scale = r.abs()[:, None]
        residual = (c - s).mul_(scale)
        c = (c * scale).contiguous()
        s = (s * scale).contiguous()
        gemm.gram_(self.candidate_gram, c)
        gemm.addmm_tn_(self.candidate_source_cross, c, s)
        gemm.addmm_tn_(self.candidate_residual_cross, c, residual)
        if self.source_gram is not None:
            gemm.gram_(self.source_gram, s)
            gemm.gram_(self.hidden_residual_gram, residual)

    def merge_(self, other: "CandidateHiddenStatistics") -> None:
        """Add the statistics of a disjoint row partition."""

        self._validate()
        other._validate()
        if other.width != self.width:
            raise ValueError("candidate statistics widths differ")
        if (self.source_gram is None) != (other.source_gram is None):
            raise ValueError("candidate statistics disagree on source-Gram retention")
        for mine, theirs in zip(self._matrices(), other._matrices()):
            mine.add_(theirs.to(mine))
        self.weight_sum += other.weight_sum
        self.weight_square_sum += other.weight_square_sum
        self.rows += other.rows

    def to(self, *, device, dtype: torch.dtype | None = None) -> "CandidateHiddenStatistics":
        """A copy on ``device`` (and ``dtype``) with the same scalar support."""

        dtype = self.candidate_gram.dtype if dtype is None else dtype
        if dtype not in (torch.float32, torch.float64):
            raise TypeError("sufficient statistics require FP32 or FP64")

        def move(t):
            return None if t is None else t.to(device=device, dtype=dtype)

        return CandidateHiddenStatistics(move(self.candidate_gram), move(self.candidate_source_cross),
                                         move(self.source_gram), move(self.candidate_residual_cross),
                                         move(self.hidden_residual_gram), self.weight_sum, self.weight_square_sum,
                                         self.rows)


@dataclass(frozen=True)
class PooledExpertEvaluation:
    """Routed-function score and W2 statistics of one candidate."""

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
    """Routed-function scores of candidates that share one source expert."""

    candidate_sse: Mapping[str, float]
    source_energy: float
    routed_occurrences: int

    def __post_init__(self) -> None:
        if (not self.candidate_sse or any(not math.isfinite(v) or v < 0 for v in self.candidate_sse.values())
                or not math.isfinite(self.source_energy) or self.source_energy <= 0 or self.routed_occurrences <= 0):
            raise ValueError("pooled portfolio evaluation is invalid")


@dataclass
class UpstreamFunctionalStatistics:
    """Per-neuron post-SiTU energy and 2x2 gate/up sensitivity metric."""

    hidden_energy: Tensor
    derivative_metric: Tensor
    weight_sum: float
    weight_square_sum: float
    rows: int

    @property
    def effective_sample_size(self) -> float:
        if self.weight_sum <= 0 or self.weight_square_sum <= 0:
            return 0.0
        return self.weight_sum ** 2 / self.weight_square_sum


def blockwise_upstream_conditioning_coefficients(derivative_metric: Tensor, *, block_size: int):
    """Per-neuron ``m01 / m00`` and ``m01 / m11`` of the gate/up metric summed
    over contiguous neuron blocks (reference pooled_calibration.py:295-360)."""

    if (derivative_metric.ndim != 3 or derivative_metric.shape[1:] != (2, 2)
            or not torch.is_floating_point(derivative_metric)):
        raise ValueError("derivative metric must have shape [neurons, 2, 2]")
    neurons = int(derivative_metric.shape[0])
    if block_size <= 0 or neurons % block_size:
        raise ValueError("block size must divide the intermediate width")
    if not _all_finite(derivative_metric):
        raise ValueError("derivative metric must be finite")
    metric = derivative_metric.double()
    metric = (metric + metric.transpose(1, 2)) * 0.5
    eps = torch.finfo(metric.dtype).eps
    if float(torch.linalg.eigvalsh(metric).min()) < -256 * eps * max(float(metric.abs().max()), 1.0):
        raise ValueError("derivative metric must be positive semidefinite")
    blocks = metric.reshape(neurons // block_size, block_size, 2, 2).sum(dim=1)
    floor = max(float(blocks.diagonal(dim1=1, dim2=2).max().clamp_min(0)) * 1e-12, torch.finfo(metric.dtype).tiny)
    gate_from_up_blocks = blocks[:, 0, 1] / blocks[:, 0, 0].clamp_min(floor)
    up_from_gate_blocks = blocks[:, 0, 1] / blocks[:, 1, 1].clamp_min(floor)

    def spread(prefix: str, v: Tensor) -> dict[str, float]:
        q = torch.quantile(v, torch.tensor((0.05, 0.5, 0.95), device=v.device, dtype=v.dtype))
        return {f"{prefix}_minimum": float(v.min()), f"{prefix}_p05": float(q[0]), f"{prefix}_median": float(q[1]),
                f"{prefix}_p95": float(q[2]), f"{prefix}_maximum": float(v.max())}

    return (gate_from_up_blocks.repeat_interleave(block_size), up_from_gate_blocks.repeat_interleave(block_size),
            {"block_size": float(block_size), "blocks": float(blocks.shape[0]), "diagonal_floor": floor,
             **spread("gate_from_up", gate_from_up_blocks), **spread("up_from_gate", up_from_gate_blocks)})


def _routed_batches(batches: Iterable[Mapping[str, Tensor]], hidden: int, *, missing: str, misaligned: str,
                    order: str):
    """Validated ``(input, route_weight, row_index)`` of each nonempty batch;
    global row indices must increase strictly across all batches."""

    previous = -1
    for batch in batches:
        if not {"input", "route_weight", "row_index"}.issubset(batch):
            raise ValueError(missing)
        rows, route, index = batch["input"], batch["route_weight"], batch["row_index"]
        if (rows.ndim != 2 or rows.shape[1] != hidden or route.ndim != 1 or index.ndim != 1
                or route.numel() != rows.shape[0] or index.numel() != rows.shape[0]):
            raise ValueError(misaligned)
        if rows.shape[0] == 0:
            continue
        if index.dtype != torch.int64:
            raise TypeError("global row indices must be int64")
        if int(index[0]) <= previous or bool(torch.any(index[1:] <= index[:-1])):
            raise ValueError(order)
        previous = int(index[-1])
        yield rows, route, index


_POOLED = dict(missing="pooled expert batch lacks input, route weight, or row index",
               misaligned="pooled expert batch tensors do not align",
               order="pooled expert rows must be globally increasing")


def collect_upstream_functional_statistics(batches, *, source: CoupledTriplet, device) -> UpstreamFunctionalStatistics:
    """Per neuron ``n``: ``sum_r w_r d_rn d_rn^T |W2[:, n]|^2`` with ``d`` the
    SiTU (gate, up) derivative pair and ``w = route^2``, plus the weighted
    post-SiTU energy (reference pooled_calibration.py:363-430)."""

    target = torch.device(device)
    source = source.to(device=target, dtype=torch.float32)
    hidden_energy = torch.zeros(source.intermediate, device=target, dtype=torch.float64)
    metric = torch.zeros(source.intermediate, 2, 2, device=target, dtype=torch.float64)
    down_energy = source.down.double().square().sum(dim=0)
    weight_sum = weight_square_sum = 0.0
    count = 0
    for rows, route, _ in _routed_batches(batches, source.hidden,
                                          missing="functional-statistics batch lacks required tensors",
                                          misaligned="functional-statistics batch tensors do not align",
                                          order="functional-statistics rows must be globally increasing"):
        rows = rows.to(device=target, dtype=torch.float32)
        w = route.to(device=target, dtype=torch.float64).square()
        gate, up = F.linear(rows, source.gate), F.linear(rows, source.up)
        hidden_energy.add_((situ(gate, up).double().square() * w[:, None]).sum(dim=0))
        d_gate, d_up = (d.double() for d in situ_derivatives(gate, up))
        wg, wu = d_gate * w[:, None], d_up * w[:, None]
        m01 = (wg * d_up).sum(dim=0)
        block = torch.stack((torch.stack(((wg * d_gate).sum(dim=0), m01), dim=1),
                             torch.stack((m01, (wu * d_up).sum(dim=0)), dim=1)), dim=1)
        metric.add_(block * down_energy[:, None, None])
        weight_sum += float(w.sum())
        weight_square_sum += float(w.square().sum())
        count += int(rows.shape[0])
    if count == 0 or weight_sum <= 0:
        raise ValueError("functional statistics require routed support")
    return UpstreamFunctionalStatistics(hidden_energy, metric, weight_sum, weight_square_sum, count)


def _device_of(candidate: CoupledTriplet, message: str) -> torch.device:
    devices = {t.device for t in candidate.tensors()}
    if len(devices) != 1:
        raise ValueError(message)
    return devices.pop()


def _check_execution(execution: CoupledHadamardExecution, source: CoupledTriplet, statistics_dtype) -> None:
    if execution.hidden != source.hidden or execution.intermediate != source.intermediate:
        raise ValueError("coupled execution geometry differs from the expert")
    if statistics_dtype not in (torch.float32, torch.float64):
        raise TypeError("statistics require FP32 or FP64")


def collect_coupled_hidden_statistics(batches, *, source: CoupledTriplet, candidate_coordinates: CoupledTriplet,
                                      execution: CoupledHadamardExecution,
                                      statistics_dtype: torch.dtype = torch.float32,
                                      retain_source_gram: bool = False) -> CandidateHiddenStatistics:
    """Statistics of a decoded gate/up candidate in the coupled basis, with no
    W2 evaluation (reference pooled_calibration.py:433-515)."""

    if source.hidden != candidate_coordinates.hidden or source.intermediate != candidate_coordinates.intermediate:
        raise ValueError("source and candidate expert geometry differ")
    _check_execution(execution, source, statistics_dtype)
    device = _device_of(candidate_coordinates, "candidate coordinate tensors must share one device")
    source = source.to(device=device, dtype=torch.float32)
    candidate = candidate_coordinates.to(device=device, dtype=torch.float32)
    source_coords = CoupledTriplet(*encode_coupled_weights(source.tensors(), execution.spec))
    stats = CandidateHiddenStatistics.zeros(source.intermediate, device=device, dtype=statistics_dtype,
                                            retain_source_gram=retain_source_gram)
    for rows, route, _ in _routed_batches(batches, source.hidden, **_POOLED):
        rows = execution.transform_inputs(rows.to(device=device, dtype=torch.float32))
        stats.update(execution.decode_middle(rows, candidate.gate, candidate.up),
                     execution.decode_middle(rows, source_coords.gate, source_coords.up),
                     route.to(device=device, dtype=torch.float32))
    if stats.rows == 0:
        raise ValueError("pooled hidden statistics require routed support")
    return stats


def evaluate_coupled_expert_batches(batches, *, source: CoupledTriplet, teacher_source: CoupledTriplet | None = None,
                                    candidate_coordinates: CoupledTriplet, execution: CoupledHadamardExecution,
                                    prefix_row_limits: Iterable[int] = (),
                                    statistics_dtype: torch.dtype = torch.float32,
                                    retain_source_gram: bool = False) -> PooledExpertEvaluation:
    """Routed-output SSE of a coupled candidate against the ordinary-basis
    teacher, with its W2 statistics and scores over global-row prefixes
    (reference pooled_calibration.py:518-658)."""

    if source.hidden != candidate_coordinates.hidden or source.intermediate != candidate_coordinates.intermediate:
        raise ValueError("source and candidate expert geometry differ")
    teacher = source if teacher_source is None else teacher_source
    if teacher.hidden != source.hidden or teacher.intermediate != source.intermediate:
        raise ValueError("teacher and coordinate-source expert geometry differ")
    _check_execution(execution, source, statistics_dtype)
    limits = tuple(sorted({int(v) for v in prefix_row_limits}))
    if any(v <= 0 for v in limits):
        raise ValueError("prefix row limits must be positive")
    device = _device_of(candidate_coordinates, "candidate coordinate tensors must share one device")
    source = source.to(device=device, dtype=torch.float32)
    teacher = teacher.to(device=device, dtype=torch.float32)
    candidate = candidate_coordinates.to(device=device, dtype=torch.float32)
    source_coords = CoupledTriplet(*encode_coupled_weights(source.tensors(), execution.spec))
    stats = CandidateHiddenStatistics.zeros(source.intermediate, device=device, dtype=statistics_dtype,
                                            retain_source_gram=retain_source_gram)
    sse = energy = 0.0
    occurrences = 0
    prefix = {limit: [0.0, 0.0, 0] for limit in limits}
    for rows, route, index in _routed_batches(batches, source.hidden, **_POOLED):
        rows = rows.to(device=device, dtype=torch.float32)
        route = route.to(device=device, dtype=torch.float32)
        transformed = execution.transform_inputs(rows)
        source_hidden = execution.decode_middle(transformed, source_coords.gate, source_coords.up)
        candidate_hidden = execution.decode_middle(transformed, candidate.gate, candidate.up)
        # The teacher output is evaluated in the ordinary basis, so roundoff of
        # the coupled change of basis never redefines the target.
        source_output = F.linear(situ(F.linear(rows, teacher.gate), F.linear(rows, teacher.up)), teacher.down)
        candidate_output = execution.decode_output(candidate_hidden @ candidate.down.T)
        stats.update(candidate_hidden, source_hidden, route)
        row_sse = ((candidate_output - source_output) * route[:, None]).square().sum(dim=1, dtype=torch.float64).cpu()
        row_energy = (source_output * route[:, None]).square().sum(dim=1, dtype=torch.float64).cpu()
        sse += float(row_sse.sum())
        energy += float(row_energy.sum())
        occurrences += int(rows.shape[0])
        cpu_index = index.cpu()
        for limit, acc in prefix.items():
            n = int(torch.searchsorted(cpu_index, limit, right=False))
            if n:
                acc[0] += float(row_sse[:n].sum())
                acc[1] += float(row_energy[:n].sum())
                acc[2] += n
    if occurrences == 0 or energy <= 0:
        raise ValueError("pooled expert evaluation requires routed support")
    return PooledExpertEvaluation(stats, sse, energy, occurrences,
                                  {k: (float(v[0]), float(v[1]), int(v[2])) for k, v in prefix.items()})


def evaluate_coupled_candidate_portfolio_batches(batches, *, source: CoupledTriplet,
                                                 candidate_coordinates: Mapping[str, CoupledTriplet],
                                                 executions: Mapping[str, CoupledHadamardExecution]
                                                 ) -> PooledPortfolioEvaluation:
    """Routed SSE of several candidates of one source expert from one shared
    source forward; every candidate must share the residual-side transform
    (reference pooled_calibration.py:661-771)."""

    names = tuple(candidate_coordinates)
    if not names or set(executions) != set(names):
        raise ValueError("candidate coordinates and executions must share identities")
    devices = {t.device for c in candidate_coordinates.values() for t in c.tensors()}
    if len(devices) != 1:
        raise ValueError("pooled portfolio candidates must share one device")
    device = devices.pop()
    source = source.to(device=device, dtype=torch.float32)
    candidates = {k: c.to(device=device, dtype=torch.float32) for k, c in candidate_coordinates.items()}
    first = executions[names[0]]
    if first.hidden != source.hidden or first.intermediate != source.intermediate:
        raise ValueError("pooled portfolio execution geometry differs from the source")
    residual = (first.spec.residual_block_size, first.spec.residual_draw)
    for name in names:
        c, e = candidates[name], executions[name]
        if (c.hidden != source.hidden or c.intermediate != source.intermediate or e.hidden != source.hidden
                or e.intermediate != source.intermediate
                or (e.spec.residual_block_size, e.spec.residual_draw) != residual):
            raise ValueError("pooled portfolio candidates do not share residual geometry")
    sse = {name: 0.0 for name in names}
    energy = 0.0
    occurrences = 0
    for rows, route, _ in _routed_batches(batches, source.hidden, missing=_POOLED["missing"],
                                          misaligned="pooled portfolio batch tensors do not align",
                                          order=_POOLED["order"]):
        rows = rows.to(device=device, dtype=torch.float32)
        route = route.to(device=device, dtype=torch.float32)
        source_output = F.linear(situ(F.linear(rows, source.gate), F.linear(rows, source.up)), source.down)
        transformed = first.transform_inputs(rows)
        energy += float((source_output * route[:, None]).square().sum(dtype=torch.float64).cpu())
        for name in names:
            c, e = candidates[name], executions[name]
            out = e.decode_output(e.decode_middle(transformed, c.gate, c.up) @ c.down.T)
            sse[name] += float(((out - source_output) * route[:, None]).square().sum(dtype=torch.float64).cpu())
        occurrences += int(rows.shape[0])
    return PooledPortfolioEvaluation(sse, energy, occurrences)


def _down_operands(statistics: CandidateHiddenStatistics, *mats: Tensor) -> list[Tensor]:
    dtype, device = statistics.candidate_gram.dtype, statistics.candidate_gram.device
    return [m.to(device=device, dtype=dtype) for m in mats]


def decoded_down_sse(statistics: CandidateHiddenStatistics, candidate_down_t: Tensor, source_down_t: Tensor) -> Tensor:
    """Routed-output SSE ``sum r^2 |c D_c - s D_s|^2`` from the statistics,
    with ``D`` in ``[intermediate, output]`` orientation (reference
    pooled_calibration.py:774-827).

    Written around ``Delta = D_c - D_s``: ``<Delta, G_cc Delta> + 2 <Delta,
    G_cr D_s> + <D_s, G_rr D_s>``, every term at the scale of the error, so no
    absolute output energies cancel."""

    statistics._validate()
    if statistics.source_gram is None:
        raise ValueError("decoded down SSE requires retained source Gram statistics")
    if candidate_down_t.ndim != 2:
        raise ValueError("candidate down projection must be two-dimensional")
    if tuple(candidate_down_t.shape) != (statistics.width, candidate_down_t.shape[1]):
        raise ValueError("candidate down projection has the wrong shape")
    if source_down_t.shape != candidate_down_t.shape:
        raise ValueError("source and candidate down projections do not align")
    candidate, source = _down_operands(statistics, candidate_down_t, source_down_t)
    delta = candidate - source
    delta_term = torch.sum(delta * (statistics.candidate_gram @ delta))
    cross_term = torch.sum(delta * (statistics.candidate_residual_cross @ source))
    residual_term = torch.sum(source * (statistics.hidden_residual_gram @ source))
    value = delta_term + 2.0 * cross_term + residual_term
    dtype = statistics.candidate_gram.dtype
    tolerance = 64 * torch.finfo(dtype).eps * max(float(delta_term.abs()), float((2.0 * cross_term).abs()),
                                                  float(residual_term.abs()), 1.0)
    if float(value) < -tolerance:
        raise ArithmeticError(f"pooled SSE is negative beyond roundoff: {float(value):.9g}")
    return value.clamp_min(0)


def decoded_down_sse_difference(statistics: CandidateHiddenStatistics, candidate_down_t: Tensor,
                                baseline_down_t: Tensor, source_down_t: Tensor) -> Tensor:
    """SSE(candidate) - SSE(baseline) without the source Gram: with
    ``delta = D_c - D_b``, ``2 <delta, G_cc (D_b - D_s) + G_cr D_s> + <delta,
    G_cc delta>`` (reference pooled_calibration.py:830-861)."""

    statistics._validate()
    if candidate_down_t.ndim != 2:
        raise ValueError("candidate down projection must be two-dimensional")
    if (tuple(candidate_down_t.shape) != (statistics.width, candidate_down_t.shape[1])
            or baseline_down_t.shape != candidate_down_t.shape or source_down_t.shape != candidate_down_t.shape):
        raise ValueError("down projections do not share the expected shape")
    candidate, baseline, source = _down_operands(statistics, candidate_down_t, baseline_down_t, source_down_t)
    delta = candidate - baseline
    gradient = statistics.candidate_gram @ (baseline - source) + statistics.candidate_residual_cross @ source
    return 2.0 * torch.sum(delta * gradient) + torch.sum(delta * (statistics.candidate_gram @ delta))


def candidate_h2(statistics: CandidateHiddenStatistics, *, max_local_alpha: float = 0.75):
    """Candidate-local covariance ``G_cc / sum w`` shrunk toward
    ``trace / d * I`` by the Oracle Approximating Shrinkage estimator of Chen,
    Wiesel, Eldar and Hero (2010) at the Kish effective sample size ``n``:
    ``rho = ((1 - 2/d) |S|_F^2 + tr(S)^2) / ((n + 1 - 2/d)(|S|_F^2 - tr(S)^2 / d))``,
    local weight ``min(max_local_alpha, 1 - rho)`` (reference
    pooled_calibration.py:864-924)."""

    statistics._validate()
    max_local_alpha = float(max_local_alpha)
    if not math.isfinite(max_local_alpha) or not 0 <= max_local_alpha <= 1:
        raise ValueError("max_local_alpha must be finite and in [0, 1]")
    if statistics.weight_sum <= 0 or statistics.effective_sample_size <= 0:
        raise ValueError("candidate H2 requires positive weighted support")
    cov = statistics.candidate_gram / statistics.weight_sum
    cov = (cov + cov.T) * 0.5
    d = statistics.width
    trace = torch.trace(cov)
    if float(trace) <= 0:
        raise ValueError("candidate covariance must have positive trace")
    trace_sq, frob_sq = trace.square(), cov.square().sum()
    den = (statistics.effective_sample_size + 1.0 - 2.0 / d) * (frob_sq - trace_sq / d)
    rho = 1.0 if float(den) <= 0 else min(1.0, max(0.0, float(((1.0 - 2.0 / d) * frob_sq + trace_sq) / den)))
    local_alpha = min(max_local_alpha, 1.0 - rho)
    scale = trace / d
    result = torch.lerp(torch.eye(d, dtype=cov.dtype, device=cov.device).mul_(scale), cov, local_alpha)
    return result.contiguous(), {
        "rows": float(statistics.rows), "weight_sum": statistics.weight_sum,
        "effective_sample_size": statistics.effective_sample_size, "oas_shrinkage": rho,
        "local_alpha": local_alpha, "max_local_alpha": max_local_alpha, "identity_scale": float(scale)}


def ridge_refit_down_from_statistics(statistics: CandidateHiddenStatistics, source_down_t: Tensor, *,
                                     regularization_ratio: float):
    """``(G_cc + lam I)^-1 (G_cs D_s + lam D_s)`` with ``lam = ratio *
    trace(G_cc) / d`` (reference pooled_calibration.py:927-958)."""

    statistics._validate()
    ratio = float(regularization_ratio)
    if not math.isfinite(ratio) or ratio <= 0:
        raise ValueError("regularization_ratio must be finite and positive")
    if source_down_t.ndim != 2 or source_down_t.shape[0] != statistics.width:
        raise ValueError("source down projection does not match candidate width")
    (source,) = _down_operands(statistics, source_down_t)
    scale = float(torch.trace(statistics.candidate_gram)) / statistics.width
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("candidate Gram matrix must have positive trace")
    lam = ratio * scale
    system = statistics.candidate_gram.clone()
    system.diagonal().add_(lam)
    refit = torch.linalg.solve(system, statistics.candidate_source_cross @ source + lam * source)
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
