"""QSRT encoder hot-path benchmark on one MI355X.

Headline workload (the largest single-GPU
configuration): the whole 384-expert Kimi-class MoE layer (gate/up
[7168 x 2048], down [2048 x 7168] per expert) encoded end to end -- the
exact coupled gate/up/down basis, H13 captured from each expert's
Zipf-routed calibration rows, batched global-scale search, BlockLDLQ with
14 K3 + 2 K4 records per matrix, H2 rebuilt from the reconstructed gate/up
SwiGLU activations, record-major packing -- followed by the decode of the
whole packed layer to bf16.  The synthetic bf16 sources and calibration rows
are resident in HBM before the timed region (288 GB holds the whole layer);
everything from them to the packed payload is timed.

``--steps K`` splits the layer into K steps of consecutive experts (each
step one or more encoder batches); ``--warmup W`` encodes a separate
warm-up expert W times first.  Prints ONE JSON line:

  value        encoded weights/s (M/s) over the whole layer
  roofline     the tile Viterbi (the dominant kernel): algorithmic FP32 flops
               (3 per trellis edge, 131,072 edges per weight at C = 128) per
               launch / its average launch time, HIP events on its stream over
               the timed region, against MI355X's 157.3 TFLOP/s FP32 peak
  cpu_baseline the CPU oracle (float64 BlockLDLQ + the C Viterbi, OpenMP on
               this host's cores) on the bottom row blocks of one layer
               matrix, with the same inputs the GPU encoded
  parity       the GPU's states on that sample against the CPU oracle's
Secondary keys: the decode of the encoded layer, the config-2 Viterbi
microbench (packing inside its step), the config-4 expert at K3 (the
north-star target) and at K2 (as BASELINE specifies it), the config-3 GLM
expert, the MFMA GEMMs and the Hadamard rotation.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import tempfile
import time
from pathlib import Path
from types import SimpleNamespace

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

CONTEXT = 128
EDGES_PER_WEIGHT = (256 + 2 * CONTEXT) / 256 * 65536  # 131,072 at C = 128
FLOPS_PER_EDGE = 3  # d = label - x (1), fma(d, d, cost) (2)
FP32_PEAK_TFLOPS = 157.3
FP32_UNPACKED_PEAK_TFLOPS = 78.6  # 256 CUs x 64 FP32 FMA lanes x 2 flops x 2.4 GHz, no packed FP32
HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f32": 157.3, "f64": 78.6}
# HBM bytes per tile of the Viterbi kernel by rate (FETCH_SIZE x 2.00 + WRITE_SIZE x 1.00 per dispatch, calibrated
# on a 4 GiB device copy; K3/K4 over every dispatch of a 20-expert layer step, K2 from the microbench;
# profiles/layer_encode_config5.md): mostly the traceback decision stream.
VITERBI_HBM_BYTES_PER_TILE = {2: 1.631e6, 3: 1.633e6, 4: 0.816e6}
# Same counters for the decode launches: 1.03 x their algorithmic bytes (profiles/decode_kernel_layer.md).
DECODE_TRAFFIC_OVER_ALGORITHMIC = 1.032
# Same counters at the bench's GEMM and Hadamard shapes (profiles/gemm_tn_kernels_expert_shapes.md,
# profiles/hadamard_kernel_expert_matrix.md): HBM bytes per launch (the Hessian capture: its main kernel and
# the fixup kernel of its K-split tiles together).
GEMM_HBM_BYTES = {"hessian_capture": 2.435e9, "ldlq_span_update": 1.485e8, "ldlq_span_update_f64": 2.950e8,
                  "ldlq_span_update_batched_f64": 6.09e9}
HADAMARD_HBM_BYTES = {"left": 1.1782e8, "right": 1.1765e8}
# Same counters for the BaKron top band's left + right launches (profiles/bakron_band_kernels_config4_gate.md):
# mostly the right product's re-reads of the input factor.
BAKRON_TOP_BAND_HBM_BYTES = 5.515e9

# Every `traffic` field is a profile constant (HBM bytes per launch from a rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
# pass of this file's own command, calibrated on a device copy), not a counter read by this run.
TRAFFIC_NOTE = ("HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes ({}), scaled by the "
                "same counters on a device copy; a profile constant, not measured in this run")

LAYER_EXPERTS = 384
LAYER_TOKENS = 65536
LAYER_ZIPF_S = 1.1
LAYER_ID = 24
LAYER_HIDDEN, LAYER_INTER = 7168, 2048
# Record rates of every layer matrix: BASELINE names 2 K4 + 22 K3 records (the 24-record H308 mode of a
# 3072-channel intermediate axis); a 2048-channel axis holds 16 records of 128 channels, so the layer keeps the
# two K4 records and fills the rest with K3 (3.125 trellis bpw).
LAYER_RECORD_BITS = (3,) * 14 + (4,) * 2
MAX_BATCH_EXPERTS = 24


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# BASELINE configs as seeded synthetic inputs
# ---------------------------------------------------------------------------


def student_t_like(shape, *, nu: int = 5, std: float, gen: torch.Generator) -> torch.Tensor:
    """Student-t(nu) scaled to standard deviation ``std``, drawn on the
    generator's device: ``z / sqrt(chi2_nu / nu)`` with the chi-square a sum
    of ``nu`` squared normals."""

    dev = gen.device
    z = torch.randn(shape, generator=gen, device=dev)
    chi2 = torch.zeros(shape, device=dev)
    for _ in range(nu):
        chi2.addcmul_(u := torch.randn(shape, generator=gen, device=dev), u)
    return z.div_(chi2.div_(nu).sqrt_()).mul_(std / math.sqrt(nu / (nu - 2.0)))


def ar1_scan(n: int, k: int, rho: float, gen: torch.Generator, *, block: int = 128) -> torch.Tensor:
    """``n`` rows of the AR(1) process along channels (x_0 = z_0,
    x_j = rho x_{j-1} + sqrt(1 - rho^2) z_j, so Sigma_ij = rho^|i-j|), FP32 on
    the generator's device: each block of ``block`` channels is one
    triangular product, then the carries run across the blocks."""

    dev = gen.device
    if k % block:
        raise ValueError("channels must be a multiple of the scan block")
    c = math.sqrt(1.0 - rho * rho)
    z = torch.randn((n, k), generator=gen, device=dev)
    z[:, 0] /= c  # x_0 = z_0: the first channel's innovation has weight 1, not c
    i = torch.arange(block, device=dev, dtype=torch.float64)
    gap = i[None, :] - i[:, None]
    T = torch.where(gap >= 0, c * rho ** gap.clamp(min=0), torch.zeros((), dtype=torch.float64, device=dev)).float()
    x = (z.view(n, k // block, block) @ T).contiguous()
    carry = (rho ** (i + 1)).float()
    for b in range(1, k // block):
        x[:, b].addcmul_(x[:, b - 1, -1:], carry[None, :])
    return x.view(n, k)


def config_expert(cfg: int, device, *, expert: int = 0, tokens: int | None = None) -> dict:
    """Seeded synthetic inputs of BASELINE configs 1, 3, 4 and 5 (one expert):
    weights ``w_gate, w_up [inter, hidden]``, ``w_down [hidden, inter]`` and
    calibration rows ``x [tokens, hidden]``.

    cfg 1: hidden 256, inter 512, FP32 weights t5 x 0.02, 4096 rows rho 0.8.
    cfg 3: hidden 5120, inter 1536, bf16 weights t5 x 0.015, 8192 rows
           rho 0.9, 8 seeded outlier channels at 20x variance.
    cfg 4: hidden 7168, inter 2048, bf16 weights t5 x 0.015, 16384 rows rho 0.85.
    cfg 5: the cfg-4 shape, one generator per expert, ``tokens`` routed rows.
    """

    shapes = {1: (256, 512, 4096, 0.8, 0.02, False), 3: (5120, 1536, 8192, 0.9, 0.015, True),
              4: (7168, 2048, 16384, 0.85, 0.015, True), 5: (7168, 2048, 0, 0.85, 0.015, True)}
    hidden, inter, n, rho, std, bf16 = shapes[cfg]
    n = n if tokens is None else tokens
    gen = torch.Generator(device=device).manual_seed((20261201 + cfg) * 1000 + expert)
    w = []
    for shape in ((inter, hidden), (inter, hidden), (hidden, inter)):
        t = student_t_like(shape, std=std, gen=gen)
        w.append(t.bfloat16().float() if bf16 else t)
    x = ar1_scan(max(n, 1), hidden, rho, gen)[:n]
    outliers = None
    if cfg == 3:
        outliers = torch.randperm(hidden, generator=gen, device=device)[:8].sort().values
        x[:, outliers] *= math.sqrt(20.0)
    return {"w_gate": w[0], "w_up": w[1], "w_down": w[2], "x": x, "hidden": hidden, "inter": inter,
            "outliers": outliers}


def zipf_token_counts(experts: int = LAYER_EXPERTS, tokens: int = LAYER_TOKENS, s: float = LAYER_ZIPF_S,
                      seed: int = 20261201 + 8) -> list[int]:
    """Routed calibration tokens per expert: c_r proportional to r^-s over the
    ranks, scaled to ``tokens`` with largest-remainder rounding, ranks mapped
    to experts by a seeded permutation."""

    w = [r ** -s for r in range(1, experts + 1)]
    total = sum(w)
    exact = [tokens * x / total for x in w]
    counts = [int(math.floor(x)) for x in exact]
    for i in sorted(range(experts), key=lambda i: exact[i] - counts[i], reverse=True)[:tokens - sum(counts)]:
        counts[i] += 1
    perm = torch.randperm(experts, generator=torch.Generator().manual_seed(seed)).tolist()
    by_expert = [0] * experts
    for rank, expert in enumerate(perm):
        by_expert[expert] = counts[rank]
    return by_expert


def expert_source(cfg: int, device, *, expert: int = 0, tokens: int | None = None) -> dict:
    """One expert's encoder inputs as they sit in HBM: bf16 weights and bf16
    calibration rows (the activations a capture hook sees), plus each routed
    row's gate value (uniform in [0.05, 1), from a generator of its own so
    the weights and rows are unchanged; BASELINE does not fix them)."""

    d = config_expert(cfg, device, expert=expert, tokens=tokens)
    n = int(d["x"].shape[0])
    gen = torch.Generator(device=device).manual_seed((20261201 + cfg) * 1000 + expert + 500_000)
    gates = 0.05 + 0.95 * torch.rand(n, generator=gen, device=device)
    return {"expert": expert, "w": tuple(d[k].bfloat16() for k in ("w_gate", "w_up", "w_down")),
            "x": d["x"].bfloat16(), "tokens": n, "gates": gates}


# ---------------------------------------------------------------------------
# Coupled-expert encode (configs 4 and 5)
# ---------------------------------------------------------------------------


def pack_records(encoded: torch.Tensor, rate_axis: str, record_bits) -> torch.Tensor:
    """``[K/16, N/16, 256]`` states -> record-major EXL words (the
    ``pack_qsrt_trellis`` container: 128-channel records along the rate axis,
    each record's tiles in row-major order at the record's rate)."""

    from qsrt_amd.qsrt import pack_trellis_edges

    tk, tn = encoded.shape[:2]
    n_rec = len(record_bits)
    if rate_axis == "k":  # a record is 8 whole tile rows: the records are already contiguous
        by_record = encoded.reshape(n_rec, 8 * tn, 256)
    else:  # a record is 8 tile columns: gather each record's tiles, row-major within it, in one copy
        by_record = encoded.reshape(tk, n_rec, 8, 256).transpose(0, 1).reshape(n_rec, 8 * tk, 256)
    pieces, r = [], 0
    while r < n_rec:  # a run of consecutive records at one rate packs in one call (tiles pack independently)
        e = r + 1
        while e < n_rec and record_bits[e] == record_bits[r]:
            e += 1
        pieces.append(pack_trellis_edges(by_record[r:e].reshape(-1, 256), record_bits[r]).reshape(-1))
        r = e
    return torch.cat(pieces)


class ExpertEncoder:
    """Encode batches of SwiGLU experts of one shape in the exact coupled
    basis, as the layer pipeline does: per expert the coupled transform and
    the H13 capture, one ``quantize_qsrt_batch`` over every gate and up
    matrix of the batch, H2 from the reconstructed gate/up SwiGLU
    activations, one ``quantize_qsrt_batch`` over the down matrices, and
    record-major packing of every payload.

    ``hessian_policy``: ``"routed"`` (default) takes H13
    as the Gram of the expert's routed rows and H2 as the Gram of its decoded
    post-activation rows.  ``"support_aware"`` is the production covariance
    policy of ``qsrt_amd.candidate_hessian.build_expert_hessians``: H13 is
    the layer's ``global_h13`` (the covariance of all the layer's
    calibration rows), H2 the gate-square weighted covariance of the decoded
    post-activation rows, OAS-shrunk toward its trace-scaled identity -- for
    a low-support expert (tens of routed rows) mostly the identity.  The
    evidence of each expert's H2 is kept in ``self.h2_evidence``."""

    def __init__(self, device, *, hidden: int, inter: int, record_bits, layer: int = LAYER_ID, scope=None,
                 hessian_policy: str = "routed", global_h13: torch.Tensor | None = None):
        from qsrt_amd.qsrt_coupled import CoupledHadamardSpec

        if inter % 128 or len(record_bits) != inter // 128:
            raise ValueError("one record rate per 128 intermediate channels")
        if hessian_policy not in ("routed", "support_aware"):
            raise ValueError("hessian_policy must be 'routed' or 'support_aware'")
        if hessian_policy == "support_aware" and (global_h13 is None or tuple(global_h13.shape) != (hidden, hidden)):
            raise ValueError("the support-aware policy needs the layer's global H13 [hidden, hidden]")
        self.policy, self.global_h13, self.h2_evidence = hessian_policy, global_h13, {}
        self.dev, self.hidden, self.inter, self.layer = device, hidden, inter, layer
        self.record_bits = tuple(record_bits)
        self.rate_map = tuple(b for b in self.record_bits for _ in range(8))  # per 16-channel tile
        self.scope = scope if scope is not None else ("bench-layer", layer)
        self.spec = CoupledHadamardSpec()  # residual 512, pre/post 128, draw 0
        self.tile_encodes = 0

    def quant_args(self, matrix: str) -> dict:
        from qsrt_amd.qsrt import MATRIX_RATE_AXIS
        from qsrt_amd.qsrt_encoder import _qsrt_quant_args
        from qsrt_amd.transform_seeds import default_qsrt_transform_seeds

        plan = SimpleNamespace(rate_axis=MATRIX_RATE_AXIS[matrix], encoder_tile_bits=self.rate_map)
        qa = _qsrt_quant_args(plan, matrix=matrix, layer=self.layer, device=self.dev, shared_scale_scope=self.scope,
                              transform_seeds=default_qsrt_transform_seeds(self.layer, matrix))
        qa["sigma_reg"] = 0.01  # BASELINE: H = X^T X / n + 1% diagonal damping
        return qa

    def encode(self, sources: list[dict], *, keep_states=()) -> list[dict]:
        """Returns one dict per expert with ``w1``/``w3``/``w2`` entries
        (record-major ``words``, ``suh``, ``svh``, ``proxy``, ``g_scale``);
        experts whose id is in ``keep_states`` also keep their states and
        quant_args."""

        from qsrt_amd import exl3_encoder_backend as be
        from qsrt_amd import gemm
        from qsrt_amd.ldlq import make_shared_h
        from qsrt_amd.qsrt import MATRIX_RATE_AXIS
        from qsrt_amd.qsrt_coupled import coupled_execution, decode_coupled_weights, encode_coupled_weights

        dev, hidden, inter = self.dev, self.hidden, self.inter
        aware = self.policy == "support_aware"
        prepared = []
        for src in sources:
            w = tuple(t.float() for t in src["w"])
            g_c, u_c, d_c = encode_coupled_weights(w, self.spec)
            ex = coupled_execution((g_c, u_c, d_c), self.spec)
            if aware:  # the layer's global input covariance (local weight 0), already normalised
                h13, count13 = ex.transform_h13(self.global_h13.to(dev).float()), 1
            else:
                h13 = ex.transform_h13(gemm.gram_(torch.zeros((hidden, hidden), device=dev), src["x"]))
                count13 = src["tokens"]
            prepared.append({"c": (g_c, u_c, d_c), "ex": ex, "h13": h13, "x": src["x"], "n": src["tokens"],
                             "n13": count13, "gates": src.get("gates"), "expert": src["expert"]})
        weights, hs, qas = [], [], []
        for p in prepared:
            for name, m in (("w1", p["c"][0]), ("w3", p["c"][1])):
                shared = make_shared_h(hidden, dev, p["h13"])
                shared["count"] = p["n13"]
                weights.append(m.T.contiguous())
                hs.append(shared)
                qas.append([self.quant_args(name)])
            del p["h13"]
        up = be.quantize_qsrt_batch(weights, hs, qas)
        kept = {}
        for i, src in enumerate(sources):  # the float64 regularised weight and factor the recursion read
            if src["expert"] in keep_states:
                kept[(i, "w1")] = (up[2 * i][0]["weight_r"], hs[2 * i]["L"])
                kept[(i, "w3")] = (up[2 * i + 1][0]["weight_r"], hs[2 * i + 1]["L"])
        del weights, hs
        weights, hs, qas_d = [], [], []
        for i, p in enumerate(prepared):
            g_hat, u_hat = up[2 * i][0]["weight_q"].T, up[2 * i + 1][0]["weight_q"].T
            gs, us, _ = decode_coupled_weights((g_hat, u_hat, p["c"][2]), self.spec)
            x = p["x"].float()
            h = (torch.nn.functional.silu(x @ gs.T) * (x @ us.T)).contiguous()
            if aware:
                from qsrt_amd.candidate_hessian import build_expert_hessians

                if p["gates"] is None:
                    raise ValueError("the support-aware policy needs each source's routed gate values")
                _, h2_cov, evidence = build_expert_hessians(x, p["gates"], h, global_h13=self.global_h13,
                                                            global_h2=torch.eye(inter, device=dev), device=dev)
                self.h2_evidence[p["expert"]] = evidence
                h2, count2 = p["ex"].transform_h2(h2_cov), 1
            else:
                h2, count2 = p["ex"].transform_h2(gemm.gram_(torch.zeros((inter, inter), device=dev), h)), p["n"]
            del h, x
            shared = make_shared_h(inter, dev, h2)
            shared["count"] = count2
            weights.append(p["c"][2].T.contiguous())
            hs.append(shared)
            qas_d.append([self.quant_args("w2")])
        down = be.quantize_qsrt_batch(weights, hs, qas_d, return_weight_q=False)
        for i, src in enumerate(sources):
            if src["expert"] in keep_states:
                kept[(i, "w2")] = (down[i][0]["weight_r"], hs[i]["L"])
        del weights, hs
        out = []
        for i, src in enumerate(sources):
            rec = {"expert": src["expert"], "tokens": src["tokens"]}
            for name, r, qa in (("w1", up[2 * i][0], qas[2 * i][0]), ("w3", up[2 * i + 1][0], qas[2 * i + 1][0]),
                                ("w2", down[i][0], qas_d[i][0])):
                axis = MATRIX_RATE_AXIS[name]
                entry = {"words": pack_records(r["encoded"], axis, self.record_bits), "suh": r["suh"],
                         "svh": r["svh"], "proxy": r["proxy"], "g_scale": r["g_scale"], "rate_axis": axis,
                         "shape": tuple(16 * s for s in r["encoded"].shape[:2])}
                if src["expert"] in keep_states:
                    entry["encoded"] = r["encoded"]
                    entry["quant_args"] = qa
                    entry["W_r"], entry["L"] = kept[(i, name)]
                rec[name] = entry
            out.append(rec)
        return out


class ViterbiLaunchTimer:
    """HIP events around every tile-Viterbi launch, on the launch stream, so
    the dominant kernel's average duration over a timed region is measured
    live."""

    def __init__(self):
        from qsrt_amd import sqg_quantizer

        self._mod = sqg_quantizer
        self._real = sqg_quantizer.viterbi_tiles
        self.events: list = []
        self.active = False

    def __enter__(self):
        real = self._real

        cus = torch.cuda.get_device_properties(0).multi_processor_count

        def timed(tiles, lut, bits, **kw):
            if not self.active:
                return real(tiles, lut, bits, **kw)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            out = real(tiles, lut, bits, **kw)
            e1.record()
            cap = int(kw.get("max_workgroups", 0)) or cus
            self.events.append((int(tiles.shape[0]), int(bits), e0, e1, min(cap, cus, int(tiles.shape[0])) / cus))
            return out

        self._mod.viterbi_tiles = timed
        return self

    def __exit__(self, *exc):
        self._mod.viterbi_tiles = self._real

    def summary(self) -> dict:
        """Launch count, tiles, summed launch time, and the GPU-equivalent
        time: each launch's duration weighted by the share of the compute
        units its grid holds (rate groups of one step run side by side on
        split grids, so their durations overlap)."""

        torch.cuda.synchronize()
        tiles = sum(ev[0] for ev in self.events)
        ms = sum(ev[2].elapsed_time(ev[3]) for ev in self.events)
        gpu_ms = sum(ev[2].elapsed_time(ev[3]) * ev[4] for ev in self.events)
        by_k: dict = {}
        for t, b, e0, e1, share in self.events:
            d = by_k.setdefault(f"K{b}", [0, 0, 0.0, 0.0])
            d[0] += 1
            d[1] += t
            d[2] += e0.elapsed_time(e1)
            d[3] += e0.elapsed_time(e1) * share
        return {"launches": len(self.events), "tiles": tiles, "ms": ms, "gpu_ms": gpu_ms,
                "by_rate": {k: {"launches": v[0], "tiles": v[1], "ms": round(v[2], 3), "gpu_ms": round(v[3], 3)}
                            for k, v in sorted(by_k.items())}}


def layer_sources(device, experts, counts) -> list[dict]:
    return [expert_source(5, device, expert=e, tokens=counts[e]) for e in experts]


def layer_bench(steps: int, warmup: int, experts: int = LAYER_EXPERTS):
    """The headline: the whole config-5 layer, encoded in ``steps`` timed
    steps of consecutive experts after ``warmup`` encodes of a warm-up
    expert, then decoded to bf16.  ``experts`` < 384 encodes only the first
    experts of the same routed layer (shorter profiling passes)."""

    from qsrt_amd import exl3_encoder_backend as be

    dev = torch.device("cuda:0")
    counts = zipf_token_counts()
    experts = max(1, min(experts, LAYER_EXPERTS))
    steps = max(1, min(steps, experts))
    bounds = [experts * i // steps for i in range(steps + 1)]
    log(f"[bench] layer inputs: {experts} experts x bf16 gate/up/down + {sum(counts[:experts])} routed rows, to HBM")
    t0 = time.perf_counter()
    sources = layer_sources(dev, range(experts), counts)
    warm = expert_source(5, dev, expert=LAYER_EXPERTS, tokens=max(counts))
    torch.cuda.synchronize()
    log(f"[bench] layer inputs ready in {time.perf_counter() - t0:.1f} s")

    warm_enc = ExpertEncoder(dev, hidden=LAYER_HIDDEN, inter=LAYER_INTER, record_bits=LAYER_RECORD_BITS,
                             scope=("bench-warmup", LAYER_ID))
    for i in range(warmup):
        t0 = time.perf_counter()
        warm_enc.encode([warm])
        torch.cuda.synchronize()
        log(f"[bench] warmup {i}: 1 expert in {time.perf_counter() - t0:.2f} s")
    enc = ExpertEncoder(dev, hidden=LAYER_HIDDEN, inter=LAYER_INTER, record_bits=LAYER_RECORD_BITS)
    for key in [k for k in be._SHARED_INPUT_SCALES if k[0] == enc.scope]:
        del be._SHARED_INPUT_SCALES[key]

    encoded: list = []
    step_s = []
    with ViterbiLaunchTimer() as timer:
        torch.cuda.synchronize()
        timer.active = True
        t_start = time.perf_counter()
        for s in range(steps):
            ts = time.perf_counter()
            group = sources[bounds[s]:bounds[s + 1]]
            for b0 in range(0, len(group), MAX_BATCH_EXPERTS):
                batch = group[b0:b0 + MAX_BATCH_EXPERTS]
                encoded += enc.encode(batch, keep_states=(0,))
            torch.cuda.synchronize()
            step_s.append(time.perf_counter() - ts)
            log(f"[bench] step {s}: experts {bounds[s]}..{bounds[s + 1] - 1} in {step_s[-1]:.2f} s")
        torch.cuda.synchronize()
        wall = time.perf_counter() - t_start
        timer.active = False
        vit = timer.summary()
    weights = experts * 3 * LAYER_HIDDEN * LAYER_INTER
    proxies = [e[m]["proxy"] for e in encoded for m in ("w1", "w3", "w2")]
    del sources
    return {"wall": wall, "steps": steps, "experts": experts, "step_s": step_s, "weights": weights, "viterbi": vit, "encoded": encoded,
            "first_step_experts": bounds[1],
            "proxy_mean": sum(proxies) / len(proxies), "proxy_max": max(proxies), "warm": warm, "counts": counts}


def layer_streamed(lay: dict) -> dict:
    """BASELINE's "work is streamed from host", measured on the layer's first
    step: the same experts with their bf16 gate/up/down and routed
    calibration rows in pinned host memory, uploaded to HBM inside the timed
    region, then encoded exactly as the resident step was.  The upload is
    not overlapped with the encode (a side-stream upload of step i + 1 during
    step i would hide it); the line reports its share."""

    dev = torch.device("cuda:0")
    n = lay["first_step_experts"]
    host = []
    for e in range(n):
        src = expert_source(5, dev, expert=e, tokens=lay["counts"][e])
        host.append({"expert": src["expert"], "tokens": src["tokens"],
                     "w": tuple(t.cpu().pin_memory() for t in src["w"]), "x": src["x"].cpu().pin_memory(),
                     "gates": src["gates"].cpu().pin_memory()})
        del src
    torch.cuda.synchronize()
    nbytes = sum(t.numel() * t.element_size() for h in host for t in (*h["w"], h["x"], h["gates"]))
    enc = ExpertEncoder(dev, hidden=LAYER_HIDDEN, inter=LAYER_INTER, record_bits=LAYER_RECORD_BITS,
                        scope=("bench-streamed", LAYER_ID))
    from qsrt_amd import exl3_encoder_backend as be
    for key in [k for k in be._SHARED_INPUT_SCALES if k[0] == enc.scope]:
        del be._SHARED_INPUT_SCALES[key]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    srcs = [{"expert": h["expert"], "tokens": h["tokens"], "w": tuple(t.to(dev, non_blocking=True) for t in h["w"]),
             "x": h["x"].to(dev, non_blocking=True), "gates": h["gates"].to(dev, non_blocking=True)} for h in host]
    torch.cuda.synchronize()
    upload = time.perf_counter() - t0
    for b0 in range(0, n, MAX_BATCH_EXPERTS):
        enc.encode(srcs[b0:b0 + MAX_BATCH_EXPERTS])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    weights = n * 3 * LAYER_HIDDEN * LAYER_INTER
    resident = lay["step_s"][0]
    return {"workload": f"the layer's first step ({n} experts) with its sources in pinned host memory, uploaded inside "
                        "the timed region, then encoded",
            "M_weights_per_s": round(weights / wall / 1e6, 3), "seconds": round(wall, 3),
            "upload_seconds": round(upload, 4), "upload_bytes": nbytes, "upload_GB_per_s": round(nbytes / upload / 1e9, 2),
            "resident_seconds": round(resident, 3), "resident_M_weights_per_s": round(weights / resident / 1e6, 3)}


def layer_store(encoded: list, directory: str) -> dict:
    """Write the encoded layer as a rate-record layer file (every expert's
    atoms assembled on the GPU, written one expert at a time), read every
    expert back and check the payloads and scales are the encoder's, byte
    for byte.  Returns the file's facts and the read-back matrices (on the
    GPU) for the decode."""

    from qsrt_amd.qsrt import Geometry
    from qsrt_amd.qsrt_rate_atoms import (SCHEMA, QSRTRateLayerLayout, QSRTRateLayerReader, RateSchedule,
                                          materialize_rate_layer)

    dev = torch.device("cuda:0")
    sched = RateSchedule(Geometry(LAYER_INTER, LAYER_HIDDEN), LAYER_RECORD_BITS)
    layout = QSRTRateLayerLayout(LAYER_ID, sched, tuple(e["expert"] for e in encoded))
    path = Path(directory) / f"qsrt-layer-{LAYER_ID:05d}.safetensors"

    def experts():
        for e in encoded:
            yield e["expert"], {m: {"trellis": e[m]["words"], "suh": e[m]["suh"], "svh": e[m]["svh"]}
                                for m in ("w1", "w3", "w2")}

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    info = materialize_rate_layer(path, layout, experts())
    t_write = time.perf_counter() - t0
    t0 = time.perf_counter()
    mats, same = [], True
    with QSRTRateLayerReader(path) as rd:
        for e in encoded:
            parts = rd.read_expert(e["expert"], device=dev)
            for m in ("w1", "w3", "w2"):
                p, r = parts[m], e[m]
                same &= bool(torch.equal(p["trellis"], r["words"]) and torch.equal(p["suh"], r["suh"])
                             and torch.equal(p["svh"], r["svh"]))
                mats.append((p["trellis"], p["suh"], p["svh"], r["rate_axis"], r["shape"]))
    torch.cuda.synchronize()
    t_read = time.perf_counter() - t0
    path.unlink()
    if not same:
        raise RuntimeError("the layer file did not read back as the encoder's payloads")
    return {"facts": {"schema": SCHEMA, "experts": info["experts"], "disk_bytes": info["disk_bytes"],
                      "payload_bytes": info["payload_bytes"], "write_s": round(t_write, 2),
                      "read_s": round(t_read, 2), "read_back_equal": same}, "mats": mats}


def layer_decode(mats: list, reps: int = 3) -> dict:
    """Decode every packed matrix of the layer to bf16 (one prepared plan,
    one launch per rate), HIP events on the launch stream.  ``mats``:
    ``(record-major words, suh, svh, rate axis, (K, N))`` per matrix, on the
    GPU."""

    from qsrt_amd.decode import DecodePlan
    from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

    dev = torch.device("cuda:0")
    payloads, outs = [], []
    for words, suh, svh, axis, (k, n) in mats:
        out = torch.empty((k, n), dtype=torch.bfloat16, device=dev)
        outs.append(out)
        payloads.append((words, LAYER_RECORD_BITS, axis, (suh.float() / 128.0).contiguous(), svh.float().contiguous(),
                         out))
    plan = DecodePlan.for_records(payloads, {b: sqg_xor_cheb_t12_bytes(b).to(dev) for b in set(LAYER_RECORD_BITS)})
    plan.run()
    torch.cuda.synchronize()
    ms = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        plan.run()
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    n_mat = len(payloads)
    weights = n_mat * LAYER_HIDDEN * LAYER_INTER
    bpw = sum(LAYER_RECORD_BITS) / len(LAYER_RECORD_BITS)
    byts = weights * (bpw / 8 + 2) + n_mat * (LAYER_HIDDEN + LAYER_INTER) * 4
    t = sum(ms) / len(ms) / 1e3
    del plan, payloads, outs
    torch.cuda.empty_cache()
    return {
        "workload": f"the stored config-5 layer read back from its layer file: {n_mat} packed matrices "
                    f"({n_mat // 3} experts x gate, up, down), records {LAYER_RECORD_BITS.count(3)} K3 + "
                    f"{LAYER_RECORD_BITS.count(4)} K4 ({bpw:.3f} trellis bpw) -> bf16",
        "kernel": "decode_block_wave_kernel (one launch per rate)",
        "ms": round(t * 1e3, 3),
        "G_weights_per_s": round(weights / t / 1e9, 2),
        "roofline": {
            "bound": "hbm", "achieved": round(byts / t / 1e9, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(byts / t / 1e9 / HBM_PEAK_GBPS, 4), "traffic": round(byts * DECODE_TRAFFIC_OVER_ALGORITHMIC),
            "traffic_note": TRAFFIC_NOTE.format("profiles/decode_kernel_layer.md"),
            "algorithmic": f"{bpw:.3f}/8 B payload + 2 B bf16 out per weight + (K + N) f32 scales per matrix "
                           f"= {byts:.4g} B per layer (both launches)",
        },
    }


# ---------------------------------------------------------------------------
# CPU baseline and parity on a sample of the layer
# ---------------------------------------------------------------------------


def cpu_model() -> str:
    """The host CPU's model name (``/proc/cpuinfo``, what ``lscpu`` prints)."""

    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _sign_draw(n: int, seed: int):
    g = torch.Generator().manual_seed(int(seed))
    return (torch.randn(n, generator=g).sign() + 1e-5).sign().double().numpy()


def layer_cpu_sample(first: dict, source: dict, blocks: int = 160) -> dict:
    """The CPU oracle on the layer's first expert, w1, over the bottom
    ``blocks`` 16-row blocks -- the first steps of the backward recursion,
    which depend on nothing above them.  Two comparisons with the GPU's
    states for the same rows:

    * recursion: the float64 BlockLDLQ with the C Viterbi, fed the GPU's
      regularised weight and block-LDL factor (this is the timed CPU
      baseline: the recursion is the per-weight work);
    * end to end: the same recursion after the oracle's own float64 Hessian
      preparation, conditioned congruence (layer-shared input profile, scale
      in sv) and block LDL from the captured ``X^T X``."""

    import numpy as np

    from oracle import encode as oenc
    from oracle import ldlq as oldlq
    from oracle import tables as otables
    from oracle import viterbi as ov
    from qsrt_amd import gemm
    from qsrt_amd.qsrt_coupled import CoupledHadamardSpec, coupled_execution, encode_coupled_weights

    dev = torch.device("cuda:0")
    rows = 16 * blocks
    kt, nt = LAYER_HIDDEN // 16, LAYER_INTER // 16
    tile_bits = np.tile(np.array([b for b in LAYER_RECORD_BITS for _ in range(8)]), (blocks, 1))
    labels = {b: otables.t12_values(b) for b in (3, 4)}
    lags = {3: 1, 4: 1}
    threads = ov.default_threads()
    r = first["w1"]
    gpu_states = r["encoded"][kt - blocks:].cpu().numpy().view(np.uint16)
    W_gpu = r["W_r"][-rows:].double().cpu().numpy()
    L_gpu = r["L"][-rows:, -rows:].double().cpu().numpy()
    t0 = time.perf_counter()
    rec = oenc.blockldlq(W_gpu, L_gpu, tile_bits, labels, lags, threads=threads)
    t_rec = time.perf_counter() - t0
    rec_stats = oenc.compare_states(gpu_states, rec, labels, tile_bits, lags)

    spec = CoupledHadamardSpec()
    w = tuple(t.float() for t in source["w"])
    g_c, u_c, d_c = encode_coupled_weights(w, spec)
    ex = coupled_execution((g_c, u_c, d_c), spec)
    h13 = ex.transform_h13(gemm.gram_(torch.zeros((LAYER_HIDDEN, LAYER_HIDDEN), device=dev), source["x"]))
    W = g_c.T.contiguous().double().cpu().numpy()
    qa = r["quant_args"]
    su_s, sv_s = _sign_draw(LAYER_HIDDEN, qa["seed"]), _sign_draw(LAYER_INTER, qa["sv_seed"])
    t0 = time.perf_counter()
    H = oenc.prepare_hessian(h13.double().cpu().numpy(), source["tokens"], 0.01)
    profile = oldlq.input_rms(W, sv_s)  # the layer's first w1 sets the shared profile
    W_r, su, _ = oldlq.regularize(W, su_s, sv_s, r["g_scale"], g_into_sv=True, input_scales=profile)
    H_c, L0 = oenc.factor(H, su)
    t_prep = time.perf_counter() - t0
    e2e = oenc.blockldlq(W_r[-rows:], L0[-rows:, -rows:], tile_bits, labels, lags, threads=threads)
    e2e_stats = oenc.compare_states(gpu_states, e2e, labels, tile_bits, lags)
    n_w = rows * LAYER_INTER

    def parity(stats, what):
        return {"what": what, "tiles": stats["tiles"], "tiles_differing": stats["differ"],
                "mismatch_rate": stats["mismatch_rate"], "near_tie_tiles": len(stats["first"]),
                "max_near_tie_sse_rel": float(max(stats["sse_rel_deltas"], default=0.0)),
                "boundary_ties": stats["kinds"].count("boundary"),
                "max_boundary_margin": float(max(stats["boundary_margins"], default=0.0))}

    return {
        "cpu": {"value": round(n_w / t_rec / 1e6, 5), "unit": "M weights/s", "cores": threads, "kind": "port",
                "model": cpu_model(),
                "sample": f"expert 0 w1 of the layer ({source['tokens']} routed rows), the bottom {blocks} of {kt} "
                          f"16-row blocks ({blocks * nt} tiles, {n_w} weights): the float64 BlockLDLQ of "
                          f"oracle/encode.py with oracle/viterbi_ref.c (AVX2) on {threads} OpenMP threads at the "
                          f"layer's record rates; the Hessian preparation and factorisation ({t_prep:.1f} s per matrix in "
                          "float64) and the global-scale search (about 22% more tile encodes on the GPU) are not "
                          "charged, so the CPU rate is an upper bound",
                "seconds": round(t_rec, 2)},
        "parity": {
            "sample": f"expert 0 w1, bottom {blocks} row blocks ({blocks * nt} tiles, K3 and K4 records)",
            "recursion": parity(rec_stats, "CPU BlockLDLQ + C Viterbi on the GPU's regularised weight and factor"),
            "end_to_end": parity(e2e_stats, "CPU float64 preparation, congruence, block LDL, regularisation and "
                                            "BlockLDLQ from the captured X^T X and the source weight"),
        },
    }


# ---------------------------------------------------------------------------
# Secondary lines
# ---------------------------------------------------------------------------


def _time_ms(fn, steps: int, min_ms: float = 2.0, warm_ms: float = 100.0) -> float:
    """Mean duration of ``fn`` over at least ``steps`` launches, HIP events on
    the current stream (the stream the kernels are launched on).  Short
    kernels get enough launches to fill ``min_ms`` of GPU time, so the mean
    is the kernel's own duration rather than launch latency; about
    ``warm_ms`` of untimed launches come first, so the clocks have left
    their idle state (the first ~20 launches of a 1 ms kernel after an idle
    gap run up to 40% slower)."""

    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    one = max(e0.elapsed_time(e1), 1e-3)
    for _ in range(min(500, math.ceil(warm_ms / one))):
        fn()
    torch.cuda.synchronize()
    reps = max(steps, min(2000, math.ceil(min_ms / one)))
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def microbench(tiles_n: int = 65536, steps: int = 3, rates=(2, 3, 4)) -> dict:
    """65,536 iid N(0,1) tiles, identity Hessian, no
    feedback, at K2, K3 and K4; a step is the tile Viterbi plus the packing
    of its states into the EXL bitstream."""

    from qsrt_amd.qsrt import pack_trellis_edges
    from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes
    from qsrt_amd.sqg_quantizer import boundary_lag, viterbi_tiles

    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(20261201 + 2)
    tiles = torch.randn((tiles_n, 256), generator=gen, dtype=torch.float32).to(dev)
    out = {}
    for b in rates:
        lut = sqg_xor_cheb_t12_bytes(b).to(dev)
        buf = (torch.empty_like(tiles), torch.empty(tiles.shape, dtype=torch.int16, device=dev))
        lag = boundary_lag(b, 6.5)

        def step():
            viterbi_tiles(tiles, lut, b, tailbite_context=CONTEXT, lag=lag, out=buf)
            return pack_trellis_edges(buf[1], b)

        step()
        torch.cuda.synchronize()
        ev = []
        for _ in range(steps):
            e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            e0.record()
            viterbi_tiles(tiles, lut, b, tailbite_context=CONTEXT, lag=lag, out=buf)
            e1.record()
            pack_trellis_edges(buf[1], b)
            e2.record()
            ev.append((e0, e1, e2))
        torch.cuda.synchronize()
        vit = sum(a.elapsed_time(c) for a, c, _ in ev) / steps
        tot = sum(a.elapsed_time(d) for a, _, d in ev) / steps
        fl = tiles_n * 256 * EDGES_PER_WEIGHT * FLOPS_PER_EDGE
        out[f"K{b}"] = {"ms_viterbi": round(vit, 3), "ms_step": round(tot, 3),
                        "M_weights_per_s": round(tiles_n * 256 / (tot / 1e3) / 1e6, 2),
                        "viterbi_TFLOPs": round(fl / (vit / 1e3) / 1e12, 2)}
    del tiles
    torch.cuda.empty_cache()
    return {"workload": f"config 2 microbench: {tiles_n} iid N(0,1) tiles x 256, C = 128, Viterbi + EXL packing per "
                        "step", **out}


def microbench_cpu(bits: int = 3, seconds: float = 6.0) -> dict:
    """The C oracle on the microbench's first tiles at one rate."""

    import numpy as np

    from oracle import tables as otables
    from oracle import viterbi as ov

    threads = ov.default_threads()
    tiles = torch.randn((max(threads, 64) * 8, 256), generator=torch.Generator().manual_seed(20261201 + 2)).numpy()
    lab = otables.t12_values(bits)
    ov.encode(tiles[:threads], lab, K=bits, boundary_lag=1, threads=threads)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        ov.encode(tiles, lab, K=bits, boundary_lag=1, threads=threads)
        n += len(tiles)
    per_tile = (time.perf_counter() - t0) / n
    return {"value": round(256 / per_tile / 1e6, 4), "unit": "M weights/s", "cores": threads, "model": cpu_model(),
            "ms_per_tile": per_tile * 1e3,
            "sample": f"{n} microbench tiles at K{bits}, oracle/viterbi_ref.c (AVX2) with {threads} OpenMP threads"}


def expert_bench(bits: int = 3, reps: int = 2) -> dict:
    """BASELINE config 4 shape at K3 (the north-star target): one coupled
    Kimi-class expert, all three matrices, LDLQ, H2 from the reconstructed
    activations, through the layer pipeline with uniform records."""

    dev = torch.device("cuda:0")
    src = expert_source(4, dev)
    enc = ExpertEncoder(dev, hidden=LAYER_HIDDEN, inter=LAYER_INTER, record_bits=(bits,) * (LAYER_INTER // 128),
                        scope=("bench-expert", bits))
    times = []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        res = enc.encode([src])[0]
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    weights = 3 * LAYER_HIDDEN * LAYER_INTER
    return {"workload": f"config 4: Kimi-class coupled expert 7168 x 2048 SwiGLU, all three matrices, K{bits}, LDLQ, "
                        "H2 from reconstructed activations, 16,384 calibration rows",
            "seconds": round(times[-1], 3), "seconds_first": round(times[0], 3),
            "M_weights_per_s": round(weights / times[-1] / 1e6, 2),
            "proxy_err": {m: round(res[m]["proxy"], 5) for m in ("w1", "w3", "w2")}}


def glm_expert_bench(reps: int = 2) -> dict:
    """the GLM-class SwiGLU expert (hidden 5120, inter
    1536) at K3 with 8 outlier channels, 128-block Hadamard rotation, H13
    from 8192 AR(1) rows (rho 0.9) and H2 from the source SwiGLU
    activations, all three matrices through ``quantize_qsrt_batch``."""

    from qsrt_amd import exl3_encoder_backend as be
    from qsrt_amd import gemm
    from qsrt_amd.ldlq import make_shared_h
    from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes
    from qsrt_amd.transform_seeds import default_qsrt_transform_seeds

    dev = torch.device("cuda:0")
    d = config_expert(3, dev)
    hidden, inter, x = d["hidden"], d["inter"], d["x"]
    luts = {b: sqg_xor_cheb_t12_bytes(b) for b in (2, 3, 4)}

    def qa(matrix, k, n):
        seeds = default_qsrt_transform_seeds(1, matrix)
        axis = "k" if matrix == "w2" else "n"
        return {"K": 3, "seed": seeds.input_sign, "sv_seed": seeds.output_sign, "sigma_reg": 0.01,
                "devices": [str(dev)], "apply_out_scales": False, "tailbite_context": CONTEXT,
                "sqg_e4m3_luts_by_bits": luts, "mixed_rate_axis": axis,
                "mixed_tile_bits": (3,) * ((k if axis == "k" else n) // 16)}

    times, proxies = [], {}
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        h13 = gemm.gram_(torch.zeros((hidden, hidden), device=dev), x)
        h = (torch.nn.functional.silu(x @ d["w_gate"].T) * (x @ d["w_up"].T)).contiguous()
        h2 = gemm.gram_(torch.zeros((inter, inter), device=dev), h)
        del h
        ws, hs, qas = [], [], []
        for matrix, w, H in (("w1", d["w_gate"], h13), ("w3", d["w_up"], h13)):
            shared = make_shared_h(hidden, dev, H)
            shared["count"] = x.shape[0]
            ws.append(w.T.contiguous())
            hs.append(shared)
            qas.append([qa(matrix, hidden, inter)])
        up = be.quantize_qsrt_batch(ws, hs, qas, return_weight_q=False)
        shared = make_shared_h(inter, dev, h2)
        shared["count"] = x.shape[0]
        down = be.quantize_qsrt_batch([d["w_down"].T.contiguous()], [shared], [[qa("w2", inter, hidden)]],
                                      return_weight_q=False)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        proxies = {"w1": up[0][0]["proxy"], "w3": up[1][0]["proxy"], "w2": down[0][0]["proxy"]}
    weights = 3 * hidden * inter
    return {"workload": "config 3: GLM-class SwiGLU expert, gate/up [5120 x 1536] and down [1536 x 5120], K3, "
                        "8 outlier channels (20x variance), H13 from 8192 AR(1) rows (rho 0.9), H2 from the source "
                        "SwiGLU activations, 128-block Hadamard, BlockLDLQ",
            "seconds": round(times[-1], 3), "seconds_first": round(times[0], 3),
            "M_weights_per_s": round(weights / times[-1] / 1e6, 2),
            "proxy_err": {m: round(v, 5) for m, v in proxies.items()}}


def k2_expert_bench(reps: int = 2) -> dict:
    """BASELINE config 4 as specified: the coupled Kimi-class expert at K2
    (one fp16 suh and svh vector per matrix, about 2.01 bpw all told)."""

    dev = torch.device("cuda:0")
    src = expert_source(4, dev)
    enc = ExpertEncoder(dev, hidden=LAYER_HIDDEN, inter=LAYER_INTER, record_bits=(2,) * (LAYER_INTER // 128),
                        scope=("bench-expert", 2))
    times = []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        res = enc.encode([src])[0]
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    weights = 3 * LAYER_HIDDEN * LAYER_INTER
    bits = sum(res[m]["words"].numel() * 16 + 16 * (res[m]["suh"].numel() + res[m]["svh"].numel())
               for m in ("w1", "w3", "w2"))
    return {"workload": "config 4: coupled Kimi-class expert 7168 x 2048 SwiGLU at K2, all three matrices, LDLQ, "
                        "H2 from reconstructed activations, fp16 suh/svh vectors",
            "seconds": round(times[-1], 3), "seconds_first": round(times[0], 3),
            "M_weights_per_s": round(weights / times[-1] / 1e6, 2), "bpw": round(bits / weights, 5),
            "proxy_err": {m: round(res[m]["proxy"], 5) for m in ("w1", "w3", "w2")}}


def gemm_bench(steps: int = 20):
    """The MFMA GEMM shapes of the config-4 expert encode: Hessian capture
    ``H += X^T X`` of 16,384 bf16 tokens x 7168 channels, and one LDLQ span
    update ``P[:begin] += L[span, :begin]^T (W - Q)[span]`` (M = 7040,
    K = 128, N = 2048) on the float64 matrix cores as the encoder runs it
    (float64 L, W and P, FP32 Q) and, for the two-sided recursion's FP32
    contract, on the FP32 ones; and the layer's batched form (40 members,
    M = 3584), one launch as the batched recursion issues it."""

    from qsrt_amd import gemm

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(20261201 + 6)
    n, k = 16384, 7168
    X = torch.randn((n, k), device=dev, generator=g).to(torch.bfloat16)
    H = torch.zeros((k, k), device=dev)
    ms_h = _time_ms(lambda: gemm.gram_(H, X, 1.0 / n), steps)
    fl_h = 1.0 * n * k * (k + 1)  # symmetric rank-n update: one triangle computed, the other mirrored
    del X, H
    m, kk, nn = 7040, 128, 2048
    L = torch.randn((kk, m), device=dev, generator=g)
    W = torch.randn((kk, nn), device=dev, generator=g)
    Q = torch.randn((kk, nn), device=dev, generator=g)
    P = torch.zeros((m, nn), device=dev)
    ms_l = _time_ms(lambda: gemm.addmm_sub_tn_(P, L, W, Q), steps)
    fl_l = 2.0 * m * kk * nn
    L64, W64, P64 = L.double(), W.double(), P.double()
    ms_l64 = _time_ms(lambda: gemm.addmm_sub_tn_(P64, L64, W64, Q), steps)
    del L, W, Q, P, L64, W64, P64
    torch.cuda.empty_cache()
    # the layer's batched span update: the 40 gate/up members of a 20-expert step in one launch, at the
    # middle of the recursion (M = begin = 3584 rows still to update)
    nb, mb = 40, 3584
    Lb = torch.randn((nb, kk, mb), device=dev, generator=g, dtype=torch.float64)
    Wb = torch.randn((nb, kk, nn), device=dev, generator=g, dtype=torch.float64)
    Qb = torch.randn((nb, kk, nn), device=dev, generator=g)
    Pb = torch.zeros((nb, mb, nn), device=dev, dtype=torch.float64)
    ms_lb = _time_ms(lambda: gemm.baddmm_sub_tn_f64_(Pb, Lb, Wb, Qb), steps)
    fl_lb = 2.0 * nb * mb * kk * nn
    del Lb, Wb, Qb, Pb
    torch.cuda.empty_cache()

    def line(key, name, ms, fl, dtype, shape, what):
        t = fl / (ms / 1e3) / 1e12
        acc = "f64" if dtype == "f64" else "f32"
        traffic = GEMM_HBM_BYTES.get(key)
        return {"kernel": name, "shape": shape, "ms": round(ms, 4), "roofline": {
            "bound": "mfma", "achieved": round(t, 1), "peak": MFMA_PEAK_TFLOPS[dtype], "unit": "TFLOP/s",
            "frac": round(t / MFMA_PEAK_TFLOPS[dtype], 4), "traffic": None if traffic is None else round(traffic),
            "traffic_note": (TRAFFIC_NOTE.format("profiles/gemm_tn_kernels_expert_shapes.md") if traffic is not None
                             else "not profiled"),
            "algorithmic": f"{what} = {fl:.4g} flops/launch ({dtype} in, {acc} accumulate)"}}

    return {
        "hessian_capture": line("hessian_capture", "gemm_tn_bf16_kernel", ms_h, fl_h, "bf16",
                                f"X [{n} x {k}] bf16 -> H [{k} x {k}] f32", "n k (k + 1) (symmetric)"),
        "ldlq_span_update": line("ldlq_span_update_f64", "gemm_tn_f64_kernel", ms_l64, fl_l, "f64",
                                 f"L^T [{m} x {kk}] (W - Q) [{kk} x {nn}] f64 (Q f32)", "2 M N K"),
        "ldlq_span_update_f32": line("ldlq_span_update", "gemm_tn_f32_kernel", ms_l, fl_l, "f32",
                                     f"L^T [{m} x {kk}] (W - Q) [{kk} x {nn}] f32", "2 M N K"),
        "ldlq_span_update_batched": line("ldlq_span_update_batched_f64", "gemm_tn_f64_kernel (batched)", ms_lb, fl_lb,
                                         "f64", f"{nb} members L^T [{mb} x {kk}] (W - Q) [{kk} x {nn}] f64 (Q f32)",
                                         "2 batch M N K"),
    }


def hadamard_bench(steps: int = 5):
    """Block-128 rotation of a 7168 x 2048 FP32 matrix along each axis with
    fused sign vectors (the ``su``/``sv`` sides of the expert's rotation):
    8 B per element per launch."""

    from qsrt_amd.hadamard import rotate_

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(20261201 + 7)
    k, n = 7168, 2048
    W = torch.randn((k, n), device=dev, generator=g)
    su = torch.randint(0, 2, (k,), device=dev, generator=g).float() * 2 - 1
    sv = torch.randint(0, 2, (n,), device=dev, generator=g).float() * 2 - 1
    out = {}
    for side, vec in (("left", su), ("right", sv)):
        ms = _time_ms(lambda: rotate_(W, 128, side=side, pre_mul=vec), steps)
        gbps = 8.0 * k * n / (ms / 1e3) / 1e9
        out[side] = {"kernel": "hadamard_kernel", "ms": round(ms, 4), "roofline": {
            "bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": round(HADAMARD_HBM_BYTES[side]),
            "traffic_note": TRAFFIC_NOTE.format("profiles/hadamard_kernel_expert_matrix.md"),
            "algorithmic": f"8 B/element x {k * n} elements/launch"}}
    del W
    torch.cuda.empty_cache()
    return {"workload": f"[{k} x {n}] f32, block 128, fused signs, in place", **out}


def _bakron_band_flops(ob: int, ib: int, first: int, middle: int, last: int, block_lower: bool = False) -> int:
    """Algorithmic flops of one fused band update: 2 * 16^3 per (target block,
    source block) pair of the left and right products (with ``block_lower``,
    the left pairs whose output-factor block is not a zero block above the
    diagonal)."""

    pairs = 0
    for d in range(first, last):
        for o in range(max(0, d - ib + 1), min(ob, d + 1)):
            i = d - o
            s_end = min(ob, middle - i, o + 1) if block_lower else min(ob, middle - i)
            pairs += max(0, s_end - max(0, first - i))
            if d >= middle:
                pairs += max(0, min(ib, middle, last - o) - max(0, first - o))
    return 2 * 16 ** 3 * pairs


def bakron_bench(steps: int = 5):
    """BaKron band propagation on the config-4 gate (weights [7168, 2048] in
    the encoder orientation: 2048 output x 7168 input rows of 16 x 16 blocks,
    575 anti-diagonals).  The top band of the divide and conquer (diagonals
    [0, 287) into [287, 575)) is the roofline line (FP32 matrix cores); the
    whole recursion's 574 band updates are timed back to back, on the HIP
    kernel and on the bounding-box torch products."""

    from qsrt_amd.sqg_quantizer import apply_bakron_block_update
    from qsrt_amd.two_sided_rounding import _propagate_band

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(20261201 + 11)
    n_out, n_in = 2048, 7168
    ob, ib = n_out // 16, n_in // 16
    diagonals = ob + ib - 1
    T = torch.randn((n_out, n_in), device=dev, generator=g)
    Q = torch.round(T * 4) / 4
    l_out = torch.randn((n_out, n_out), device=dev, generator=g) / n_out ** 0.5
    l_in = torch.randn((n_in, n_in), device=dev, generator=g) / n_in ** 0.5
    l_out = l_out * torch.kron(torch.tril(torch.ones(ob, ob, device=dev)), torch.ones(16, 16, device=dev))
    l_in = l_in * torch.kron(torch.tril(torch.ones(ib, ib, device=dev)), torch.ones(16, 16, device=dev))
    inter = torch.empty_like(T)
    bands = []

    def rec(first, last):
        if last == first + 1:
            return
        mid = (first + last) // 2
        rec(first, mid)
        bands.append((first, mid, last))
        rec(mid, last)

    rec(0, diagonals)
    top = (0, diagonals // 2, diagonals)

    def hip(band):
        apply_bakron_block_update(T, Q, l_out, l_in, inter, first_diagonal=band[0], middle_diagonal=band[1],
                                  last_diagonal=band[2], block_size=16)

    top_ms = _time_ms(lambda: hip(top), steps)
    top_flops = _bakron_band_flops(ob, ib, *top)
    achieved = top_flops / (top_ms / 1e3) / 1e12

    def hip_lower(band):
        apply_bakron_block_update(T, Q, l_out, l_in, inter, first_diagonal=band[0], middle_diagonal=band[1],
                                  last_diagonal=band[2], block_size=16, block_lower=True)

    lower_ms = _time_ms(lambda: hip_lower(top), steps)
    lower_flops = _bakron_band_flops(ob, ib, *top, block_lower=True)

    def all_hip():
        for band in bands:
            hip(band)

    def all_torch():
        for band in bands:
            _propagate_band(T, Q, l_out, l_in, first=band[0], middle=band[1], last=band[2], block_size=16)

    all_ms = _time_ms(all_hip, 2, min_ms=0.0, warm_ms=0.0)
    all_flops = sum(_bakron_band_flops(ob, ib, *b) for b in bands)
    torch_ms = _time_ms(all_torch, 2, min_ms=0.0, warm_ms=0.0)
    del T, Q, l_out, l_in, inter
    torch.cuda.empty_cache()
    return {"workload": f"{n_out} x {n_in} FP32 (config-4 gate, encoder orientation), 16 x 16 blocks, "
                        f"{diagonals} anti-diagonals",
            "kernel": "bakron_left_kernel + bakron_right_kernel",
            "top_band": {"diagonals": list(top), "ms": round(top_ms, 4), "roofline": {
                "bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / FP32_PEAK_TFLOPS, 4), "traffic": round(BAKRON_TOP_BAND_HBM_BYTES),
                "traffic_note": TRAFFIC_NOTE.format("profiles/bakron_band_kernels_config4_gate.md"),
                "algorithmic": f"2 x 16^3 flops per (target, source) block pair x {top_flops // 8192} pairs"},
                "block_lower": {"ms": round(lower_ms, 4),
                                "tflops": round(lower_flops / (lower_ms / 1e3) / 1e12, 2),
                                "pairs": lower_flops // 8192}},
            "recursion": {"bands": len(bands), "hip_ms": round(all_ms, 3), "torch_bounding_box_ms": round(torch_ms, 3),
                          "hip_tflops": round(all_flops / (all_ms / 1e3) / 1e12, 2)}}


def copy_calibration(nbytes: int) -> None:
    """A plain device copy of ``nbytes`` (the known-size reference for the
    HBM byte counters)."""

    x = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda:0").fill_(1.0)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    y.copy_(x)
    torch.cuda.synchronize()
    log(f"[bench] copied {nbytes} bytes")


LINES = ("layer", "microbench", "expert", "glm", "k2", "gemm", "hadamard", "bakron")


def headline(lay: dict, warmup: int) -> dict:
    vit = lay["viterbi"]
    # a launch on a split grid holds only its share of the GPU: its duration counts at that share
    mean_launch_ms = vit["gpu_ms"] / max(vit["launches"], 1)
    mean_tiles = vit["tiles"] / max(vit["launches"], 1)
    flops_per_launch = mean_tiles * 256 * EDGES_PER_WEIGHT * FLOPS_PER_EDGE
    achieved = flops_per_launch / (mean_launch_ms / 1e3) / 1e12
    value = lay["weights"] / lay["wall"] / 1e6
    experts = lay["experts"]
    for d in vit["by_rate"].values():
        d["mean_ms"] = round(d["ms"] / max(d["launches"], 1), 4)
        d["tiles_per_launch"] = round(d["tiles"] / max(d["launches"], 1), 1)
    log(f"[bench] layer: {lay['wall']:.1f} s, {value:.2f} M weights/s; Viterbi {achieved:.1f} TFLOP/s, "
        f"{100 * vit['gpu_ms'] / 1e3 / lay['wall']:.1f}% of wall")
    return {
        "metric": "encoded weights/sec (M/s) at K=2/3 on one GPU",
        "value": round(value, 3),
        "unit": "M weights/s",
        "n_gpus": 1,
        "steps": lay["steps"],
        "warmup": warmup,
        "ms_per_step": round(lay["wall"] / lay["steps"] * 1e3, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded Student-t(5) bf16 weights (std 0.015), AR(1) rho 0.85 calibration rows",
        "config": {
            "workload": "config 5 (BASELINE configs[4]): full Kimi-class MoE layer encode, 384 experts x "
                        "(gate, up [7168 x 2048], down [2048 x 7168]), exact coupled basis, Zipf s=1.1 routing of "
                        "65,536 calibration tokens, records 14 K3 + 2 K4 per matrix, BlockLDLQ, H2 from the "
                        "reconstructed SwiGLU activations, L=16, C=128, sqg_xor_cheb_t12"
                        + ("" if experts == LAYER_EXPERTS else f" -- PARTIAL: only the first {experts} experts"),
            "experts": experts, "weights": lay["weights"], "layer_seconds": round(lay["wall"], 2),
            "experts_per_step": sorted({experts * (i + 1) // lay["steps"] - experts * i // lay["steps"]
                                        for i in range(lay["steps"])}),
        },
        "roofline": {
            "bound": "valu",
            "achieved": round(achieved, 3),
            "peak": FP32_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
            "traffic": round(sum(VITERBI_HBM_BYTES_PER_TILE[int(k[1:])] * d["tiles"] for k, d in vit["by_rate"].items())
                             / max(vit["launches"], 1)),
            "traffic_note": TRAFFIC_NOTE.format("profiles/layer_encode_config5.md"),
            "kernel": "viterbi_tiles_kernel",
            "algorithmic": f"{FLOPS_PER_EDGE} FP32 flops/edge x {int(EDGES_PER_WEIGHT)} edges/weight x 256 weights/tile "
                           f"x {mean_tiles:.1f} tiles/launch (mean over {vit['launches']} launches in the timed region)",
            "mean_launch_ms": round(mean_launch_ms, 4),
            "mean_launch_ms_note": "HIP events around every launch on its stream, each duration weighted by the share "
                                   "of the CUs its grid holds (the K3 and K4 groups of a step run side by side on "
                                   "split grids); per rate, mean_ms is the unweighted event mean",
            "launches": vit["by_rate"],
            "viterbi_share_of_wall": round(vit["gpu_ms"] / 1e3 / lay["wall"], 4),
            # The 157.3 TFLOP/s peak counts packed FP32; this build disables packed FP32 ops (a miscompare hazard
            # on this pool), which halves the vector ceiling for this instruction mix.
            "peak_without_packed_fp32": FP32_UNPACKED_PEAK_TFLOPS,
            "frac_without_packed_fp32": round(achieved / FP32_UNPACKED_PEAK_TFLOPS, 4),
        },
        "quality": {"proxy_err_mean": round(lay["proxy_mean"], 6), "proxy_err_max": round(lay["proxy_max"], 6)},
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20, help="timed steps the 384-expert layer is split into")
    ap.add_argument("--warmup", type=int, default=2, help="untimed encodes of a warm-up expert")
    ap.add_argument("--no-secondary", action="store_true", help="only the layer encode, its decode and its CPU sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default=",".join(LINES),
                    help=f"comma list of lines to run, from {','.join(LINES)} (profiling passes)")
    ap.add_argument("--experts", type=int, default=LAYER_EXPERTS,
                    help="encode only the first experts of the layer (profiling passes; the headline needs 384)")
    ap.add_argument("--tiles", type=int, default=65536, help="tiles per rate of the config-2 microbench")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a device copy of BYTES (reference for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build runs the encoder on one GPU and does not shard it "
              "across GPUs (experts would shard with no exchange; see the repository's design notes)",
              file=sys.stderr)
        return 2
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return 0
    lines = [x for x in args.only.split(",") if x]
    bad = [x for x in lines if x not in LINES]
    if bad:
        print(f"bench.py: unknown --only lines {bad}; choose from {LINES}", file=sys.stderr)
        return 2
    if args.no_secondary:
        lines = ["layer"]

    result: dict = {}
    if "layer" in lines:
        lay = layer_bench(args.steps, args.warmup, args.experts)
        result = headline(lay, args.warmup)
        value = result["value"]
        log("[bench] layer file: write, read back, compare")
        with tempfile.TemporaryDirectory(prefix="qsrt-bench-") as tmp:
            stored = layer_store(lay["encoded"], tmp)
        log(f"[bench] layer file {json.dumps(stored['facts'])}")
        log("[bench] decode of the stored layer")
        result["decode"] = layer_decode(stored["mats"])
        result["decode"]["layer_file"] = stored["facts"]
        del stored
        log(f"[bench] decode {result['decode']['ms']} ms, {result['decode']['roofline']['achieved']} GB/s")
        first = next(e for e in lay["encoded"] if "encoded" in e["w1"])
        sample_src = expert_source(5, torch.device("cuda:0"), expert=first["expert"], tokens=first["tokens"])
        del lay["encoded"]
        torch.cuda.empty_cache()
        if not args.no_cpu_baseline:
            log("[bench] CPU baseline and parity on a sample of the layer")
            cs = layer_cpu_sample(first, sample_src)
            result["cpu_baseline"] = cs["cpu"]
            result["cpu_baseline"]["gpu_speedup"] = round(value / cs["cpu"]["value"], 1)
            result["parity"] = cs["parity"]
            log(f"[bench] CPU {cs['cpu']['value']} M w/s on {cs['cpu']['cores']} threads; "
                f"parity {json.dumps(cs['parity'])}")
        del first, sample_src
        if not args.no_secondary:
            log("[bench] layer step streamed from host")
            result["streamed_from_host"] = layer_streamed(lay)
            log(f"[bench] streamed {json.dumps(result['streamed_from_host'])}")
    else:
        result = {"metric": "encoded weights/sec (M/s) at K=2/3 on one GPU", "value": None,
                  "note": f"headline not run (--only {args.only})"}
    if "microbench" in lines:
        log("[bench] config-2 microbench")
        result["microbench"] = microbench(args.tiles)
        if not args.no_cpu_baseline:
            result["microbench"]["cpu"] = microbench_cpu()
    if "expert" in lines:
        log("[bench] config-4 expert (K3)")
        result["expert_encode"] = expert_bench()
        if "cpu_baseline" in result:
            result["expert_encode"]["speedup_vs_cpu_baseline"] = round(
                result["expert_encode"]["M_weights_per_s"] / result["cpu_baseline"]["value"], 1)
    if "glm" in lines:
        log("[bench] config-3 GLM expert (K3)")
        result["glm_expert_encode"] = glm_expert_bench()
    if "k2" in lines:
        log("[bench] config-4 expert at K2")
        result["expert_encode_k2"] = k2_expert_bench()
    if "gemm" in lines:
        log("[bench] GEMM kernels")
        result["gemm"] = gemm_bench()
    if "hadamard" in lines:
        log("[bench] Hadamard kernel")
        result["hadamard"] = hadamard_bench()
    if "bakron" in lines:
        log("[bench] BaKron band update")
        result["bakron"] = bakron_bench()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
