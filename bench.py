"""QSRT encoder hot-path benchmark on one MI355X.

Workload (the Viterbi-only microbench): 65,536
independent 256-weight tiles of iid N(0,1) FP32 (seeded), identity Hessian,
no feedback, tail-bite context 128, encoded at K=2 and K=3 against the
frozen sqg_xor_cheb_t12 tables.  One "step" = both rates over the whole
batch.  Inputs are resident in HBM before the timed region.

Prints ONE JSON line:
  value      encoded weights/s (M/s) over the K2 + K3 runs
  roofline   the tile Viterbi: algorithmic FP32 flops (3 per trellis edge,
             131,072 edges per weight at C=128) / measured kernel time,
             against MI355X's 157.3 TFLOP/s FP32 peak
  cpu_baseline  the C oracle (oracle/viterbi_ref.c, OpenMP over tiles) on
             a bounded sample of the same tiles on this host's cores
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

TILES = 65536
RATES = (2, 3)
CONTEXT = 128
EDGES_PER_WEIGHT = (256 + 2 * CONTEXT) / 256 * 65536  # 131,072 at C=128
FLOPS_PER_EDGE = 3  # d = label - x (1), fma(d, d, cost) (2)
FP32_PEAK_TFLOPS = 157.3
FP32_UNPACKED_PEAK_TFLOPS = 78.6  # 256 CUs x 64 FP32 FMA lanes x 2 flops x 2.4 GHz, no packed FP32
# VALU issue-slot occupancy of viterbi_tiles_kernel by PMC (K3, K2; profiles/viterbi_tiles_kernel_microbench.md)
VITERBI_VALU_ISSUE_FRAC_PMC = {"K2": 1.06, "K3": 0.94}
# HBM bytes per tile of the Viterbi kernel (FETCH_SIZE x 2.00 + WRITE_SIZE x 1.00 per dispatch, calibrated on a
# 4 GiB device copy; profiles/viterbi_tiles_kernel_microbench.md): mostly the traceback decision stream.
VITERBI_HBM_BYTES_PER_TILE = 1.629e6
# Same counters for the decode launches: 1.013 x their algorithmic bytes (profiles/decode_kernel_layer.md).
DECODE_TRAFFIC_OVER_ALGORITHMIC = 1.013
# Same counters at the bench's GEMM and Hadamard shapes (profiles/gemm_tn_kernels_expert_shapes.md,
# profiles/hadamard_kernel_expert_matrix.md): HBM bytes per launch.
GEMM_HBM_BYTES = {"hessian_capture": 2.415e9, "ldlq_span_update": 1.485e8}
HADAMARD_HBM_BYTES = {"left": 1.1782e8, "right": 1.1765e8}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# BASELINE configs as seeded synthetic inputs
# ---------------------------------------------------------------------------


def student_t(shape, *, nu: float, std: float, gen: torch.Generator) -> torch.Tensor:
    """Student-t(nu) from N(0,1) and a chi-square built from nu normals,
    scaled to standard deviation ``std``."""

    z = torch.randn(shape, generator=gen)
    chi2 = torch.zeros(shape)
    for _ in range(int(nu)):
        chi2 += torch.randn(shape, generator=gen).square()
    t = z / torch.sqrt(chi2 / nu)
    return t * (std / math.sqrt(nu / (nu - 2.0)))


def ar1_rows(n: int, k: int, rho: float, gen: torch.Generator, device) -> torch.Tensor:
    """Rows x with x_0 = z_0, x_j = rho x_{j-1} + sqrt(1 - rho^2) z_j (Sigma_ij =
    rho^|i-j|), built on the device as Z @ T with T the AR(1) Toeplitz factor."""

    z = torch.randn((n, k), generator=gen).to(device)
    j = torch.arange(k, device=device, dtype=torch.float64)
    gap = j[None, :] - j[:, None]
    coef = torch.full((k,), math.sqrt(1.0 - rho * rho), device=device, dtype=torch.float64)
    coef[0] = 1.0
    T = torch.where(gap >= 0, coef[:, None] * torch.pow(torch.tensor(rho, device=device, dtype=torch.float64), gap.clamp(min=0)), torch.zeros((), device=device, dtype=torch.float64))
    return (z.double() @ T).float()


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


def run_expert_encode(bits: int = 3, hidden: int = 7168, inter: int = 2048, tokens: int = 16384, rho: float = 0.85, log=print):
    """BASELINE config 4 at rate ``bits``: one Kimi-class SwiGLU expert in the
    exact coupled basis (qsrt_amd.qsrt_coupled, draw 0), H13 = X^T X from
    ``tokens`` AR(1) rows (captured before the timed region, as the reference
    receives it), H2 rebuilt inside the timed region from the reconstructed
    gate/up SwiGLU activations, all three matrices encoded with BlockLDLQ.
    Returns timing and quality figures."""

    from qsrt_amd import exl3_encoder_backend as be
    from qsrt_amd.decode import decode_words
    from qsrt_amd.ldlq import make_shared_h
    from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

    from qsrt_amd import gemm
    from qsrt_amd.qsrt_coupled import CoupledHadamardSpec, coupled_execution, decode_coupled_weights, encode_coupled_weights

    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(20261201 + 4)
    w_gate = student_t((inter, hidden), nu=5, std=0.015, gen=gen).bfloat16().float().to(dev)
    w_up = student_t((inter, hidden), nu=5, std=0.015, gen=gen).bfloat16().float().to(dev)
    w_down = student_t((hidden, inter), nu=5, std=0.015, gen=gen).bfloat16().float().to(dev)
    x = ar1_rows(tokens, hidden, rho, gen, dev)
    torch.cuda.synchronize()
    spec = CoupledHadamardSpec()  # residual 512, pre/post 128, draw 0
    g_c, u_c, d_c = encode_coupled_weights((w_gate, w_up, w_down), spec)
    ex = coupled_execution((g_c, u_c, d_c), spec)
    h13 = gemm.gram_(torch.zeros((hidden, hidden), device=dev), x)  # H13 = X^T X on the FP32 matrix cores
    h13 = ex.transform_h13(h13)
    lut = sqg_xor_cheb_t12_bytes(bits)
    tiles_encoded = [0]
    real = be.quantize_tiles_multigpu

    def counting(tiles, qa):
        tiles_encoded[0] += tiles.shape[0]
        return real(tiles, qa)

    def qargs(seed, sv_seed):
        return {"K": bits, "seed": seed, "sv_seed": sv_seed, "sigma_reg": 0.01, "devices": [str(dev)],
                "apply_out_scales": False, "tailbite_context": 128, "sqg_e4m3_lut": lut}

    be.quantize_tiles_multigpu = counting
    try:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        shared13 = make_shared_h(hidden, dev, h13)
        shared13["count"] = tokens
        qa_g, qa_u = qargs(1_000_000, 1_499_979), qargs(1_000_002, 1_499_981)
        (pg, tg), (pu, tu) = be.quantize_uniform_batch([g_c.T.contiguous(), u_c.T.contiguous()], [shared13, shared13], [qa_g, qa_u])
        torch.cuda.synchronize()
        t_upstream = time.perf_counter() - t0
        # H2 from the reconstructed gate/up SwiGLU activations (source basis), then the coupled transform
        dec = lambda t: decode_words(t["trellis"], t["suh"], t["svh"], bits, lut, out_dtype=torch.float32).T
        g_hat, u_hat, _ = decode_coupled_weights((dec(tg), dec(tu), d_c), spec)
        h = (torch.nn.functional.silu(x @ g_hat.T) * (x @ u_hat.T)).contiguous()
        h2 = ex.transform_h2(gemm.gram_(torch.zeros((inter, inter), device=dev), h))
        del h
        shared2 = make_shared_h(inter, dev, h2)
        shared2["count"] = tokens
        qa_d = qargs(1_000_001, 1_499_980)
        t1 = time.perf_counter()
        _, pd, td = be.quantize_qsrt(d_c.T.contiguous(), shared2, qa_d, False)
        torch.cuda.synchronize()
        t_down = time.perf_counter() - t1
        total = time.perf_counter() - t0
    finally:
        be.quantize_tiles_multigpu = real
    weights = 3 * hidden * inter
    out = {
        "bits": bits,
        "weights": weights,
        "seconds": total,
        "seconds_upstream": t_upstream,
        "seconds_down": t_down,
        "seconds_h2_rebuild": total - t_upstream - t_down,
        "M_weights_per_s": weights / total / 1e6,
        "tile_encodes": tiles_encoded[0],
        "proxy": {"gate": pg, "up": pu, "down": pd},
        "g_scale": {"gate": qa_g["g_scale"], "up": qa_u["g_scale"], "down": qa_d["g_scale"]},
    }
    log(f"[bench] expert K{bits}: {total:.2f} s ({out['M_weights_per_s']:.1f} M w/s), {tiles_encoded[0]} tile encodes")
    return out


LAYER_EXPERTS = 384
LAYER_TOKENS = 65536
LAYER_ZIPF_S = 1.1


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


def layer_encode_bench(sample: int = 8, batch: int = 8, rho: float = 0.85):
    """BASELINE config 5 encode: ``sample`` experts of the 384-expert layer,
    ``batch`` experts per encoder batch (their gate/up traversals share tile
    launches, then their down traversals), mixed record rates (14 K3 + 2 K4
    records per matrix, the decode line's schedule), exact coupled basis,
    H13 from each expert's Zipf-routed tokens (captured before the timed
    region), H2 rebuilt in the timed region from the reconstructed SwiGLU
    activations.  The layer time is the sample's time scaled to 384 experts."""

    from types import SimpleNamespace

    from qsrt_amd import exl3_encoder_backend as be
    from qsrt_amd import gemm
    from qsrt_amd.ldlq import make_shared_h
    from qsrt_amd.qsrt_coupled import CoupledHadamardSpec, coupled_execution, decode_coupled_weights, encode_coupled_weights
    from qsrt_amd.qsrt_encoder import _qsrt_quant_args
    from qsrt_amd.transform_seeds import default_qsrt_transform_seeds

    dev = torch.device("cuda:0")
    hidden, inter = 7168, 2048
    counts = zipf_token_counts()
    # experts spread over the routing ranks (every expert of the sample has tokens)
    order = sorted(range(LAYER_EXPERTS), key=lambda e: -counts[e])
    chosen = [order[int(i * (LAYER_EXPERTS - 1) / max(sample - 1, 1))] for i in range(sample)]
    chosen = [e if counts[e] > 0 else order[0] for e in chosen]
    rate_map = tuple(b for b in DECODE_RECORD_BITS for _ in range(8))  # per 16-channel tile of the rate axis
    spec = CoupledHadamardSpec()
    gen = torch.Generator().manual_seed(20261201 + 9)
    experts = []
    for e in chosen:
        w = [student_t(shape, nu=5, std=0.015, gen=gen).bfloat16().float().to(dev)
             for shape in ((inter, hidden), (inter, hidden), (hidden, inter))]
        x = ar1_rows(max(counts[e], 1), hidden, rho, gen, dev)
        g_c, u_c, d_c = encode_coupled_weights(tuple(w), spec)
        ex = coupled_execution((g_c, u_c, d_c), spec)
        h13 = ex.transform_h13(gemm.gram_(torch.zeros((hidden, hidden), device=dev), x, 1.0 / x.shape[0]))
        experts.append({"expert": e, "tokens": x.shape[0], "x": x, "c": (g_c, u_c, d_c), "ex": ex, "h13": h13})
    torch.cuda.synchronize()

    def qa(matrix, axis, scope):
        plan = SimpleNamespace(rate_axis=axis, encoder_tile_bits=rate_map)
        return _qsrt_quant_args(plan, matrix=matrix, layer=24, device=dev, shared_scale_scope=scope,
                                transform_seeds=default_qsrt_transform_seeds(24, matrix))

    def run_sample():
        proxies = []
        for g0 in range(0, sample, batch):
            group = experts[g0:g0 + batch]
            weights, hs, qas = [], [], []
            for item in group:
                g_c, u_c, _ = item["c"]
                for name, m in (("w1", g_c), ("w3", u_c)):
                    shared = make_shared_h(hidden, dev, item["h13"])
                    shared["count"] = item["tokens"]
                    weights.append(m.T.contiguous())
                    hs.append(shared)
                    qas.append([qa(name, "n", ("layer-bench", g0))])
            up = be.quantize_qsrt_batch(weights, hs, qas)
            weights, hs, qas = [], [], []
            for i, item in enumerate(group):
                g_c, u_c, d_c = item["c"]
                g_hat, u_hat = up[2 * i][0]["weight_q"].T, up[2 * i + 1][0]["weight_q"].T
                gs, us, _ = decode_coupled_weights((g_hat, u_hat, d_c), spec)
                x = item["x"]
                h = (torch.nn.functional.silu(x @ gs.T) * (x @ us.T)).contiguous()
                h2 = item["ex"].transform_h2(gemm.gram_(torch.zeros((inter, inter), device=dev), h, 1.0 / x.shape[0]))
                shared = make_shared_h(inter, dev, h2)
                shared["count"] = item["tokens"]
                weights.append(d_c.T.contiguous())
                hs.append(shared)
                qas.append([qa("w2", "k", ("layer-bench", g0))])
            down = be.quantize_qsrt_batch(weights, hs, qas)
            proxies += [r[0]["proxy"] for r in up] + [r[0]["proxy"] for r in down]
        torch.cuda.synchronize()
        return proxies

    # The first pass pays one-time costs (library code objects loaded on first use of each kernel and shape,
    # allocator growth); a whole layer pays them once, so the layer time is the cold pass plus the warm
    # pass's time for every further batch of the same shape.
    t0 = time.perf_counter()
    run_sample()
    cold = time.perf_counter() - t0
    t0 = time.perf_counter()
    proxies = run_sample()
    seconds = time.perf_counter() - t0
    weights_per_expert = 3 * hidden * inter
    return {
        "workload": f"config 5 layer encode: {sample} of {LAYER_EXPERTS} Kimi-class experts (Zipf s={LAYER_ZIPF_S} over "
                    f"{LAYER_TOKENS} routed tokens), {batch} experts per batch, records 14 K3 + 2 K4, coupled basis, "
                    f"LDLQ, H2 from reconstructed activations",
        "sample_experts": chosen,
        "sample_tokens": [item["tokens"] for item in experts],
        "sample_seconds": round(seconds, 3),
        "sample_seconds_cold": round(cold, 3),
        "M_weights_per_s": round(sample * weights_per_expert / seconds / 1e6, 2),
        "layer_seconds_extrapolated": round(cold + seconds * (LAYER_EXPERTS / sample - 1), 1),
        "proxy_err_mean": round(sum(proxies) / len(proxies), 5),
    }


def cpu_baseline(tiles_np, seconds_target: float = 12.0):
    """Time the oracle on a bounded sample (first tiles), K2 and K3."""

    import numpy as np

    from oracle import tables as otables
    from oracle import viterbi as ov

    threads = ov.default_threads()
    total_w = 0
    total_t = 0.0
    sample = max(threads, 8)
    for bits in RATES:
        lab = otables.t12_values(bits)
        # calibrate on a small batch, then size the sample to the time budget
        t0 = time.perf_counter()
        ov.encode(tiles_np[:threads], lab, K=bits, threads=threads)
        per_tile = (time.perf_counter() - t0) / threads
        n = int(min(len(tiles_np), max(threads, (seconds_target / len(RATES)) / max(per_tile, 1e-6))))
        n = max(threads, (n // threads) * threads)
        t0 = time.perf_counter()
        ov.encode(tiles_np[:n], lab, K=bits, threads=threads)
        total_t += time.perf_counter() - t0
        total_w += n * 256
        sample = n
    return {
        "value": total_w / total_t / 1e6,
        "unit": "M weights/s",
        "cores": threads,
        "kind": "port",
        "sample": f"first {sample} of the {TILES} microbench tiles at each of K2 and K3, C=128, oracle/viterbi_ref.c with {threads} OpenMP threads",
    }


DECODE_EXPERTS = 384  # a layer of Kimi-class experts
# Per-matrix record rates of the decoded layer: H308's 2 K4 + 22 K3 needs 24 records; the 7168 x 2048 expert has
# 16 records of 128 intermediate channels, so its record-granular analogue is 2 K4 + 14 K3 (3.125 trellis bpw).
DECODE_RECORD_BITS = (3,) * 14 + (4,) * 2
HBM_PEAK_GBPS = 8000.0


def decode_bench(steps: int = 3, experts: int = DECODE_EXPERTS):
    """Whole-layer decode: ``experts`` x (gate, up, down)
    record-major payloads with mixed record rates -> bf16.  Gate/up
    [7168 x 2048] carry their records along N, down [2048 x 7168] along K, as
    the encoder stores them.  One prepared plan, one launch per rate per step.
    Payload words are random (any word stream is a valid cyclic path)."""

    from qsrt_amd.decode import DecodePlan
    from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

    dev = torch.device("cuda:0")
    h, i = 7168, 2048
    bits = DECODE_RECORD_BITS
    words_per = h * i * sum(bits) // (16 * len(bits))
    n_mat = 3 * experts
    g = torch.Generator(device=dev).manual_seed(20261201 + 5)
    words = torch.randint(-32768, 32767, (n_mat, words_per), dtype=torch.int16, device=dev, generator=g)
    su = (torch.rand((n_mat, 7168), device=dev, generator=g) + 0.5) / 128.0
    sv = torch.rand((n_mat, 7168), device=dev, generator=g) - 0.5
    out = torch.empty((n_mat, h * i), dtype=torch.bfloat16, device=dev)
    payloads = []
    for m in range(n_mat):
        down = m % 3 == 2
        k, n = (i, h) if down else (h, i)
        payloads.append((words[m], bits, "k" if down else "n", su[m, :k], sv[m, :n], out[m].view(k, n)))
    plan = DecodePlan.for_records(payloads, {b: sqg_xor_cheb_t12_bytes(b).to(dev) for b in set(bits)})
    plan.run()
    torch.cuda.synchronize()
    ms = []
    for _ in range(steps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        plan.run()
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    weights = n_mat * h * i
    bpw = sum(bits) / len(bits)
    byts = weights * (bpw / 8 + 2) + n_mat * (h + i) * 4
    t = min(ms) / 1e3
    del words, out, plan, payloads
    torch.cuda.empty_cache()
    return {
        "workload": f"config 5 layer: {experts} experts x (gate, up [{h} x {i}], down [{i} x {h}]), records "
                    f"{bits.count(3)} K3 + {bits.count(4)} K4 ({bpw:.3f} trellis bpw) -> bf16",
        "kernel": "decode_kernel (one launch per rate)",
        "ms": round(min(ms), 3),
        "G_weights_per_s": round(weights / t / 1e9, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(byts / t / 1e9, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(byts / t / 1e9 / HBM_PEAK_GBPS, 4),
            "traffic": round(byts * DECODE_TRAFFIC_OVER_ALGORITHMIC),
            "algorithmic": f"{bpw:.3f}/8 B payload + 2 B bf16 out per weight + (K + N) f32 scales per matrix "
                           f"= {byts:.4g} B per layer (both launches)",
        },
    }


def expert_bench(bits: int = 3, cpu_seconds: float = 4.0):
    """BASELINE config 4 at K3 (the north-star target): one warm-up and one
    timed end-to-end encode of the coupled Kimi-class expert, and the CPU
    oracle's per-tile time scaled by the timed run's tile-encode count (a lower
    bound on the CPU encoder: the LDLQ products, Hessian and activation work
    are not charged to the CPU)."""

    run_expert_encode(bits=bits, log=log)
    r = run_expert_encode(bits=bits, log=log)
    import numpy as np
    from oracle import tables as otables
    from oracle import viterbi as ov

    threads = ov.default_threads()
    g = np.random.default_rng(20261201 + 4)
    sample = g.standard_normal((max(threads, 256), 256)).astype(np.float32)
    lab = otables.t12_values(bits)
    ov.encode(sample[:threads], lab, K=bits, threads=threads)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < cpu_seconds:
        ov.encode(sample, lab, K=bits, boundary_lag=1, threads=threads)
        n += len(sample)
    per_tile = (time.perf_counter() - t0) / n
    cpu_s = per_tile * r["tile_encodes"]
    return {
        "workload": "config 4: Kimi-class coupled expert 7168 x 2048 SwiGLU, all three matrices, K3, LDLQ, H2 from reconstructed activations",
        "seconds": round(r["seconds"], 3),
        "M_weights_per_s": round(r["M_weights_per_s"], 2),
        "tile_encodes": r["tile_encodes"],
        "phases_s": {"gate_up": round(r["seconds_upstream"], 3), "h2_rebuild": round(r["seconds_h2_rebuild"], 3),
                     "down": round(r["seconds_down"], 3)},
        "proxy_err": {k: round(v, 5) for k, v in r["proxy"].items()},
        "cpu_extrapolated_seconds": round(cpu_s, 1),
        "cpu_basis": f"oracle/viterbi_ref.c, {threads} threads, {per_tile * 1e3:.3f} ms/tile (K3, C=128) x {r['tile_encodes']} tile encodes",
        "speedup_vs_cpu": round(cpu_s / r["seconds"], 1),
    }


MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f32": 157.3}


def _time_ms(fn, steps: int, min_ms: float = 2.0) -> float:
    """Mean duration of ``fn`` over at least ``steps`` launches, HIP events on
    the current stream (the stream the kernels are launched on).  Short
    kernels get enough launches to fill ``min_ms`` of GPU time, so the mean
    is the kernel's own duration rather than launch latency."""

    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    reps = max(steps, min(2000, math.ceil(min_ms / max(e0.elapsed_time(e1), 1e-3))))
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def gemm_bench(steps: int = 5):
    """The two MFMA GEMM shapes of the config-4 expert encode:
    Hessian capture ``H += X^T X / n`` of 16,384 bf16 tokens x 7168 channels,
    and one LDLQ span update ``P[:begin] += L[span, :begin]^T (W - Q)[span]``
    (M = 7040, K = 128, N = 2048, FP32)."""

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
    del L, W, Q, P
    torch.cuda.empty_cache()

    def line(key, name, ms, fl, dtype, shape, what):
        t = fl / (ms / 1e3) / 1e12
        return {"kernel": name, "shape": shape, "ms": round(ms, 4), "roofline": {
            "bound": "mfma", "achieved": round(t, 1), "peak": MFMA_PEAK_TFLOPS[dtype], "unit": "TFLOP/s",
            "frac": round(t / MFMA_PEAK_TFLOPS[dtype], 4), "traffic": round(GEMM_HBM_BYTES[key]),
            "algorithmic": f"{what} = {fl:.4g} flops/launch ({dtype} in, f32 accumulate)"}}

    return {
        "hessian_capture": line("hessian_capture", "gemm_tn_bf16_kernel", ms_h, fl_h, "bf16",
                                f"X [{n} x {k}] bf16 -> H [{k} x {k}] f32", "n k (k + 1) (symmetric)"),
        "ldlq_span_update": line("ldlq_span_update", "gemm_tn_f32_kernel", ms_l, fl_l, "f32",
                                 f"L^T [{m} x {kk}] (W - Q) [{kk} x {nn}] f32", "2 M N K"),
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
            "algorithmic": f"8 B/element x {k * n} elements/launch"}}
    del W
    torch.cuda.empty_cache()
    return {"workload": f"[{k} x {n}] f32, block 128, fused signs, in place", **out}


def copy_calibration(nbytes: int) -> None:
    """A plain device copy of ``nbytes`` (the known-size reference for the
    HBM byte counters)."""

    x = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda:0").fill_(1.0)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    y.copy_(x)
    torch.cuda.synchronize()
    log(f"[bench] copied {nbytes} bytes")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--tiles", type=int, default=TILES)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-expert", action="store_true", help="skip the config-4 expert encode")
    ap.add_argument("--no-decode", action="store_true", help="skip the layer decode")
    ap.add_argument("--no-kernels", action="store_true", help="skip the GEMM and Hadamard kernel lines")
    ap.add_argument("--no-layer", action="store_true", help="skip the config-5 layer encode sample")
    ap.add_argument("--layer-sample", type=int, default=8, help="experts encoded for the config-5 layer estimate")
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

    import numpy as np

    from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes
    from qsrt_amd.sqg_quantizer import boundary_lag, viterbi_tiles

    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(20261201 + 2)
    tiles_cpu = torch.randn((args.tiles, 256), generator=gen, dtype=torch.float32)
    tiles = tiles_cpu.to(dev)
    luts = {b: sqg_xor_cheb_t12_bytes(b).to(dev) for b in RATES}
    lags = {b: boundary_lag(b, 6.5) for b in RATES}
    outs = {b: (torch.empty_like(tiles), torch.empty(tiles.shape, dtype=torch.int16, device=dev)) for b in RATES}

    def step(events=None):
        for b in RATES:
            if events is not None:
                events[b][0].record()
            viterbi_tiles(tiles, luts[b], b, tailbite_context=CONTEXT, lag=lags[b], out=outs[b])
            if events is not None:
                events[b][1].record()

    log(f"[bench] warmup {args.warmup} step(s) of {args.tiles} tiles x K{RATES}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    per_k_ms = {b: [] for b in RATES}
    log(f"[bench] timing {args.steps} step(s)")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev = {b: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for b in RATES}
        step(ev)
        torch.cuda.synchronize()
        for b in RATES:
            per_k_ms[b].append(ev[b][0].elapsed_time(ev[b][1]))
        log(f"[bench] step {i}: " + ", ".join(f"K{b} {per_k_ms[b][-1]:.1f} ms" for b in RATES))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3

    weights_per_k = args.tiles * 256
    value = weights_per_k * len(RATES) * args.steps / wall / 1e6
    kernel_ms = {b: float(np.mean(per_k_ms[b])) for b in RATES}
    per_k_rate = {f"K{b}": weights_per_k / (kernel_ms[b] / 1e3) / 1e6 for b in RATES}
    # roofline of the dominant kernel: average over the measured launches
    mean_launch_s = float(np.mean([kernel_ms[b] for b in RATES])) / 1e3
    flops_per_launch = weights_per_k * EDGES_PER_WEIGHT * FLOPS_PER_EDGE
    achieved = flops_per_launch / mean_launch_s / 1e12

    result = {
        "metric": "encoded weights/sec (M/s) at K=2/3 on one GPU",
        "value": round(value, 3),
        "unit": "M weights/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: iid N(0,1) tiles, seed 20261203",
        "config": {
            "workload": "viterbi-microbench (BASELINE configs[1]): 65,536 tiles x 256 weights, K2 and K3, L=16, C=128, sqg_xor_cheb_t12",
            "tiles": args.tiles,
            "rates": list(RATES),
            "tailbite_context": CONTEXT,
        },
        "per_rate_M_weights_per_s": {k: round(v, 3) for k, v in per_k_rate.items()},
        "roofline": {
            "bound": "valu",
            "achieved": round(achieved, 3),
            "peak": FP32_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
            "traffic": round(VITERBI_HBM_BYTES_PER_TILE * args.tiles),
            "kernel": "viterbi_tiles_kernel",
            "algorithmic": f"{FLOPS_PER_EDGE} FP32 flops/edge x {int(EDGES_PER_WEIGHT)} edges/weight x {weights_per_k} weights/launch",
            # The 157.3 TFLOP/s peak counts packed FP32; this build disables packed FP32 ops, which halves the
            # vector ceiling.  PMC on the same kernel puts VALU issue at 94-106% of slots (K2 above 1: its compares
            # into SGPR masks retire in fewer than 4 cycles).
            "peak_without_packed_fp32": FP32_UNPACKED_PEAK_TFLOPS,
            "frac_without_packed_fp32": round(achieved / FP32_UNPACKED_PEAK_TFLOPS, 4),
            "valu_issue_frac_pmc": VITERBI_VALU_ISSUE_FRAC_PMC,
        },
    }
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle) on a bounded sample")
        result["cpu_baseline"] = cpu_baseline(tiles_cpu.numpy())
        result["cpu_baseline"]["gpu_speedup"] = round(value / result["cpu_baseline"]["value"], 1)
    del tiles, outs
    torch.cuda.empty_cache()
    if not args.no_kernels:
        log("[bench] GEMM and Hadamard kernels")
        result["gemm"] = gemm_bench()
        result["hadamard"] = hadamard_bench()
        log("[bench] gemm " + ", ".join(f"{k} {v['roofline']['achieved']} TFLOP/s" for k, v in result["gemm"].items())
            + "; hadamard " + ", ".join(f"{k} {result['hadamard'][k]['roofline']['achieved']} GB/s"
                                        for k in ("left", "right")))
    if not args.no_decode:
        log("[bench] layer decode")
        result["decode"] = decode_bench()
        log(f"[bench] decode {result['decode']['roofline']['achieved']} GB/s")
    if not args.no_expert:
        log("[bench] config-4 expert encode (K3)")
        result["expert_encode"] = expert_bench()
        log(f"[bench] expert {result['expert_encode']['seconds']} s, {result['expert_encode']['speedup_vs_cpu']}x CPU")
    if not args.no_layer:
        log("[bench] config-5 layer encode sample")
        result["layer_encode"] = layer_encode_bench(sample=args.layer_sample)
        log(f"[bench] layer sample {result['layer_encode']['sample_seconds']} s, "
            f"{result['layer_encode']['M_weights_per_s']} M w/s, layer ~{result['layer_encode']['layer_seconds_extrapolated']} s")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
