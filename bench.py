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
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

TILES = 65536
RATES = (2, 3)
CONTEXT = 128
EDGES_PER_WEIGHT = (256 + 2 * CONTEXT) / 256 * 65536  # 131,072 at C=128
FLOPS_PER_EDGE = 3  # d = label - x (1), fma(d, d, cost) (2)
FP32_PEAK_TFLOPS = 157.3


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--tiles", type=int, default=TILES)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the encoder hot path is a single-GPU kernel here; "
              "multi-GPU sharding is design-only (see DESIGN.md)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

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
            "traffic": None,
            "kernel": "viterbi_tiles_kernel",
            "algorithmic": f"{FLOPS_PER_EDGE} FP32 flops/edge x {int(EDGES_PER_WEIGHT)} edges/weight x {weights_per_k} weights/launch",
        },
    }
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle) on a bounded sample")
        result["cpu_baseline"] = cpu_baseline(tiles_cpu.numpy())
        result["cpu_baseline"]["gpu_speedup"] = round(value / result["cpu_baseline"]["value"], 1)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
