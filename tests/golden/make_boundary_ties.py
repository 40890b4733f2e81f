"""Writes ``boundary_ties_k3.npz``: tiles whose MI355X encode chose another
boundary state than the CPU oracle (``oracle/viterbi_ref.c``) on the same
BlockLDLQ target.  Runs on a GPU box:

    python tests/golden/make_boundary_ties.py --out /tmp/boundary_ties_k3.npz

It encodes the config-3 strip of ``tests/test_e2e_parity_gpu.py`` with
``quantize_qsrt`` at global scales a few float32 steps from the searched one
(each choice moves the FP32 targets by rounding), runs the CPU encode on the
same inputs, and keeps every tile that differs while all tiles below it in
its column agree and whose boundary state (``codeword[0] >> K``) differs.
Stored per tile: the CPU target (float32 [256]) and the GPU's and CPU's
codewords (uint16 [256]); K = 3, boundary_lag = 1, context 128.
"""

from __future__ import annotations

import argparse
import os
import sys

import numpy as np
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", ".."))

import bench  # noqa: E402
from oracle import encode as oenc  # noqa: E402
from oracle import fmt as ofmt  # noqa: E402
from oracle import tables as otables  # noqa: E402
from qsrt_amd import exl3_encoder_backend as be  # noqa: E402
from qsrt_amd.ldlq import make_shared_h  # noqa: E402
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes  # noqa: E402
from qsrt_amd.transform_seeds import default_qsrt_transform_seeds  # noqa: E402


def _signs(n: int, seed: int) -> np.ndarray:
    g = torch.Generator().manual_seed(int(seed))
    return (torch.randn(n, generator=g).sign() + 1e-5).sign().double().numpy()


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", required=True)
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed((20261201 + 3) * 1000 + 7)
    k, n, rows, bits = 1024, 1536, 8192, 3
    x = bench.ar1_scan(rows, k, 0.9, gen)
    x[:, torch.randperm(k, generator=gen)[:8]] *= 20.0 ** 0.5
    W = bench.student_t_like((n, k), std=0.015, gen=gen).bfloat16().float().T.contiguous()
    H_sum = (x.double().T @ x.double()).float()
    seeds = default_qsrt_transform_seeds(1, "w1")
    labels, lags = {bits: otables.t12_values(bits)}, {bits: 1}
    tile_bits = np.full((k // 16, n // 16), bits)
    targets, gpu, cpu_states, g_scales = [], [], [], []
    searched = None
    for step in (0, -1, 1, -2, 2, 3):
        shared = make_shared_h(k, dev, H_sum)
        shared["count"] = rows
        qa = {"K": bits, "seed": seeds.input_sign, "sv_seed": seeds.output_sign, "sigma_reg": 0.01,
              "devices": [str(dev)], "apply_out_scales": False, "tailbite_context": 128,
              "sqg_e4m3_lut": sqg_xor_cheb_t12_bytes(bits)}
        if searched is not None:
            g = np.float32(searched)
            for _ in range(abs(step)):
                g = np.nextafter(g, np.float32(np.inf if step > 0 else -np.inf))
            qa["g_scale_override"] = float(g)
        _, _, tensors = be.quantize_qsrt(W.to(dev).clone(), shared, qa, False)
        torch.cuda.synchronize()
        if searched is None:
            searched = qa["g_scale"]
        trellis = tensors["trellis"].cpu().numpy().view(np.uint16)
        g_states = ofmt.cyclic_states(ofmt.unpack_symbols(trellis, bits), bits)
        cpu = oenc.encode_matrix(W.double().numpy(), H_sum.double().numpy(), rows, _signs(k, seeds.input_sign),
                                 _signs(n, seeds.output_sign), qa["g_scale"], tile_bits, labels, lags,
                                 sigma_reg=0.01)
        stats = oenc.compare_states(g_states, cpu, labels, tile_bits, lags)
        kept = 0
        for (rb, col), kind in zip(stats["first"], stats["kinds"]):
            if kind == "boundary":
                targets.append(cpu["targets"][rb, col])
                gpu.append(g_states[rb, col])
                cpu_states.append(cpu["states"][rb, col])
                g_scales.append(qa["g_scale"])
                kept += 1
        print(f"g {qa['g_scale']!r}: {stats['differ']} tiles differ, {len(stats['first'])} near-ties, "
              f"{kept} at the boundary", flush=True)
    np.savez(args.out, targets=np.array(targets, dtype=np.float32), gpu_states=np.array(gpu, dtype=np.uint16),
             cpu_states=np.array(cpu_states, dtype=np.uint16), g_scale=np.array(g_scales))
    print(f"{len(targets)} boundary tiles -> {args.out}", flush=True)


if __name__ == "__main__":
    main()
