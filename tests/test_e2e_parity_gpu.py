"""End-to-end payload parity: ``quantize_qsrt`` on the GPU against an
untethered CPU encode (``oracle.encode``) on the same seeded inputs.

The CPU side receives only what the GPU side receives -- the weight, the
captured ``X^T X`` sum and its count, the seeds -- plus the global scale the
GPU's search picked (that search is pinned on its own in
``test_gscale.py``).  It then runs the float64 Hessian preparation,
congruence, block LDL, regularisation and BlockLDLQ with the C oracle
Viterbi on every 16-row block.  Nothing of the GPU run feeds the CPU
recursion.

Bar: the payloads are equal, tile for tile and byte for byte (0 differing
tiles at every size, the full config-3, config-4 and config-5 gates
included).  Both sides keep everything before the tile Viterbi in float64
and round each target to FP32 once, and the Viterbi is bit-exact on equal
input, so any differing tile would come from a target that differs; for the
uniform-rate encodes the test also compares every target the GPU handed the
Viterbi with the CPU's, which must be equal except for rare elements that a
float64 discrepancy moved across an FP32 rounding boundary (a sum in another
order, amplified by the factor's conditioning).  The tile mismatch rate and the
near-tie classification of any differing tile (``compare_states``) are
printed, so a failure says what kind of difference it met.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import bench
from oracle import encode as oenc
from oracle import fmt as ofmt
from oracle import ldlq as oldlq
from oracle import tables as otables
from qsrt_amd import exl3_encoder_backend as be
from qsrt_amd.ldlq import make_shared_h
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes
from qsrt_amd.transform_seeds import default_qsrt_transform_seeds

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _signs(n: int, seed: int) -> np.ndarray:
    """The reference's sign draw on a CPU generator (qsrt/rng.py:8-20)."""

    g = torch.Generator().manual_seed(int(seed))
    return (torch.randn(n, generator=g).sign() + 1e-5).sign().double().numpy()


def _gpu_encode(W: torch.Tensor, H_sum: torch.Tensor, count: int, bits: int, seeds, monkeypatch=None) -> tuple:
    """``quantize_qsrt`` on the device; with ``monkeypatch`` every tile call
    is recorded, and the last ``K / 16`` calls (the BlockLDLQ steps, after
    the global-scale search) give the targets the Viterbi saw."""

    shared = make_shared_h(W.shape[0], DEV, H_sum)
    shared["count"] = count
    qa = {"K": bits, "seed": seeds.input_sign, "sv_seed": seeds.output_sign, "sigma_reg": 0.01,
          "devices": [str(DEV)], "apply_out_scales": False, "tailbite_context": 128,
          "sqg_e4m3_lut": sqg_xor_cheb_t12_bytes(bits)}
    calls = []
    if monkeypatch is not None:
        real = be.quantize_tiles_multigpu

        def recording(tiles, quant_args):
            calls.append(tiles.cpu().numpy())
            return real(tiles, quant_args)

        monkeypatch.setattr(be, "quantize_tiles_multigpu", recording)
    weight_q, proxy, tensors = be.quantize_qsrt(W.to(DEV).clone(), shared, qa, False)
    torch.cuda.synchronize()
    if monkeypatch is not None:
        monkeypatch.undo()
    kt = W.shape[0] // 16
    targets = np.stack(calls[-kt:][::-1]) if calls else None  # step i quantizes row block kt - 1 - i
    return weight_q, proxy, tensors, qa, shared, targets


def _check_equal_payload(name: str, stats: dict) -> None:
    """Every tile equal.  A differing tile is reported with its near-tie
    classification first, so a failure says what it met."""

    if stats["differ"]:
        for (rb, col), kind, d, m in zip(stats["first"], stats["kinds"], stats["sse_rel_deltas"],
                                         stats["boundary_margins"]):
            _say(f"[e2e] {name}: differing tile ({rb}, {col}) is a {kind} near tie: SSE delta {d:.3e}, "
                 f"boundary margin {m:.3e}")
    assert stats["differ"] == 0, f"{name}: {stats['differ']} of {stats['tiles']} tiles differ from the CPU encode"


def _check_targets(name: str, gpu_targets: np.ndarray, cpu_targets: np.ndarray) -> None:
    """The GPU's Viterbi inputs against the CPU's float64 targets rounded
    once: equal, except rare elements that a float64 discrepancy (sums in
    another order, amplified by the factor's conditioning) moved across a
    rounding boundary -- one FP32 ulp apart, or, for a target near zero,
    within 1e-10 of the largest target."""

    g = np.ascontiguousarray(gpu_targets, dtype=np.float32)
    c = np.ascontiguousarray(cpu_targets, dtype=np.float32)
    assert g.shape == c.shape
    ulps = np.abs(g.view(np.int32).astype(np.int64) - c.view(np.int32).astype(np.int64))
    absd = np.abs(g.astype(np.float64) - c.astype(np.float64))
    scale = float(np.abs(c).max())
    n_diff = int(np.count_nonzero(ulps))
    far = (ulps > 1) & (absd > 1e-10 * scale)
    _say(f"[e2e] {name}: {g.size - n_diff} of {g.size} Viterbi inputs equal the CPU's bit for bit, "
         f"{n_diff} differ (max {int(ulps.max())} ulp, max {float(absd.max()) / scale:.2e} of the largest target)")
    assert not far.any(), f"{name}: {int(far.sum())} targets beyond float64-rounding distance of the CPU's"
    assert n_diff <= max(4, g.size // 10_000), f"{name}: {n_diff} targets differ from the CPU's"


def _tie_summary(stats: dict) -> str:
    d, m = stats["sse_rel_deltas"], stats["boundary_margins"]
    return (f"{stats['kinds'].count('path')} path and {stats['kinds'].count('boundary')} boundary near-ties, "
            f"max SSE delta {max(d, default=0.0):.3e}, max boundary margin {max(m, default=0.0):.3e}")


def _check_matrix(name: str, W: torch.Tensor, H_sum: torch.Tensor, count: int, bits: int, seeds,
                  monkeypatch) -> dict:
    k, n = W.shape
    _say(f"[e2e] {name}: [{k} x {n}] K{bits} on cuda:0")
    weight_q, proxy, tensors, qa, shared, targets = _gpu_encode(W, H_sum, count, bits, seeds, monkeypatch)
    trellis = tensors["trellis"].cpu().numpy().view(np.uint16)
    g_states = ofmt.cyclic_states(ofmt.unpack_symbols(trellis, bits), bits)
    _say(f"[e2e] {name}: GPU proxy {proxy:.6f}, g_scale {qa['g_scale']:.6f}; CPU encode")
    labels = {bits: otables.t12_values(bits)}
    lags = {bits: 0 if bits == 2 else 1}
    cpu = oenc.encode_matrix(W.double().cpu().numpy(), H_sum.double().cpu().numpy(), count,
                             _signs(k, seeds.input_sign), _signs(n, seeds.output_sign), qa["g_scale"],
                             np.full((k // 16, n // 16), bits), labels, lags, sigma_reg=0.01)
    stats = oenc.compare_states(g_states, cpu, labels, np.full((k // 16, n // 16), bits), lags)
    words = ofmt.pack_words(cpu["states"], bits)
    same_tile = ~np.any(g_states != cpu["states"], axis=2)
    cpu_proxy = oenc.proxy(cpu["W_r"], cpu["Q"], cpu["H_c"])
    _say(f"[e2e] {name}: {stats['differ']} of {stats['tiles']} tiles differ (mismatch rate "
         f"{stats['mismatch_rate']:.5f}; {stats['propagated']} downstream of {_tie_summary(stats)}); "
         f"proxy GPU {proxy:.6f} CPU {cpu_proxy:.6f}")
    # words of every agreeing tile are the oracle's, byte for byte
    assert np.array_equal(trellis[same_tile], words[same_tile])
    # GPU's float64 factor and FP32 conditioned metric against the float64 congruence + block LDL
    assert shared["L"].dtype == torch.float64
    L = shared["L"].cpu().numpy()
    H_c = shared["H"].double().cpu().numpy()
    h_err = np.max(np.abs(H_c - cpu["H_c"])) / np.abs(cpu["H_c"]).max()
    l_err = np.max(np.abs(L - cpu["L0"])) / max(np.abs(cpu["L0"]).max(), 1.0)
    _say(f"[e2e] {name}: conditioned H max rel {h_err:.2e}, L max rel {l_err:.2e}")
    assert h_err <= 1e-6 and l_err <= 1e-8
    _check_targets(name, targets, cpu["targets"])
    _check_equal_payload(name, stats)
    # the GPU's reconstruction (regularised basis) is its states' labels
    assert np.array_equal(weight_q.cpu().numpy(), cpu["Q"].astype(np.float32))
    assert abs(proxy - cpu_proxy) <= 1e-4 * cpu_proxy
    return stats


def test_config1_expert_all_three_matrices_match_cpu_encode(monkeypatch):
    """BASELINE config 1 (hidden 256, inter 512, K2): gate and up under
    H13 = X^T X, down under H2 from the source SwiGLU activations."""

    d = bench.config_expert(1, torch.device("cpu"))
    x = d["x"].double()
    h13 = (x.T @ x).float()
    h = torch.nn.functional.silu(x @ d["w_gate"].double().T) * (x @ d["w_up"].double().T)
    h2 = (h.T @ h).float()
    n_rows = x.shape[0]
    total = {"tiles": 0, "differ": 0}
    for matrix, W, H in (("w1", d["w_gate"].T, h13), ("w3", d["w_up"].T, h13), ("w2", d["w_down"].T, h2)):
        stats = _check_matrix(f"config 1 {matrix}", W.contiguous(), H, n_rows, 2,
                              default_qsrt_transform_seeds(1, matrix), monkeypatch)
        total["tiles"] += stats["tiles"]
        total["differ"] += stats["differ"]
    _say(f"[e2e] config 1 expert: tile mismatch rate {total['differ'] / total['tiles']:.5f} "
         f"({total['differ']} of {total['tiles']})")


def test_config3_strip_matches_cpu_encode(monkeypatch):
    """A 1,024-row strip of the config-3 gate matrix (K3): rows 0..1023 of
    W^T [5120 x 1536] under the matching 1024 x 1024 block of H13, from 8192
    AR(1) rows (rho 0.9) whose 8 outlier channels (20x variance) are placed
    inside the strip."""

    gen = torch.Generator().manual_seed((20261201 + 3) * 1000 + 7)
    k, n, rows = 1024, 1536, 8192
    x = bench.ar1_scan(rows, k, 0.9, gen)
    outliers = torch.randperm(k, generator=gen)[:8]
    x[:, outliers] *= 20.0 ** 0.5
    W = bench.student_t_like((n, k), std=0.015, gen=gen).bfloat16().float().T.contiguous()
    xd = x.double()
    _check_matrix("config 3 strip", W, (xd.T @ xd).float(), rows, 3, default_qsrt_transform_seeds(1, "w1"),
                  monkeypatch)


def test_config4_gate_full_size_matches_cpu_encode(monkeypatch):
    """BASELINE config 4 at full size: the 7168 x 2048 gate matrix at K2
    (57,344 tiles, 448 BlockLDLQ steps) under H13 from the config's 16,384
    AR(1) rows (rho 0.85), against the untethered CPU encode of the same
    inputs.  H13 is summed in float64 on the device and handed to both sides
    as FP32."""

    d = bench.config_expert(4, DEV)
    xd = d["x"].double()
    H_sum = (xd.T @ xd).float().cpu()
    del xd
    _check_matrix("config 4 gate (full size)", d["w_gate"].T.contiguous().cpu(), H_sum, d["x"].shape[0], 2,
                  default_qsrt_transform_seeds(1, "w1"), monkeypatch)


def test_config3_gate_full_size_matches_cpu_encode(monkeypatch):
    """BASELINE config 3 at full size: the 5120 x 1536 gate matrix at K3
    (30,720 tiles) under H13 from the config's 8192 AR(1) rows (rho 0.9)
    with 8 outlier channels at 20x variance."""

    d = bench.config_expert(3, DEV)
    xd = d["x"].double()
    H_sum = (xd.T @ xd).float().cpu()
    del xd
    _check_matrix("config 3 gate (full size)", d["w_gate"].T.contiguous().cpu(), H_sum, d["x"].shape[0], 3,
                  default_qsrt_transform_seeds(1, "w1"), monkeypatch)


def test_config5_rarely_routed_expert_full_size_matches_cpu_encode(monkeypatch):
    """BASELINE config 5's hardest conditioning at full size: the gate
    matrix (7168 x 2048, K3) of a layer expert that the Zipf routing gives
    only 19 of 65,536 calibration rows, so H13 is rank 19 plus the 1%
    damping.  An FP32 factorisation of it would move decisions against any
    other; the float64 one keeps the payload equal."""

    counts = bench.zipf_token_counts()
    expert = counts.index(min(counts))
    d = bench.config_expert(5, DEV, expert=expert, tokens=counts[expert])
    xd = d["x"].double()
    H_sum = (xd.T @ xd).float().cpu()
    del xd
    _check_matrix(f"config 5 expert {expert} gate ({counts[expert]} rows)", d["w_gate"].T.contiguous().cpu(), H_sum,
                  d["x"].shape[0], 3, default_qsrt_transform_seeds(1, "w1"), monkeypatch)


def test_few_row_hessian_matches_cpu_encode(monkeypatch):
    """A Hessian from 48 calibration rows (rank 48 of 256 plus 1% damping, the
    conditioning of a rarely routed expert): the device factorisation must
    still agree with the float64 one closely enough that the payloads match."""

    d = bench.config_expert(1, torch.device("cpu"), tokens=48)
    x = d["x"].double()
    _check_matrix("config 1 w1, 48 rows", d["w_gate"].T.contiguous(), (x.T @ x).float(), 48, 2,
                  default_qsrt_transform_seeds(1, "w1"), monkeypatch)


def test_batch_conditioned_path_matches_cpu_encode():
    """``quantize_qsrt_batch`` (the layer pipeline's path): w1 and w3 of one
    expert share a 96-row Hessian; the congruence uses the regularised su,
    the input profile is layer-shared (taken from w1), the global scale goes
    into sv, and the records along N mix K3 and K4."""

    k, n, rows = 512, 256, 96
    gen = torch.Generator().manual_seed(20261201 + 51)
    x = bench.ar1_scan(rows, k, 0.85, gen).double()
    H_sum = (x.T @ x).float()
    Ws = [bench.student_t_like((n, k), std=0.015, gen=gen).bfloat16().float().T.contiguous() for _ in range(2)]
    bits_map = (3,) * 8 + (4,) * 8
    scope = ("e2e-batch-test", 1)
    hds, groups = [], []
    for matrix in ("w1", "w3"):
        seeds = default_qsrt_transform_seeds(1, matrix)
        hd = make_shared_h(k, DEV, H_sum)
        hd["count"] = rows
        hds.append(hd)
        groups.append([{"K": 3, "seed": seeds.input_sign, "sv_seed": seeds.output_sign, "sigma_reg": 0.01,
                        "devices": [str(DEV)], "apply_out_scales": False, "tailbite_context": 128,
                        "sqg_e4m3_luts_by_bits": {b: sqg_xor_cheb_t12_bytes(b) for b in (2, 3, 4)},
                        "mixed_rate_axis": "n", "mixed_tile_bits": bits_map,
                        "shared_input_scales_key": (scope, "w1"), "g_scale_into_sv": True}])
    _say(f"[e2e] quantize_qsrt_batch: w1, w3 [{k} x {n}], {rows}-row Hessian, records K3/K4 along N")
    out = be.quantize_qsrt_batch([W.to(DEV).clone() for W in Ws], hds, groups)
    torch.cuda.synchronize()
    be._SHARED_INPUT_SCALES.pop((scope, "w1"), None)
    labels = {b: otables.t12_values(b) for b in (3, 4)}
    lags = {3: 1, 4: 1}
    tile_bits = np.tile(np.array(bits_map), (k // 16, 1))
    profile = None
    for (matrix, W, res, qa) in zip(("w1", "w3"), Ws, out, groups):
        seeds = default_qsrt_transform_seeds(1, matrix)
        su_s, sv_s = _signs(k, seeds.input_sign), _signs(n, seeds.output_sign)
        Wd = W.double().numpy()
        if profile is None:
            profile = oldlq.input_rms(Wd, sv_s)
        cpu = oenc.encode_matrix(Wd, H_sum.double().numpy(), rows, su_s, sv_s, res[0]["g_scale"], tile_bits, labels,
                                 lags, sigma_reg=0.01, conditioned=True, g_into_sv=True, input_scales=profile)
        g_states = res[0]["encoded"].cpu().numpy().view(np.uint16)
        stats = oenc.compare_states(g_states, cpu, labels, tile_bits, lags)
        _say(f"[e2e] batch {matrix}: {stats['differ']} of {stats['tiles']} tiles differ, {_tie_summary(stats)}; "
             f"proxy GPU {res[0]['proxy']:.6f} CPU {oenc.proxy(cpu['W_r'], cpu['Q'], cpu['H_c']):.6f}")
        cpu_proxy = oenc.proxy(cpu["W_r"], cpu["Q"], cpu["H_c"])
        assert abs(res[0]["proxy"] - cpu_proxy) <= 1e-4 * cpu_proxy
        # the regularised weight the recursion read is the oracle's, to float64 rounding
        w_err = np.max(np.abs(res[0]["weight_r"].cpu().numpy() - cpu["W_r"])) / np.abs(cpu["W_r"]).max()
        assert w_err <= 1e-13, f"batch {matrix}: regularised weight {w_err:.2e} from the oracle's"
        _check_equal_payload(f"batch {matrix}", stats)
