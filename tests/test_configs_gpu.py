"""Every BASELINE config on the GPU at its own shape (config 1 is compared
end to end with the CPU encode in ``test_e2e_parity_gpu.py``).

* config 2: the 65,536-tile microbench at K4 (K2 and K3 in
  ``test_full_size_gpu.py``): closure, labels, a seeded sample bit-exact with
  the oracle; the packed EXL bitstream of every rate equals the oracle's
  packing of the sampled tiles byte for byte;
* config 3: the GLM expert (hidden 5120, inter 1536, K3, 8 outlier channels)
  gate and down through ``quantize_qsrt``: closure, exactly 3 bits per
  weight, decode of the stored payload equals the reconstruction, sampled
  LDLQ tile calls replay bit-exactly on the oracle;
* config 4: the Kimi-class coupled expert at K2 through the layer pipeline
  (coupled basis, H2 rebuilt from the reconstruction): closure at K2, the
  payload's bit accounting (2 trellis bits per weight plus the fp16 suh/svh
  vectors), sampled tile calls replayed;
* config 5: two Zipf-routed experts of the 384-expert layer in one batch with
  14 K3 + 2 K4 records: every record closes at its rate, sampled tile calls
  replay, and the stored record-major payloads decode -- through the
  oracle's own container reader and float64 decode -- to what the fused HIP
  decode produces.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import bench
from oracle import fmt as ofmt
from oracle import tables as otables
from oracle import viterbi as ov
from qsrt_amd import exl3_encoder_backend as be
from qsrt_amd import qsrt as Q
from qsrt_amd.decode import DecodePlan
from qsrt_amd.exl3_reference import decode_regularized_weight, reconstruct_trellis_states
from qsrt_amd.ldlq import make_shared_h
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes
from qsrt_amd.sqg_quantizer import boundary_lag, quantize_tiles_sqg, viterbi_tiles
from qsrt_amd.transform_seeds import default_qsrt_transform_seeds

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
LAGS = {2: 0, 3: 1, 4: 1}


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class _Recorder:
    """Keeps chosen LDLQ tile-quantizer calls (not the global-scale search's)
    for an oracle replay."""

    def __init__(self, monkeypatch, keep):
        self.keep, self.count, self.calls, self.in_search = set(keep), 0, [], False
        real_q, real_s = be.quantize_tiles_multigpu, be.g_scale_search_batch

        def q(tiles, qa):
            out = real_q(tiles, qa)
            if not self.in_search:
                if self.count in self.keep:
                    self.calls.append((self.count, tiles.cpu().numpy(), int(qa["K"]), out[0].cpu().numpy(),
                                       out[1].cpu().numpy().view(np.uint16)))
                self.count += 1
            return out

        def s(samples, qa):
            self.in_search = True
            try:
                return real_s(samples, qa)
            finally:
                self.in_search = False

        monkeypatch.setattr(be, "quantize_tiles_multigpu", q)
        monkeypatch.setattr(be, "g_scale_search_batch", s)

    def replay(self):
        assert len(self.calls) == len(self.keep), "a kept LDLQ call was never made"
        for i, tiles, bits, recon, states in self.calls:
            o_recon, o_states = ov.encode(tiles, otables.t12_values(bits), K=bits, boundary_lag=LAGS[bits])
            assert np.array_equal(states, o_states), f"call {i} (K{bits}, {len(tiles)} tiles): states differ"
            assert np.array_equal(recon, o_recon), f"call {i}: labels differ"
        return len(self.calls)


def _closed(states: torch.Tensor, bits) -> bool:
    s64 = states.to(torch.int64) & 0xFFFF
    return bool(torch.equal(states.to(torch.int16), reconstruct_trellis_states(s64 & ((1 << bits) - 1), bits)
                            .to(torch.int16)))


def test_config2_k4_full_size_and_packed_bitstreams():
    tiles_n = 65536
    gen = torch.Generator().manual_seed(20261201 + 2)
    source = torch.randn((tiles_n, 256), generator=gen).to(DEV)
    pick = torch.randperm(tiles_n, generator=torch.Generator().manual_seed(99))[:16]
    for bits in (4, 3, 2):
        _say(f"[configs] config 2 microbench K{bits}: {tiles_n} tiles, Viterbi + packing")
        lut = sqg_xor_cheb_t12_bytes(bits).to(DEV)
        recon, states = viterbi_tiles(source, lut, bits, tailbite_context=128, lag=boundary_lag(bits, 6.5))
        words = Q.pack_trellis_edges(states, bits)
        torch.cuda.synchronize()
        assert tuple(words.shape) == (tiles_n, 16 * bits)
        if bits == 4:
            s64 = states.to(torch.int64) & 0xFFFF
            assert _closed(states, bits)
            assert torch.equal(recon, lut.view(torch.float8_e4m3fn).float()[s64])
        sample = source[pick.to(DEV)].cpu().numpy()
        o_recon, o_states = ov.encode(sample, otables.t12_values(bits), K=bits, boundary_lag=LAGS[bits])
        got_states = states[pick.to(DEV)].cpu().numpy().view(np.uint16)
        assert np.array_equal(got_states, o_states) and np.array_equal(recon[pick.to(DEV)].cpu().numpy(), o_recon)
        assert np.array_equal(words[pick.to(DEV)].cpu().numpy().view(np.uint16), ofmt.pack_words(o_states, bits))


def _quantize(W, H_sum, count, bits, seeds):
    shared = make_shared_h(W.shape[0], DEV, H_sum)
    shared["count"] = count
    qa = {"K": bits, "seed": seeds.input_sign, "sv_seed": seeds.output_sign, "sigma_reg": 0.01,
          "devices": [str(DEV)], "apply_out_scales": False, "tailbite_context": 128,
          "sqg_e4m3_lut": sqg_xor_cheb_t12_bytes(bits)}
    weight_q, proxy, tensors = be.quantize_qsrt(W.clone(), shared, qa, False)
    torch.cuda.synchronize()
    return weight_q, proxy, tensors, qa


def test_config3_glm_expert_full_size(monkeypatch):
    from qsrt_amd import gemm

    d = bench.config_expert(3, DEV)
    x = d["x"]
    _say(f"[configs] config 3: GLM expert, {x.shape[0]} rows, outlier channels {d['outliers'].tolist()}")
    h13 = gemm.gram_(torch.zeros((5120, 5120), device=DEV), x)
    h = (torch.nn.functional.silu(x @ d["w_gate"].T) * (x @ d["w_up"].T)).contiguous()
    h2 = gemm.gram_(torch.zeros((1536, 1536), device=DEV), h)
    del h
    for matrix, W, H, keep in (("w1", d["w_gate"].T.contiguous(), h13, (5, 200)),
                               ("w2", d["w_down"].T.contiguous(), h2, (3, 90))):
        k, n = W.shape
        rec = _Recorder(monkeypatch, keep)
        weight_q, proxy, tensors, qa = _quantize(W, H, x.shape[0], 3, default_qsrt_transform_seeds(1, matrix))
        trellis = tensors["trellis"]
        _say(f"[configs] config 3 {matrix} [{k} x {n}]: {rec.count} LDLQ calls, proxy {proxy:.5f}, "
             f"g {qa['g_scale']:.4f}")
        assert rec.count == k // 16
        assert trellis.numel() * 16 == k * n * 3
        states = Q.unpack_trellis_states(trellis, 3)
        assert _closed(states, 3)
        assert torch.equal(decode_regularized_weight(states.cpu(), bits=3), weight_q.cpu())
        assert 0.0 < proxy < 0.05
        assert rec.replay() == 2
        monkeypatch.undo()


def _layer_experts(monkeypatch, cfg, experts, tokens, record_bits, keep, scope):
    enc = bench.ExpertEncoder(DEV, hidden=7168, inter=2048, record_bits=record_bits, scope=scope)
    sources = [bench.expert_source(cfg, DEV, expert=e, tokens=t) for e, t in zip(experts, tokens)]
    rec = _Recorder(monkeypatch, keep)
    out = enc.encode(sources, keep_states=set(experts))
    torch.cuda.synchronize()
    for key in [k for k in be._SHARED_INPUT_SCALES if k[0] == scope]:
        del be._SHARED_INPUT_SCALES[key]
    return enc, out, rec


def test_config4_coupled_expert_at_k2(monkeypatch):
    _say("[configs] config 4: coupled Kimi-class expert at K2 (16,384 rows), H2 from the reconstruction")
    enc, out, rec = _layer_experts(monkeypatch, 4, [0], [16384], (2,) * 16, keep=(7, 440, 460),
                                   scope=("configs-test", 4))
    e = out[0]
    total_bits = 0
    for m in ("w1", "w3", "w2"):
        r = e[m]
        k, n = r["shape"]
        assert _closed(r["encoded"], 2), m
        assert r["words"].numel() * 16 == k * n * 2
        assert r["suh"].dtype == torch.float16 and r["suh"].numel() == k and r["svh"].numel() == n
        assert 0.0 < r["proxy"] < 0.2
        total_bits += r["words"].numel() * 16 + 16 * (k + n)
    bpw = total_bits / (3 * 7168 * 2048)
    _say(f"[configs] config 4 K2: {bpw:.5f} bpw including the fp16 suh/svh vectors; proxies "
         f"{[round(e[m]['proxy'], 4) for m in ('w1', 'w3', 'w2')]}")
    assert bpw == pytest.approx(2.0 + 16 * (7168 + 2048) / (7168 * 2048))
    assert rec.replay() == 3  # two gate/up batch steps, one down step


def test_config5_two_layer_experts_records_and_decode(monkeypatch):
    counts = bench.zipf_token_counts()
    order = sorted(range(bench.LAYER_EXPERTS), key=lambda i: -counts[i])
    experts = [order[0], order[-1]]  # the most and the least routed expert
    _say(f"[configs] config 5: experts {experts} with {[counts[i] for i in experts]} routed rows, "
         f"records 14 K3 + 2 K4")
    enc, out, rec = _layer_experts(monkeypatch, 5, experts, [counts[i] for i in experts], bench.LAYER_RECORD_BITS,
                                   keep=(0, 201, 447, 800, 950), scope=("configs-test", 5))
    luts = {b: sqg_xor_cheb_t12_bytes(b).to(DEV) for b in (3, 4)}
    payloads, meta = [], []
    for e in out:
        for m in ("w1", "w3", "w2"):
            r = e[m]
            k, n = r["shape"]
            axis = r["rate_axis"]
            tile_bits = np.array([b for b in bench.LAYER_RECORD_BITS for _ in range(8)])
            st = r["encoded"]
            for t, b in enumerate(tile_bits):
                sl = st[t] if axis == "k" else st[:, t]
                assert _closed(sl, int(b)), f"expert {e['expert']} {m} tile line {t}"
            outb = torch.empty((k, n), dtype=torch.float32, device=DEV)
            payloads.append((r["words"], bench.LAYER_RECORD_BITS, axis, (r["suh"].float() / 128).contiguous(),
                             r["svh"].float().contiguous(), outb))
            meta.append((r, axis))
    DecodePlan.for_records(payloads, luts, out_dtype=torch.float32).run()
    torch.cuda.synchronize()
    for (r, axis), p in zip(meta, payloads):
        k, n = r["shape"]
        states, tile_bits = ofmt.unpack_records(r["words"].cpu().numpy(), bench.LAYER_RECORD_BITS, axis, k // 16,
                                                n // 16)
        assert np.array_equal(states, r["encoded"].cpu().numpy().view(np.uint16))
        labels = np.zeros(states.shape)
        for b in (3, 4):
            mask = tile_bits == b
            labels[mask] = otables.t12_values(b)[states[mask].astype(np.int64)]
        rows = slice(0, 512)  # the decode is separable by 128-row block rows
        want = ofmt.decode_tile_values(labels[:32], r["suh"].float().cpu().numpy()[rows], r["svh"].float().cpu().numpy())
        got = p[5][rows].double().cpu().numpy()
        assert np.max(np.abs(got - want)) <= 2e-6 * np.abs(want).max()
    _say(f"[configs] config 5: {len(payloads)} stored payloads decoded; proxies "
         f"{[round(e[m]['proxy'], 4) for e in out for m in ('w1', 'w3', 'w2')]}")
    assert rec.replay() == 5
