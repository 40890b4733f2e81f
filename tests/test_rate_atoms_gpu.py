"""A rate-record layer file at BASELINE config-5 geometry decodes, through
the fused HIP decode, exactly as the payloads it was written from: two
experts of 7168 x 2048 with 14 K3 + 2 K4 records per matrix, atoms
assembled on the GPU, the file read back to the GPU."""

from __future__ import annotations

import sys

import pytest
import torch

from qsrt_amd.decode import DecodePlan
from qsrt_amd.qsrt import Geometry
from qsrt_amd.qsrt_rate_atoms import MATRICES, QSRTRateLayerLayout, QSRTRateLayerReader, RateSchedule, \
    materialize_rate_layer
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
BITS = (3,) * 14 + (4,) * 2
SHAPES = {"w1": (7168, 2048), "w3": (7168, 2048), "w2": (2048, 7168)}
AXES = {"w1": "n", "w3": "n", "w2": "k"}


def _decode(mats: dict) -> dict:
    outs, payloads = {}, []
    for (e, m), p in mats.items():
        k, n = SHAPES[m]
        out = torch.empty((k, n), dtype=torch.bfloat16, device=DEV)
        outs[(e, m)] = out
        payloads.append((p["trellis"], BITS, AXES[m], (p["suh"].float() / 128.0).contiguous(),
                         p["svh"].float().contiguous(), out))
    DecodePlan.for_records(payloads, {b: sqg_xor_cheb_t12_bytes(b).to(DEV) for b in (3, 4)}).run()
    torch.cuda.synchronize()
    return outs


def test_config5_layer_file_decodes_like_its_payloads(tmp_path):
    print("[rate-atoms] config-5 geometry, experts 0 and 5", file=sys.stderr, flush=True)
    sched = RateSchedule(Geometry(2048, 7168), BITS)
    g = torch.Generator(device=DEV).manual_seed(2048)
    shared = {m: ((torch.rand(7168, device=DEV, generator=g) - 0.5) * 0.02).half() for m in MATRICES}
    experts = {}
    for e in (0, 5):
        experts[e] = {}
        for m in MATRICES:
            words = torch.randint(-32768, 32768, (sched.matrix_words,), device=DEV, generator=g,
                                  dtype=torch.int32).to(torch.int16)
            local = ((torch.rand(2048, device=DEV, generator=g) + 0.5) * 0.01).half()
            experts[e][m] = ({"trellis": words, "suh": shared[m], "svh": local} if m != "w2"
                             else {"trellis": words, "suh": local, "svh": shared[m]})
    layout = QSRTRateLayerLayout(24, sched, (0, 5))
    path = tmp_path / "qsrt-layer-00024.safetensors"
    materialize_rate_layer(path, layout, experts.items())
    with QSRTRateLayerReader(path) as rd:
        back = {(e, m): p for e in (0, 5) for m, p in rd.read_expert(e, device=DEV).items()}
    for (e, m), p in back.items():
        for part in ("trellis", "suh", "svh"):
            assert torch.equal(p[part], experts[e][m][part]), (e, m, part)
    want = _decode({(e, m): experts[e][m] for e in (0, 5) for m in MATRICES})
    got = _decode(back)
    for key in want:
        assert torch.equal(got[key], want[key]), key
        assert bool(torch.isfinite(got[key].float()).all())
