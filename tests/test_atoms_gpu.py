"""A materialised atom layer decodes on the GPU straight from the file:
``QSRTAtomLayerReader.decode_expert`` equals the fused decode of the original
candidate payloads bit for bit, and the float64 reference decode within
bf16 rounding."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from qsrt_amd import qsrt_atoms as qa
from qsrt_amd.decode import decode_packed
from qsrt_amd.qsrt import (INTERMEDIATE_CHANNELS, LATENT_CHANNELS, MATRIX_TRELLIS_BYTES, ExpertFormatSpec,
                           PackedQSRTTrellis, decode_qsrt_exl3_weight)
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

pytestmark = pytest.mark.gpu


def test_decode_expert_from_layer_file(tmp_path):
    print("[atoms] decode an expert from a materialised layer", file=sys.stderr, flush=True)
    layer, expert, fmt = 40, 285, ExpertFormatSpec.compressed(2, 1)
    g = torch.Generator().manual_seed(9)
    cands = {}
    for m in ("w1", "w3", "w2"):
        local = (torch.rand(INTERMEDIATE_CHANNELS, generator=g) + 0.5).half()
        shared = (torch.rand(LATENT_CHANNELS, generator=g) - 0.5).half()
        suh, svh = (local, shared) if m == "w2" else (shared, local)
        trellis = torch.randint(-32768, 32768, (MATRIX_TRELLIS_BYTES // 2,), generator=g, dtype=torch.int32)
        cands[m] = {"trellis": trellis.to(torch.int16), "suh": suh, "svh": svh}
    d = tmp_path / "pool" / "candidates"
    d.mkdir(parents=True)
    save_file({qa.candidate_tensor_name(layer, expert, m, p): v.clone() for m, pp in cands.items() for p, v in pp.items()},
              str(d / f"qsrt-layer-{layer:05d}.safetensors"))
    formats = tuple(fmt if e == expert else ExpertFormatSpec.x4t() for e in range(896))
    spec = qa.QSRTAtomLayerSpec(layer, formats, (expert,), tuple(e for e in range(896) if e != expert))
    dest = tmp_path / qa.layer_filename(layer)
    qa.materialize_atom_layer(tmp_path / "pool", dest, spec)
    luts = {b: sqg_xor_cheb_t12_bytes(b) for b in (2, 3, 4)}
    with qa.QSRTAtomLayerReader(dest) as reader:
        got = reader.decode_expert(expert, luts, out_dtype=torch.float32)
    dev = torch.device("cuda:0")
    for m in ("w1", "w3", "w2"):
        desc = qa._matrix_descriptor(m, fmt.r2 if m == "w2" else fmt.r13)
        packed = PackedQSRTTrellis(desc, cands[m]["trellis"].to(dev))
        direct = decode_packed(packed, cands[m]["suh"].to(dev), cands[m]["svh"].to(dev),
                               {b: l.to(dev) for b, l in luts.items()}, out_dtype=torch.float32)
        assert torch.equal(got[m], direct), m
    ref = decode_qsrt_exl3_weight(PackedQSRTTrellis(qa._matrix_descriptor("w2", fmt.r2), cands["w2"]["trellis"]),
                                  cands["w2"]["suh"], cands["w2"]["svh"]).double().numpy()
    assert np.max(np.abs(got["w2"].cpu().double().numpy() - ref)) <= 2e-6 * np.abs(ref).max()
