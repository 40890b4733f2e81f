"""Matrix and expert encode callers on the GPU (qsrt_amd.qsrt_encoder):
every stored payload must close exactly (edges and states), decode to the
encoder's own reconstruction, carry exactly the mode's bit budget, and agree
with the fused HIP decode kernel.  Small generic geometry (512 intermediate x
256 latent channels, four records) so each case runs in well under a second."""

from __future__ import annotations

import sys

import pytest
import torch

from qsrt_amd import qsrt_encoder as enc
from qsrt_amd.decode import decode_packed
from qsrt_amd.qsrt import ExpertFormatSpec, Geometry, decode_qsrt_exl3_weight, resolve_mode
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

pytestmark = pytest.mark.gpu
GEO = Geometry(512, 256)
DEV = torch.device("cuda:0")


def _contexts(seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    ctx = torch.arange(GEO.records).repeat_interleave(32)
    return ctx[torch.randperm(ctx.numel(), generator=g)]


def _hessian(d: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(4 * d, d, generator=g) @ (torch.eye(d) + 0.3 * torch.randn(d, d, generator=g) / d ** 0.5)
    h = x.T @ x / x.shape[0]
    return (h + 0.01 * h.diagonal().mean() * torch.eye(d)).to(DEV)


def _source(matrix: str, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    shape = (GEO.latent_channels, GEO.intermediate_channels) if matrix == "w2" else (GEO.intermediate_channels,
                                                                                     GEO.latent_channels)
    return (0.02 * torch.randn(shape, generator=g)).to(DEV)


def _rel(a, b) -> float:
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("matrix,mode", [("w1", "R1"), ("w3", "R0"), ("w2", "R2")])
def test_quantize_qsrt_matrix_closes_and_decodes(matrix, mode):
    print(f"[encoder] {matrix} {mode}", file=sys.stderr, flush=True)
    d = GEO.intermediate_channels if matrix == "w2" else GEO.latent_channels
    source, hessian = _source(matrix, 11), _hessian(d, 12)
    out = enc.quantize_qsrt_matrix(source, _contexts(3), matrix=matrix, mode=mode, hessian=hessian, layer=7,
                                   device=DEV, shared_scale_scope=("test-matrix", matrix, mode))
    c = out.coding
    assert c["reference_edge_roundtrip"] and c["reference_state_roundtrip"]
    assert c["index_bits"] == source.numel() * 3
    # the stored su / sv are fp16 (the encoder's own reconstruction keeps them in FP32): ~2^-12 relative
    assert c["stored_decode_vs_encoder"]["relative_l2"] < 1e-3
    assert out.packed.descriptor.schema == enc.GENERIC_SCHEMA
    # a 3-bit-average trellis code of a Gaussian source: about 0.13 relative error in the rotated domain
    assert 0.02 < _rel(out.reconstruction, source) < 0.35
    # the stored payload through the fused HIP decode equals the reference decode
    ref = decode_qsrt_exl3_weight(out.packed, out.tensors["suh"], out.tensors["svh"])
    luts = {b: sqg_xor_cheb_t12_bytes(b).to(DEV) for b in (2, 3, 4)}
    hip = decode_packed(out.packed, out.tensors["suh"].float(), out.tensors["svh"].float(), luts,
                        out_dtype=torch.float32)
    assert _rel(hip, ref) < 1e-5


def test_quantize_qsrt_expert_shares_one_physical_order():
    print("[encoder] expert R1/R2", file=sys.stderr, flush=True)
    sources = {m: _source(m, 20 + i) for i, m in enumerate(("w1", "w3", "w2"))}
    out = enc.quantize_qsrt_expert(sources, _contexts(4), format_spec=ExpertFormatSpec.compressed(1, 2),
                                   h13=_hessian(GEO.latent_channels, 31), h2=_hessian(GEO.intermediate_channels, 32),
                                   layer=9, device=DEV, shared_scale_scope="test-expert")
    assert out.coding["format"] == "R1/R2" and out.coding["common_physical_permutation"]
    assert out.coding["trellis_bytes"] == 3 * GEO.intermediate_channels * GEO.latent_channels * 3 // 8
    for m in ("w1", "w3", "w2"):
        assert torch.equal(out.matrices[m].plan.physical_permutation, out.physical_permutation)
        assert out.matrices[m].coding["stored_decode_vs_encoder"]["relative_l2"] < 1e-3
        assert _rel(out.matrices[m].reconstruction, sources[m]) < 0.35
    assert out.matrices["w2"].coding["mode"] == "R2" and out.matrices["w1"].coding["mode"] == "R1"


@pytest.mark.parametrize("layout", ["importance_ordered", "qsrt_pair_prefix_reuse"])
def test_batched_candidates_finalize_to_their_scoring_reconstruction(layout):
    print(f"[encoder] batched candidates {layout}", file=sys.stderr, flush=True)
    modes = tuple(resolve_mode(m, GEO) for m in ("R0", "R1", "R2"))
    sources = {"w1": _source("w1", 41), "w3": _source("w3", 42)}
    h13 = _hessian(GEO.latent_channels, 43)
    cands = enc.quantize_qsrt_matrix_candidates_batched(sources, _contexts(5), modes=modes,
                                                        hessians={"w1": h13, "w3": h13}, layer=11, device=DEV,
                                                        shared_scale_scope=("test-batch", layout), layout=layout)
    assert set(cands) == {"w1", "w3"} and all(set(v) == {0, 1, 2} for v in cands.values())
    for m, by_mode in cands.items():
        for mode_id, cand in by_mode.items():
            fin = enc.finalize_qsrt_matrix_candidate(cand, layer=11)
            assert fin.coding["scoring_reconstruction_vs_stored"]["relative_l2"] < 1e-3
            assert fin.coding["mode_id"] == mode_id and fin.coding["index_bits"] == sources[m].numel() * 3
            assert _rel(fin.reconstruction, sources[m]) < 0.35
