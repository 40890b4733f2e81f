"""Atom-major layer files (qsrt_amd.qsrt_atoms): materialise two compressed
experts of a Kimi-K3 layer from a candidate file and read every view back
bit-exactly (reference tests/test_qsrt_storage.py:217-262)."""

from __future__ import annotations

import pytest
import torch
from safetensors.torch import save_file

from qsrt_amd import qsrt_atoms as qa
from qsrt_amd import qsrt_storage as st
from qsrt_amd.qsrt import INTERMEDIATE_CHANNELS, LATENT_CHANNELS, MATRIX_TRELLIS_BYTES, ExpertFormatSpec

LAYER = 24
EXPERTS = {3: ExpertFormatSpec.compressed(1, 2), 700: ExpertFormatSpec.compressed(0, 0)}


def _candidates(seed: int):
    g = torch.Generator().manual_seed(seed)
    shared = {m: torch.randn(LATENT_CHANNELS, generator=g).half() for m in ("w1", "w3", "w2")}
    out = {}
    for expert in EXPERTS:
        parts = {}
        for m in ("w1", "w3", "w2"):
            trellis = torch.randint(-32768, 32768, (MATRIX_TRELLIS_BYTES // 2,), generator=g, dtype=torch.int32)
            local = torch.randn(INTERMEDIATE_CHANNELS, generator=g).half()
            suh, svh = (local, shared[m]) if m == "w2" else (shared[m], local)
            parts[m] = {"trellis": trellis.to(torch.int16), "suh": suh, "svh": svh}
        out[expert] = parts
    return out


def _write(tmp_path, cands):
    d = tmp_path / "pool" / "candidates"
    d.mkdir(parents=True)
    tensors = {qa.candidate_tensor_name(LAYER, e, m, p): v.clone()
               for e, parts in cands.items() for m, pp in parts.items() for p, v in pp.items()}
    save_file(tensors, str(d / f"qsrt-layer-{LAYER:05d}.safetensors"))
    formats = tuple(EXPERTS.get(e, ExpertFormatSpec.x4t()) for e in range(896))
    spec = qa.QSRTAtomLayerSpec(LAYER, formats, tuple(sorted(EXPERTS)), tuple(e for e in range(896) if e not in EXPERTS))
    return tmp_path / "pool", spec


def test_materialised_layer_reads_back_bit_exactly(tmp_path):
    cands = _candidates(5)
    root, spec = _write(tmp_path, cands)
    dest = tmp_path / "out" / qa.layer_filename(LAYER)
    info = qa.materialize_atom_layer(root, dest, spec)
    assert info["disk_bytes"] == dest.stat().st_size == st.QSRTLayerLayout(2, 894).disk_bytes
    expected = [qa.assemble_candidate_atoms(layer=LAYER, expert=e, format_spec=EXPERTS[e], tensors=cands[e])[0]
                for e in sorted(EXPERTS)]
    with qa.QSRTAtomLayerReader(dest) as reader:
        assert reader.header.layout == st.QSRTLayerLayout(2, 894)
        assert reader.compressed == (3, 700) and len(reader.x4t) == 894
        assert reader.formats[3] == "R1/R2" and reader.formats[700] == EXPERTS[700].name and reader.formats[0] == "X4T"
        assert all(torch.equal(a.view(torch.int16), b.view(torch.int16))
                   for a, b in zip(reader.shared_scales, (cands[3]["w1"]["suh"], cands[3]["w3"]["suh"],
                                                          cands[3]["w2"]["svh"])))
        for slot, atoms in enumerate(expected):
            assert torch.equal(reader.read_expert_atoms(slot), atoms)
        both = torch.stack(expected, dim=1)  # [96, 2, bundle]
        assert torch.equal(torch.cat([reader.read_shard(12, i, require_equal=True) for i in range(12)]), both)
        assert torch.equal(torch.cat([reader.read_shard(5, i) for i in range(5)]), both)
        for e in EXPERTS:
            for m in ("w1", "w3", "w2"):
                got = reader.read_compressed_matrix(e, m)
                for p in ("trellis", "suh", "svh"):
                    assert torch.equal(got[p].view(torch.int16), cands[e][m][p].view(torch.int16)), (e, m, p)
        with pytest.raises(ValueError):
            reader.read_compressed_matrix(0, "w1")  # an X4T expert
    with pytest.raises(FileExistsError):
        qa.materialize_atom_layer(root, dest, spec)


def test_shared_scale_drift_is_rejected_and_leaves_no_file(tmp_path):
    cands = _candidates(6)
    cands[700]["w3"]["suh"] = cands[700]["w3"]["suh"].clone()
    cands[700]["w3"]["suh"][0] += 1
    root, spec = _write(tmp_path, cands)
    dest = tmp_path / "out" / qa.layer_filename(LAYER)
    with pytest.raises(ValueError, match="drifted"):
        qa.materialize_atom_layer(root, dest, spec)
    assert not dest.exists() and not dest.with_name(f".{dest.name}.partial").exists()


def test_names_specs_and_argument_checks():
    assert qa.layer_filename(7) == "qsrt-layer-00007.safetensors"
    assert qa.candidate_tensor_name(3, 12, "w2", "svh").endswith("layers.3.block_sparse_moe.experts.12.w2.qsrt_svh")
    with pytest.raises(ValueError):
        qa.layer_filename(93)
    with pytest.raises(ValueError):
        qa.candidate_tensor_name(3, 1, "w4", "suh")
    formats = (ExpertFormatSpec.x4t(),) * 896
    with pytest.raises(ValueError, match="tiers"):
        qa.QSRTAtomLayerSpec(3, formats, (0,), tuple(range(1, 896)))
    with pytest.raises(ValueError):
        qa.assemble_candidate_atoms(layer=3, expert=0, format_spec=ExpertFormatSpec.x4t(), tensors={})
