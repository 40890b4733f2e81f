"""The global-scale search and its tile sample, pinned by closed forms (no
GPU: the tile quantizer is replaced by a stand-in whose error at every
scale is known exactly).

* ``g_scale_search_batch`` (reference ``qsrt/exl3_encoder_backend.py:2413-2476``):
  - on an exactly quadratic error curve the search returns the vertex, since
    the parabola through three samples of a quadratic is the quadratic;
  - on a curve with a narrow quadratic well centred between coarse points,
    the coarse stage must land on the one grid point inside the well (0.7 of
    0.1, 0.3, ..., 1.9) and the fine stage then recovers the well's vertex;
  - the coarse stage sees every third sample tile, the fine stage all;
  - a vertex beyond the fine grid's edge returns the edge point itself.
* ``sample_scale_tiles`` (``:2383-2410``): on a matrix whose tiles hold
  their own index, the sample is exactly the wrapped diagonal of width 3
  followed by the highest- and lowest-RMS tiles.
"""

from __future__ import annotations

import pytest
import torch

from qsrt_amd import exl3_encoder_backend as be


def _marked_tiles(n: int) -> torch.Tensor:
    """Tiles whose element 0 is 1 (so a scaled batch reveals its scale) and
    element 1 is the tile's index (so a call reveals which tiles it got)."""

    t = torch.zeros((n, 256))
    t[:, 0] = 1.0
    t[:, 1] = torch.arange(n, dtype=torch.float32)
    return t


def _stand_in(curve, seen):
    """Quantizer whose reconstruction error at scale s is sqrt(curve(s)) per
    element, so that mean((recon / s - tiles)^2) == curve(s)."""

    def quantize(batch, quant_args):
        scale = batch[:, 0:1]
        err = torch.tensor([curve(float(s)) for s in scale.flatten()]).sqrt().unsqueeze(1)
        seen.append((sorted({round(float(s), 6) for s in scale.flatten()}), batch[:, 1] / scale.flatten()))
        return batch + scale * err, torch.zeros(batch.shape, dtype=torch.int16)

    return quantize


def _search(monkeypatch, curve, n_tiles=30):
    seen = []
    monkeypatch.setattr(be, "quantize_tiles_multigpu", _stand_in(curve, seen))
    (g, mse), = be.g_scale_search_batch([_marked_tiles(n_tiles)], {"K": 2})
    return g, float(mse), seen


@pytest.mark.parametrize("vertex", [0.4567, 0.83, 1.0, 1.2345, 1.61])
def test_quadratic_curve_returns_its_vertex(monkeypatch, vertex):
    g, mse, _ = _search(monkeypatch, lambda s: 0.02 + 0.3 * (s - vertex) ** 2)
    assert g == pytest.approx(vertex, abs=2e-4)
    assert mse == pytest.approx(0.02 + 0.3 * min((vertex - p) ** 2 for p in _fine_points(vertex)), rel=1e-4)


def _fine_points(vertex):
    coarse = [0.1 + 0.2 * i for i in range(10)]
    c = min(coarse, key=lambda p: abs(p - vertex))
    return [c + 0.075 * (i - 2) for i in range(5)]


def test_narrow_well_between_coarse_points(monkeypatch):
    # a deep well of half-width 0.09 around 0.71: only the coarse point 0.7 falls inside it; outside the well
    # the curve is a shallow bowl whose own minimum (1.3) the coarse grid would otherwise pick
    def curve(s):
        return 0.5 + 20.0 * (s - 0.71) ** 2 if abs(s - 0.71) < 0.09 else 1.0 + 0.01 * (s - 1.3) ** 2

    g, _, seen = _search(monkeypatch, curve)
    assert g == pytest.approx(0.71, abs=2e-4)
    coarse_scales = sorted({s for scales, _ in seen[:1] for s in scales})
    assert coarse_scales == pytest.approx([0.1 + 0.2 * i for i in range(10)])


def test_coarse_stage_uses_every_third_tile(monkeypatch):
    _, _, seen = _search(monkeypatch, lambda s: (s - 1.0) ** 2 + 1.0, n_tiles=31)
    coarse_ids = seen[0][1]
    fine_ids = seen[-1][1]
    assert torch.equal(coarse_ids[:11].round(), torch.arange(0, 31, 3, dtype=torch.float32))
    assert torch.equal(fine_ids[-31:].round(), torch.arange(31, dtype=torch.float32))


def test_vertex_outside_the_fine_grid_returns_the_edge(monkeypatch):
    # strictly decreasing curve: coarse picks 1.9, fine grid 1.75 .. 2.05 is still decreasing -> edge 2.05
    g, _, _ = _search(monkeypatch, lambda s: 5.0 - s)
    assert g == pytest.approx(1.9 + 0.15, abs=1e-6)


def test_sample_scale_tiles_is_the_wrapped_diagonal_plus_extreme_rms():
    kt, nt = 5, 12  # 80 x 192 matrix, tile (i, j) filled with 1 + i * nt + j
    w = torch.zeros((16 * kt, 16 * nt))
    for i in range(kt):
        for j in range(nt):
            w[16 * i:16 * i + 16, 16 * j:16 * j + 16] = 1 + i * nt + j
    tiles = be.sample_scale_tiles(w)
    ids = (tiles[:, 0] - 1).round().long().tolist()
    assert torch.all(tiles == tiles[:, :1])  # each sampled tile is one whole tile
    diag_len, width = max(kt, nt), 3
    diagonal = [(i % kt) * nt + (i + d) % nt for i in range(diag_len) for d in range(width)]
    extremes = min(max(8, diag_len * width // 16), (kt * nt + 1) // 2)
    hi = list(range(kt * nt - 1, kt * nt - 1 - extremes, -1))
    lo = list(range(extremes))
    assert ids == diagonal + hi + lo


def test_sample_scale_tiles_elements_in_tensor_core_order():
    # element (r, c) of every tile holds its row-major index r * 16 + c, so each sampled tile must read back as
    # the tensor-core permutation itself; a ragged shape (3 x 7 tiles) exercises the wrap in both directions
    kt, nt = 3, 7
    idx = torch.arange(256, dtype=torch.float32).view(16, 16)
    w = idx.repeat(kt, nt).contiguous()
    tiles = be.sample_scale_tiles(w, width=2)
    perm = be.tensor_core_perm("cpu").float()
    assert tiles.dtype == torch.float32 and tiles.shape[1] == 256
    assert torch.equal(tiles, perm.expand_as(tiles))
    assert sorted(set(perm.long().tolist())) == list(range(256))
