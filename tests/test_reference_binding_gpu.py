"""The binding a maintainer would add to the reference, driven as the
reference's caller drives its extension (qsrt/sqg_quantizer.py:478-654):
the K2..K4 codebook transposed to [out-edge pair][predecessor][2], FP16 cost
and uint8 traceback temporaries sized like ``_sqg_temp_buffers``
(qsrt/sqg_quantizer.py:410-427), and ``lut_abs_max`` choosing the boundary
rule.  The stub's results must equal this build's own tile quantizer bit for
bit."""

from __future__ import annotations

import ctypes
import sys

import pytest
import torch

from qsrt_amd import _native
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes
from qsrt_amd.sqg_quantizer import boundary_lag, viterbi_tiles

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _reference_inputs(bits: int, batch: int):
    """What the reference's caller hands its extension."""

    edges = 65536 >> bits
    decisions = edges // 4 if bits == 2 else edges // 2 if bits <= 4 else edges
    costs = torch.zeros((batch, 2, edges), dtype=torch.float16, device=DEV)
    traceback = torch.empty((batch, 256, decisions), dtype=torch.uint8, device=DEV)
    lut = sqg_xor_cheb_t12_bytes(bits).to(DEV).contiguous()
    lut_abs_max = float(lut.view(torch.float8_e4m3fn).to(torch.float32).abs().amax())
    if bits in (2, 3, 4):
        lut = lut.reshape(1 << bits, (65536 >> bits) // 2, 2).permute(1, 0, 2).contiguous().reshape(-1)
    return costs, traceback, lut, lut_abs_max


def quantize_tiles_sqg(input_tiles, output_tiles, output_indices, temp_costs, temp_edges, codebook, K,
                       tailbite_context, lut_abs_max):
    """The ctypes stub: the reference extension's signature, tensor for tensor."""

    lib = _native.lib()
    rc = lib.qsrt_quantize_tiles_sqg(
        input_tiles.data_ptr(), output_tiles.data_ptr(), output_indices.data_ptr(), input_tiles.shape[0],
        temp_costs.data_ptr(), temp_costs.numel() * temp_costs.element_size(), temp_edges.data_ptr(),
        temp_edges.numel(), codebook.data_ptr(), int(K), int(tailbite_context), ctypes.c_double(lut_abs_max),
        _native.stream_handle(DEV))
    if rc != 0:
        raise RuntimeError(lib.qsrt_last_error().decode())


@pytest.mark.parametrize("bits", (2, 3, 4, 5))
@pytest.mark.parametrize("batch", (768, 40))
def test_reference_call_shape_matches_the_native_quantizer(bits, batch):
    print(f"[binding] K{bits}, traceback buffer of {batch} tiles", file=sys.stderr, flush=True)
    gen = torch.Generator().manual_seed(100 * bits + batch)
    tiles = torch.randn((1500, 256), generator=gen).to(DEV)
    costs, traceback, lut, lut_abs_max = _reference_inputs(bits, batch)
    out = torch.empty_like(tiles)
    idx = torch.empty(tiles.shape, dtype=torch.int16, device=DEV)
    quantize_tiles_sqg(tiles, out, idx, costs, traceback, lut, bits, 128, lut_abs_max)
    lag = boundary_lag(bits, lut_abs_max)
    recon, states = viterbi_tiles(tiles, sqg_xor_cheb_t12_bytes(bits).to(DEV), bits, tailbite_context=128, lag=lag)
    torch.cuda.synchronize()
    assert torch.equal(out, recon)
    assert torch.equal(idx, states)


def test_k2_boundary_rule_follows_the_label_bound():
    """A K2 table whose bound exceeds 16 takes the reference's generic kernel
    rule (lag 1) even though it is passed through the same entry point."""

    gen = torch.Generator().manual_seed(7)
    tiles = torch.randn((300, 256), generator=gen).to(DEV)
    costs, traceback, lut, _ = _reference_inputs(2, 768)
    out = torch.empty_like(tiles)
    idx = torch.empty(tiles.shape, dtype=torch.int16, device=DEV)
    quantize_tiles_sqg(tiles, out, idx, costs, traceback, lut, 2, 128, 17.0)
    recon, states = viterbi_tiles(tiles, sqg_xor_cheb_t12_bytes(2).to(DEV), 2, tailbite_context=128, lag=1)
    torch.cuda.synchronize()
    assert torch.equal(out, recon)
    assert torch.equal(idx, states)


def test_reference_call_shape_rejects_what_the_reference_rejects():
    tiles = torch.zeros((4, 256), device=DEV)
    costs, traceback, lut, amax = _reference_inputs(3, 768)
    out, idx = torch.empty_like(tiles), torch.empty(tiles.shape, dtype=torch.int16, device=DEV)
    with pytest.raises(RuntimeError, match="K1--K6"):
        quantize_tiles_sqg(tiles, out, idx, costs, traceback, lut, 7, 128, amax)
    with pytest.raises(RuntimeError, match="tailbite_context"):
        quantize_tiles_sqg(tiles, out, idx, costs, traceback, lut, 3, 0, amax)
    with pytest.raises(RuntimeError, match="temp_edges too small"):
        quantize_tiles_sqg(tiles, out, idx, costs, traceback[:1], lut, 3, 128, amax)  # 1 MiB < one workgroup's 2 MiB
