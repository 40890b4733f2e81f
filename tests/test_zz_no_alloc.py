"""``qsrt_decode_noalloc`` (the decode whose job table is the library's own
device array) against ``qsrt_decode`` (the same decode with a caller
workspace), through the C-ABI: bit-identical outputs on two calls in a row,
the second with a smaller input, and the size limit rejected with a clear
error before any GPU work."""

from __future__ import annotations

import ctypes
import sys

import pytest
import torch

from qsrt_amd import _native
from qsrt_amd.exl3_reference import reconstruct_trellis_states
from qsrt_amd.qsrt import pack_trellis_edges
from qsrt_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
MAX_JOBS = 4096


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _matrix(k: int, n: int, bits: int, seed: int):
    """Closed random paths for a [k, n] matrix at rate ``bits``: device words,
    scales and the two output buffers."""

    g = torch.Generator().manual_seed(seed)
    edges = torch.randint(0, 1 << bits, (k // 16, n // 16, 256), generator=g)
    states = reconstruct_trellis_states(edges, bits)
    words = pack_trellis_edges(states.reshape(-1, 256), bits).reshape(k // 16, n // 16, 16 * bits).to(DEV)
    su = ((torch.rand(k, generator=g) + 0.5) / 128.0).to(DEV)
    sv = (torch.rand(n, generator=g) - 0.5).to(DEV)
    outs = [torch.full((k, n), float("nan"), dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    return words.contiguous(), su, sv, outs


def _job(words, su, sv, out, bits):
    kt, nt, _ = words.shape
    return _native.DecodeJob(words.data_ptr(), nt * 16 * bits, 16 * bits, su.data_ptr(), sv.data_ptr(), out.data_ptr(),
                             out.stride(0), 16 * kt, 16 * nt, 0, 0)


def _decode_both(mats, bits):
    lib = _native.lib()
    lut = sqg_xor_cheb_t12_bytes(bits).to(DEV)
    stream = _native.stream_handle(DEV)
    for slot in (0, 1):
        jobs = [_job(w, su, sv, outs[slot], bits) for w, su, sv, outs in mats]
        arr = (_native.DecodeJob * len(jobs))(*jobs)
        if slot == 0:
            ws = torch.empty(int(lib.qsrt_decode_workspace_bytes(len(jobs))), dtype=torch.uint8, device=DEV)
            rc = lib.qsrt_decode(ctypes.cast(arr, ctypes.c_void_p), len(jobs), bits, lut.data_ptr(), 1, 0,
                                 ws.data_ptr(), ws.numel(), stream)
        else:
            rc = lib.qsrt_decode_noalloc(ctypes.cast(arr, ctypes.c_void_p), len(jobs), bits, lut.data_ptr(), 1, 0,
                                         stream)
        _native.check(rc, "qsrt_decode" if slot == 0 else "qsrt_decode_noalloc")
    torch.cuda.synchronize()
    for _, _, _, outs in mats:
        assert not torch.isnan(outs[1].float()).any(), "the no-allocation decode left outputs unwritten"
        assert torch.equal(outs[0], outs[1])


def test_noalloc_decode_matches_workspace_decode_twice_then_smaller():
    _say("[noalloc] call 1: 20 K3 matrices (512 x 256 .. 1024 x 768), 20 jobs")
    first = [_matrix(512 + 128 * (i % 5), 256 + 128 * (i % 5), 3, 100 + i) for i in range(20)]
    _decode_both(first, 3)
    _say("[noalloc] call 2: 3 smaller K2 matrices (256 x 128), 3 jobs")
    second = [_matrix(256, 128, 2, 200 + i) for i in range(3)]
    _decode_both(second, 2)


def test_noalloc_decode_rejects_more_jobs_than_its_table():
    _say("[noalloc] size limit")
    lib = _native.lib()
    words, su, sv, outs = _matrix(128, 128, 2, 300)
    jobs = [_job(words, su, sv, outs[0], 2)] * (MAX_JOBS + 1)
    arr = (_native.DecodeJob * len(jobs))(*jobs)
    lut = sqg_xor_cheb_t12_bytes(2).to(DEV)
    rc = lib.qsrt_decode_noalloc(ctypes.cast(arr, ctypes.c_void_p), len(jobs), 2, lut.data_ptr(), 1, 0,
                                 _native.stream_handle(DEV))
    assert rc == -1
    assert b"at most 4096 jobs" in lib.qsrt_last_error()
    torch.cuda.synchronize()
    assert torch.isnan(outs[0].float()).all()  # nothing ran
