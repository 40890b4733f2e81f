"""HIP BaKron band update (qsrt_bakron_band_update_f32, through
qsrt_amd.sqg_quantizer.apply_bakron_block_update and the C ABI) against the
float64 oracle (oracle/bakron.py).

Bar: FP32 on the matrix cores, so every element of the updated targets and
of the intermediate is within 1e-5 of the float64 value relative to the same
sums taken over absolute values (|Lout| |Q - T| |Lin|^T), plus one FP32 ulp
of the result (the kernel stores T + update rounded to FP32) and 1e-7.
Blocks outside the bands must be untouched bit for bit; the intermediate is
pre-filled with NaN, so a read of a block the call did not write shows up.
At the full config-4 gate shape the reference is the dense masked product in
float64 on the device.  The encoders: a lockstep batch equals independent
encodes bit for bit, and a
shared rank-2 factor equals the same factor expanded per member (the
reference's tests/test_two_sided_rounding.py:244-326)."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import oracle.bakron as bk
from qsrt_amd import _native
from qsrt_amd.sqg_quantizer import apply_bakron_block_update
from qsrt_amd.two_sided_rounding import (bakron_block_round_encoder, bakron_block_round_encoder_batch,
                                         bakron_block_round_encoder_prepared_batch, factor_bakron_hessian)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
B = 16
REL = 1e-5
ABS = 1e-7
ULP = 2.0 ** -23  # one FP32 ulp relative to the value


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _block_lower(n, rng):
    m = n // B
    f = rng.standard_normal((n, n)) / np.sqrt(n)
    f *= np.kron(np.tril(np.ones((m, m))), np.ones((B, B)))
    for j in range(m):
        f[j * B:(j + 1) * B, j * B:(j + 1) * B] = np.eye(B)
    return f


def _inputs(batch, n_out, n_in, seed, shared):
    rng = np.random.default_rng(seed)
    T = rng.standard_normal((batch, n_out, n_in)).astype(np.float32)
    Q = (np.round(T * 4) / 4 + 0.01 * rng.standard_normal(T.shape)).astype(np.float32)
    if shared:
        lo, li = _block_lower(n_out, rng).astype(np.float32), _block_lower(n_in, rng).astype(np.float32)
    else:
        lo = np.stack([_block_lower(n_out, rng) for _ in range(batch)]).astype(np.float32)
        li = np.stack([_block_lower(n_in, rng) for _ in range(batch)]).astype(np.float32)
    return T, Q, lo, li


def _run(T, Q, lo, li, first, middle, last, block_lower=False):
    ws = torch.from_numpy(T.copy()).to(DEV)
    inter = torch.full(T.shape, float("nan"), dtype=torch.float32, device=DEV)
    apply_bakron_block_update(ws, torch.from_numpy(Q).to(DEV), torch.from_numpy(lo).to(DEV),
                              torch.from_numpy(li).to(DEV), inter, first_diagonal=first, middle_diagonal=middle,
                              last_diagonal=last, block_size=B, block_lower=block_lower)
    torch.cuda.synchronize()
    return ws.cpu().numpy(), inter.cpu().numpy()


def _check(T, Q, lo, li, first, middle, last):
    got_t, got_i = _run(T, Q, lo, li, first, middle, last)
    # the block-lower entry point skips the zero blocks of these factors: the same values (== also equates -0, 0)
    low_t, low_i = _run(T, Q, lo, li, first, middle, last, block_lower=True)
    assert np.array_equal(low_t, got_t) and np.array_equal(low_i, got_i, equal_nan=True)
    T64, Q64 = T.astype(np.float64), Q.astype(np.float64)
    want_t, want_i = bk.band_update_batch(T64, Q64, lo.astype(np.float64), li.astype(np.float64), first, middle,
                                          last)
    abs_t, abs_i = bk.band_update_batch(np.zeros_like(T64), np.abs(Q64 - T64), np.abs(lo.astype(np.float64)),
                                        np.abs(li.astype(np.float64)), first, middle, last)
    n_out, n_in = T.shape[-2:]
    band_i = bk.band_mask(n_out, n_in, first, last)
    band_t = bk.band_mask(n_out, n_in, middle, last)
    worst = 0.0
    for j in range(T.shape[0]):
        assert np.array_equal(got_t[j][~band_t], T[j][~band_t]), "targets outside the next band changed"
        assert np.all(np.isnan(got_i[j][~band_i])), "intermediate written outside [first, last)"
        assert np.all(np.isfinite(got_i[j][band_i])) and np.all(np.isfinite(got_t[j]))
        err_t = np.abs(got_t[j][band_t] - want_t[j][band_t])
        err_i = np.abs(got_i[j][band_i] - want_i[j][band_i])
        assert np.all(err_t <= REL * abs_t[j][band_t] + ULP * np.abs(want_t[j][band_t]) + ABS), float(err_t.max())
        assert np.all(err_i <= REL * abs_i[j][band_i] + ULP * np.abs(want_i[j][band_i]) + ABS), float(err_i.max())
        worst = max(worst, float((err_t / (abs_t[j][band_t] + 1e-30)).max()))
    return worst


CASES = [
    (1, 64, 96, 0, 4, 9, False), (1, 64, 96, 2, 3, 5, False), (1, 96, 48, 0, 1, 8, False),
    (1, 96, 48, 3, 6, 8, False), (1, 48, 48, 0, 2, 5, False), (1, 128, 32, 1, 5, 9, False),
    (1, 16, 16, 0, 0, 0, False),
    (1, 256, 768, 0, 31, 63, False), (1, 768, 256, 20, 41, 63, False), (1, 512, 512, 5, 6, 63, False),
    (3, 128, 192, 0, 9, 19, False), (3, 128, 192, 4, 11, 17, True),
]


@pytest.mark.parametrize("batch,n_out,n_in,first,middle,last,shared", CASES)
def test_band_update_matches_the_float64_oracle(batch, n_out, n_in, first, middle, last, shared):
    if last == 0:  # 16 x 16: a single diagonal, no band pair exists; the call must be rejected
        T, Q, lo, li = _inputs(1, 16, 16, 1, False)
        with pytest.raises(ValueError):
            _run(T, Q, lo, li, 0, 1, 2)
        return
    _say(f"[bakron] band update batch={batch} {n_out}x{n_in} [{first},{middle},{last}) shared={shared}")
    T, Q, lo, li = _inputs(batch, n_out, n_in, 100 + n_out + n_in + first + last, shared)
    worst = _check(T, Q, lo, li, first, middle, last)
    _say(f"[bakron]   worst error / |terms| {worst:.2e}")


def test_every_band_of_a_recursion_matches_the_oracle():
    n_out, n_in = 96, 160
    D = n_out // B + n_in // B - 1
    T, Q, lo, li = _inputs(1, n_out, n_in, 77, False)
    bands = []

    def rec(first, last):
        if last == first + 1:
            return
        mid = (first + last) // 2
        rec(first, mid)
        bands.append((first, mid, last))
        rec(mid, last)

    rec(0, D)
    _say(f"[bakron] {len(bands)} bands of a {n_out}x{n_in} recursion")
    for first, mid, last in bands:
        _check(T, Q, lo, li, first, mid, last)


def test_the_c_abi_rejects_bad_arguments():
    lib = _native.lib()
    ws, q, inter = (torch.zeros((64, 96), device=DEV) for _ in range(3))
    f_out, f_in = torch.eye(64, device=DEV), torch.eye(96, device=DEV)
    p = [ws.data_ptr(), q.data_ptr(), f_out.data_ptr(), f_in.data_ptr(), inter.data_ptr()]
    s = _native.stream_handle(DEV)
    assert lib.qsrt_bakron_band_update_f32(*p, 1, 64, 96, 0, 0, 0, 4, 9, s) == 0
    for args in ((1, 64, 96, 0, 0, 0, 4, 10), (1, 64, 96, 0, 0, 4, 4, 9), (1, 64, 90, 0, 0, 0, 4, 9),
                 (0, 64, 96, 0, 0, 0, 4, 9), (2, 64, 96, 100, 0, 0, 4, 9), (1, 64, 96, 0, 0, -1, 4, 9)):
        assert lib.qsrt_bakron_band_update_f32(*p, *args, s) == -1, args
    assert lib.qsrt_bakron_band_update_f32(None, *p[1:], 1, 64, 96, 0, 0, 0, 4, 9, s) == -1
    torch.cuda.synchronize()


def test_overlapping_buffers_are_rejected():
    ws = torch.zeros((64, 96), device=DEV)
    q = torch.zeros_like(ws)
    f_out, f_in = torch.eye(64, device=DEV), torch.eye(96, device=DEV)
    big = torch.zeros((2, 64, 96), device=DEV)
    kw = dict(first_diagonal=0, middle_diagonal=4, last_diagonal=9, block_size=16)
    with pytest.raises(ValueError, match="intermediate"):
        apply_bakron_block_update(ws, q, f_out, f_in, ws, **kw)
    with pytest.raises(ValueError, match="intermediate"):
        apply_bakron_block_update(big[0], q, f_out, f_in, big.view(-1)[100:100 + 64 * 96].view(64, 96), **kw)
    with pytest.raises(ValueError, match="workspace"):
        apply_bakron_block_update(ws, ws, f_out, f_in, torch.empty_like(ws), **kw)
    apply_bakron_block_update(big[0], q, f_out, f_in, big[1], **kw)  # adjacent, not overlapping
    torch.cuda.synchronize()


def _spd(n, seed):
    g = torch.Generator().manual_seed(seed)
    root = torch.randn((3 * n, n), generator=g)
    return root.T @ root / (3 * n) + 0.3 * torch.eye(n)


def _round_tiles(tiles):
    code = torch.round(tiles * 4).to(torch.int16)
    return code.to(tiles.dtype) / 4, code


def test_lockstep_batch_equals_independent_hip_encodes_exactly():
    _say("[bakron] batch of 2 x 32x48 vs independent, HIP updates")
    g = torch.Generator().manual_seed(8100)
    w = torch.randn((2, 32, 48), generator=g).to(DEV)
    h_in = torch.stack((_spd(32, 8101), _spd(32, 8102))).to(DEV)
    h_out = torch.stack((_spd(48, 8103), _spd(48, 8104))).to(DEV)
    batched = bakron_block_round_encoder_batch(w, h_in, h_out, _round_tiles)
    for j in range(2):
        one = bakron_block_round_encoder(w[j], h_in[j], h_out[j], _round_tiles, work_dtype=torch.float32,
                                         update_backend="cuda")
        assert torch.equal(batched.reconstruction[j], one.reconstruction)
        assert torch.equal(batched.payload[j], one.payload)


def test_prepared_shared_factor_equals_the_expanded_batch():
    _say("[bakron] prepared batch with one shared input factor")
    g = torch.Generator().manual_seed(8200)
    w = torch.randn((3, 32, 48), generator=g).to(DEV)
    h_in = _spd(32, 8201).to(DEV)
    h_out = torch.stack([_spd(48, 8202 + j) for j in range(3)]).to(DEV)
    f_in, r_in = factor_bakron_hessian(h_in)
    outs = [factor_bakron_hessian(h_out[j]) for j in range(3)]
    prepared = bakron_block_round_encoder_prepared_batch(w, f_in, torch.stack([f for f, _ in outs]), r_in,
                                                         outs[0][1], _round_tiles)
    expected = bakron_block_round_encoder_batch(w, h_in.expand(3, -1, -1).contiguous(), h_out, _round_tiles)
    assert torch.equal(prepared.reconstruction, expected.reconstruction)
    assert torch.equal(prepared.payload, expected.payload)


def test_hip_updates_choose_the_float64_path():
    k, n = 256, 384
    _say(f"[bakron] {k}x{n} encode, HIP FP32 updates vs float64 products")
    g = torch.Generator().manual_seed(8300)
    w = torch.randn((k, n), generator=g)
    h_in, h_out = _spd(k, 8301), _spd(n, 8302)
    hip = bakron_block_round_encoder(w.to(DEV), h_in.to(DEV), h_out.to(DEV), _round_tiles,
                                     work_dtype=torch.float32)
    ref = bakron_block_round_encoder(w.double(), h_in.double(), h_out.double(), _round_tiles,
                                     work_dtype=torch.float64)
    differ = float((hip.payload.cpu().long() != ref.payload.long()).double().mean())
    _say(f"[bakron]   payload elements differing from the float64 encode: {differ:.2e}")
    assert differ <= 1e-3


def _band_mask_t(ob, ib, first, last):
    o = torch.arange(ob, device=DEV)[:, None]
    i = torch.arange(ib, device=DEV)[None, :]
    m = ((o + i) >= first) & ((o + i) < last)
    return m.repeat_interleave(B, 0).repeat_interleave(B, 1)


@pytest.mark.parametrize("first,middle,last", [(0, 287, 575), (143, 215, 287), (500, 501, 575)])
def test_config4_gate_bands_match_the_dense_float64_product(first, middle, last):
    """Full config-4 gate shape (2048 x 7168 in the encoder orientation): the
    kernel against T + M2 (Lout (M1 (Q - T)) Lin^T) in float64 on the device,
    the dense form the CPU tests pin to the block oracle for block-lower
    factors; same bar as above."""

    n_out, n_in = 2048, 7168
    ob, ib = n_out // B, n_in // B
    _say(f"[bakron] config-4 gate {n_out}x{n_in} band [{first},{middle},{last})")
    g = torch.Generator(device=DEV).manual_seed(9000 + first)
    T = torch.randn((n_out, n_in), device=DEV, generator=g)
    Q = torch.round(T * 4) / 4 + 0.01 * torch.randn((n_out, n_in), device=DEV, generator=g)
    lo = torch.randn((n_out, n_out), device=DEV, generator=g) / n_out ** 0.5
    li = torch.randn((n_in, n_in), device=DEV, generator=g) / n_in ** 0.5
    lo *= torch.kron(torch.tril(torch.ones(ob, ob, device=DEV)), torch.ones(B, B, device=DEV))
    li *= torch.kron(torch.tril(torch.ones(ib, ib, device=DEV)), torch.ones(B, B, device=DEV))
    ws = T.clone()
    inter = torch.full_like(T, float("nan"))
    apply_bakron_block_update(ws, Q, lo, li, inter, first_diagonal=first, middle_diagonal=middle,
                              last_diagonal=last, block_size=B)
    ws_low, inter_low = T.clone(), torch.full_like(T, float("nan"))
    apply_bakron_block_update(ws_low, Q, lo, li, inter_low, first_diagonal=first, middle_diagonal=middle,
                              last_diagonal=last, block_size=B, block_lower=True)
    torch.cuda.synchronize()
    assert torch.equal(ws_low, ws) and torch.equal(inter_low.nan_to_num(7.0), inter.nan_to_num(7.0))
    m1 = _band_mask_t(ob, ib, first, middle)
    m2 = _band_mask_t(ob, ib, middle, last)
    mi = _band_mask_t(ob, ib, first, last)
    delta = torch.where(m1, (Q - T).double(), 0.0)
    left = lo.double() @ delta
    want = T.double() + torch.where(m2, left @ li.double().t().contiguous(), 0.0)
    abs_left = lo.double().abs() @ delta.abs()
    abs_upd = abs_left @ li.double().abs().t().contiguous()
    assert torch.equal(ws[~m2], T[~m2]), "targets outside the next band changed"
    assert bool(torch.isnan(inter[~mi]).all()), "intermediate written outside [first, last)"
    err_t = (ws.double() - want).abs()[m2]
    err_i = (inter.double() - left).abs()[mi]
    assert bool((err_t <= REL * abs_upd[m2] + ULP * want[m2].abs() + ABS).all()), float(err_t.max())
    assert bool((err_i <= REL * abs_left[mi] + ULP * left[mi].abs() + ABS).all()), float(err_i.max())
    _say(f"[bakron]   worst error / |terms| {float((err_t / (abs_upd[m2] + 1e-30)).max()):.2e}")
