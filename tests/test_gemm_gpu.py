"""HIP matrix-core GEMM (qsrt_gemm_tn) against float64: the fused BlockLDLQ
feedback product C += alpha A^T (B - B2) in FP32 and the bf16 Hessian
capture H += X^T X, at ragged shapes, strided views and the LDLQ shapes."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from qsrt_amd import _native, gemm

pytestmark = pytest.mark.gpu


def _rel(got, want):
    return float(np.max(np.abs(got - want)) / max(np.abs(want).max(), 1e-30))


@pytest.mark.parametrize("M,N,K", [(16, 256, 112), (200, 300, 77), (128, 128, 16), (1, 5, 3), (640, 4096, 128),
                                   (96, 200, 129), (300, 260, 1000)])
def test_fused_feedback_product_matches_float64(M, N, K):
    print(f"[gemm] f32 M{M} N{N} K{K}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(M * 7 + N + K)
    A = torch.randn(K, M, generator=g)
    B = torch.randn(K, N, generator=g)
    B2 = torch.randn(K, N, generator=g)
    C = torch.randn(M, N, generator=g)
    want = C.double().numpy() + 0.5 * (A.double().numpy().T @ (B.double().numpy() - B2.double().numpy()))
    Cg = C.cuda()
    gemm.addmm_sub_tn_(Cg, A.cuda(), B.cuda(), B2.cuda(), alpha=0.5)
    assert _rel(Cg.cpu().double().numpy(), want) < 1e-5
    Cg = C.cuda()
    gemm.addmm_tn_(Cg, A.cuda(), B.cuda())
    assert _rel(Cg.cpu().double().numpy(), C.double().numpy() + A.double().numpy().T @ B.double().numpy()) < 1e-5


def test_strided_ldlq_views():
    # L[begin:end, :begin]^T (W - Q)[begin:end] into prod_cache[:begin], the span update of the recursion
    g = torch.Generator().manual_seed(3)
    k, n, begin, end = 512, 384, 256, 384
    L = torch.randn(k, k, generator=g).cuda()
    W = torch.randn(k, n, generator=g).cuda()
    Q = torch.randn(k, n, generator=g).cuda()
    P = torch.zeros(k, n).cuda()
    gemm.addmm_sub_tn_(P[:begin], L[begin:end, :begin], W[begin:end], Q[begin:end])
    want = L[begin:end, :begin].double().cpu().numpy().T @ (W[begin:end] - Q[begin:end]).double().cpu().numpy()
    assert _rel(P[:begin].cpu().double().numpy(), want) < 1e-5
    assert bool((P[begin:] == 0).all())
    # the per-block product with a 16-column slice of L (unaligned to the 128 tile)
    blk, blk_end = 272, 288
    comp = torch.zeros(16, n).cuda()
    gemm.addmm_sub_tn_(comp, L[blk_end:end, blk:blk_end], W[blk_end:end], Q[blk_end:end])
    want = L[blk_end:end, blk:blk_end].double().cpu().numpy().T @ (W[blk_end:end] - Q[blk_end:end]).double().cpu().numpy()
    assert _rel(comp.cpu().double().numpy(), want) < 1e-5


@pytest.mark.parametrize("n,k", [(4096, 256), (1000, 200), (777, 600), (130, 203), (64, 8), (3, 520)])
def test_bf16_gram_matches_float64(n, k):
    """Symmetric path: tiles on and above the diagonal plus their mirror;
    ragged k (padded leading dimension), ragged n (zero-filled K edge) and an
    accumulated, non-zero H."""

    print(f"[gemm] bf16 gram n{n} k{k}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(n + k)
    X = torch.randn(n, k, generator=g).bfloat16()
    H0 = torch.randn(k, k, generator=g)
    H = H0.cuda()
    gemm.gram_(H, X.cuda(), alpha=1.0 / n)
    x64 = X.double().numpy()
    want = H0.double().numpy() + x64.T @ x64 / n
    assert _rel(H.cpu().double().numpy(), want) < 1e-5
    Hf = torch.zeros(k, k).cuda()
    gemm.gram_(Hf, X.float().cuda())
    assert _rel(Hf.cpu().double().numpy(), x64.T @ x64) < 1e-5


def test_bf16_gram_full_size_matches_float64():
    """The Hessian capture at the config-4 shape: 16,384 bf16 rows x 7168
    channels.  Reference: the float64 product on the device (rocBLAS DGEMM),
    itself pinned on 64 sampled entries by float64 dot products on the CPU."""

    n, k = 16384, 7168
    print(f"[gemm] bf16 gram full size n{n} k{k}", file=sys.stderr, flush=True)
    g = torch.Generator(device="cuda").manual_seed(7168)
    X = torch.randn(n, k, device="cuda", generator=g).bfloat16()
    H = torch.zeros(k, k, device="cuda")
    gemm.gram_(H, X, alpha=1.0 / n)
    X64 = X.double()
    ref = (X64.T @ X64) / n
    del X64
    scale = ref.abs().max().item()
    assert (H.double() - ref).abs().max().item() / scale < 1e-5
    rng = np.random.default_rng(5)
    idx = rng.integers(0, k, size=(64, 2))
    xc = X.cpu().double().numpy()
    for i, j in idx:
        exact = float(xc[:, i] @ xc[:, j]) / n
        assert abs(ref[i, j].item() - exact) <= 1e-12 * scale
        assert abs(H[i, j].item() - exact) <= 1e-5 * scale
        assert H[i, j].item() == H[j, i].item()


@pytest.mark.parametrize("K,M,N", [(1000, 520, 264), (64, 256, 256), (129, 8, 600)])
def test_bf16_general_product_matches_float64(K, M, N):
    """Distinct operands take the full tile grid (no mirroring)."""

    print(f"[gemm] bf16 general K{K} M{M} N{N}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(K + M + N)
    A = torch.randn(K, M, generator=g).bfloat16()
    B = torch.randn(K, N, generator=g).bfloat16()
    C0 = torch.randn(M, N, generator=g)
    C = C0.cuda()
    gemm._launch(C, gemm._aligned(A.cuda(), 8), gemm._aligned(B.cuda(), 8), None, 0.25, 1)
    want = C0.double().numpy() + 0.25 * (A.double().numpy().T @ B.double().numpy())
    assert _rel(C.cpu().double().numpy(), want) < 1e-5


def _bf16_call(C, A, B, alpha, workspace=None, nbytes=None):
    """qsrt_gemm_tn_ws with an explicit workspace (None: qsrt_gemm_tn)."""

    lib = _native.lib()
    K, M = A.shape
    N = B.shape[1]
    stream = _native.stream_handle(C.device)
    if workspace is None:
        rc = lib.qsrt_gemm_tn(C.data_ptr(), A.data_ptr(), B.data_ptr(), None, M, N, K, A.stride(0), B.stride(0),
                              C.stride(0), float(alpha), 1, stream)
    else:
        rc = lib.qsrt_gemm_tn_ws(C.data_ptr(), A.data_ptr(), B.data_ptr(), None, M, N, K, A.stride(0), B.stride(0),
                                 C.stride(0), float(alpha), 1, workspace.data_ptr(),
                                 workspace.numel() if nbytes is None else nbytes, stream)
    assert rc == 0, lib.qsrt_last_error().decode()


@pytest.mark.parametrize("K,M,N,sym", [(640, 5888, 5888, True), (1000, 4504, 4504, False), (640, 4352, 4600, False),
                                       (16384, 7168, 7168, False)])
def test_bf16_split_last_round(K, M, N, sym):
    """Tile counts that leave the last round of CUs part-empty split that
    round's tiles along K (partials in the workspace, added in K order by the
    fixup kernel): the result matches float64 and the unsplit kernel to FP32
    rounding, is identical from call to call, and a short workspace runs the
    unsplit kernel bit for bit."""

    print(f"[gemm] bf16 split K{K} M{M} N{N} sym={sym}", file=sys.stderr, flush=True)
    g = torch.Generator(device="cuda").manual_seed(K + M + N)
    A = torch.randn(K, M, device="cuda", generator=g).bfloat16()
    B = A if sym else torch.randn(K, N, device="cuda", generator=g).bfloat16()
    C0 = torch.randn(M, N, device="cuda", generator=g)
    if sym:
        C0 = C0 + C0.T
    lib = _native.lib()
    nbytes = lib.qsrt_gemm_tn_workspace_bytes(C0.data_ptr(), A.data_ptr(), B.data_ptr(), M, N, K, A.stride(0),
                                              B.stride(0), C0.stride(0), 1)
    assert nbytes > 0 and nbytes % (256 * 1024) == 0  # split tiles x parts partials of 256 KiB
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    split = C0.clone()
    _bf16_call(split, A, B, 0.5, ws)
    again = C0.clone()
    _bf16_call(again, A, B, 0.5, ws)
    whole = C0.clone()
    _bf16_call(whole, A, B, 0.5)
    short = C0.clone()
    _bf16_call(short, A, B, 0.5, ws, nbytes - 16)
    torch.cuda.synchronize()
    assert torch.equal(split, again)
    assert torch.equal(short, whole)
    ref = C0.double() + 0.5 * (A.double().T @ B.double())
    scale = ref.abs().max().item()
    assert (split.double() - ref).abs().max().item() / scale < 1e-5
    assert (split - whole).abs().max().item() / scale < 1e-5
    if sym:
        assert torch.equal(split, split.T)
    assert not torch.equal(split, whole) or K < 128  # the split tiles did take the partial path
    # only the last round's tiles changed path: every other tile is the unsplit kernel's, bit for bit,
    # whichever wave of workgroups ran it
    tm, tn = -(-M // 256), -(-N // 256)
    tiles = tm * (tm + 1) // 2 if sym else tm * tn
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    pad = torch.zeros(tm * 256, tn * 256, dtype=torch.bool, device="cuda")
    pad[:M, :N] = split != whole
    moved = pad.view(tm, 256, tn, 256).any(dim=3).any(dim=1)
    if sym:
        moved = torch.triu(moved)
    assert int(moved.sum()) <= tiles % cus


def test_gemm_rejects_bad_arguments():
    A = torch.randn(4, 4).cuda()
    with pytest.raises(ValueError):
        gemm.addmm_sub_tn_(torch.zeros(4, 5).cuda(), A, torch.randn(4, 4).cuda())


@pytest.mark.parametrize("M,N,K", [(16, 256, 112), (200, 300, 77), (128, 128, 16), (2, 6, 3), (640, 2048, 128),
                                   (96, 200, 129), (7040, 256, 128)])
def test_float64_feedback_product_matches_float64(M, N, K):
    """qsrt_gemm_tn_f64: C (f64) += alpha A^T (B - B2) with float64 A, B and
    an FP32 B2 on the float64 matrix cores, against the same product on the
    CPU; both sides are float64, so they agree to float64 rounding."""

    print(f"[gemm] f64 M{M} N{N} K{K}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(M * 5 + N + K)
    A = torch.randn(K, M, generator=g, dtype=torch.float64)
    B = torch.randn(K, N, generator=g, dtype=torch.float64)
    B2 = torch.randn(K, N, generator=g)
    C = torch.randn(M, N, generator=g, dtype=torch.float64)
    for alpha, b2 in ((1.0, B2), (0.5, B2), (1.0, None)):
        rhs = B.numpy() - (0.0 if b2 is None else b2.double().numpy())
        want = C.numpy() + alpha * (A.numpy().T @ rhs)
        Cg = C.cuda()
        gemm.addmm_sub_tn_(Cg, A.cuda(), B.cuda(), None if b2 is None else b2.cuda(), alpha=alpha)
        assert _rel(Cg.cpu().numpy(), want) < 1e-13


def test_float64_span_update_is_width_independent():
    """Each column of C sums its K terms in one order whatever N is: a column
    block computed in a narrow launch equals the same columns of a wide one
    bit for bit (the candidate-reuse paths of the recursion rely on it), and
    repeated calls are identical."""

    g = torch.Generator().manual_seed(5)
    k, n, begin, end = 1024, 2048, 768, 896
    L = torch.randn(k, k, generator=g, dtype=torch.float64).cuda()
    W = torch.randn(k, n, generator=g, dtype=torch.float64).cuda()
    Q = torch.randn(k, n, generator=g).cuda()
    P0 = torch.randn(k, n, generator=g, dtype=torch.float64).cuda()
    wide = P0.clone()
    gemm.addmm_sub_tn_(wide[:begin], L[begin:end, :begin], W[begin:end], Q[begin:end])
    again = P0.clone()
    gemm.addmm_sub_tn_(again[:begin], L[begin:end, :begin], W[begin:end], Q[begin:end])
    assert torch.equal(wide, again)
    cols = slice(336, 336 + 48)
    narrow = P0[:, cols].contiguous()
    gemm.addmm_sub_tn_(narrow[:begin], L[begin:end, :begin], W[begin:end, cols].contiguous(),
                       Q[begin:end, cols].contiguous())
    assert torch.equal(narrow, wide[:, cols])
    want = P0[:begin].cpu().numpy() + L[begin:end, :begin].cpu().numpy().T @ (
        W[begin:end].cpu().numpy() - Q[begin:end].double().cpu().numpy())
    assert _rel(wide[:begin].cpu().numpy(), want) < 1e-13


@pytest.mark.parametrize("batch,k,n,begin,end", [(5, 1024, 2048, 768, 896), (3, 512, 200, 128, 256),
                                                 (40, 768, 384, 512, 640), (2, 256, 130, 112, 240)])
def test_float64_batched_span_update_equals_the_member_loop(batch, k, n, begin, end):
    """qsrt_gemm_tn_f64_batched over the views the recursion passes
    (prod_cache[:, :begin], Ls[:, begin:end, :begin], W[:, begin:end],
    Q[:, begin:end]) equals the per-member qsrt_gemm_tn_f64 loop bit for bit,
    with and without B2 and at a scaled alpha, and equals float64 on the CPU."""

    print(f"[gemm] f64 batched {batch} x [{begin} x {n}] K{end - begin}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(batch * 7 + k + n)
    L = torch.randn(batch, k, k, generator=g, dtype=torch.float64).cuda()
    W = torch.randn(batch, k, n, generator=g, dtype=torch.float64).cuda()
    Q = torch.randn(batch, k, n, generator=g).cuda()
    P0 = torch.randn(batch, k, n, generator=g, dtype=torch.float64).cuda()
    for alpha, q in ((1.0, Q), (-0.5, Q), (1.0, None)):
        loop = P0.clone()
        for b in range(batch):
            gemm.addmm_sub_tn_(loop[b, :begin], L[b, begin:end, :begin], W[b, begin:end],
                               None if q is None else q[b, begin:end], alpha=alpha)
        one = P0.clone()
        gemm.baddmm_sub_tn_f64_(one[:, :begin], L[:, begin:end, :begin], W[:, begin:end],
                                None if q is None else q[:, begin:end], alpha=alpha)
        assert torch.equal(one, loop)
    b = batch - 1
    want = P0[b, :begin].cpu().numpy() + L[b, begin:end, :begin].cpu().numpy().T @ W[b, begin:end].cpu().numpy()
    assert _rel(one[b, :begin].cpu().numpy(), want) < 1e-13


def test_float64_batched_span_update_argument_rules():
    """Overlapping members of C and odd member strides are refused by the
    C-ABI entry point with an error, before any launch; the Python wrapper
    falls back to the member loop for views the batched kernel cannot take."""

    C = torch.zeros(2, 64, 64, dtype=torch.float64).cuda()
    A = torch.zeros(2, 16, 64, dtype=torch.float64).cuda()
    B = torch.zeros(2, 16, 64, dtype=torch.float64).cuda()
    lib = _native.lib()
    stream = _native.stream_handle(C.device)
    # stride_c of 64 elements: member 1 would start on row 1 of member 0
    rc = lib.qsrt_gemm_tn_f64_batched(C.data_ptr(), A.data_ptr(), B.data_ptr(), None, 2, 64, 64, 16, 64, 64, 0, 64,
                                      64, 16 * 64, 16 * 64, 0, 1.0, stream)
    assert rc != 0 and b"overlap" in lib.qsrt_last_error()
    rc = lib.qsrt_gemm_tn_f64_batched(C.data_ptr(), A.data_ptr(), B.data_ptr(), None, 2, 64, 64, 16, 64, 64, 0, 64,
                                      64 * 64, 16 * 64 + 1, 16 * 64, 0, 1.0, stream)
    assert rc != 0 and b"even" in lib.qsrt_last_error()
    with pytest.raises(ValueError, match="incompatible"):
        gemm.baddmm_sub_tn_f64_(C, A, B[:, :8])
    # a column slice of C has members that the kernel could take, a transposed A does not: the loop serves it
    At = torch.randn(2, 64, 16, dtype=torch.float64).cuda().transpose(1, 2)
    Bm = torch.randn(2, 16, 64, dtype=torch.float64).cuda()
    want = C.clone()
    for b in range(2):
        want[b] += At[b].T @ Bm[b]
    gemm.baddmm_sub_tn_f64_(C, At, Bm)
    assert _rel(C.cpu().numpy(), want.cpu().numpy()) < 1e-13
