// Diagonal-block step of a blocked float64 Cholesky factorisation.
//
// block_ldl (reference qsrt/exl3_encoder_backend.py:323-393) factors the damped
// Hessian H = C C^T before forming L = C blockdiag(C_ii)^-1; here that
// factorisation runs in float64.  A right-looking blocked Cholesky spends its
// flops in the trailing updates A22 -= L21 L21^T, which are plain DGEMMs on
// the matrix cores; what a library factorisation of one matrix loses time on
// is the chain of small diagonal-block factorisations between them.  This
// kernel does one diagonal block in a single workgroup (registers and LDS), and
// also returns the block's inverse so that the panel solve
// L21 = A21 L11^-T becomes one more DGEMM.
//
// Block of nb <= 128 rows, 1024 threads: thread (ti, tj) = (t / 32, t % 32) keeps the 4 x 4 sub-block of
// rows 4 ti .. 4 ti + 3 and columns 4 tj .. 4 tj + 3 in registers for the whole call,
// so each elimination step is a branch-free outer-product update from one published column:
//   Cholesky  step k: the owners of column k publish it below the diagonal (zeros at and above it) and the
//             pivot a_kk; every thread computes d = sqrt(a_kk), l_ik = a_ik * (1 / d) (the reciprocal
//             multiply of LAPACK's dpotf2) for its rows and columns and does a_ij -= l_ik l_jk (fma); the
//             owners of column k then keep d and l_ik.  Entries above the diagonal are updated too and
//             never read.
//   inverse   X = L11^-1, X = I to start; step k: the owners of row k divide it by l_kk and publish it,
//             the owners of column k of L11 publish it below the diagonal, and every thread does
//             x_ic -= l_ik x_kc (fma).
// A wave whose rows all lie above row k has nothing left to update and skips the step.  Two barriers
// per step of each pass.  One workgroup per matrix of a batch.

#include "common.h"
#include "qsrt_amd.h"

namespace {

constexpr int kMaxNb = 128;
constexpr int kSub = 4;                              // rows and columns of a thread's sub-block
constexpr int kGroups = kMaxNb / kSub;               // sub-blocks per row of the block (32)
constexpr int kThreadsChol = kGroups * kGroups;      // 1024
constexpr int kRowGroupsPerWave = 64 / kGroups;      // 2

// The nb x nb diagonal block at (j0, j0) of matrix blockIdx.x (leading dimension n, batch stride
// `stride`): its lower triangle is read, the factor L11 is written over it with zeros above the
// diagonal, and L11^-1 goes to inv (nb x nb row-major per matrix, zeros above the diagonal).  A pivot
// k that is not positive (or NaN) stops the factorisation; info[b] then receives j0 + k + 1 unless it
// already holds an earlier failure, and the block and its inverse are left undefined.
__global__ __launch_bounds__(kThreadsChol) void chol_diag_block_f64_kernel(double* __restrict__ A, int64_t n,
                                                                           int64_t stride, int64_t j0, int nb,
                                                                           double* __restrict__ inv,
                                                                           int32_t* __restrict__ info) {
    __shared__ double colv[kMaxNb];  // the published column (Cholesky: a_ik; inverse: l_ik), zero at i <= k
    __shared__ double rowv[kMaxNb];  // inverse: the published row k of X
    __shared__ double diag[kMaxNb];  // l_kk
    __shared__ double pivot;
    const int t = static_cast<int>(threadIdx.x);
    const int ti = t / kGroups, tj = t % kGroups;
    const int i0 = kSub * ti, c0 = kSub * tj;
    const int wave_last_row = kSub * ((t >> 6) * kRowGroupsPerWave + kRowGroupsPerWave) - 1;  // of this wave
    double* M = A + static_cast<int64_t>(blockIdx.x) * stride + j0 * n + j0;
    double* Xo = inv + static_cast<int64_t>(blockIdx.x) * nb * nb;

    double a[kSub][kSub];
#pragma unroll
    for (int r = 0; r < kSub; ++r)
#pragma unroll
        for (int c = 0; c < kSub; ++c) {
            const int i = i0 + r, j = c0 + c;
            a[r][c] = i < nb && j <= i ? M[static_cast<int64_t>(i) * n + j] : 0.0;
        }

    int failed = 0;
    for (int k = 0; k < nb; ++k) {
        const int kc = k % kSub;
        if (tj == k / kSub) {
#pragma unroll
            for (int c = 0; c < kSub; ++c)
                if (c == kc) {  // uniform: k is the same for every thread
#pragma unroll
                    for (int r = 0; r < kSub; ++r) {
                        const int i = i0 + r;
                        colv[i] = i > k ? a[r][c] : 0.0;
                        if (i == k) pivot = a[r][c];
                    }
                }
        }
        __syncthreads();
        const double piv = pivot;  // the same value for every thread: the branch is uniform
        if (!(piv > 0.0)) {
            failed = k + 1;
            break;
        }
        if (wave_last_row >= k) {  // the wave holding row k finalises a_kk
            const double d = sqrt(piv), rd = 1.0 / d;
            double li[kSub], lj[kSub];
#pragma unroll
            for (int q = 0; q < kSub; ++q) {
                li[q] = colv[i0 + q] * rd;
                lj[q] = colv[c0 + q] * rd;
            }
#pragma unroll
            for (int r = 0; r < kSub; ++r)
#pragma unroll
                for (int c = 0; c < kSub; ++c) a[r][c] = fma(-li[r], lj[c], a[r][c]);
            if (tj == k / kSub) {
#pragma unroll
                for (int c = 0; c < kSub; ++c)
                    if (c == kc) {
#pragma unroll
                        for (int r = 0; r < kSub; ++r) {
                            const int i = i0 + r;
                            a[r][c] = i == k ? d : i > k ? li[r] : a[r][c];
                        }
                    }
            }
        }
        __syncthreads();
    }
    if (failed) {
        if (t == 0) atomicCAS(info + blockIdx.x, 0, static_cast<int32_t>(j0 + failed));
        return;
    }
#pragma unroll
    for (int r = 0; r < kSub; ++r)
#pragma unroll
        for (int c = 0; c < kSub; ++c) {
            const int i = i0 + r, j = c0 + c;
            if (i < nb && j < nb) M[static_cast<int64_t>(i) * n + j] = j <= i ? a[r][c] : 0.0;
            if (i == j && i < nb) diag[i] = a[r][c];
        }

    double x[kSub][kSub];
#pragma unroll
    for (int r = 0; r < kSub; ++r)
#pragma unroll
        for (int c = 0; c < kSub; ++c) x[r][c] = i0 + r == c0 + c && i0 + r < nb ? 1.0 : 0.0;
    __syncthreads();
    for (int k = 0; k < nb; ++k) {
        const int kc = k % kSub;
        if (ti == k / kSub) {
            const double lkk = diag[k];
#pragma unroll
            for (int r = 0; r < kSub; ++r)
                if (r == kc) {  // uniform
#pragma unroll
                    for (int c = 0; c < kSub; ++c) {
                        x[r][c] = x[r][c] / lkk;
                        rowv[c0 + c] = x[r][c];
                    }
                }
        }
        if (tj == k / kSub) {
#pragma unroll
            for (int c = 0; c < kSub; ++c)
                if (c == kc) {
#pragma unroll
                    for (int r = 0; r < kSub; ++r) colv[i0 + r] = i0 + r > k ? a[r][c] : 0.0;
                }
        }
        __syncthreads();
        if (wave_last_row > k) {
            double li[kSub], xk[kSub];
#pragma unroll
            for (int q = 0; q < kSub; ++q) {
                li[q] = colv[i0 + q];
                xk[q] = rowv[c0 + q];
            }
#pragma unroll
            for (int r = 0; r < kSub; ++r)
#pragma unroll
                for (int c = 0; c < kSub; ++c) x[r][c] = fma(-li[r], xk[c], x[r][c]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < kSub; ++r)
#pragma unroll
        for (int c = 0; c < kSub; ++c) {
            const int i = i0 + r, j = c0 + c;
            if (i < nb && j < nb) Xo[i * nb + j] = j <= i ? x[r][c] : 0.0;
        }
}

}  // namespace

// Unit block-lower factor from a lower Cholesky factor, in place: row i of column block j (i past the block's
// diagonal) becomes C[i, 16 j : 16 j + 16] inv_j, the diagonal 16 x 16 blocks become the identity, and the zero
// blocks above the diagonal are not touched.  One workgroup per (row chunk, column block, matrix); inv_j is
// staged in LDS and each thread owns one row: sixteen doubles read, sixteen 16-term products, sixteen written.
// Element (i, c) sits at i * ld + c (row-major, 16-byte loads along the row) or at c * ld + i (column-major, the
// layout torch's batched Cholesky returns: a wave's 64 rows are then 512 contiguous bytes per column).
constexpr int kUnitRows = 256;

template <bool kRowMajor>
__global__ __launch_bounds__(kUnitRows) void block_unit_lower_f64_kernel(double* __restrict__ C,
                                                                         const double* __restrict__ inv, int64_t n,
                                                                         int64_t ld, int64_t batch_stride) {
    const int64_t j = blockIdx.y, mat = blockIdx.z;
    const int64_t col0 = 16 * j;
    const int64_t row0 = col0 + static_cast<int64_t>(blockIdx.x) * kUnitRows;
    if (row0 >= n) return;  // the whole workgroup is past the last row
    __shared__ double iv[16][17];
    const double* ij = inv + (mat * (n / 16) + j) * 256;
    for (int e = threadIdx.x; e < 256; e += kUnitRows) iv[e >> 4][e & 15] = ij[e];
    __syncthreads();
    const int64_t row = row0 + threadIdx.x;
    if (row >= n) return;
    double* base = C + mat * batch_stride;
    const int64_t rs = kRowMajor ? ld : 1, cs = kRowMajor ? 1 : ld;
    double* r = base + row * rs + col0 * cs;
    if (row < col0 + 16) {  // the diagonal block
#pragma unroll
        for (int l = 0; l < 16; ++l) r[l * cs] = (row - col0 == l) ? 1.0 : 0.0;
        return;
    }
    double x[16];
    if constexpr (kRowMajor) {
#pragma unroll
        for (int k = 0; k < 16; k += 2) {
            const double2 v = *reinterpret_cast<const double2*>(r + k);
            x[k] = v.x;
            x[k + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) x[k] = r[k * cs];
    }
#pragma unroll
    for (int l = 0; l < 16; l += 2) {
        double a0 = 0.0, a1 = 0.0;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            a0 = __builtin_fma(x[k], iv[k][l], a0);
            a1 = __builtin_fma(x[k], iv[k][l + 1], a1);
        }
        if constexpr (kRowMajor) {
            *reinterpret_cast<double2*>(r + l) = make_double2(a0, a1);
        } else {
            r[l * cs] = a0;
            r[(l + 1) * cs] = a1;
        }
    }
}

extern "C" {

int qsrt_block_unit_lower_f64(double* C, const double* inv, int64_t batch, int64_t n, int64_t row_stride,
                              int64_t col_stride, int64_t batch_stride, void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (!C || !inv) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (n <= 0 || batch <= 0) return qsrt::fail(qsrt::kBadArgument, "n and batch must be positive");
    if (n % 16) return qsrt::fail(qsrt::kBadArgument, "n must be a multiple of 16");
    const bool row_major = col_stride == 1;
    if (!row_major && row_stride != 1)
        return qsrt::fail(qsrt::kBadArgument, "one of row_stride and col_stride must be 1");
    const int64_t ld = row_major ? row_stride : col_stride;
    if (ld < n) return qsrt::fail(qsrt::kBadArgument, "the leading dimension must be at least n");
    if (row_major && (ld % 2 || reinterpret_cast<uintptr_t>(C) % 16 || (batch > 1 && batch_stride % 2)))
        return qsrt::fail(qsrt::kBadArgument, "row-major matrices need 16-byte aligned rows");
    if (batch > 1 && batch_stride < (n - 1) * ld + n)
        return qsrt::fail(qsrt::kBadArgument, "the batch stride must keep the matrices apart");
    if (batch > 65535 || n / 16 > 65535) return qsrt::fail(qsrt::kBadArgument, "batch or n too large for one launch");
    const dim3 grid(static_cast<unsigned>((n + kUnitRows - 1) / kUnitRows), static_cast<unsigned>(n / 16),
                    static_cast<unsigned>(batch));
    const int64_t bs = batch > 1 ? batch_stride : 0;
    if (row_major)
        hipLaunchKernelGGL(block_unit_lower_f64_kernel<true>, grid, dim3(kUnitRows), 0, stream, C, inv, n, ld, bs);
    else
        hipLaunchKernelGGL(block_unit_lower_f64_kernel<false>, grid, dim3(kUnitRows), 0, stream, C, inv, n, ld, bs);
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

int qsrt_chol_diag_block_f64(double* A, int64_t n, int64_t batch, int64_t batch_stride, int64_t j0, int nb,
                             double* inv, int32_t* info, void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (!A || !inv || !info) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (n <= 0 || batch <= 0) return qsrt::fail(qsrt::kBadArgument, "n and batch must be positive");
    if (nb < 1 || nb > kMaxNb) return qsrt::fail(qsrt::kBadArgument, "nb must be in 1..%d", kMaxNb);
    if (j0 < 0 || j0 + nb > n) return qsrt::fail(qsrt::kBadArgument, "block [j0, j0 + nb) outside the matrix");
    if (batch > 1 && batch_stride < n * n) return qsrt::fail(qsrt::kBadArgument, "batch stride below n * n");
    if (batch > 0x7fffffff) return qsrt::fail(qsrt::kBadArgument, "batch too large for one launch");
    hipLaunchKernelGGL(chol_diag_block_f64_kernel, dim3(static_cast<unsigned>(batch)), dim3(kThreadsChol), 0, stream,
                       A, n, batch_stride, j0, nb, inv, info);
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

}  // extern "C"
