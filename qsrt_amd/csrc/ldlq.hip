// BlockLDLQ step kernels: the per-16-row-block work of the recursion around
// the tile Viterbi, for a batch of members in one launch each.
//
// Reference (qsrt/exl3_encoder_backend.py:420-539 ldlq, :1190-1478
// ldlq_mixed_batched): for the 16-row block [blk, blk + 16) of a span
// [begin, end), member m (weight of source s = src[m]) is quantized against
//   T = W_s[blk] + mult_m * (P_m[blk] + L_s[blk_end:end, blk]^T (W_s - Q_m)[blk_end:end])
// with P_m the product cache of the spans already committed.  The reference
// runs that as a clone, a product, an add, a stack, a tensor-core gather and
// a rate-group gather per step; here it is one launch that writes each
// member's target tiles, in tensor-core order, straight into their slot of
// the rate-grouped tile buffer the Viterbi reads.  After the Viterbi a second
// launch writes the reconstruction back into Q_m's rows and the states into
// the member's encoded tile row.
//
// Precision: W, L and P are float64 and Q is FP32 (exact labels); every sum is
// float64 and the target is rounded to FP32 once, on its way into the tile
// buffer.  Sum order: every target element accumulates P first, then the
// products in increasing row order, whatever the batch or matrix width -- so
// candidates encoded in different batch shapes stay bit-identical.

#include "common.h"
#include "qsrt_amd.h"

namespace {

constexpr int kThreads = 256;  // one 16 x 16 tile per workgroup
constexpr int kChunk = 64;     // feedback rows staged in LDS per round

// Position of row r, column c of a 16 x 16 tile in tensor-core order: lane
// t holds rows 2 (t % 4) + {0, 1, 8, 9} and columns t / 4 + {0, 8}, 8
// values per lane (qsrt/exl3_reference.py:86-105).
__device__ __forceinline__ int tc_pos(int r, int c) {
    const int lane = 4 * (c & 7) + ((r & 7) >> 1);
    return 8 * lane + 4 * (c >> 3) + (r & 1) + 2 * (r >> 3);
}

__global__ __launch_bounds__(kThreads) void ldlq_targets_kernel(
    float* __restrict__ tiles, const double* __restrict__ W, const double* __restrict__ L,
    const float* __restrict__ Q, const double* __restrict__ P, const int32_t* __restrict__ src,
    const double* __restrict__ mult, const int32_t* __restrict__ slot, int64_t K, int64_t N, int64_t sW, int64_t sL,
    int64_t sQ, int64_t sP, int64_t blk, int64_t rows) {
    __shared__ double ls[kChunk][16];  // L_s[blk_end + j, blk + r]
    __shared__ double ds[kChunk][17];  // (W_s - Q_m)[blk_end + j, 16 t + c], padded against bank conflicts
    const int t = blockIdx.x, m = blockIdx.y, nt = gridDim.x;
    const int tid = threadIdx.x, r = tid >> 4, c = tid & 15;
    const int64_t s = src[m];
    const double* Ws = W + s * sW;
    const double* Ls = L + s * sL;
    const float* Qm = Q + m * sQ;
    const int64_t e = (blk + r) * N + 16 * t + c;
    double acc = P[m * sP + e];
    for (int64_t j0 = 0; j0 < rows; j0 += kChunk) {
        const int n = static_cast<int>(rows - j0 < kChunk ? rows - j0 : kChunk);
        for (int i = tid; i < n * 16; i += kThreads) {
            const int j = i >> 4, cc = i & 15;
            const int64_t row = blk + 16 + j0 + j;
            ls[j][cc] = Ls[row * K + blk + cc];
            ds[j][cc] = Ws[row * N + 16 * t + cc] - static_cast<double>(Qm[row * N + 16 * t + cc]);
        }
        __syncthreads();
        for (int j = 0; j < n; ++j) acc = __builtin_fma(ls[j][r], ds[j][c], acc);
        __syncthreads();
    }
    const double w = Ws[e];
    const double k = mult[m];
    const double target = k == 1.0 ? w + acc : (k == 0.0 ? w : w + k * acc);
    tiles[static_cast<int64_t>(slot[m * nt + t]) * 256 + tc_pos(r, c)] = static_cast<float>(target);
}

__global__ __launch_bounds__(kThreads) void ldlq_commit_kernel(
    float* __restrict__ Q, int16_t* __restrict__ E, const float* __restrict__ recon, const uint16_t* __restrict__ states,
    const int32_t* __restrict__ slot, int64_t N, int64_t sQ, int64_t sE, int64_t blk) {
    const int t = blockIdx.x, m = blockIdx.y, nt = gridDim.x;
    const int tid = threadIdx.x, r = tid >> 4, c = tid & 15;
    const int64_t g = slot[m * nt + t];
    Q[m * sQ + (blk + r) * N + 16 * t + c] = recon[g * 256 + tc_pos(r, c)];
    E[m * sE + ((blk >> 4) * nt + t) * 256 + tid] = static_cast<int16_t>(states[g * 256 + tid]);
}

}  // namespace

extern "C" {

int qsrt_ldlq_targets(float* tiles, const double* W, const double* L, const float* Q, const double* P,
                      const int32_t* src, const double* mult, const int32_t* slot, int B, int64_t K, int64_t N,
                      int64_t sW, int64_t sL, int64_t sQ, int64_t sP, int64_t blk, int64_t end, void* stream) {
    if (B < 0 || K <= 0 || N <= 0 || N % 16 || K % 16)
        return qsrt::fail(qsrt::kBadArgument, "ldlq targets: need B >= 0 and K, N positive multiples of 16");
    if (blk < 0 || blk % 16 || blk + 16 > end || end > K)
        return qsrt::fail(qsrt::kBadArgument, "ldlq targets: need a 16-aligned block inside [0, end], end <= K");
    if (B == 0) return qsrt::kOk;
    if (!tiles || !W || !L || !Q || !P || !src || !mult || !slot)
        return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (N / 16 > 65535 || B > 65535) return qsrt::fail(qsrt::kBadArgument, "ldlq targets: grid too large");
    hipLaunchKernelGGL(ldlq_targets_kernel, dim3(static_cast<unsigned>(N / 16), static_cast<unsigned>(B)),
                       dim3(kThreads), 0, static_cast<hipStream_t>(stream), tiles, W, L, Q, P, src, mult, slot, K, N,
                       sW, sL, sQ, sP, blk, end - blk - 16);
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

int qsrt_ldlq_commit(float* Q, int16_t* encoded, const float* recon, const uint16_t* states, const int32_t* slot,
                     int B, int64_t K, int64_t N, int64_t sQ, int64_t sE, int64_t blk, void* stream) {
    if (B < 0 || K <= 0 || N <= 0 || N % 16 || K % 16)
        return qsrt::fail(qsrt::kBadArgument, "ldlq commit: need B >= 0 and K, N positive multiples of 16");
    if (blk < 0 || blk % 16 || blk + 16 > K) return qsrt::fail(qsrt::kBadArgument, "ldlq commit: bad block");
    if (B == 0) return qsrt::kOk;
    if (!Q || !encoded || !recon || !states || !slot) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (N / 16 > 65535 || B > 65535) return qsrt::fail(qsrt::kBadArgument, "ldlq commit: grid too large");
    hipLaunchKernelGGL(ldlq_commit_kernel, dim3(static_cast<unsigned>(N / 16), static_cast<unsigned>(B)),
                       dim3(kThreads), 0, static_cast<hipStream_t>(stream), Q, encoded, recon, states, slot, N, sQ, sE,
                       blk);
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

}  // extern "C"
