// Dense contractions of the encoder on the matrix cores:
//
//   C[M, N] += alpha * A^T (B - B2)       A: [K, M], B, B2: [K, N], all row-major
//
// * FP32 operands (the BlockLDLQ feedback products, reference
//   qsrt/exl3_encoder_backend.py:496 and :534: prod_cache += L^T (W - Q)):
//   v_mfma_f32_16x16x4_f32, exact FP32 products with FP32 accumulation; the
//   subtraction W - Q is fused into the operand load (B2 may be NULL).
// * bf16 operands (Hessian capture H += X^T X of BASELINE's kernel (c)):
//   v_mfma_f32_16x16x32_bf16 with FP32 accumulation; B2 must be NULL.
//
// One 256-thread workgroup per 128 x 128 tile of C (four waves of 64 x 64,
// sixteen 16 x 16 MFMA tiles each).  K is walked in chunks staged through
// LDS with double buffering: the next chunk's global loads are issued before
// the current chunk's MFMAs.  Edges of M, N and K are zero-filled on load and
// masked on store.

#include "common.h"
#include "qsrt_amd.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kBM = 128, kBN = 128, kThreads = 256;

// ---------------------------------------------------------------- FP32 path
constexpr int kBK32 = 16;
constexpr int kPad32 = 4;  // row pad of the [k][m] LDS tiles

struct F32Chunk {
    float4 a[2], b[2];
};

__device__ __forceinline__ float4 ld4_masked(const float* p, int64_t row, int64_t col, int64_t rows, int64_t cols,
                                             int64_t ld) {
    if (row >= rows) return make_float4(0.f, 0.f, 0.f, 0.f);
    const float* q = p + row * ld + col;
    if (col + 3 < cols) return *reinterpret_cast<const float4*>(q);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (col < cols) v.x = q[0];
    if (col + 1 < cols) v.y = q[1];
    if (col + 2 < cols) v.z = q[2];
    return v;
}

__device__ __forceinline__ void load_f32(F32Chunk& ch, const float* A, const float* B, const float* B2, int64_t k0,
                                         int64_t m0, int64_t n0, int64_t M, int64_t N, int64_t K, int64_t lda,
                                         int64_t ldb, int t) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int f = t + kThreads * i;  // 512 float4 per operand chunk: 16 rows x 32 float4
        const int r = f >> 5, q = f & 31;
        ch.a[i] = ld4_masked(A, k0 + r, m0 + 4 * q, K, M, lda);
        float4 b = ld4_masked(B, k0 + r, n0 + 4 * q, K, N, ldb);
        if (B2) {
            const float4 s = ld4_masked(B2, k0 + r, n0 + 4 * q, K, N, ldb);
            b.x -= s.x; b.y -= s.y; b.z -= s.z; b.w -= s.w;
        }
        ch.b[i] = b;
    }
}

__device__ __forceinline__ void store_f32(const F32Chunk& ch, float (*As)[kBM + kPad32], float (*Bs)[kBN + kPad32],
                                          int t) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int f = t + kThreads * i;
        const int r = f >> 5, q = f & 31;
        *reinterpret_cast<float4*>(&As[r][4 * q]) = ch.a[i];
        *reinterpret_cast<float4*>(&Bs[r][4 * q]) = ch.b[i];
    }
}

__global__ __launch_bounds__(kThreads) void gemm_tn_f32_kernel(float* __restrict__ C, const float* __restrict__ A,
                                                               const float* __restrict__ B,
                                                               const float* __restrict__ B2, int64_t M, int64_t N,
                                                               int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                                                               float alpha, int64_t tiles_n) {
    __shared__ __attribute__((aligned(16))) float As[2][kBK32][kBM + kPad32];
    __shared__ __attribute__((aligned(16))) float Bs[2][kBK32][kBN + kPad32];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int64_t m0 = (blockIdx.x / tiles_n) * kBM, n0 = (blockIdx.x % tiles_n) * kBN;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    F32Chunk ch;
    load_f32(ch, A, B, B2, 0, m0, n0, M, N, K, lda, ldb, t);
    store_f32(ch, As[0], Bs[0], t);
    __syncthreads();
    const int64_t chunks = (K + kBK32 - 1) / kBK32;
    for (int64_t kc = 0; kc < chunks; ++kc) {
        const int cur = kc & 1;
        if (kc + 1 < chunks) load_f32(ch, A, B, B2, (kc + 1) * kBK32, m0, n0, M, N, K, lda, ldb, t);
#pragma unroll
        for (int kk = 0; kk < kBK32 / 4; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[cur][4 * kk + g][wm + 16 * i + c];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[cur][4 * kk + g][wn + 16 * j + c];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kc + 1 < chunks) store_f32(ch, As[cur ^ 1], Bs[cur ^ 1], t);
        __syncthreads();
    }
    // lane holds C[wm + 16 i + 4 g + r][wn + 16 j + c]
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = m0 + wm + 16 * i + 4 * g + r;
            if (row >= M) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t col = n0 + wn + 16 * j + c;
                if (col < N) C[row * ldc + col] += alpha * acc[i][j][r];
            }
        }
}

// ---------------------------------------------------------------- bf16 path
constexpr int kBK16 = 32;
constexpr int kPad16 = 8;  // k-contiguous LDS rows: [m][k]

__global__ __launch_bounds__(kThreads) void gemm_tn_bf16_kernel(float* __restrict__ C, const uint16_t* __restrict__ A,
                                                                const uint16_t* __restrict__ B, int64_t M, int64_t N,
                                                                int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                                                                float alpha, int64_t tiles_n) {
    // transposed staging: row = m (or n), 32 contiguous k per row
    __shared__ __attribute__((aligned(16))) uint16_t As[kBM][kBK16 + kPad16];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[kBN][kBK16 + kPad16];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int64_t m0 = (blockIdx.x / tiles_n) * kBM, n0 = (blockIdx.x % tiles_n) * kBN;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int64_t k0 = 0; k0 < K; k0 += kBK16) {
        // 32 k-rows x 128 columns per operand: thread t takes k-row t / 8, columns 16 (t % 8) .. +15
        const int r = t >> 3, q = (t & 7) * 16;
        const int64_t krow = k0 + r;
#pragma unroll
        for (int op = 0; op < 2; ++op) {
            const uint16_t* P = op == 0 ? A : B;
            const int64_t cols = op == 0 ? M : N, base = op == 0 ? m0 : n0, ld = op == 0 ? lda : ldb;
            uint16_t (*S)[kBK16 + kPad16] = op == 0 ? As : Bs;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t col = base + q + e;
                S[q + e][r] = (krow < K && col < cols) ? P[krow * ld + col] : static_cast<uint16_t>(0);
            }
        }
        __syncthreads();
        bf16x8 a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const bf16x8*>(&As[wm + 16 * i + c][8 * g]);
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const bf16x8*>(&Bs[wn + 16 * j + c][8 * g]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = m0 + wm + 16 * i + 4 * g + r;
            if (row >= M) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t col = n0 + wn + 16 * j + c;
                if (col < N) C[row * ldc + col] += alpha * acc[i][j][r];
            }
        }
}

}  // namespace

extern "C" {

int qsrt_gemm_tn(float* C, const void* A, const void* B, const void* B2, int64_t M, int64_t N, int64_t K,
                 int64_t lda, int64_t ldb, int64_t ldc, float alpha, int dtype, void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (dtype != 0 && dtype != 1) return qsrt::fail(qsrt::kBadArgument, "dtype must be 0 (f32) or 1 (bf16)");
    if (M < 0 || N < 0 || K < 0) return qsrt::fail(qsrt::kBadArgument, "negative GEMM extent");
    if (M == 0 || N == 0 || K == 0) return qsrt::kOk;
    if (!C || !A || !B) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (lda < M || ldb < N || ldc < N)
        return qsrt::fail(qsrt::kBadArgument, "leading dimensions must cover the rows (lda >= M, ldb >= N, ldc >= N)");
    const int64_t tiles_n = (N + kBN - 1) / kBN;
    const int64_t tiles = ((M + kBM - 1) / kBM) * tiles_n;
    if (tiles > 0x7fffffff) return qsrt::fail(qsrt::kBadArgument, "GEMM too large for one launch");
    if (dtype == 0) {
        if (lda % 4 || ldb % 4 || reinterpret_cast<uintptr_t>(A) % 16 || reinterpret_cast<uintptr_t>(B) % 16 ||
            (B2 && reinterpret_cast<uintptr_t>(B2) % 16))
            return qsrt::fail(qsrt::kBadArgument, "f32 operands must be 16-byte aligned with lda, ldb multiples of 4");
        hipLaunchKernelGGL(gemm_tn_f32_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, stream, C,
                           static_cast<const float*>(A), static_cast<const float*>(B), static_cast<const float*>(B2),
                           M, N, K, lda, ldb, ldc, alpha, tiles_n);
    } else {
        if (B2) return qsrt::fail(qsrt::kBadArgument, "the bf16 path has no fused subtraction");
        hipLaunchKernelGGL(gemm_tn_bf16_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, stream, C,
                           static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), M, N, K, lda, ldb, ldc,
                           alpha, tiles_n);
    }
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

}  // extern "C"
