// Dense contractions of the encoder on the matrix cores:
//
//   C[M, N] += alpha * A^T (B - B2)       A: [K, M], B, B2: [K, N], all row-major
//
// * FP32 operands (the BlockLDLQ feedback products, reference
//   qsrt/exl3_encoder_backend.py:496 and :534: prod_cache += L^T (W - Q)):
//   v_mfma_f32_16x16x4_f32, exact FP32 products with FP32 accumulation; the
//   subtraction W - Q is fused into the operand load (B2 may be NULL).
// * bf16 operands (Hessian capture H += X^T X / n, the H_data["H"] that
//   qsrt/exl3_encoder_backend.py:2077-2122 finalises; the reference's in-tree
//   accumulator, qsrt/kimi_reverse_pipeline.py:95-111, is an FP32 addmm_):
//   v_mfma_f32_16x16x32_bf16 with FP32 accumulation; B2 must be NULL.
//
// FP32: one 256-thread workgroup per 128 x 128 tile of C (four waves of
// 64 x 64, sixteen 16 x 16 MFMA tiles each); K is walked in chunks staged
// through LDS with double buffering, the next chunk's global loads issued
// before the current chunk's MFMAs; edges of M, N and K are zero-filled on
// load and masked on store.  bf16: see the comment above its kernel.

#include "common.h"
#include "qsrt_amd.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kBM = 128, kBN = 128, kThreads = 256;

// ---------------------------------------------------------------- FP32 path
constexpr int kBK32 = 16;
constexpr int kPad32 = 16;  // row pad of the [k][m] LDS tiles: rows 4 apart start 64 banks apart, so the
                             // four k-rows of a fragment read hit distinct banks

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

// Occupancy floor of three waves per SIMD: unconstrained, the allocator takes 184 VGPRs (two waves); held to
// the floor it fits 122 with no spill, and the K = 128 BlockLDLQ products run 15% faster.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) void gemm_tn_f32_kernel(float* __restrict__ C, const float* __restrict__ A,
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

    // With alpha == 1 (the BlockLDLQ products) the accumulators start from C: its reads are issued with the
    // first operand chunk instead of after the last MFMA, and the epilogue is a plain store.
    const bool seed = alpha == 1.0f;
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (seed) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm + 16 * i + 4 * g + r;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t col = n0 + wn + 16 * j + c;
                    if (row < M && col < N) acc[i][j][r] = C[row * ldc + col];
                }
            }
    }

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
                if (col < N) {
                    if (seed)
                        C[row * ldc + col] = acc[i][j][r];
                    else
                        C[row * ldc + col] += alpha * acc[i][j][r];
                }
            }
        }
}

// ---------------------------------------------------------------- bf16 path
// 256 x 256 tile of C per 512-thread workgroup: eight waves of 128 x 64
// (thirty-two 16 x 16 x 32 MFMA accumulators each), 64 k per stage.
// Operands arrive k-major ([k][m] in memory) and are copied to LDS as they
// are: 64 k-rows of 256 columns per operand and stage, 16-byte chunks,
// coalesced 512-byte row segments.  MFMA fragments want 8 consecutive k of
// one column; gfx950's transposing LDS read (ds_read_b64_tr_b16) delivers
// them: within each 16 lanes, lane a addresses the 4 columns 4 (a & 3) of
// k-row a >> 2, and lane i receives column i of the 4 k-rows.  Two such
// reads (k-rows 0..3 and 4..7 of the lane's k octet) make one fragment.
// LDS rows are 256 + 32 bf16 (576 bytes), and the 16-byte chunk index of
// every row in an odd group of eight rows is XORed with 2: the transposing
// reads of 32 lanes and the 16-byte writes of 16 lanes then all hit distinct
// banks.  LDS is double-buffered; half-way through a stage each thread
// writes the next stage to LDS and requests the one after, so global loads
// have a stage and a half to land: one barrier per stage.  With
// A == B (the Gram matrix X^T X) only tiles on and above the diagonal run;
// off-diagonal tiles also add their transpose (float4 stores along m).
constexpr int kT16 = 256;
constexpr int kBK16 = 64;
constexpr int kRow16 = kT16 + 32;  // LDS row: 256 columns + 32 pad (bf16) = 576 B
constexpr int kThreads16 = 512;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

// physical element offset of (k-row r, column col) in one operand's LDS tile
__device__ __forceinline__ int lds_pos(int r, int col) {
    return r * kRow16 + ((((col >> 3) ^ (((r >> 3) & 1) << 1))) << 3) + (col & 7);
}

struct Bf16Stage {
    u32x4 v[4];  // chunks t % 32 of k-rows t / 32 + 16 q, q = 0..3
};

// Four 16-byte chunks of one operand's stage through a buffer resource that
// ends at the last 16-byte group of valid columns of the stage's last row
// (row min(K, k0 + 64) - 1): reads past it return zero (the K edge and the
// last row's tail), so no load is predicated and nothing past the matrix is
// read.  Columns past M or N in earlier rows read the following row; they
// only feed rows or columns of C that are never stored.  `span` is the number
// of columns from the tile's first column to the end of its valid 16-byte
// groups.
__device__ __forceinline__ void load_stage(Bf16Stage& u, const uint16_t* P, int64_t k0, int64_t K, int64_t ld,
                                           int span, int t) {
    const int64_t left = K - k0;
    const int rows = static_cast<int>(left < kBK16 ? left : kBK16);
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P + k0 * ld), 0, ((rows - 1) * static_cast<int>(ld) + span) * 2, 0x00020000);
    const int r0 = t >> 5, ch = t & 31;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        u.v[q] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, ((r0 + 16 * q) * static_cast<int>(ld) + 8 * ch) * 2, 0, 0);
}

__device__ __forceinline__ void store_stage(const Bf16Stage& u, uint16_t* S, int t) {
    const int r0 = t >> 5, ch = t & 31;
#pragma unroll
    for (int q = 0; q < 4; ++q) *reinterpret_cast<u32x4*>(S + lds_pos(r0 + 16 * q, 8 * ch)) = u.v[q];
}

// fragment of 16 columns col0 .. col0 + 15 and the lane's k octet kk + 8 (lane / 16)
__device__ __forceinline__ bf16x8 fragment(const uint16_t* S, int kk, int col0, int lane) {
    const int a = lane & 15, r = kk + 8 * (lane >> 4) + (a >> 2), col = col0 + 4 * (a & 3);
    typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(S + lds_pos(r, col)));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(S + lds_pos(r + 4, col)));
    const i16x4 w[2] = {lo, hi};
    bf16x8 f;
    __builtin_memcpy(&f, w, sizeof(f));
    return f;
}

template <bool SYM>
__global__ __launch_bounds__(kThreads16) void gemm_tn_bf16_kernel(float* __restrict__ C, const uint16_t* __restrict__ A,
                                                                  const uint16_t* __restrict__ B, int64_t M,
                                                                  int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                                                  int64_t ldc, float alpha, int tiles_n) {
    __shared__ __attribute__((aligned(16))) uint16_t S[2][2][kBK16 * kRow16];  // [buffer][operand][k-row, column]
    // Workgroup i runs on XCD i % 8: give every XCD a contiguous run of the tile order below, so the
    // workgroups resident on one XCD at a time cover a compact 4 x 8 group of tiles and share 4 A and 8 B
    // operand panels in that XCD's L2.  Tile order: groups row-major, tiles row-major inside a group; with
    // SYM only tiles on or above the diagonal exist.
    const unsigned nwg = gridDim.x, xcd = blockIdx.x % 8u, per = nwg / 8u, rem = nwg % 8u;
    int rest = static_cast<int>(xcd * per + (xcd < rem ? xcd : rem) + blockIdx.x / 8u);
    constexpr int GM = 4, GN = 8;
    const int tiles_m = static_cast<int>((M + kT16 - 1) / kT16);
    int tm = 0, tn = 0;
    for (int gr = 0; gr * GM < tiles_m; ++gr) {
        for (int gc = 0; gc * GN < tiles_n; ++gc) {
            for (int i = 0; i < GM && gr * GM + i < tiles_m; ++i) {
                const int row = gr * GM + i;
                int lo = gc * GN, hi = gc * GN + GN < tiles_n ? gc * GN + GN : tiles_n;
                if (SYM && lo < row) lo = row;
                const int cnt = hi > lo ? hi - lo : 0;
                if (rest < cnt) {
                    tm = row;
                    tn = lo + rest;
                    goto found;
                }
                rest -= cnt;
            }
        }
    }
    return;  // not reached: the grid holds exactly the tiles of the order
found:
    const int64_t m0 = static_cast<int64_t>(tm) * kT16, n0 = static_cast<int64_t>(tn) * kT16;

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
    const int64_t endA = ((M + 7) & ~int64_t{7}) < lda ? ((M + 7) & ~int64_t{7}) : lda;
    const int64_t endB = ((N + 7) & ~int64_t{7}) < ldb ? ((N + 7) & ~int64_t{7}) : ldb;
    const int spanA = static_cast<int>(endA - m0), spanB = static_cast<int>(endB - n0);
    const uint16_t* PA = A + m0;
    const uint16_t* PB = B + n0;

    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int64_t stages = (K + kBK16 - 1) / kBK16;
    Bf16Stage ua, ub;
    load_stage(ua, PA, 0, K, lda, spanA, t);
    load_stage(ub, PB, 0, K, ldb, spanB, t);
    store_stage(ua, S[0][0], t);
    store_stage(ub, S[0][1], t);
    if (stages > 1) {
        load_stage(ua, PA, kBK16, K, lda, spanA, t);
        load_stage(ub, PB, kBK16, K, ldb, spanB, t);
    }
    __syncthreads();
    for (int64_t s = 0; s < stages; ++s) {
        const int cur = static_cast<int>(s & 1);
#pragma unroll
        for (int kk = 0; kk < kBK16; kk += 32) {
            bf16x8 a[8], b[4];
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = fragment(S[cur][0], kk, wm + 16 * i, lane);
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = fragment(S[cur][1], kk, wn + 16 * j, lane);
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
            if (kk == 0) {
                // Between the two halves of the stage (the other buffer is free since the last barrier): the
                // next stage goes to LDS and the one after is requested, so the waves' store phases overlap
                // the second half's MFMAs and the loads have a stage and a half to land.
                if (s + 1 < stages) {
                    store_stage(ua, S[cur ^ 1][0], t);
                    store_stage(ub, S[cur ^ 1][1], t);
                }
                if (s + 2 < stages) {
                    load_stage(ua, PA, (s + 2) * kBK16, K, lda, spanA, t);
                    load_stage(ub, PB, (s + 2) * kBK16, K, ldb, spanB, t);
                }
            }
        }
        __syncthreads();
    }

    // lane holds C[m0 + wm + 16 i + 4 g + r][n0 + wn + 16 j + c], r = 0..3
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int64_t row0 = m0 + wm + 16 * i + 4 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t col = n0 + wn + 16 * j + c;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (row0 + r < M) C[(row0 + r) * ldc + col] += alpha * acc[i][j][r];
            if (SYM && tm != tn) {  // the transposed tile: C[col][row0 .. row0 + 3]
                float* q = C + col * ldc + row0;
                if (row0 + 3 < M) {
                    f32x4 v = *reinterpret_cast<const f32x4*>(q);
                    v += alpha * acc[i][j];
                    *reinterpret_cast<f32x4*>(q) = v;
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (row0 + r < M) q[r] += alpha * acc[i][j][r];
                }
            }
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
        if (lda % 8 || ldb % 8 || reinterpret_cast<uintptr_t>(A) % 16 || reinterpret_cast<uintptr_t>(B) % 16)
            return qsrt::fail(qsrt::kBadArgument, "bf16 operands must be 16-byte aligned with lda, ldb multiples of 8");
        if (lda > (1 << 23) || ldb > (1 << 23))
            return qsrt::fail(qsrt::kBadArgument, "bf16 leading dimensions above 2^23 are not supported");
        const int64_t tm = (M + kT16 - 1) / kT16, tn = (N + kT16 - 1) / kT16;
        const bool sym = A == B && lda == ldb && M == N && ldc % 4 == 0 && reinterpret_cast<uintptr_t>(C) % 16 == 0;
        const int64_t n = sym ? tm * (tm + 1) / 2 : tm * tn;
        if (n > 0x7fffffff || tn > 0x7fffffff) return qsrt::fail(qsrt::kBadArgument, "GEMM too large for one launch");
        if (sym)
            hipLaunchKernelGGL(gemm_tn_bf16_kernel<true>, dim3(static_cast<unsigned>(n)), dim3(kThreads16), 0, stream,
                               C, static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), M, N, K, lda, ldb,
                               ldc, alpha, static_cast<int>(tn));
        else
            hipLaunchKernelGGL(gemm_tn_bf16_kernel<false>, dim3(static_cast<unsigned>(n)), dim3(kThreads16), 0,
                               stream, C, static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), M, N, K,
                               lda, ldb, ldc, alpha, static_cast<int>(tn));
    }
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

}  // extern "C"
