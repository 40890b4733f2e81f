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
// One workgroup per CU (the LDS buffers take 144 KiB), so a tile count that
// is not a multiple of the CU count leaves CUs idle in the last round (the
// 406 Gram tiles of 7168 channels: 150 tiles in a second round on 256 CUs);
// given a workspace, those tiles are split along K (bf16_plan below).
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

// Tile order: groups of 4 x 8 tiles, groups row-major, tiles row-major inside a group; with SYM only tiles
// on or above the diagonal exist.  Returns false past the last tile.
__device__ __forceinline__ bool tile_at(int idx, int tiles_m, int tiles_n, bool sym, int& tm, int& tn) {
    constexpr int GM = 4, GN = 8;
    int rest = idx;
    for (int gr = 0; gr * GM < tiles_m; ++gr) {
        // a whole group row at once: tiles of its rows (with SYM, columns from the row's own onwards)
        int row_tiles = 0;
        for (int i = 0; i < GM && gr * GM + i < tiles_m; ++i)
            row_tiles += sym ? (tiles_n > gr * GM + i ? tiles_n - (gr * GM + i) : 0) : tiles_n;
        if (rest >= row_tiles) {
            rest -= row_tiles;
            continue;
        }
        for (int gc = 0; gc * GN < tiles_n; ++gc)
            for (int i = 0; i < GM && gr * GM + i < tiles_m; ++i) {
                const int row = gr * GM + i;
                int lo = gc * GN;
                const int hi = gc * GN + GN < tiles_n ? gc * GN + GN : tiles_n;
                if (sym && lo < row) lo = row;
                const int cnt = hi > lo ? hi - lo : 0;
                if (rest < cnt) {
                    tm = row;
                    tn = lo + rest;
                    return true;
                }
                rest -= cnt;
            }
        return false;  // not reached: the group row holds the tile
    }
    return false;
}

// Workgroup q of a range of n runs on XCD q % 8: it takes slot xcd_slot(q, n), so every XCD owns a
// contiguous run of the range and the workgroups resident on one XCD at a time share operand panels
// (a 4 x 8 group: 4 A and 8 B panels) in that XCD's L2.
__device__ __forceinline__ int xcd_slot(int q, int n) {
    const int x = q % 8, per = n / 8, rem = n % 8;
    return x * per + (x < rem ? x : rem) + q / 8;
}

typedef uint16_t Bf16Lds[2][2][kBK16 * kRow16];  // [buffer][operand][k-row, column]

// acc += A[k0 .. k1)^T B[k0 .. k1) over the tile's columns m0 .. m0 + 255 of A and n0 .. n0 + 255 of B
__device__ __forceinline__ void bf16_mainloop(f32x4 (&acc)[8][4], Bf16Lds& S, const uint16_t* __restrict__ A,
                                              const uint16_t* __restrict__ B, int64_t M, int64_t N, int64_t k0,
                                              int64_t k1, int64_t lda, int64_t ldb, int64_t m0, int64_t n0, int t) {
    const int lane = t & 63, wave = t >> 6;
    const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
    const int64_t endA = ((M + 7) & ~int64_t{7}) < lda ? ((M + 7) & ~int64_t{7}) : lda;
    const int64_t endB = ((N + 7) & ~int64_t{7}) < ldb ? ((N + 7) & ~int64_t{7}) : ldb;
    const int spanA = static_cast<int>(endA - m0), spanB = static_cast<int>(endB - n0);
    const uint16_t* PA = A + k0 * lda + m0;
    const uint16_t* PB = B + k0 * ldb + n0;
    const int64_t K = k1 - k0;
    const int64_t stages = (K + kBK16 - 1) / kBK16;
    if (stages <= 0) return;
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
}

// C tile (tm, tn) += alpha * acc over the 16-row blocks i0 .. i0 + IB - 1 of every wave's 128 x 64 block;
// with SYM an off-diagonal tile also adds its transpose.
// lane holds C[m0 + wm + 16 i + 4 g + r][n0 + wn + 16 j + c], r = 0..3
template <bool SYM, int IB>
__device__ __forceinline__ void bf16_epilogue(float* __restrict__ C, const f32x4 (&acc)[IB][4], int i0, int64_t M,
                                              int64_t N, int64_t ldc, float alpha, int tm, int tn, int t) {
    const int lane = t & 63, wave = t >> 6, c = lane & 15, g = lane >> 4;
    const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
    const int64_t m0 = static_cast<int64_t>(tm) * kT16, n0 = static_cast<int64_t>(tn) * kT16;
    if (m0 + kT16 <= M && n0 + kT16 <= N) {
        // Interior tile: no per-element bounds, so the C loads of a 16-row block (and of its transposed
        // block) are issued together and waited for once, not one load round trip per element.
#pragma unroll
        for (int ii = 0; ii < IB; ++ii) {
            const int64_t row0 = m0 + wm + 16 * (i0 + ii) + 4 * g;
            float v[4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) v[j][r] = C[(row0 + r) * ldc + n0 + wn + 16 * j + c];
            f32x4 w[4];
            if (SYM && tm != tn) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    w[j] = *reinterpret_cast<const f32x4*>(C + (n0 + wn + 16 * j + c) * ldc + row0);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    C[(row0 + r) * ldc + n0 + wn + 16 * j + c] = v[j][r] + alpha * acc[ii][j][r];
            if (SYM && tm != tn) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    *reinterpret_cast<f32x4*>(C + (n0 + wn + 16 * j + c) * ldc + row0) = w[j] + alpha * acc[ii][j];
            }
        }
        return;
    }
#pragma unroll
    for (int ii = 0; ii < IB; ++ii) {
        const int64_t row0 = m0 + wm + 16 * (i0 + ii) + 4 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t col = n0 + wn + 16 * j + c;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (row0 + r < M) C[(row0 + r) * ldc + col] += alpha * acc[ii][j][r];
            if (SYM && tm != tn) {  // the transposed tile: C[col][row0 .. row0 + 3]
                float* q = C + col * ldc + row0;
                if (row0 + 3 < M) {
                    f32x4 v = *reinterpret_cast<const f32x4*>(q);
                    v += alpha * acc[ii][j];
                    *reinterpret_cast<f32x4*>(q) = v;
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (row0 + r < M) q[r] += alpha * acc[ii][j][r];
                }
            }
        }
    }
}

// One partial of a split tile in the workspace: 32 accumulators x 512 threads x 16 bytes, accumulator-major
// so a wave's stores and loads are contiguous.
constexpr int64_t kPartialVec = 32 * kThreads16;  // f32x4 per partial (256 KiB)

// Workgroups [0, dp) each own a whole tile: order[xcd_slot(b, dp)].  When the tile count is not a multiple
// of the CU count, the tiles order[dp .. dp + sk) of the last, partial round are instead split into `parts`
// K ranges and the workgroups [dp, dp + sk * parts) compute one range each into the workspace, range-major
// (all first ranges, then all second ranges, ...), so the workgroups resident on one XCD at a time walk the
// same K range of neighbouring tiles; gemm_tn_bf16_fixup adds the ranges to C in K order.
template <bool SYM>
__global__ __launch_bounds__(kThreads16) void gemm_tn_bf16_kernel(float* __restrict__ C, const uint16_t* __restrict__ A,
                                                                  const uint16_t* __restrict__ B, int64_t M,
                                                                  int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                                                  int64_t ldc, float alpha, int tiles_n, int dp,
                                                                  int sk, int parts, f32x4* __restrict__ ws) {
    __shared__ __attribute__((aligned(16))) Bf16Lds S;
    const int b = static_cast<int>(blockIdx.x), t = static_cast<int>(threadIdx.x);
    const int tiles_m = static_cast<int>((M + kT16 - 1) / kT16);
    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    int tm = 0, tn = 0;
    if (b < dp) {
        if (!tile_at(xcd_slot(b, dp), tiles_m, tiles_n, SYM, tm, tn)) return;  // not reached: dp <= tiles
        bf16_mainloop(acc, S, A, B, M, N, 0, K, lda, ldb, static_cast<int64_t>(tm) * kT16,
                      static_cast<int64_t>(tn) * kT16, t);
        bf16_epilogue<SYM, 8>(C, acc, 0, M, N, ldc, alpha, tm, tn, t);
        return;
    }
    const int q = xcd_slot(b - dp, sk * parts), part = q / sk, s = q % sk;
    if (!tile_at(dp + s, tiles_m, tiles_n, SYM, tm, tn)) return;  // not reached
    const int64_t stages = (K + kBK16 - 1) / kBK16;
    const int64_t k0 = stages * part / parts * kBK16, k1 = stages * (part + 1) / parts * kBK16;
    bf16_mainloop(acc, S, A, B, M, N, k0, k1 < K ? k1 : K, lda, ldb, static_cast<int64_t>(tm) * kT16,
                  static_cast<int64_t>(tn) * kT16, t);
    f32x4* w = ws + static_cast<int64_t>(part * sk + s) * kPartialVec;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) w[(i * 4 + j) * kThreads16 + t] = acc[i][j];
}

// Eight workgroups per split tile, one per 16-row block i of every wave's 128 x 64 block: the tile's K
// ranges summed in K order, then the epilogue of those rows (and of their transpose).
template <bool SYM>
__global__ __launch_bounds__(kThreads16) void gemm_tn_bf16_fixup(float* __restrict__ C, int64_t M, int64_t N,
                                                                 int64_t ldc, float alpha, int tiles_n, int dp,
                                                                 int sk, int parts,
                                                                 const f32x4* __restrict__ ws) {
    const int s = static_cast<int>(blockIdx.x) / 8, i = static_cast<int>(blockIdx.x) % 8;
    const int t = static_cast<int>(threadIdx.x);
    int tm = 0, tn = 0;
    if (!tile_at(dp + s, static_cast<int>((M + kT16 - 1) / kT16), tiles_n, SYM, tm, tn)) return;  // not reached
    const f32x4* w = ws + static_cast<int64_t>(s) * kPartialVec;
    f32x4 acc[1][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[0][j] = w[(i * 4 + j) * kThreads16 + t];
    for (int part = 1; part < parts; ++part) {
        const f32x4* wp = w + static_cast<int64_t>(part) * sk * kPartialVec;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[0][j] += wp[(i * 4 + j) * kThreads16 + t];
    }
    bf16_epilogue<SYM, 1>(C, acc, i, M, N, ldc, alpha, tm, tn, t);
}

// Launch plan of the bf16 path: `tiles` tiles on `cus` compute units.  A last round that would leave CUs
// idle is split along K into `parts` ranges, chosen to minimise (rounds of ranges) / parts + 0.09 x
// (ranges per CU) in units of one tile's time: the first term is the split round's length, the second the
// cost of writing and re-reading each range's partial (fitted on MI355X to the Gram of a 16384 x 7168
// operand at 2, 3, 4, 5 and 8 parts; 3 parts there, 8 for the 28 x 28 tiles of the full product).
struct Bf16Plan {
    int64_t tiles = 0, dp = 0, sk = 0;
    int parts = 1;
    size_t workspace_bytes() const { return sk ? static_cast<size_t>(sk * parts) * kPartialVec * sizeof(f32x4) : 0; }
};

Bf16Plan bf16_plan(int64_t tiles, int64_t stages, int cus) {
    Bf16Plan p;
    p.tiles = p.dp = tiles;
    if (cus <= 0 || tiles <= cus || tiles % cus == 0 || stages < 2) return p;
    const int64_t sk = tiles % cus;
    double best = 1.0;  // an unsplit last round: one tile's time
    int best_parts = 1;
    for (int parts = 2; parts <= 8 && parts <= stages; ++parts) {
        const double rounds = static_cast<double>((sk * parts + cus - 1) / cus);
        const double cost = rounds / parts + 0.09 * static_cast<double>(sk * parts) / cus;
        if (cost < best - 1e-9) {
            best = cost;
            best_parts = parts;
        }
    }
    if (best_parts == 1) return p;
    p.dp = tiles - sk;
    p.sk = sk;
    p.parts = best_parts;
    return p;
}

int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cached[dev] = n;
    }
    return cached[dev];
}

bool bf16_symmetric(const float* C, const void* A, const void* B, int64_t M, int64_t N, int64_t lda, int64_t ldb,
                    int64_t ldc) {
    return A == B && lda == ldb && M == N && ldc % 4 == 0 && reinterpret_cast<uintptr_t>(C) % 16 == 0;
}

int64_t bf16_tiles(bool sym, int64_t M, int64_t N) {
    const int64_t tm = (M + kT16 - 1) / kT16, tn = (N + kT16 - 1) / kT16;
    return sym ? tm * (tm + 1) / 2 : tm * tn;
}

}  // namespace

extern "C" {

size_t qsrt_gemm_tn_workspace_bytes(const float* C, const void* A, const void* B, int64_t M, int64_t N, int64_t K,
                                    int64_t lda, int64_t ldb, int64_t ldc, int dtype) {
    if (dtype != 1 || M <= 0 || N <= 0 || K <= 0) return 0;
    const bool sym = bf16_symmetric(C, A, B, M, N, lda, ldb, ldc);
    return bf16_plan(bf16_tiles(sym, M, N), (K + kBK16 - 1) / kBK16, device_cus()).workspace_bytes();
}

int qsrt_gemm_tn_ws(float* C, const void* A, const void* B, const void* B2, int64_t M, int64_t N, int64_t K,
                    int64_t lda, int64_t ldb, int64_t ldc, float alpha, int dtype, void* workspace,
                    size_t workspace_bytes, void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (dtype != 0 && dtype != 1) return qsrt::fail(qsrt::kBadArgument, "dtype must be 0 (f32) or 1 (bf16)");
    if (M < 0 || N < 0 || K < 0) return qsrt::fail(qsrt::kBadArgument, "negative GEMM extent");
    if (M == 0 || N == 0 || K == 0) return qsrt::kOk;
    if (!C || !A || !B) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (lda < M || ldb < N || ldc < N)
        return qsrt::fail(qsrt::kBadArgument, "leading dimensions must cover the rows (lda >= M, ldb >= N, ldc >= N)");
    if (dtype == 0) {
        const int64_t tiles_n = (N + kBN - 1) / kBN;
        const int64_t tiles = ((M + kBM - 1) / kBM) * tiles_n;
        if (tiles > 0x7fffffff) return qsrt::fail(qsrt::kBadArgument, "GEMM too large for one launch");
        if (lda % 4 || ldb % 4 || reinterpret_cast<uintptr_t>(A) % 16 || reinterpret_cast<uintptr_t>(B) % 16 ||
            (B2 && reinterpret_cast<uintptr_t>(B2) % 16))
            return qsrt::fail(qsrt::kBadArgument, "f32 operands must be 16-byte aligned with lda, ldb multiples of 4");
        hipLaunchKernelGGL(gemm_tn_f32_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, stream, C,
                           static_cast<const float*>(A), static_cast<const float*>(B), static_cast<const float*>(B2),
                           M, N, K, lda, ldb, ldc, alpha, tiles_n);
        QSRT_HIP_TRY(hipGetLastError());
        return qsrt::kOk;
    }
    if (B2) return qsrt::fail(qsrt::kBadArgument, "the bf16 path has no fused subtraction");
    if (lda % 8 || ldb % 8 || reinterpret_cast<uintptr_t>(A) % 16 || reinterpret_cast<uintptr_t>(B) % 16)
        return qsrt::fail(qsrt::kBadArgument, "bf16 operands must be 16-byte aligned with lda, ldb multiples of 8");
    if (lda > (1 << 23) || ldb > (1 << 23))
        return qsrt::fail(qsrt::kBadArgument, "bf16 leading dimensions above 2^23 are not supported");
    const int64_t tn = (N + kT16 - 1) / kT16;
    const bool sym = bf16_symmetric(C, A, B, M, N, lda, ldb, ldc);
    const int64_t tiles = bf16_tiles(sym, M, N);
    if (tiles > 0x7fffffff / 8 || tn > 0x7fffffff) return qsrt::fail(qsrt::kBadArgument, "GEMM too large for one launch");
    Bf16Plan plan = bf16_plan(tiles, (K + kBK16 - 1) / kBK16, device_cus());
    if (plan.sk && (!workspace || workspace_bytes < plan.workspace_bytes() ||
                    reinterpret_cast<uintptr_t>(workspace) % 16)) {
        plan.dp = tiles;  // no room for the split tiles' partials: every tile whole, as qsrt_gemm_tn runs them
        plan.sk = 0;
        plan.parts = 1;
    }
    const unsigned grid = static_cast<unsigned>(plan.dp + plan.sk * plan.parts);
    auto* ws = static_cast<f32x4*>(workspace);
    const auto* a = static_cast<const uint16_t*>(A);
    const auto* b = static_cast<const uint16_t*>(B);
    const int dp = static_cast<int>(plan.dp), sk = static_cast<int>(plan.sk), ti = static_cast<int>(tn);
    if (sym)
        hipLaunchKernelGGL(gemm_tn_bf16_kernel<true>, dim3(grid), dim3(kThreads16), 0, stream, C, a, b, M, N, K, lda,
                           ldb, ldc, alpha, ti, dp, sk, plan.parts, ws);
    else
        hipLaunchKernelGGL(gemm_tn_bf16_kernel<false>, dim3(grid), dim3(kThreads16), 0, stream, C, a, b, M, N, K, lda,
                           ldb, ldc, alpha, ti, dp, sk, plan.parts, ws);
    QSRT_HIP_TRY(hipGetLastError());
    if (plan.sk) {
        if (sym)
            hipLaunchKernelGGL(gemm_tn_bf16_fixup<true>, dim3(static_cast<unsigned>(sk) * 8u), dim3(kThreads16), 0, stream,
                               C, M, N, ldc, alpha, ti, dp, sk, plan.parts, ws);
        else
            hipLaunchKernelGGL(gemm_tn_bf16_fixup<false>, dim3(static_cast<unsigned>(sk) * 8u), dim3(kThreads16), 0, stream,
                               C, M, N, ldc, alpha, ti, dp, sk, plan.parts, ws);
        QSRT_HIP_TRY(hipGetLastError());
    }
    return qsrt::kOk;
}

int qsrt_gemm_tn(float* C, const void* A, const void* B, const void* B2, int64_t M, int64_t N, int64_t K,
                 int64_t lda, int64_t ldb, int64_t ldc, float alpha, int dtype, void* stream_handle) {
    return qsrt_gemm_tn_ws(C, A, B, B2, M, N, K, lda, ldb, ldc, alpha, dtype, nullptr, 0, stream_handle);
}

}  // extern "C"

// ---------------------------------------------------------------- FP64 path
// C[M, N] += alpha * A^T (B - B2) with A, B, C float64 and B2 FP32: the
// BlockLDLQ product cache P += L[span]^T (W - Q)[span] under the encoder's
// float64 contract (the factor L and the regularised weight W stay float64,
// the reconstruction Q is FP32 labels, exact in float64), so that the
// targets the tile Viterbi sees are the float64 sums rounded once.
//
// v_mfma_f64_16x16x4_f64: lane l holds A[m = l % 16][k = l / 16] and
// B[k = l / 16][n = l % 16]; its accumulator r is C[l / 16 + 4 r][l % 16] (rows
// interleaved by four, unlike the FP32 16x16x4 form's C[4 (l / 16) + r]).
// One 256-thread workgroup per 128 x 128 tile of C (four waves of 64 x 64,
// sixteen 16 x 16 accumulator tiles each, 128 accumulator registers), K in
// chunks of 16 rows staged through double-buffered LDS, the next chunk's
// global loads issued before the current chunk's products.  Each element of
// C sums its K terms in increasing chunk order, the same for any M and N, so
// a column's result does not depend on the width of the launch.
namespace {

typedef double f64x4 __attribute__((ext_vector_type(4)));

constexpr int kBM64 = 64;   // float64 tile: 64 rows of C x kBN columns, four waves of 32 x 64
constexpr int kBK64 = 8;    // k-rows per LDS chunk (28 KB double-buffered: four workgroups per CU)
constexpr int kPad64 = 16;  // row pad (doubles): the four k-rows of a fragment read start 32 banks apart
constexpr int kMI64 = kBM64 / 32;                  // 16-row MFMA tiles per wave
constexpr int kNA64 = kBK64 * kBM64 / 2 / kThreads;  // double2 of A per thread per chunk
constexpr int kNB64 = kBK64 * kBN / 2 / kThreads;    // double2 of B per thread per chunk
static_assert(kNA64 >= 1 && kNB64 >= 1 && kBK64 % 4 == 0, "float64 chunk shape");

struct F64Chunk {
    double2 a[kNA64], b[kNB64];
};

__device__ __forceinline__ double2 ld2_masked(const double* p, int64_t row, int64_t col, int64_t rows, int64_t cols,
                                              int64_t ld) {
    if (row >= rows) return make_double2(0.0, 0.0);
    const double* q = p + row * ld + col;
    if (col + 1 < cols) return *reinterpret_cast<const double2*>(q);
    return make_double2(col < cols ? q[0] : 0.0, 0.0);
}

__device__ __forceinline__ double2 ld2_masked_f32(const float* p, int64_t row, int64_t col, int64_t rows,
                                                  int64_t cols, int64_t ld) {
    if (row >= rows) return make_double2(0.0, 0.0);
    const float* q = p + row * ld + col;
    if (col + 1 < cols) {
        const float2 v = *reinterpret_cast<const float2*>(q);
        return make_double2(v.x, v.y);
    }
    return make_double2(col < cols ? static_cast<double>(q[0]) : 0.0, 0.0);
}

__device__ __forceinline__ void load_f64(F64Chunk& ch, const double* A, const double* B, const float* B2, int64_t k0,
                                         int64_t m0, int64_t n0, int64_t M, int64_t N, int64_t K, int64_t lda,
                                         int64_t ldb, int64_t ldb2, int t) {
#pragma unroll
    for (int i = 0; i < kNA64; ++i) {  // kBK64 rows x kBM64 / 2 double2 of A
        const int f = t + kThreads * i;
        const int r = f / (kBM64 / 2), q = f % (kBM64 / 2);
        ch.a[i] = ld2_masked(A, k0 + r, m0 + 2 * q, K, M, lda);
    }
#pragma unroll
    for (int i = 0; i < kNB64; ++i) {  // kBK64 rows x kBN / 2 double2 of B - B2
        const int f = t + kThreads * i;
        const int r = f / (kBN / 2), q = f % (kBN / 2);
        double2 b = ld2_masked(B, k0 + r, n0 + 2 * q, K, N, ldb);
        if (B2) {
            const double2 s = ld2_masked_f32(B2, k0 + r, n0 + 2 * q, K, N, ldb2);
            b.x -= s.x;
            b.y -= s.y;
        }
        ch.b[i] = b;
    }
}

__device__ __forceinline__ void store_f64(const F64Chunk& ch, double (*As)[kBM64 + kPad64], double (*Bs)[kBN + kPad64],
                                          int t) {
#pragma unroll
    for (int i = 0; i < kNA64; ++i) {
        const int f = t + kThreads * i;
        *reinterpret_cast<double2*>(&As[f / (kBM64 / 2)][2 * (f % (kBM64 / 2))]) = ch.a[i];
    }
#pragma unroll
    for (int i = 0; i < kNB64; ++i) {
        const int f = t + kThreads * i;
        *reinterpret_cast<double2*>(&Bs[f / (kBN / 2)][2 * (f % (kBN / 2))]) = ch.b[i];
    }
}

// Four workgroups per CU (four waves per SIMD): 64 accumulator registers per lane, 28 KB of LDS per workgroup,
// so one workgroup's loads and stores of its C tile overlap the others' matrix-core work.
// Batch members are consecutive runs of tiles_m * tiles_n workgroups (member-major, so a member's operands stay
// in L2 while its tiles run); member b reads A + b * sa, B + b * sb, B2 + b * sb2 and updates C + b * sc.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void gemm_tn_f64_kernel(double* __restrict__ C, const double* __restrict__ A,
                                                               const double* __restrict__ B,
                                                               const float* __restrict__ B2, int64_t M, int64_t N,
                                                               int64_t K, int64_t lda, int64_t ldb, int64_t ldb2,
                                                               int64_t ldc, double alpha, int64_t tiles_n,
                                                               int64_t tiles_per_member, int64_t sc, int64_t sa,
                                                               int64_t sb, int64_t sb2) {
    __shared__ __attribute__((aligned(16))) double As[2][kBK64][kBM64 + kPad64];
    __shared__ __attribute__((aligned(16))) double Bs[2][kBK64][kBN + kPad64];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int64_t member = blockIdx.x / tiles_per_member, tile = blockIdx.x - member * tiles_per_member;
    C += member * sc;
    A += member * sa;
    B += member * sb;
    if (B2) B2 += member * sb2;
    const int64_t m0 = (tile / tiles_n) * kBM64, n0 = (tile % tiles_n) * kBN;
    const int wm = (wave >> 1) * (kBM64 / 2), wn = (wave & 1) * 64;

    const bool seed = alpha == 1.0;  // accumulators start from C (plain store at the end)
    f64x4 acc[kMI64][4];
#pragma unroll
    for (int i = 0; i < kMI64; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};
    if (seed) {
#pragma unroll
        for (int i = 0; i < kMI64; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm + 16 * i + g + 4 * r;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t col = n0 + wn + 16 * j + c;
                    if (row < M && col < N) acc[i][j][r] = C[row * ldc + col];
                }
            }
    }

    F64Chunk ch;
    load_f64(ch, A, B, B2, 0, m0, n0, M, N, K, lda, ldb, ldb2, t);
    store_f64(ch, As[0], Bs[0], t);
    __syncthreads();
    const int64_t chunks = (K + kBK64 - 1) / kBK64;
    for (int64_t kc = 0; kc < chunks; ++kc) {
        const int cur = kc & 1;
        if (kc + 1 < chunks) load_f64(ch, A, B, B2, (kc + 1) * kBK64, m0, n0, M, N, K, lda, ldb, ldb2, t);
#pragma unroll
        for (int kk = 0; kk < kBK64 / 4; ++kk) {
            double a[kMI64], b[4];
#pragma unroll
            for (int i = 0; i < kMI64; ++i) a[i] = As[cur][4 * kk + g][wm + 16 * i + c];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[cur][4 * kk + g][wn + 16 * j + c];
#pragma unroll
            for (int i = 0; i < kMI64; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kc + 1 < chunks) store_f64(ch, As[cur ^ 1], Bs[cur ^ 1], t);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < kMI64; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = m0 + wm + 16 * i + g + 4 * r;
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

}  // namespace

extern "C" {

int qsrt_gemm_tn_f64_batched(double* C, const double* A, const double* B, const float* B2, int batch, int64_t M,
                             int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldb2, int64_t ldc, int64_t stride_c,
                             int64_t stride_a, int64_t stride_b, int64_t stride_b2, double alpha,
                             void* stream_handle) {
    if (batch < 0 || M < 0 || N < 0 || K < 0) return qsrt::fail(qsrt::kBadArgument, "gemm f64: negative extent");
    if (batch == 0 || M == 0 || N == 0 || K == 0) return qsrt::kOk;
    if (!C || !A || !B) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (lda < M || ldb < N || ldc < N || (B2 && ldb2 < N))
        return qsrt::fail(qsrt::kBadArgument, "gemm f64: leading dimension smaller than the row");
    if (lda % 2 || ldb % 2 || (B2 && ldb2 % 2) || reinterpret_cast<uintptr_t>(A) % 16 ||
        reinterpret_cast<uintptr_t>(B) % 16 || (B2 && reinterpret_cast<uintptr_t>(B2) % 8))
        return qsrt::fail(qsrt::kBadArgument,
                          "gemm f64: A and B must be 16-byte aligned, B2 8-byte aligned, leading dimensions even");
    if (batch > 1 && (stride_a % 2 || stride_b % 2 || (B2 && stride_b2 % 2) || stride_c < 0 || stride_a < 0 ||
                      stride_b < 0 || stride_b2 < 0))
        return qsrt::fail(qsrt::kBadArgument, "gemm f64: member strides must be non-negative and even");
    if (batch > 1 && stride_c < (M - 1) * ldc + N)
        return qsrt::fail(qsrt::kBadArgument, "gemm f64: members of C overlap (stride_c < (M - 1) * ldc + N)");
    const int64_t tiles_m = (M + kBM64 - 1) / kBM64, tiles_n = (N + kBN - 1) / kBN;
    if (tiles_m * tiles_n * batch > 0x7fffffff) return qsrt::fail(qsrt::kBadArgument, "gemm f64: too many tiles");
    hipLaunchKernelGGL(gemm_tn_f64_kernel, dim3(static_cast<unsigned>(tiles_m * tiles_n * batch)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream_handle), C, A, B, B2, M, N, K, lda, ldb, ldb2, ldc, alpha,
                       tiles_n, tiles_m * tiles_n, batch > 1 ? stride_c : 0, batch > 1 ? stride_a : 0,
                       batch > 1 ? stride_b : 0, batch > 1 ? stride_b2 : 0);
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

int qsrt_gemm_tn_f64(double* C, const double* A, const double* B, const float* B2, int64_t M, int64_t N, int64_t K,
                     int64_t lda, int64_t ldb, int64_t ldb2, int64_t ldc, double alpha, void* stream_handle) {
    return qsrt_gemm_tn_f64_batched(C, A, B, B2, 1, M, N, K, lda, ldb, ldb2, ldc, 0, 0, 0, 0, alpha, stream_handle);
}

}  // extern "C"
