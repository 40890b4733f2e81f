// Fused trellis decode: packed EXL words -> cyclic states -> E4M3 labels ->
// W = diag(su) . H128 X H128 . diag(sv) -> bf16 (or f32), one 128x128 block
// per workgroup iteration.  Each workgroup walks a contiguous run of blocks
// (runs differ by at most one block); the block cursor advances by carries,
// with no per-block division.
//
// Reference semantics (qsrt/exl3_reference.py:61-302, qsrt/qsrt.py:1175-1209):
//   X[K, N]  = labels of the states, tile-major, tensor-core order in a tile
//   W        = H_R( H_L(X) * su[:, None] ) * sv[None, :]
// with H_L / H_R the normalised 128-block Sylvester Hadamards.  Row scaling
// commutes with the right product, so per 128x128 block
//   W_blk = su . (H128 X_blk H128) . sv / 128   (unnormalised +-1 Hadamards)
// and H128 = H8 (x) H16 (Kronecker over the 8x8 tiles of a block and the
// 16x16 positions of a tile).
//
// Per workgroup (8 waves, two workgroups per CU), per block:
//  A. wave w decodes tile-column w.  Lane (c = lane % 16, g = lane / 16)
//     takes, in every tile, the 4 values of column c at rows 2g + {0,1,8,9}:
//     trellis positions 32 (c % 8) + 8 g + 4 (c / 8) + 0..3 (tensor-core
//     order), one 16 + 3K-bit window of the tile's MSB-first bitstream (EXL
//     stores adjacent 16-bit words swapped, so a little-endian u32 read is the
//     big-endian 32-bit chunk of the stream).  Labels come from the
//     state-indexed E4M3 LUT in LDS; the lane's 32 labels of the tile-column
//     (8 tiles x 4 rows) are written to a 16 KB LDS label area.
//  B. wave w produces output tile-row w.  For each tile-column a', the whole
//     left transform (H8 (x) H16 over the 128 rows) is ONE fp8 MFMA
//     (16x16x128): A = the lane's 32 labels of that tile-column, B = +-1 with
//     B[(a, row)][col] = H8[w][a] H16[row][col].  Exact for |label| <= 6 (sums
//     of at most 128 x 6 on multiples of 2^-9).  The eight results of the
//     tile-row stay in registers; the right H8 across tile-columns runs on
//     VALU (exact: < 2^22 units of 2^-9).  Each value is split into fp16
//     hi + lo (exact, 11 + 11 bits: hi by rounding, lo by a mixed-precision
//     fma), and the right H16 is two accumulating f16 MFMAs (16x16x16) per
//     tile, on hi then lo, sharing A = H16 with row i scaled by the fp16 sv
//     of output column i.  Finally times su/128, conversion, four
//     consecutive outputs per lane per tile.
//  Memory traffic is shaped for the vector-memory pipe: a wave's 8 tiles of
//  packed words arrive with one 16-byte load per lane and are staged through
//  the wave's own slice of the LDS label area; outputs are staged through the
//  same slice (XOR-swizzled 16-byte chunks) so each store instruction writes
//  full 128-byte row segments.  Words, su and sv of the next block are loaded
//  before this block's stores (vector-memory counters retire in issue order,
//  so a load issued after a store would wait for the store to drain).
// Tables whose labels exceed 6 in magnitude use FP32 MFMAs for both products
// (labels widened exactly to FP32), with the same data movement.

#include <algorithm>
#include <mutex>

#include "common.h"
#include "qsrt_amd.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) uint32_t* gu32;
typedef const __attribute__((address_space(1))) float* gf32;
typedef const __attribute__((address_space(1))) f32x4* gf4;

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kLabelBytes = 64 * 256;  // one byte per weight of a block

__device__ __forceinline__ int hsign(int i, int j) { return (__builtin_popcount(i & j) & 1) ? -1 : 1; }

struct Job {
    const int16_t* words;
    int64_t tile_row_stride;
    int64_t tile_col_stride;
    int64_t block_row_stride;  // words between vertically adjacent 128 x 128 blocks
    int64_t block_col_stride;  // words between horizontally adjacent blocks
    const float* row_scale;
    const float* col_scale;
    void* out;
    int64_t out_ld;
    int32_t nbr, nbc;     // 128 x 128 blocks along rows and columns (both > 0)
    int64_t first_block;  // prefix over jobs (filled by the host)
};

// Position of a workgroup in its run of blocks: job and block coordinates,
// all wave-uniform.  Runs are contiguous, so moving to the next block is a
// carry chain instead of a division.
struct Cursor {
    int j, br, bc;
};

__device__ __forceinline__ Cursor cursor_at(const Job* jobs, int n_jobs, int64_t blk) {
    int j = 0;
    while (j + 1 < n_jobs && jobs[j + 1].first_block <= blk) ++j;
    const int64_t local = blk - jobs[j].first_block;
    const int br = static_cast<int>(local / jobs[j].nbc);
    return Cursor{j, br, static_cast<int>(local - static_cast<int64_t>(br) * jobs[j].nbc)};
}

__device__ __forceinline__ void cursor_next(const Job* jobs, Cursor& cu) {
    if (++cu.bc == jobs[cu.j].nbc) {
        cu.bc = 0;
        if (++cu.br == jobs[cu.j].nbr) {
            cu.br = 0;
            ++cu.j;
        }
    }
}

struct BlockCtx {
    const int16_t* words;  // tile (8 br, 8 bc) of the block
    int64_t trs, tcs;
    const float* su;       // row 128 br
    const float* sv;       // col 128 bc
    char* out;             // element (128 br, 128 bc)
    int64_t ld;
};

__device__ __forceinline__ BlockCtx block_ctx(const Job* jobs, const Cursor& cu, int out_size) {
    const Job& J = jobs[cu.j];
    BlockCtx x;
    x.words = J.words + cu.br * J.block_row_stride + cu.bc * J.block_col_stride;
    x.trs = J.tile_row_stride;
    x.tcs = J.tile_col_stride;
    x.su = J.row_scale + 128 * cu.br;
    x.sv = J.col_scale + 128 * cu.bc;
    x.out = static_cast<char*>(J.out) + (128 * cu.br * J.out_ld + 128 * cu.bc) * out_size;
    x.ld = J.out_ld;
    return x;
}

// 16 bytes of the wave's tile-column: lane l < 16 K loads chunk l % (2 K) of
// tile-row l / (2 K) (each tile is 32 K bytes of words).
template <int K>
__device__ __forceinline__ u32x4 fetch_words(const BlockCtx& x, int w, int lane) {
    if (lane >= 16 * K) return u32x4{0u, 0u, 0u, 0u};
    const int a = lane / (2 * K), q = lane % (2 * K);
    const int16_t* tile = x.words + a * x.trs + w * x.tcs;
    return *(const __attribute__((address_space(1))) u32x4*)(tile + 8 * q);
}

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// fp16 pair {e0 - hi.x, e1 - hi.y} with hi a packed fp16 pair: each value is
// one mixed-precision fma (fp16 source, fp32 addend, result rounded once to
// fp16, v_fma_mixlo/mixhi_f16) written straight into its half of the result.
// `neg_one` lives in a register so the fma is not rewritten as a subtraction,
// which has no mixed-precision form; callers pass `hi` through an opaque copy
// so the halves are read from the packed register (op_sel) rather than
// converted again.
__device__ __forceinline__ uint32_t residual_pair(uint32_t hi, float e0, float e1, float neg_one) {
    const f16x2 h = __builtin_bit_cast(f16x2, hi);
    const f16x2 lo = {static_cast<_Float16>(__builtin_fmaf(static_cast<float>(h.x), neg_one, e0)),
                      static_cast<_Float16>(__builtin_fmaf(static_cast<float>(h.y), neg_one, e1))};
    return __builtin_bit_cast(uint32_t, lo);
}

template <int K, bool FP8, typename OutT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void decode_kernel(const Job* __restrict__ jobs, int n_jobs, int64_t total_blocks, const uint8_t* __restrict__ lut) {
    static_assert(sizeof(OutT) == 2 || sizeof(OutT) == 4, "bf16 or f32 output");
    __shared__ __attribute__((aligned(16))) uint8_t lut_s[65536];
    // Label area, 2 KB per wave.  During B1: labels of tile-column a', lane l,
    // half h (tile-rows 4h..4h+3) at ((a' * 2 + h) * 64 + l) * 16.  Wave w's
    // slice [2 KB w, 2 KB (w + 1)) also stages its packed words (phase A) and
    // its outputs (phase B2), when no other wave reads it.
    __shared__ __attribute__((aligned(16))) uint8_t labels[kLabelBytes];

    // this workgroup's run of blocks: [begin, end), sizes differ by at most one
    const int64_t begin = total_blocks * blockIdx.x / gridDim.x;
    const int64_t end = total_blocks * (blockIdx.x + 1) / gridDim.x;
    if (begin >= end) return;

    for (int i = threadIdx.x; i < 65536 / 16; i += kThreads)
        reinterpret_cast<uint4*>(lut_s)[i] = reinterpret_cast<const uint4*>(lut)[i];

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15;
    const int g = lane >> 4;
    const int rho[4] = {2 * g, 2 * g + 1, 2 * g + 8, 2 * g + 9};

    // Left-product B operand (fp8 +-1): byte j <-> tile-row j / 4, row rho(j % 4); value H8[w][j/4] H16[rho][c].
    i32x8 bl;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        uint32_t v = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int j = 4 * r + b;
            const int s = hsign(w, j >> 2) * hsign(rho[j & 3], c);
            v |= (s > 0 ? 0x38u : 0xB8u) << (8 * b);  // E4M3 +1 / -1
        }
        bl[r] = static_cast<int>(v);
    }
    // Right-product A operand rows: H16[c][4g + q]
    float hr[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) hr[q] = static_cast<float>(hsign(c, 4 * g + q));
    float hl[4];  // FP32 path: H16[rho(i)][c]
#pragma unroll
    for (int i = 0; i < 4; ++i) hl[i] = static_cast<float>(hsign(rho[i], c));
    // fp16 sign masks of H16[c][4g + q], q = 0..3, as two packed pairs
    uint32_t hsg[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
        hsg[h] = (hr[2 * h] < 0.f ? 0x8000u : 0u) | (hr[2 * h + 1] < 0.f ? 0x80000000u : 0u);
#pragma unroll
    for (int h = 0; h < 2; ++h) asm volatile("" : "+v"(hsg[h]));
    float neg_one = -1.0f;
    asm volatile("" : "+v"(neg_one));
    // Keep the operand constants in registers instead of recomputing them in the loop.
#pragma unroll
    for (int r = 0; r < 8; ++r) asm volatile("" : "+v"(bl[r]));
#pragma unroll
    for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(hr[q]));

    // The lane's 16 + 3K-bit window starts at stream bit b0; sh = b0 % 32 is never 0 for K = 2, 3, 4 and these
    // positions (b0 = (p0 + 1) K - 16 with p0 = 32 (c % 8) + 8 g + 4 (c / 8)), so one funnel shift extracts it.
    const int p0 = 32 * (c & 7) + 8 * g + 4 * (c >> 3);
    int b0 = (p0 + 1) * K - 16;
    if (b0 < 0) b0 += 256 * K;
    const int m0 = b0 >> 5;
    const int m1 = (m0 + 1) % (8 * K);
    const uint32_t rsh = 32u - static_cast<uint32_t>(b0 & 31);

    uint8_t* slice = labels + 2048 * w;
    uint4* lab_w = reinterpret_cast<uint4*>(labels) + (w * 2) * 64 + lane;
    const uint4* lab_r = reinterpret_cast<const uint4*>(labels) + lane;
    const uint32_t* wstage = reinterpret_cast<const uint32_t*>(slice);

    Cursor cu = cursor_at(jobs, n_jobs, begin);
    BlockCtx ctx = block_ctx(jobs, cu, sizeof(OutT));
    u32x4 words = fetch_words<K>(ctx, w, lane);
    float su = ((gf32)ctx.su)[16 * w + c];
    float sv[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) sv[a] = ((gf32)ctx.sv)[16 * a + c];
    __syncthreads();

    for (int64_t blk = begin; blk < end; ++blk) {
        // ---- A: stage the tile-column's words, decode the lane's labels.  From here to the end of B1 the wave
        // runs at raised issue priority and drops back for B2: a wave in its right product and stores then
        // yields issue slots to waves still gathering labels or in the left product, so the two workgroups'
        // phases overlap better (bit-identical output; 0.82-0.86 ms against 0.89-0.96 ms on 96 K3 matrices).
        __builtin_amdgcn_s_setprio(2);
        if (lane < 16 * K) reinterpret_cast<u32x4*>(slice)[lane] = words;
        uint32_t lab[8];
#pragma unroll
        for (int a = 0; a < 8; ++a) {
            const uint32_t lo = wstage[a * 8 * K + m0], hi = wstage[a * 8 * K + m1];
            const uint32_t win = __builtin_amdgcn_alignbit(lo, hi, rsh);  // stream bits [b0, b0 + 32)
            const uint32_t v01 = lut_s[win >> 16] | (static_cast<uint32_t>(lut_s[(win >> (16 - K)) & 0xFFFFu]) << 16);
            const uint32_t v23 = lut_s[(win >> (16 - 2 * K)) & 0xFFFFu] |
                                 (static_cast<uint32_t>(lut_s[(win >> (16 - 3 * K)) & 0xFFFFu]) << 16);
            lab[a] = __builtin_amdgcn_perm(v23, v01, 0x06040200u);
        }
        lab_w[0] = make_uint4(lab[0], lab[1], lab[2], lab[3]);
        lab_w[64] = make_uint4(lab[4], lab[5], lab[6], lab[7]);
        // this block's scale operands, before the prefetch below replaces su and sv
        uint32_t sv2[8];  // FP8 path: fp16 pairs
        float svf[8];     // FP32 path
#pragma unroll
        for (int a = 0; a < 8; ++a) {
            if constexpr (FP8)
                sv2[a] = __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(sv[a]), static_cast<_Float16>(sv[a])});
            else
                svf[a] = sv[a];
        }
        const float su_cur = su;
        const BlockCtx cur = ctx;
        // ---- prefetch the next block (before this block's stores)
        if (blk + 1 < end) {
            cursor_next(jobs, cu);
            ctx = block_ctx(jobs, cu, sizeof(OutT));
            words = fetch_words<K>(ctx, w, lane);
            su = ((gf32)ctx.su)[16 * w + c];
#pragma unroll
            for (int a = 0; a < 8; ++a) sv[a] = ((gf32)ctx.sv)[16 * a + c];
        }
        __syncthreads();

        // ---- B1: output tile-row w, left transform per tile-column
        f32x4 e[8];
#pragma unroll
        for (int a2 = 0; a2 < 8; ++a2) {
            const uint4 x0 = lab_r[(a2 * 2) * 64], x1 = lab_r[(a2 * 2 + 1) * 64];
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            if constexpr (FP8) {
                const i32x8 av = {static_cast<int>(x0.x), static_cast<int>(x0.y), static_cast<int>(x0.z),
                                  static_cast<int>(x0.w), static_cast<int>(x1.x), static_cast<int>(x1.y),
                                  static_cast<int>(x1.z), static_cast<int>(x1.w)};
                // format 0 = E4M3 for A and B; E8M0 scales 127 = 1.0
                acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bl, acc, 0, 0, 0, 127, 0, 127);
            } else {
                const uint32_t words8[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int a = 0; a < 8; ++a) {
                    const float sgn = static_cast<float>(hsign(w, a));
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float x = sgn * qsrt::e4m3_to_float((words8[a] >> (8 * i)) & 0xFFu);
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x, hl[i], acc, 0, 0, 0);
                    }
                }
            }
            e[a2] = acc;
        }
        __syncthreads();  // every wave is done reading labels: slices are private again
        __builtin_amdgcn_s_setprio(0);

        // ---- B2: right H8 across tile-columns (exact on the fp8 path)
#pragma unroll
        for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
            for (int a = 0; a < 8; ++a) {
                if (a & h) continue;
                const f32x4 x = e[a], y = e[a + h];
                e[a] = x + y;
                e[a + h] = x - y;
            }
        }
        // right H16 per tile (sv folded into the rows of A), su/128, stage, store
        constexpr int kRowBytes = 128;                                     // 16 rows x 128 B = the 2 KB slice
        constexpr int kChunks = kRowBytes / 16;                            // 16-byte chunks per staged row
        constexpr int kTilesPerRound = kRowBytes / (16 * static_cast<int>(sizeof(OutT)));  // 4 bf16, 2 f32
        constexpr int kRounds = 8 / kTilesPerRound;
        char* out_row0 = cur.out + (16 * w) * cur.ld * sizeof(OutT);
#pragma unroll
        for (int rd = 0; rd < kRounds; ++rd) {
#pragma unroll
            for (int t = 0; t < kTilesPerRound; ++t) {
                const int a = rd * kTilesPerRound + t;
                f32x4 d = {0.f, 0.f, 0.f, 0.f};
                if constexpr (FP8) {
                    // exact split: hi = e rounded to fp16 (11 significant bits), lo = e - hi, formed by a
                    // mixed-precision fma straight into fp16.  e is a multiple of 2^-9 below 2^13, so
                    // |lo| <= ulp(hi) / 2 is a multiple of 2^-9 with at most 11 significant bits: exact.
                    uint32_t hi01 = __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(e[a][0]),
                                                                              static_cast<_Float16>(e[a][1])});
                    uint32_t hi23 = __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(e[a][2]),
                                                                              static_cast<_Float16>(e[a][3])});
                    asm volatile("" : "+v"(hi01), "+v"(hi23));
                    typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
                    const u32x2v hraw = {hi01, hi23};
                    const u32x2v lraw = {residual_pair(hi01, e[a][0], e[a][1], neg_one), residual_pair(hi23, e[a][2], e[a][3], neg_one)};
                    // A rows: +-sv of the output column (sign bits from H16 via XOR), shared by the hi and lo
                    // products (k = the lane group's four columns 4 g .. 4 g + 3)
                    const u32x2v araw = {sv2[a] ^ hsg[0], sv2[a] ^ hsg[1]};
                    const f16x4 avh = __builtin_bit_cast(f16x4, araw);
                    d = __builtin_amdgcn_mfma_f32_16x16x16f16(avh, __builtin_bit_cast(f16x4, hraw), d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x16f16(avh, __builtin_bit_cast(f16x4, lraw), d, 0, 0, 0);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(hr[q] * svf[a], e[a][q], d, 0, 0, 0);
                }
                d = d * su_cur;
                // row c, staged columns 16 t + 4 g .. +3 -> byte offset, 16-byte chunks XOR-swizzled by row
                const int byte = (16 * t + 4 * g) * static_cast<int>(sizeof(OutT));
                const int chunk = (byte >> 4) ^ (c & (kChunks - 1));
                char* dst = reinterpret_cast<char*>(slice) + c * kRowBytes + chunk * 16 + (byte & 15);
                if constexpr (sizeof(OutT) == 2) {
                    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
                    const bf16x4 o = {static_cast<__bf16>(d[0]), static_cast<__bf16>(d[1]), static_cast<__bf16>(d[2]),
                                      static_cast<__bf16>(d[3])};
                    *reinterpret_cast<bf16x4*>(dst) = o;
                } else {
                    *reinterpret_cast<f32x4*>(dst) = d;
                }
            }
            // 16 rows x kRowBytes: lane -> (row, chunk), 16 bytes each
#pragma unroll
            for (int r0 = 0; r0 < 16; r0 += 64 / kChunks) {
                const int row = r0 + lane / kChunks, chunk = lane % kChunks;
                const u32x4 v = *reinterpret_cast<const u32x4*>(slice + row * kRowBytes + ((chunk ^ (row & (kChunks - 1))) * 16));
                char* dst = out_row0 + row * cur.ld * sizeof(OutT) + rd * kRowBytes + chunk * 16;
                *(__attribute__((address_space(1))) u32x4*)dst = v;
            }
        }
    }
}

template <int K, bool FP8>
void launch(const Job* jobs, int n_jobs, int64_t total, const uint8_t* lut, int out_dtype, int cus,
            hipStream_t stream) {
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(2 * static_cast<int64_t>(cus), total));  // 2 per CU
    if (out_dtype == 0)
        hipLaunchKernelGGL((decode_kernel<K, FP8, __bf16>), dim3(grid), dim3(kThreads), 0, stream, jobs, n_jobs, total,
                           lut);
    else
        hipLaunchKernelGGL((decode_kernel<K, FP8, float>), dim3(grid), dim3(kThreads), 0, stream, jobs, n_jobs, total,
                           lut);
}

// Job-table upload by kernel argument: the host validates and converts up to
// kUploadChunk jobs into a by-value argument, and one small kernel writes them
// to the device table.  Arguments are captured when the launch is enqueued,
// so there is no host buffer whose lifetime must outlast an asynchronous
// copy, no allocation, and the upload is stream-ordered like any launch.
constexpr int kUploadChunk = 16;

struct JobChunk {
    Job jobs[kUploadChunk];
    int count;
};

__global__ __launch_bounds__(64) void upload_jobs_kernel(JobChunk chunk, Job* __restrict__ dst) {
    const int i = static_cast<int>(threadIdx.x);
    if (i < chunk.count) dst[i] = chunk.jobs[i];
}

bool job_ok(const qsrt_decode_job& s) {
    return s.words && s.row_scale && s.col_scale && s.out && s.rows >= 0 && s.cols >= 0 && s.rows % 128 == 0 &&
           s.cols % 128 == 0 && s.out_ld >= s.cols && s.out_ld % 8 == 0 &&
           reinterpret_cast<uintptr_t>(s.words) % 16 == 0 && s.tile_row_stride % 8 == 0 &&
           s.tile_col_stride % 8 == 0 && s.block_row_stride % 8 == 0 && s.block_col_stride % 8 == 0 &&
           reinterpret_cast<uintptr_t>(s.out) % 16 == 0 && reinterpret_cast<uintptr_t>(s.col_scale) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(s.row_scale) % 16 == 0;
}

// Most jobs the no-allocation decode holds (its job table is `scratch`).
constexpr int kStaticJobs = 4096;

}  // namespace

// Device job table of qsrt_decode_noalloc: every GPU the library runs on holds
// one copy (352 KiB) until the process ends.  Host code never uses this name
// as an address; it uses the per-device address from hipGetSymbolAddress.
static __device__ __align__(256) Job scratch[kStaticJobs];

namespace {

std::mutex g_scratch_mutex;
void* g_scratch_ptr[64] = {nullptr};

// Address of this device's `scratch`, looked up once per device with that
// device current (each GPU holds its own copy at its own address).
int scratch_table(Job** out) {
    int dev = 0;
    QSRT_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return qsrt::fail(qsrt::kBadArgument, "device %d is out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return qsrt::fail(qsrt::kHipError, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                              hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = static_cast<Job*>(g_scratch_ptr[dev]);
    return qsrt::kOk;
}

}  // namespace

extern "C" {

size_t qsrt_decode_workspace_bytes(int n_jobs) {
    if (n_jobs < 0) return 0;
    return static_cast<size_t>(n_jobs) * sizeof(Job);
}

int qsrt_decode_prepare(const qsrt_decode_job* jobs, int n_jobs, int K, void* workspace, size_t workspace_bytes,
                        qsrt_decode_plan* plan, void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (!plan) return qsrt::fail(qsrt::kBadArgument, "null plan pointer");
    *plan = qsrt_decode_plan{workspace, 0, K, 0};
    if (K < 2 || K > 4) return qsrt::fail(qsrt::kBadArgument, "K%d decode is not supported (K2..K4)", K);
    if (n_jobs < 0) return qsrt::fail(qsrt::kBadArgument, "n_jobs must be non-negative");
    if (n_jobs == 0) return qsrt::kOk;
    if (!jobs || !workspace) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (workspace_bytes < qsrt_decode_workspace_bytes(n_jobs))
        return qsrt::fail(qsrt::kWorkspaceTooSmall, "decode workspace needs %zu bytes",
                          qsrt_decode_workspace_bytes(n_jobs));
    if (reinterpret_cast<uintptr_t>(workspace) % 16) return qsrt::fail(qsrt::kBadArgument, "workspace must be 16-byte aligned");
    // pass 1: validate everything before any upload
    for (int i = 0; i < n_jobs; ++i) {
        const qsrt_decode_job& s = jobs[i];
        if (!job_ok(s))
            return qsrt::fail(qsrt::kBadArgument,
                              "decode job %d: need rows, cols multiples of 128, out_ld >= cols and a multiple of 8, "
                              "16-byte aligned words, out, row_scale and col_scale, tile and block strides multiples of 8, "
                              "non-null pointers",
                              i);
        if (s.rows / 128 >= (1 << 30) || s.cols / 128 >= (1 << 30))
            return qsrt::fail(qsrt::kBadArgument, "decode job %d is too large", i);
    }
    // pass 2: convert and upload in chunks (empty jobs are dropped: the kernel never sees them)
    Job* table = static_cast<Job*>(workspace);
    JobChunk chunk;
    chunk.count = 0;
    int64_t total = 0;
    int kept = 0;
    for (int i = 0; i < n_jobs; ++i) {
        const qsrt_decode_job& s = jobs[i];
        if (s.rows == 0 || s.cols == 0) continue;
        chunk.jobs[chunk.count++] = Job{s.words,
                                        s.tile_row_stride,
                                        s.tile_col_stride,
                                        s.block_row_stride ? s.block_row_stride : 8 * s.tile_row_stride,
                                        s.block_col_stride ? s.block_col_stride : 8 * s.tile_col_stride,
                                        s.row_scale,
                                        s.col_scale,
                                        s.out,
                                        s.out_ld,
                                        static_cast<int32_t>(s.rows / 128),
                                        static_cast<int32_t>(s.cols / 128),
                                        total};
        total += (s.rows / 128) * (s.cols / 128);
        if (chunk.count == kUploadChunk || i == n_jobs - 1) {
            hipLaunchKernelGGL(upload_jobs_kernel, dim3(1), dim3(64), 0, stream, chunk, table + kept);
            QSRT_HIP_TRY(hipGetLastError());
            kept += chunk.count;
            chunk.count = 0;
        }
    }
    if (chunk.count) {  // the last job was empty: flush what is pending
        hipLaunchKernelGGL(upload_jobs_kernel, dim3(1), dim3(64), 0, stream, chunk, table + kept);
        QSRT_HIP_TRY(hipGetLastError());
        kept += chunk.count;
    }
    *plan = qsrt_decode_plan{workspace, kept, K, total};
    return qsrt::kOk;
}

int qsrt_decode_execute(const qsrt_decode_plan* plan, const uint8_t* lut_e4m3, int exact_fp8, int out_dtype,
                        void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (!plan) return qsrt::fail(qsrt::kBadArgument, "null plan pointer");
    if (out_dtype != 0 && out_dtype != 1) return qsrt::fail(qsrt::kBadArgument, "out_dtype must be 0 (bf16) or 1 (f32)");
    if (plan->K < 2 || plan->K > 4) return qsrt::fail(qsrt::kBadArgument, "plan holds an unsupported K%d", plan->K);
    if (plan->n_jobs < 0 || plan->total_blocks < 0) return qsrt::fail(qsrt::kBadArgument, "malformed decode plan");
    if (plan->n_jobs == 0 || plan->total_blocks == 0) return qsrt::kOk;
    if (!plan->jobs || !lut_e4m3) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (reinterpret_cast<uintptr_t>(lut_e4m3) % 16) return qsrt::fail(qsrt::kBadArgument, "LUT must be 16-byte aligned");
    int cus = 0;
    if (const int rc = qsrt::current_cu_count(&cus)) return rc;
    const Job* dj = static_cast<const Job*>(plan->jobs);
    const int n = plan->n_jobs;
    const int64_t total = plan->total_blocks;
    switch (plan->K * 2 + (exact_fp8 ? 1 : 0)) {
        case 5: launch<2, true>(dj, n, total, lut_e4m3, out_dtype, cus, stream); break;
        case 4: launch<2, false>(dj, n, total, lut_e4m3, out_dtype, cus, stream); break;
        case 7: launch<3, true>(dj, n, total, lut_e4m3, out_dtype, cus, stream); break;
        case 6: launch<3, false>(dj, n, total, lut_e4m3, out_dtype, cus, stream); break;
        case 9: launch<4, true>(dj, n, total, lut_e4m3, out_dtype, cus, stream); break;
        default: launch<4, false>(dj, n, total, lut_e4m3, out_dtype, cus, stream); break;
    }
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

int qsrt_decode(const qsrt_decode_job* jobs, int n_jobs, int K, const uint8_t* lut_e4m3, int exact_fp8,
                int out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
    if (out_dtype != 0 && out_dtype != 1) return qsrt::fail(qsrt::kBadArgument, "out_dtype must be 0 (bf16) or 1 (f32)");
    if (n_jobs > 0 && !lut_e4m3) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    qsrt_decode_plan plan;
    if (const int rc = qsrt_decode_prepare(jobs, n_jobs, K, workspace, workspace_bytes, &plan, stream)) return rc;
    return qsrt_decode_execute(&plan, lut_e4m3, exact_fp8, out_dtype, stream);
}

}  // extern "C"

extern "C" int qsrt_decode_noalloc(const qsrt_decode_job* jobs, int n_jobs, int K, const uint8_t* lut_e4m3,
                                   int exact_fp8, int out_dtype, void* stream) {
    if (out_dtype != 0 && out_dtype != 1) return qsrt::fail(qsrt::kBadArgument, "out_dtype must be 0 (bf16) or 1 (f32)");
    if (n_jobs > kStaticJobs)
        return qsrt::fail(qsrt::kBadArgument, "qsrt_decode_noalloc holds at most %d jobs; got %d (use qsrt_decode "
                          "with a workspace)", kStaticJobs, n_jobs);
    if (n_jobs > 0 && !lut_e4m3) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    Job* table = nullptr;
    if (const int rc = scratch_table(&table)) return rc;
    qsrt_decode_plan plan;
    if (const int rc = qsrt_decode_prepare(jobs, n_jobs, K, table, sizeof(Job) * kStaticJobs, &plan, stream)) return rc;
    return qsrt_decode_execute(&plan, lut_e4m3, exact_fp8, out_dtype, stream);
}
