// Fused trellis decode: packed EXL words -> cyclic states -> E4M3 labels ->
// W = diag(su) . H128 X H128 . diag(sv) -> bf16 (or f32), one 128 x 128
// block at a time.
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
// Labels: lane (c = lane % 16, g = lane / 16) takes, in a tile, the 4
// values of column c at rows 2g + {0,1,8,9}: trellis positions 32 (c % 8) +
// 8 g + 4 (c / 8) + 0..3 (tensor-core order), one 16 + 3K-bit window of the
// tile's MSB-first bitstream (EXL stores adjacent 16-bit words swapped, so a
// little-endian u32 read is the big-endian 32-bit chunk of the stream); the
// labels come from the state-indexed E4M3 LUT in LDS.  A tile-column's words
// arrive with one 16-byte load per lane and are staged through LDS.
//
// decode_block_wave_kernel (tables with |label| <= 6: the T12 tables): one
// wave per block, twelve waves per CU; see the kernel.  The left transform of
// a tile is one fp8 MFMA (16x16x128) over the 128 rows of its column, exact
// for |label| <= 6 (sums of at most 128 x 6 on multiples of 2^-9); the right
// H8 = H2 (x) H4 across tile-columns: its two stages over tile-column bits 1
// and 2 run on VALU (exact: < 2^22 units of 2^-9); each value is split into
// fp16 hi + lo (exact, 11 + 11 bits: hi by rounding, lo by a mixed-precision
// fma); the stage over bit 0 and the right H16 are two accumulating f16 MFMAs
// (16x16x32) per output tile, on hi then lo of the tile-column pair (2p,
// 2p + 1), with A = H16 with row i scaled by the fp16 sv of output column i,
// repeated over the pair with the sign of H2; then times su/128 and the
// conversion.
//
// decode_fp32_kernel (tables with larger labels): one workgroup of 8 waves
// per block, two per CU.  Wave w decodes tile-column w into a 16 KB LDS
// label area, then produces output tile-row w with FP32 MFMAs for both
// products (labels widened exactly to FP32).
//
// Both stage outputs through LDS (XOR-swizzled 16-byte chunks) so each store
// instruction writes full 128-byte row segments, and both issue the next
// block's loads before this block's stores: vector-memory counters retire in
// issue order, so a load issued after stores returns only once they drain.

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

// Cursor of block `blk`: binary search over the jobs' block prefix.
__device__ __forceinline__ Cursor cursor_at(const Job* jobs, int n_jobs, int64_t blk) {
    int lo = 0, hi = n_jobs - 1;  // jobs[lo].first_block <= blk < jobs[hi + 1].first_block
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (jobs[mid].first_block <= blk) lo = mid; else hi = mid - 1;
    }
    const int64_t local = blk - jobs[lo].first_block;
    const int br = static_cast<int>(local / jobs[lo].nbc);
    return Cursor{lo, br, static_cast<int>(local - static_cast<int64_t>(br) * jobs[lo].nbc)};
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
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

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

template <int K, typename OutT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void decode_fp32_kernel(const Job* __restrict__ jobs, int n_jobs, int64_t total_blocks, const uint8_t* __restrict__ lut) {
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

    // Right-product A operand rows: H16[c][4g + q]; left-product operand: H16[rho(i)][c]
    float hr[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) hr[q] = static_cast<float>(hsign(c, 4 * g + q));
    float hl[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) hl[i] = static_cast<float>(hsign(rho[i], c));
    // Keep the operand constants in registers instead of recomputing them in the loop.
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
        // ---- A: stage the tile-column's words, decode the lane's labels (raised issue priority through B1)
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
        float svf[8];
#pragma unroll
        for (int a = 0; a < 8; ++a) svf[a] = sv[a];
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
            e[a2] = acc;
        }
        __syncthreads();  // every wave is done reading labels: slices are private again
        __builtin_amdgcn_s_setprio(0);

        // ---- B2: right H8 across tile-columns
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
#pragma unroll
                for (int q = 0; q < 4; ++q) d = __builtin_amdgcn_mfma_f32_16x16x4f32(hr[q] * svf[a], e[a][q], d, 0, 0, 0);
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

// ---------------------------------------------------------------------------
// One wave per block.  Each wave owns whole 128 x 128 blocks: it decodes all
// 64 tiles' labels straight into registers -- lane (c, g) holds, for every
// tile-column a', the 32 labels that are the left product's A operand of
// that column (64 VGPRs) -- and then produces the block's eight output
// tile-rows one after another: for tile-row r, eight fp8 MFMAs (one per
// tile-column, B = H8[r][.] (x) H16 in E4M3 +-1), the right H8's stages over
// tile-column bits 1 and 2 on VALU, its stage over bit 0 with the right H16 as
// two f16 MFMAs (K = 32) per tile on the exact hi/lo split of a tile-column
// pair, times su/128, bf16 or f32, staged through the wave's 2 KB LDS slice
// into full 128-byte row segments.  Successive tile-rows are visited in
// Gray-code order, so B changes by one sign flip on four of its eight
// registers between them.  Nothing is shared between waves but the LUT: no
// label exchange and no barrier after the LUT load, so the workgroup's twelve
// waves drift into different phases (gathers, MFMAs, VALU, stores) and keep
// every pipe busy at once.
constexpr int kBlockWaves = 12;  // one workgroup of 12 waves per CU (3 per SIMD)
constexpr int kBlockThreads = 64 * kBlockWaves;
constexpr int kSliceBytes = 2048;  // half an output tile-row of bf16 (16 rows x 128 B); a tile-column's words
constexpr int kScaleBytes = 1024;  // a block's su (128 f32) and fp16-paired sv (128 x 2 fp16)


// Wave-uniform values computed on the vector unit, moved to scalar registers
// (the block context would otherwise hold 32 VGPRs across the label phase).
__device__ __forceinline__ int64_t sgpr64(int64_t v) {
    const uint64_t u = static_cast<uint64_t>(v);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}
template <typename T>
__device__ __forceinline__ T* sgpr_ptr(T* p) {
    return reinterpret_cast<T*>(sgpr64(reinterpret_cast<int64_t>(p)));
}
__device__ __forceinline__ BlockCtx uniform_ctx(BlockCtx x) {
    x.words = sgpr_ptr(x.words);
    x.trs = sgpr64(x.trs);
    x.tcs = sgpr64(x.tcs);
    x.su = sgpr_ptr(x.su);
    x.sv = sgpr_ptr(x.sv);
    x.out = sgpr_ptr(x.out);
    x.ld = sgpr64(x.ld);
    return x;
}

template <int K, typename OutT>
__global__ __launch_bounds__(kBlockThreads) __attribute__((amdgpu_waves_per_eu(3, 3)))
void decode_block_wave_kernel(const Job* __restrict__ jobs, int n_jobs, int64_t total_blocks,
                              const uint8_t* __restrict__ lut) {
    static_assert(sizeof(OutT) == 2 || sizeof(OutT) == 4, "bf16 or f32 output");
    __shared__ __attribute__((aligned(16))) uint8_t lut_s[65536];
    __shared__ __attribute__((aligned(16))) uint8_t slices[kBlockWaves * kSliceBytes];
    __shared__ __attribute__((aligned(16))) uint8_t scales[kBlockWaves * kScaleBytes];

    for (int i = threadIdx.x; i < 65536 / 16; i += kBlockThreads)
        reinterpret_cast<uint4*>(lut_s)[i] = reinterpret_cast<const uint4*>(lut)[i];
    __syncthreads();  // the kernel's only barrier

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t gw = static_cast<int64_t>(blockIdx.x) * kBlockWaves + w;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * kBlockWaves;
    const int64_t begin = sgpr64(total_blocks * gw / nw);
    const int64_t end = sgpr64(total_blocks * (gw + 1) / nw);
    if (begin >= end) return;

    const int c = lane & 15;
    const int g = lane >> 4;
    const int rho[4] = {2 * g, 2 * g + 1, 2 * g + 8, 2 * g + 9};
    // B of tile-row 0: byte i of every register is H16[rho(i)][c] in E4M3 (+1 0x38, -1 0xB8)
    uint32_t bbase = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) bbase |= (hsign(rho[i], c) > 0 ? 0x38u : 0xB8u) << (8 * i);
    uint32_t hsg[2];  // fp16 sign masks of H16[c][4g + q], q = 0..3, as two packed pairs
#pragma unroll
    for (int h = 0; h < 2; ++h)
        hsg[h] = (hsign(c, 4 * g + 2 * h) < 0 ? 0x8000u : 0u) | (hsign(c, 4 * g + 2 * h + 1) < 0 ? 0x80000000u : 0u);
    float neg_one = -1.0f;
    asm volatile("" : "+v"(neg_one));

    const int p0 = 32 * (c & 7) + 8 * g + 4 * (c >> 3);
    int b0 = (p0 + 1) * K - 16;
    if (b0 < 0) b0 += 256 * K;
    const int m0 = b0 >> 5;
    const int m1 = (m0 + 1) % (8 * K);
    const uint32_t rsh = 32u - static_cast<uint32_t>(b0 & 31);

    uint8_t* slice = slices + kSliceBytes * w;
    const uint32_t* wstage = reinterpret_cast<const uint32_t*>(slice);
    float* su_s = reinterpret_cast<float*>(scales + kScaleBytes * w);  // [128] row scales
    uint32_t* sv_s = reinterpret_cast<uint32_t*>(su_s + 128);          // [8][16]: sv of column 16 a + c, fp16 pair

    // Loads of a block are issued before the previous block's stores: vector-memory counters retire in issue
    // order, so a load issued after stores returns only once they have drained.
    Cursor cu = cursor_at(jobs, n_jobs, begin);
    BlockCtx ctx = uniform_ctx(block_ctx(jobs, cu, sizeof(OutT)));
    u32x4 words[8];
#pragma unroll
    for (int col = 0; col < 8; ++col) words[col] = fetch_words<K>(ctx, col, lane);
    float su_n[8], sv_n[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) {
        su_n[a] = ((gf32)ctx.su)[16 * a + c];
        sv_n[a] = ((gf32)ctx.sv)[16 * a + c];
    }

    for (int64_t blk = begin; blk < end; ++blk) {
        const BlockCtx cur = ctx;
        // ---- labels of all 64 tiles, tile-column by tile-column (high issue priority: the gathers are the
        // phase other waves' MFMA and store phases can hide behind)
        __builtin_amdgcn_s_setprio(2);
        i32x8 av[8];
#pragma unroll
        for (int col = 0; col < 8; ++col) {
            if (lane < 16 * K) reinterpret_cast<u32x4*>(slice)[lane] = words[col];
            words[col] = u32x4{0u, 0u, 0u, 0u};  // dead until the next block's prefetch (not held across it)
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
            // pack the column's labels here (its 32 gathers in flight together), not after all 256 gathers
#pragma unroll
            for (int a = 0; a < 8; ++a) {
                asm volatile("" : "+v"(lab[a]));
                av[col][a] = static_cast<int>(lab[a]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // this block's scales into the wave's LDS scale area (lanes of one c write the same values), then the
        // next block's loads, all before this block's first store
#pragma unroll
        for (int a = 0; a < 8; ++a) {
            su_s[16 * a + c] = su_n[a];
            sv_s[16 * a + c] =
                __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(sv_n[a]), static_cast<_Float16>(sv_n[a])});
        }
        const bool more = blk + 1 < end;
#pragma unroll
        for (int a = 0; a < 8; ++a) su_n[a] = sv_n[a] = 0.f;  // likewise
        if (more) {
            cursor_next(jobs, cu);
            ctx = uniform_ctx(block_ctx(jobs, cu, sizeof(OutT)));
#pragma unroll
            for (int a = 0; a < 8; ++a) {
                su_n[a] = ((gf32)ctx.su)[16 * a + c];
                sv_n[a] = ((gf32)ctx.sv)[16 * a + c];
            }
        }
        // ---- output tile-rows in Gray-code order; the left MFMAs at priority 1, the rest at 0
        uint32_t bb = bbase;
        asm volatile("" : "+v"(bb));  // eight copies per block, not eight registers held across it
        i32x8 bl;
#pragma unroll
        for (int a = 0; a < 8; ++a) bl[a] = static_cast<int>(bb);
        auto tile_row = [&](const int step, const bool last) {
            const int r = step ^ (step >> 1);
            const float su_r = su_s[16 * r + c];
            if (step > 0) {
                const int m = __builtin_ctz(step);  // the bit of r that changed: H8[r][a] flips where a has it
#pragma unroll
                for (int a = 0; a < 8; ++a)
                    bl[a] = static_cast<int>(static_cast<uint32_t>(bl[a]) ^ (((a >> m) & 1) ? 0x80808080u : 0u));
            }
            __builtin_amdgcn_s_setprio(1);
            f32x4 e[8];
#pragma unroll
            for (int a2 = 0; a2 < 8; ++a2) {
                const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
                e[a2] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[a2], bl, zero, 0, 0, 0, 127, 0, 127);
            }
            // the labels are dead after the last tile-row's left products: the next block's words take their
            // registers, loaded before this tile-row's stores (only earlier tile-rows' stores are ahead of them)
            if (last && more) {
                __builtin_amdgcn_sched_barrier(0);  // not above the MFMAs that still read the labels
#pragma unroll
                for (int col = 0; col < 8; ++col) words[col] = fetch_words<K>(ctx, col, lane);
            }
            __builtin_amdgcn_s_setprio(0);
            // right H8 over tile-column bits 1 and 2 (exact); bit 0 runs inside the right MFMAs
#pragma unroll
            for (int h = 2; h < 8; h <<= 1) {
#pragma unroll
                for (int a = 0; a < 8; ++a) {
                    if (a & h) continue;
                    const f32x4 x = e[a], y = e[a + h];
                    e[a] = x + y;
                    e[a + h] = x - y;
                }
            }
            constexpr int kRowBytes = 128;
            constexpr int kChunks = kRowBytes / 16;
            constexpr int kTilesPerRound = kRowBytes / (16 * static_cast<int>(sizeof(OutT)));
            constexpr int kRounds = 8 / kTilesPerRound;
            static_assert(kTilesPerRound % 2 == 0, "a tile-column pair stays within one staging round");
            char* out_row0 = cur.out + (16 * r) * cur.ld * sizeof(OutT);
#pragma unroll
            for (int rd = 0; rd < kRounds; ++rd) {
#pragma unroll
                for (int tp = 0; tp < kTilesPerRound; tp += 2) {
                    // tile-column pair (2p, 2p + 1) = (a0, a0 + 1): K = 32 slots 0-3 carry a0's values (rows 4g..4g+3
                    // of the lane's column), slots 4-7 those of a0 + 1; A repeats the H16 row for both, negated on
                    // slots 4-7 for the odd output tile (H2[1][1] = -1)
                    const int a0 = rd * kTilesPerRound + tp;
                    uint32_t hi[4];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        hi[2 * u] = __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(e[a0 + u][0]),
                                                                      static_cast<_Float16>(e[a0 + u][1])});
                        hi[2 * u + 1] = __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(e[a0 + u][2]),
                                                                          static_cast<_Float16>(e[a0 + u][3])});
                    }
                    asm volatile("" : "+v"(hi[0]), "+v"(hi[1]), "+v"(hi[2]), "+v"(hi[3]));
                    const u32x4 hraw = {hi[0], hi[1], hi[2], hi[3]};
                    const u32x4 lraw = {residual_pair(hi[0], e[a0][0], e[a0][1], neg_one),
                                        residual_pair(hi[1], e[a0][2], e[a0][3], neg_one),
                                        residual_pair(hi[2], e[a0 + 1][0], e[a0 + 1][1], neg_one),
                                        residual_pair(hi[3], e[a0 + 1][2], e[a0 + 1][3], neg_one)};
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int t = tp + u, a = a0 + u;
                        const uint32_t sv2 = sv_s[16 * a + c];
                        const uint32_t x0 = sv2 ^ hsg[0], x1 = sv2 ^ hsg[1];
                        const uint32_t flip = u ? 0x80008000u : 0u;
                        const u32x4 araw = {x0, x1, x0 ^ flip, x1 ^ flip};
                        const f16x8 avh = __builtin_bit_cast(f16x8, araw);
                        f32x4 d = {0.f, 0.f, 0.f, 0.f};
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(avh, __builtin_bit_cast(f16x8, hraw), d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(avh, __builtin_bit_cast(f16x8, lraw), d, 0, 0, 0);
                        d = d * su_r;
                        const int byte = (16 * t + 4 * g) * static_cast<int>(sizeof(OutT));
                        const int chunk = (byte >> 4) ^ (c & (kChunks - 1));
                        char* dst = reinterpret_cast<char*>(slice) + c * kRowBytes + chunk * 16 + (byte & 15);
                        if constexpr (sizeof(OutT) == 2) {
                            typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
                            const bf16x4 o = {static_cast<__bf16>(d[0]), static_cast<__bf16>(d[1]),
                                              static_cast<__bf16>(d[2]), static_cast<__bf16>(d[3])};
                            *reinterpret_cast<bf16x4*>(dst) = o;
                        } else {
                            *reinterpret_cast<f32x4*>(dst) = d;
                        }
                    }
                }
#pragma unroll
                for (int r0 = 0; r0 < 16; r0 += 64 / kChunks) {
                    const int row = r0 + lane / kChunks, chunk = lane % kChunks;
                    const u32x4 v =
                        *reinterpret_cast<const u32x4*>(slice + row * kRowBytes + ((chunk ^ (row & (kChunks - 1))) * 16));
                    char* dst = out_row0 + row * cur.ld * sizeof(OutT) + rd * kRowBytes + chunk * 16;
                    *(__attribute__((address_space(1))) u32x4*)dst = v;
                }
            }
        };
#pragma unroll 1
        for (int step = 0; step < 7; ++step) tile_row(step, false);
        tile_row(7, true);  // peeled: the labels die inside it, which makes room for the next block's words
    }
}

// One workgroup of kBlockWaves waves per CU (fewer when there are fewer blocks).
template <int K>
void launch_block_wave_k(const Job* jobs, int n_jobs, int64_t total, const uint8_t* lut, int out_dtype, int cus,
                         hipStream_t stream) {
    const int64_t groups = (total + kBlockWaves - 1) / kBlockWaves;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(cus, groups));
    if (out_dtype == 0)
        hipLaunchKernelGGL((decode_block_wave_kernel<K, __bf16>), dim3(grid), dim3(kBlockThreads), 0, stream, jobs,
                           n_jobs, total, lut);
    else
        hipLaunchKernelGGL((decode_block_wave_kernel<K, float>), dim3(grid), dim3(kBlockThreads), 0, stream, jobs,
                           n_jobs, total, lut);
}

template <int K, bool FP8>
void launch(const Job* jobs, int n_jobs, int64_t total, const uint8_t* lut, int out_dtype, int cus,
            hipStream_t stream) {
    if constexpr (FP8) {
        launch_block_wave_k<K>(jobs, n_jobs, total, lut, out_dtype, cus, stream);
    } else {
        const unsigned grid = static_cast<unsigned>(std::min<int64_t>(2 * static_cast<int64_t>(cus), total));  // 2 per CU
        if (out_dtype == 0)
            hipLaunchKernelGGL((decode_fp32_kernel<K, __bf16>), dim3(grid), dim3(kThreads), 0, stream, jobs, n_jobs,
                               total, lut);
        else
            hipLaunchKernelGGL((decode_fp32_kernel<K, float>), dim3(grid), dim3(kThreads), 0, stream, jobs, n_jobs,
                               total, lut);
    }
}

// Job-table upload by kernel argument: the host validates and converts up to
// kUploadChunk jobs into a by-value argument, and one small kernel writes them
// to the device table.  Arguments are captured when the launch is enqueued,
// so there is no host buffer whose lifetime must outlast an asynchronous
// copy, no allocation, and the upload is stream-ordered like any launch.
constexpr int kUploadChunk = 44;  // 44 x 88-byte jobs: one launch's 4 KiB argument block

struct JobChunk {
    Job jobs[kUploadChunk];
    int count;
};

static_assert(sizeof(Job) == 88 && sizeof(JobChunk) <= 4096, "a job chunk must fit one kernel argument block");

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
