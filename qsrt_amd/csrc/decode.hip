// Fused trellis decode: packed EXL words -> cyclic states -> E4M3 labels ->
// W = diag(su) . H128 X H128 . diag(sv) -> bf16 (or f32), one 128x128 block
// per workgroup iteration.
//
// Reference semantics (qsrt/exl3_reference.py:61-302, qsrt/qsrt.py:1175-1209):
//   X[K, N]  = labels of the states, tile-major, tensor-core order in a tile
//   W        = H_R( H_L(X) * su[:, None] ) * sv[None, :]
// with H_L / H_R the normalised 128-block Sylvester Hadamards.  Row scaling
// commutes with the right product, so per 128x128 block
//   W_blk = su . (H128 X_blk H128) . sv / 128   (unnormalised +-1 Hadamards).
// H128 = H8 (x) H16 (Kronecker over the 8x8 tiles of the block and the 16x16
// positions in a tile), so the block transform factors into per-tile H16
// products on the matrix cores and 8-point butterflies across tiles.
//
// Per workgroup (8 waves), per block:
//  1. wave w owns tile-column w.  Lane (c = lane % 16, g = lane / 16) holds,
//     for every tile, the 4 values of column c at rows 2g + {0,1,8,9}: the
//     four consecutive trellis positions 32 (c % 8) + 8 g + 4 (c / 8) + 0..3
//     (tensor-core order), i.e. one 16 + 3K-bit window of the tile's
//     MSB-first bitstream.  EXL stores adjacent 16-bit words swapped, so a
//     little-endian u32 read is the big-endian 32-bit chunk of the stream.
//  2. labels come from the state-indexed E4M3 LUT in LDS and are used as fp8
//     MFMA operands directly: A = [X_a ; X_(a+1)]^T (k = the 32 rows of two
//     vertically adjacent tiles), B = [H16 ; +-H16]: the two products are
//     (X_a +- X_(a+1))^T H16 -- the per-tile left H16 fused with the first
//     H8 butterfly stage across tile-rows (bit 0 of a).
//     (fp8 MFMA sums are exact for |label| <= 6; larger tables take the
//     FP32-MFMA variant below.)
//  3. the other two H8 stages across tile-rows on VALU; multiply by su/128.
//  4. right H16 per tile on FP32 MFMA (16x16x4, +-1 operands): exact
//     products.  Output lane layout = row c, columns 4g..4g+3 of the tile.
//  5. exchange through LDS (wave w now owns tile-row w), H8 across
//     tile-columns on VALU, multiply by sv, convert, store 4 consecutive
//     outputs per lane per tile.

#include "common.h"
#include "qsrt_amd.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kXchFloat4 = 8 * 8 * 64;  // 64 tiles x 64 lanes x float4

__device__ __forceinline__ int hsign(int i, int j) { return (__builtin_popcount(i & j) & 1) ? -1 : 1; }

struct Job {
    const int16_t* words;
    int64_t tile_row_stride;
    int64_t tile_col_stride;
    const float* row_scale;
    const float* col_scale;
    void* out;
    int64_t out_ld;
    int64_t rows;
    int64_t cols;
    int64_t first_block;  // prefix over jobs (filled by the host)
};

template <typename OutT>
__device__ __forceinline__ void store4(OutT* p, float a, float b, float c, float d);

template <>
__device__ __forceinline__ void store4<float>(float* p, float a, float b, float c, float d) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}

template <>
__device__ __forceinline__ void store4<__bf16>(__bf16* p, float a, float b, float c, float d) {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    bf16x4 v = {static_cast<__bf16>(a), static_cast<__bf16>(b), static_cast<__bf16>(c), static_cast<__bf16>(d)};
    *reinterpret_cast<bf16x4*>(p) = v;
}

// 16-bit states of trellis positions p0..p0+3 of one tile from its u32 stream.
template <int K>
__device__ __forceinline__ uint32_t window(const uint32_t* u, int m0, int m1, int sh) {
    const uint64_t two = (static_cast<uint64_t>(u[m0]) << 32) | u[m1];
    return static_cast<uint32_t>(two >> (32 - sh));
}

template <int K, bool FP8, typename OutT>
__global__ __launch_bounds__(kThreads, 1) void decode_kernel(const Job* __restrict__ jobs, int n_jobs,
                                                             int64_t total_blocks, const uint8_t* __restrict__ lut) {
    __shared__ __attribute__((aligned(16))) uint8_t lut_s[65536];
    __shared__ f32x4 xch[kXchFloat4];

    for (int i = threadIdx.x; i < 65536 / 16; i += kThreads)
        reinterpret_cast<uint4*>(lut_s)[i] = reinterpret_cast<const uint4*>(lut)[i];

    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int c = lane & 15;
    const int g = lane >> 4;
    const int rho[4] = {2 * g, 2 * g + 1, 2 * g + 8, 2 * g + 9};

    // fp8 +-1 operands of the left products: B[k = (g, j)][c] = H16[rho(j & 3)][c] (* -1 for j >= 4 in diff)
    uint64_t b_sum = 0, b_diff = 0;
    // FP32 operands for the left products of the FP32 variant: lane (c, g) holds H16[rho][c] for its rows
    float hl[4];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int s = hsign(rho[j & 3], c);
        const uint64_t pos = 0x38, neg = 0xB8;  // E4M3 +1 / -1
        b_sum |= (s > 0 ? pos : neg) << (8 * j);
        b_diff |= ((j < 4 ? s : -s) > 0 ? pos : neg) << (8 * j);
        if (j < 4) hl[j] = static_cast<float>(s);
    }
    // A operands of the right product: A_q[i = c][k = g] = H16[c][4g + q]
    float hr[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) hr[q] = static_cast<float>(hsign(c, 4 * g + q));

    // bit window of this lane's four positions
    const int p0 = 32 * (c & 7) + 8 * g + 4 * (c >> 3);
    int b0 = (p0 + 1) * K - 16;
    if (b0 < 0) b0 += 256 * K;
    const int m0 = b0 >> 5;
    const int m1 = (m0 + 1) % (8 * K);
    const int sh = b0 & 31;

    __syncthreads();

    for (int64_t blk = blockIdx.x; blk < total_blocks; blk += gridDim.x) {
        // job containing blk (uniform across the workgroup)
        int lo = 0, hi = n_jobs - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (jobs[mid].first_block <= blk) lo = mid; else hi = mid - 1;
        }
        const Job& J = jobs[lo];
        const int64_t local = blk - J.first_block;
        const int64_t nbc = J.cols >> 7;
        const int64_t br = local / nbc, bc = local - br * nbc;

        // ---- phase 1: tile-column w of the block
        f32x4 d[8];
        uint8_t lab[8][4];
#pragma unroll
        for (int a = 0; a < 8; ++a) {
            const uint32_t* u = reinterpret_cast<const uint32_t*>(
                J.words + (8 * br + a) * J.tile_row_stride + (8 * bc + w) * J.tile_col_stride);
            const uint32_t win = window<K>(u, m0, m1, sh);
#pragma unroll
            for (int i = 0; i < 4; ++i) lab[a][i] = lut_s[(win >> (16 - i * K)) & 0xFFFFu];
        }
        if constexpr (FP8) {
#pragma unroll
            for (int a = 0; a < 8; a += 2) {
                uint64_t av = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    av |= static_cast<uint64_t>(lab[a][i]) << (8 * i);
                    av |= static_cast<uint64_t>(lab[a + 1][i]) << (8 * (i + 4));
                }
                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                d[a] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(static_cast<long>(av), static_cast<long>(b_sum), z, 0, 0, 0);
                d[a + 1] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(static_cast<long>(av), static_cast<long>(b_diff), z, 0, 0, 0);
            }
        } else {
            // D1 = X^T H16 as four rank-4 FP32 products per tile, then the bit-0 butterfly.
#pragma unroll
            for (int a = 0; a < 8; ++a) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // A[c][k = g] = X[rho(i)][c]; B[k = g][col] = H16[rho(i)][col]
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qsrt::e4m3_to_float(lab[a][i]), hl[i], acc, 0, 0, 0);
                }
                d[a] = acc;
            }
#pragma unroll
            for (int a = 0; a < 8; a += 2) {
                const f32x4 x = d[a], y = d[a + 1];
                d[a] = x + y;
                d[a + 1] = x - y;
            }
        }
        // H8 stages on bits 1 and 2 of the tile-row index
#pragma unroll
        for (int h = 2; h < 8; h <<= 1) {
#pragma unroll
            for (int a = 0; a < 8; ++a) {
                if (a & h) continue;
                const f32x4 x = d[a], y = d[a + h];
                d[a] = x + y;
                d[a + h] = x - y;
            }
        }
        // su / 128 of output row 16 a + c; right H16 on FP32 MFMA
#pragma unroll
        for (int a = 0; a < 8; ++a) {
            const float su = J.row_scale[128 * br + 16 * a + c];
            const f32x4 v = d[a] * su;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(hr[q], v[q], acc, 0, 0, 0);
            xch[(a * 8 + w) * 64 + lane] = acc;
        }
        __syncthreads();

        // ---- phase 2: tile-row w of the block
        f32x4 e[8];
#pragma unroll
        for (int a = 0; a < 8; ++a) e[a] = xch[(w * 8 + a) * 64 + lane];
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
        OutT* out = static_cast<OutT*>(J.out);
        const int64_t row = 128 * br + 16 * w + c;
#pragma unroll
        for (int a = 0; a < 8; ++a) {
            const int64_t col = 128 * bc + 16 * a + 4 * g;
            const float4 sv = *reinterpret_cast<const float4*>(J.col_scale + col);
            store4<OutT>(out + row * J.out_ld + col, e[a][0] * sv.x, e[a][1] * sv.y, e[a][2] * sv.z, e[a][3] * sv.w);
        }
        __syncthreads();
    }
}

template <int K, bool FP8>
void launch(const Job* jobs, int n_jobs, int64_t total, const uint8_t* lut, int out_dtype, unsigned grid,
            hipStream_t stream) {
    if (out_dtype == 0)
        hipLaunchKernelGGL((decode_kernel<K, FP8, __bf16>), dim3(grid), dim3(kThreads), 0, stream, jobs, n_jobs, total, lut);
    else
        hipLaunchKernelGGL((decode_kernel<K, FP8, float>), dim3(grid), dim3(kThreads), 0, stream, jobs, n_jobs, total, lut);
}

}  // namespace

extern "C" {

size_t qsrt_decode_workspace_bytes(int n_jobs) {
    if (n_jobs < 0) return 0;
    return static_cast<size_t>(n_jobs) * sizeof(Job);
}

int qsrt_decode(const qsrt_decode_job* jobs, int n_jobs, int K, const uint8_t* lut_e4m3, int exact_fp8,
                int out_dtype, void* workspace, size_t workspace_bytes, void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (K < 2 || K > 4) return qsrt::fail(qsrt::kBadArgument, "K%d decode is not supported (K2..K4)", K);
    if (n_jobs < 0) return qsrt::fail(qsrt::kBadArgument, "n_jobs must be non-negative");
    if (out_dtype != 0 && out_dtype != 1) return qsrt::fail(qsrt::kBadArgument, "out_dtype must be 0 (bf16) or 1 (f32)");
    if (n_jobs == 0) return qsrt::kOk;
    if (!jobs || !lut_e4m3 || !workspace) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (workspace_bytes < qsrt_decode_workspace_bytes(n_jobs))
        return qsrt::fail(qsrt::kWorkspaceTooSmall, "decode workspace needs %zu bytes",
                          qsrt_decode_workspace_bytes(n_jobs));
    if (reinterpret_cast<uintptr_t>(lut_e4m3) % 16 || reinterpret_cast<uintptr_t>(workspace) % 16)
        return qsrt::fail(qsrt::kBadArgument, "LUT and workspace must be 16-byte aligned");
    const size_t out_align = out_dtype == 0 ? 8 : 16;
    Job* host = static_cast<Job*>(malloc(sizeof(Job) * n_jobs));
    if (!host) return qsrt::fail(qsrt::kHipError, "host allocation failed");
    int64_t total = 0;
    for (int i = 0; i < n_jobs; ++i) {
        const qsrt_decode_job& s = jobs[i];
        const bool ok = s.words && s.row_scale && s.col_scale && s.out && s.rows >= 0 && s.cols >= 0 &&
                        s.rows % 128 == 0 && s.cols % 128 == 0 && s.out_ld >= s.cols && s.out_ld % 4 == 0 &&
                        reinterpret_cast<uintptr_t>(s.words) % 4 == 0 && s.tile_row_stride % 2 == 0 &&
                        s.tile_col_stride % 2 == 0 && reinterpret_cast<uintptr_t>(s.out) % out_align == 0 &&
                        reinterpret_cast<uintptr_t>(s.col_scale) % 16 == 0;
        if (!ok) {
            free(host);
            return qsrt::fail(qsrt::kBadArgument,
                              "decode job %d: need rows, cols multiples of 128, out_ld >= cols and % 4, 4-byte "
                              "aligned words with even tile strides, aligned out and col_scale, non-null pointers",
                              i);
        }
        host[i] = Job{s.words, s.tile_row_stride, s.tile_col_stride, s.row_scale, s.col_scale, s.out, s.out_ld,
                      s.rows, s.cols, total};
        total += (s.rows / 128) * (s.cols / 128);
    }
    const hipError_t cp = hipMemcpyAsync(workspace, host, sizeof(Job) * n_jobs, hipMemcpyHostToDevice, stream);
    free(host);
    if (cp != hipSuccess) return qsrt::fail(qsrt::kHipError, "job upload failed: %s", hipGetErrorString(cp));
    if (total == 0) return qsrt::kOk;
    int cus = 0;
    if (const int rc = qsrt::current_cu_count(&cus)) return rc;
    const unsigned grid = static_cast<unsigned>(total < cus ? total : cus);
    const Job* dj = static_cast<const Job*>(workspace);
    switch (K * 2 + (exact_fp8 ? 1 : 0)) {
        case 5: launch<2, true>(dj, n_jobs, total, lut_e4m3, out_dtype, grid, stream); break;
        case 4: launch<2, false>(dj, n_jobs, total, lut_e4m3, out_dtype, grid, stream); break;
        case 7: launch<3, true>(dj, n_jobs, total, lut_e4m3, out_dtype, grid, stream); break;
        case 6: launch<3, false>(dj, n_jobs, total, lut_e4m3, out_dtype, grid, stream); break;
        case 9: launch<4, true>(dj, n_jobs, total, lut_e4m3, out_dtype, grid, stream); break;
        default: launch<4, false>(dj, n_jobs, total, lut_e4m3, out_dtype, grid, stream); break;
    }
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

}  // extern "C"
