// Band propagation of the recursive BaKron two-sided rounding: the fused FP32
// update that reference qsrt/csrc/sqg_quantize.cu:141-270 (kernels) and
// :991-1100 (launcher) implement, bound in Python as
// qsrt/sqg_quantizer.py:383-407 and called from the divide and conquer of
// qsrt/two_sided_rounding.py:777-799.
//
// Matrices are FP32 row-major [batch, n_out, n_in]: the running targets T, the
// quantized reconstruction Q and the intermediate I.  The factors are
// [n_out, n_out] and [n_in, n_in] per member (a batch stride of 0 shares one).
// Blocks are 16 x 16; block (o, i) lies on anti-diagonal o + i.  For the
// finished band of diagonals [first, middle) and the next band [middle, last):
//
//   left   I(o, i)  = sum over s in [max(0, first - i), min(ob, middle - i))  of  Lout(o, s) (Q - T)(s, i)
//                     for every block with first <= o + i < last
//   right  T(o, c) += sum over s in [max(0, first - o), min(ib, middle, last - o))  of  I(o, s) Lin(c, s)^T
//                     for every block with middle <= o + c < last
//
// (the left sum takes every source row of the finished band in the block's column; the right sum stops at
// last - o because the factors are block-lower, Lin(c, s) = 0 for s > c).  The sums run over s in
// ascending order; each source block is one 16 x 16 x 16 product.
//
// Four waves per 256-thread workgroup, no LDS and no barriers; each wave computes a tile of target blocks (below),
// and each (target, source) block product is four v_mfma_f32_16x16x4_f32.  The sixteen k of a block product
// are split as k = 4 g + q over the instruction q = 0..3 and the lane's group g = lane / 16, so that a
// lane's A operands for the four instructions are one float4 of a row (row lane % 16, columns 4 g .. 4 g + 3),
// as are the right product's B operands (rows of Lin); the left product's B operands are rows 4 g .. 4 g + 3
// of one column of Q - T.  The next source block's operands are loaded before the current block's products.
// A wave whose targets lie past its column's (row's) end returns at once.

#include "common.h"
#include "qsrt_amd.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kB = 16;
constexpr int kWaves = 4;

// Target tile of a wave, each block with its own accumulator: kLRows row blocks by kLCols column blocks in the
// left product, kRRows by kRCols in the right one.
constexpr int kLRows = 8, kLCols = 1;
constexpr int kRRows = 2, kRCols = 4;

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

__device__ __forceinline__ f32x4 mfma4(float4 a, f32x4 b, f32x4 acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b[3], acc, 0, 0, 0);
    return acc;
}

// Left: wave w handles column blocks i0 .. i0 + kLCols - 1 (i0 = kLCols (w / chunks)) and rows
// o0 .. o0 + kLRows - 1 of the
// union of those columns' targets [max(0, first - i), min(ob, last - i)), every (row, column) a target of its
// own or skipped; a column's sources are the rows [max(0, first - i), min(ob, middle - i)), so a column takes
// part in the source steps inside its range only (a wave-uniform branch).  Each Lout block loaded serves kLCols
// columns and each error block kLRows rows.

__global__ __launch_bounds__(kWaves * 64) void bakron_left_kernel(const float* __restrict__ T,
                                                                   const float* __restrict__ Q,
                                                                   const float* __restrict__ Lout,
                                                                   float* __restrict__ I, int n_out, int n_in,
                                                                   int first, int middle, int last,
                                                                   int64_t lout_stride, int lower) {
    const int ob = n_out / kB, ib = n_in / kB;
    const int chunks = (min(ob, last - first + kLCols - 1) + kLRows - 1) / kLRows;
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    const int col_groups = (ib + kLCols - 1) / kLCols;
    if (slot >= static_cast<int64_t>(col_groups) * chunks) return;
    const int i0 = kLCols * static_cast<int>(slot / chunks), chunk = static_cast<int>(slot % chunks);
    const int i_last = min(ib, i0 + kLCols) - 1;
    // union of the columns' target rows and sources
    const int o_lo = max(0, first - i_last), o_hi = min(ob, last - i0);
    const int o0 = o_lo + kLRows * chunk;
    if (o0 >= o_hi) return;
    int sb[kLCols], se[kLCols];
    bool col_ok[kLCols];
    int s_lo = ob, s_hi = 0;
#pragma unroll
    for (int u = 0; u < kLCols; ++u) {
        const int i = i0 + u;
        col_ok[u] = i < ib;
        sb[u] = max(0, first - i);
        se[u] = col_ok[u] ? min(ob, middle - i) : 0;
        if (sb[u] < se[u]) {
            s_lo = min(s_lo, sb[u]);
            s_hi = max(s_hi, se[u]);
        }
    }
    // a block-lower Lout has Lout(o, s) = 0 for s > o: the tile's rows need no source past its last row
    if (lower) s_hi = min(s_hi, min(o0 + kLRows, o_hi));
    const int64_t mat = static_cast<int64_t>(n_out) * n_in;
    T += blockIdx.y * mat;
    Q += blockIdx.y * mat;
    I += blockIdx.y * mat;
    Lout += blockIdx.y * lout_stride;
    const int c = lane & 15, g = lane >> 4;
    // lane's A rows: Lout rows 16 o + c for the tile's row blocks (a block past o_hi repeats the last one and is
    // not stored), columns 16 s + 4 g ..; B: rows 16 s + 4 g + q of columns 16 i + c
    const float* a_row[kLRows];
#pragma unroll
    for (int t = 0; t < kLRows; ++t)
        a_row[t] = Lout + static_cast<int64_t>(kB * min(o0 + t, o_hi - 1) + c) * n_out + 4 * g;
    int64_t b_col[kLCols];
#pragma unroll
    for (int u = 0; u < kLCols; ++u) b_col[u] = static_cast<int64_t>(4 * g) * n_in + kB * min(i0 + u, ib - 1) + c;
    f32x4 acc[kLCols][kLRows];
#pragma unroll
    for (int u = 0; u < kLCols; ++u)
#pragma unroll
        for (int t = 0; t < kLRows; ++t) acc[u][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float4 a_nx[kLRows] = {};
    f32x4 b_nx[kLCols] = {};
    if (s_lo < s_hi) {
#pragma unroll
        for (int t = 0; t < kLRows; ++t) a_nx[t] = ld4(a_row[t] + kB * s_lo);
#pragma unroll
        for (int u = 0; u < kLCols; ++u) {
            const int64_t off = static_cast<int64_t>(kB * s_lo) * n_in + b_col[u];
#pragma unroll
            for (int q = 0; q < 4; ++q) b_nx[u][q] = Q[off + q * n_in] - T[off + q * n_in];
        }
    }
    for (int s = s_lo; s < s_hi; ++s) {
        float4 a[kLRows];
        f32x4 b[kLCols];
#pragma unroll
        for (int t = 0; t < kLRows; ++t) a[t] = a_nx[t];
#pragma unroll
        for (int u = 0; u < kLCols; ++u) b[u] = b_nx[u];
        if (s + 1 < s_hi) {
#pragma unroll
            for (int t = 0; t < kLRows; ++t) a_nx[t] = ld4(a_row[t] + kB * (s + 1));
#pragma unroll
            for (int u = 0; u < kLCols; ++u) {
                const int64_t off = static_cast<int64_t>(kB * (s + 1)) * n_in + b_col[u];
#pragma unroll
                for (int q = 0; q < 4; ++q) b_nx[u][q] = Q[off + q * n_in] - T[off + q * n_in];
            }
        }
#pragma unroll
        for (int u = 0; u < kLCols; ++u) {
            if (s < sb[u] || s >= se[u]) continue;  // uniform: the column's own source range
#pragma unroll
            for (int t = 0; t < kLRows; ++t) {
                if (lower && s > o0 + t) continue;  // uniform: a zero block of a block-lower Lout
                acc[u][t] = mfma4(a[t], b[u], acc[u][t]);
            }
        }
    }
    // acc[u][t][r] = I(o0 + t, i0 + u)[4 g + r][c]; every target of the tile is written, zero when its column
    // has no sources
#pragma unroll
    for (int u = 0; u < kLCols; ++u) {
        const int i = i0 + u;
        if (!col_ok[u]) continue;
        const int ob_lo = max(0, first - i), ob_hi = min(ob, last - i);
#pragma unroll
        for (int t = 0; t < kLRows; ++t) {
            const int o = o0 + t;
            if (o < ob_lo || o >= ob_hi) continue;
            float* out = I + static_cast<int64_t>(kB * o + 4 * g) * n_in + kB * i + c;
#pragma unroll
            for (int r = 0; r < 4; ++r) out[static_cast<int64_t>(r) * n_in] = acc[u][t][r];
        }
    }
}

// Right: wave w handles row blocks o0 .. o0 + kRRows - 1 (o0 = kRRows (w / chunks)) and columns
// c0 .. c0 + kRCols - 1 of the
// union of those rows' targets [max(0, middle - o), min(ib, last - o)), every (row, column) a target of its own
// or skipped; a row's sources are [max(0, first - o), min(ib, middle, last - o)), so a row takes part in the
// source steps inside its range only (a wave-uniform branch).  Each Lin block loaded serves kRRows rows and each
// I block kRCols columns.

__global__ __launch_bounds__(kWaves * 64) void bakron_right_kernel(float* __restrict__ T,
                                                                    const float* __restrict__ Lin,
                                                                    const float* __restrict__ I, int n_out,
                                                                    int n_in, int first, int middle, int last,
                                                                    int64_t lin_stride) {
    const int ob = n_out / kB, ib = n_in / kB;
    const int chunks = (min(ib, last - middle + kRRows - 1) + kRCols - 1) / kRCols;
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    const int row_groups = (ob + kRRows - 1) / kRRows;
    if (slot >= static_cast<int64_t>(row_groups) * chunks) return;
    const int o0 = kRRows * static_cast<int>(slot / chunks), chunk = static_cast<int>(slot % chunks);
    const int o_last = min(ob, o0 + kRRows) - 1;
    // union of the rows' target columns and sources
    const int c_lo = max(0, middle - o_last), c_hi = min(ib, last - o0);
    const int c0 = c_lo + kRCols * chunk;
    if (c0 >= c_hi) return;
    int sb[kRRows], se[kRRows];
    bool row_ok[kRRows];
    int s_lo = ib, s_hi = 0;
#pragma unroll
    for (int a = 0; a < kRRows; ++a) {
        const int o = o0 + a;
        row_ok[a] = o < ob;
        sb[a] = max(0, first - o);
        se[a] = row_ok[a] ? min(ib, min(middle, last - o)) : 0;
        if (sb[a] < se[a]) {
            s_lo = min(s_lo, sb[a]);
            s_hi = max(s_hi, se[a]);
        }
    }
    if (s_lo >= s_hi) return;
    const int64_t mat = static_cast<int64_t>(n_out) * n_in;
    T += blockIdx.y * mat;
    I += blockIdx.y * mat;
    Lin += blockIdx.y * lin_stride;
    const int c = lane & 15, g = lane >> 4;
    // lane's A rows: I rows 16 o + c; B rows: Lin rows 16 cb + c for the tile's column blocks cb (a block past
    // c_hi repeats the last one and is not stored); columns 16 s + 4 g ..
    const float* a_row[kRRows];
#pragma unroll
    for (int a = 0; a < kRRows; ++a) a_row[a] = I + static_cast<int64_t>(kB * min(o0 + a, ob - 1) + c) * n_in + 4 * g;
    const float* b_row[kRCols];
#pragma unroll
    for (int t = 0; t < kRCols; ++t)
        b_row[t] = Lin + static_cast<int64_t>(kB * min(c0 + t, c_hi - 1) + c) * n_in + 4 * g;
    f32x4 acc[kRRows][kRCols];
#pragma unroll
    for (int a = 0; a < kRRows; ++a)
#pragma unroll
        for (int t = 0; t < kRCols; ++t) acc[a][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float4 a_nx[kRRows], b_nx[kRCols];
#pragma unroll
    for (int a = 0; a < kRRows; ++a) a_nx[a] = ld4(a_row[a] + kB * s_lo);
#pragma unroll
    for (int t = 0; t < kRCols; ++t) b_nx[t] = ld4(b_row[t] + kB * s_lo);
    for (int s = s_lo; s < s_hi; ++s) {
        float4 av[kRRows], b[kRCols];
#pragma unroll
        for (int a = 0; a < kRRows; ++a) av[a] = a_nx[a];
#pragma unroll
        for (int t = 0; t < kRCols; ++t) b[t] = b_nx[t];
        if (s + 1 < s_hi) {
#pragma unroll
            for (int a = 0; a < kRRows; ++a) a_nx[a] = ld4(a_row[a] + kB * (s + 1));
#pragma unroll
            for (int t = 0; t < kRCols; ++t) b_nx[t] = ld4(b_row[t] + kB * (s + 1));
        }
#pragma unroll
        for (int a = 0; a < kRRows; ++a) {
            if (s < sb[a] || s >= se[a]) continue;  // uniform: the row's own source range
#pragma unroll
            for (int t = 0; t < kRCols; ++t) acc[a][t] = mfma4(av[a], f32x4{b[t].x, b[t].y, b[t].z, b[t].w}, acc[a][t]);
        }
    }
#pragma unroll
    for (int a = 0; a < kRRows; ++a) {
        const int o = o0 + a;
        if (!row_ok[a] || sb[a] >= se[a]) continue;
        const int ce = min(ib, last - o), cb = max(0, middle - o);
#pragma unroll
        for (int t = 0; t < kRCols; ++t) {
            const int col = c0 + t;
            if (col < cb || col >= ce) continue;
            float* out = T + static_cast<int64_t>(kB * o + 4 * g) * n_in + kB * col + c;
#pragma unroll
            for (int r = 0; r < 4; ++r) out[static_cast<int64_t>(r) * n_in] += acc[a][t][r];
        }
    }
}

}  // namespace

extern "C" {

static int band_update(float* workspace, const float* quantized, const float* output_factor,
                       const float* input_factor, float* intermediate, int64_t batch, int64_t n_out, int64_t n_in,
                       int64_t output_factor_batch_stride, int64_t input_factor_batch_stride, int64_t first_diagonal,
                       int64_t middle_diagonal, int64_t last_diagonal, void* stream_handle, int lower) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (!workspace || !quantized || !output_factor || !input_factor || !intermediate)
        return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (batch < 1 || batch > 65535) return qsrt::fail(qsrt::kBadArgument, "batch must be in 1..65535");
    if (n_out < kB || n_in < kB || n_out % kB || n_in % kB)
        return qsrt::fail(qsrt::kBadArgument, "BaKron dimensions must be positive multiples of 16");
    if (n_out > (1 << 20) || n_in > (1 << 20) || n_out * n_in > (int64_t(1) << 31))
        return qsrt::fail(qsrt::kBadArgument, "BaKron matrix too large for one launch");
    if ((output_factor_batch_stride != 0 && output_factor_batch_stride < n_out * n_out) ||
        (input_factor_batch_stride != 0 && input_factor_batch_stride < n_in * n_in) ||
        output_factor_batch_stride < 0 || input_factor_batch_stride < 0)
        return qsrt::fail(qsrt::kBadArgument, "factor batch stride must be 0 (shared) or at least n * n");
    const int64_t ob = n_out / kB, ib = n_in / kB, diagonals = ob + ib - 1;
    if (!(first_diagonal >= 0 && first_diagonal < middle_diagonal && middle_diagonal < last_diagonal &&
          last_diagonal <= diagonals))
        return qsrt::fail(qsrt::kBadArgument, "diagonals must satisfy 0 <= first < middle < last <= %lld",
                          static_cast<long long>(diagonals));
    const int64_t left_span_union = ob < last_diagonal - first_diagonal + kLCols - 1 ? ob
                                                                                 : last_diagonal - first_diagonal + kLCols - 1;
    const int64_t left_waves = ((ib + kLCols - 1) / kLCols) * ((left_span_union + kLRows - 1) / kLRows);
    const int64_t right_span_union = ib < last_diagonal - middle_diagonal + kRRows - 1 ? ib
                                                                                   : last_diagonal - middle_diagonal + kRRows - 1;
    const int64_t right_waves = ((ob + kRRows - 1) / kRRows) * ((right_span_union + kRCols - 1) / kRCols);
    const dim3 block(kWaves * 64);
    hipLaunchKernelGGL(bakron_left_kernel, dim3(static_cast<unsigned>((left_waves + kWaves - 1) / kWaves),
                                                static_cast<unsigned>(batch)),
                       block, 0, stream, workspace, quantized, output_factor, intermediate, static_cast<int>(n_out),
                       static_cast<int>(n_in), static_cast<int>(first_diagonal), static_cast<int>(middle_diagonal),
                       static_cast<int>(last_diagonal), output_factor_batch_stride, lower);
    QSRT_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(bakron_right_kernel, dim3(static_cast<unsigned>((right_waves + kWaves - 1) / kWaves),
                                                 static_cast<unsigned>(batch)),
                       block, 0, stream, workspace, input_factor, intermediate, static_cast<int>(n_out),
                       static_cast<int>(n_in), static_cast<int>(first_diagonal), static_cast<int>(middle_diagonal),
                       static_cast<int>(last_diagonal), input_factor_batch_stride);
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

int qsrt_bakron_band_update_f32(float* workspace, const float* quantized, const float* output_factor,
                                const float* input_factor, float* intermediate, int64_t batch, int64_t n_out,
                                int64_t n_in, int64_t output_factor_batch_stride, int64_t input_factor_batch_stride,
                                int64_t first_diagonal, int64_t middle_diagonal, int64_t last_diagonal,
                                void* stream_handle) {
    return band_update(workspace, quantized, output_factor, input_factor, intermediate, batch, n_out, n_in,
                       output_factor_batch_stride, input_factor_batch_stride, first_diagonal, middle_diagonal,
                       last_diagonal, stream_handle, 0);
}

int qsrt_bakron_band_update_lower_f32(float* workspace, const float* quantized, const float* output_factor,
                                      const float* input_factor, float* intermediate, int64_t batch, int64_t n_out,
                                      int64_t n_in, int64_t output_factor_batch_stride,
                                      int64_t input_factor_batch_stride, int64_t first_diagonal,
                                      int64_t middle_diagonal, int64_t last_diagonal, void* stream_handle) {
    return band_update(workspace, quantized, output_factor, input_factor, intermediate, batch, n_out, n_in,
                       output_factor_batch_stride, input_factor_batch_stride, first_diagonal, middle_diagonal,
                       last_diagonal, stream_handle, 1);
}

}  // extern "C"
