// Blockwise normalised Sylvester-Hadamard rotation of an FP32 or float64 matrix, in place.
//
// side 0 ("left", reference preapply_had_l / blockwise_preapply_had_l_,
// qsrt/exl3_encoder_backend.py:275-320): every group of `block` consecutive
// rows is replaced by H_block @ rows.  side 1 ("right", preapply_had_r):
// every group of `block` consecutive columns by cols @ H_block.
// H_block[i][j] = (-1)^popcount(i & j) / sqrt(block), the matrix of
// exl3_reference.py:210-227 and of the butterfly in qsrt_coupled.py:49-83.
//
// Optional vectors indexed along the transformed axis fuse the sign and
// scale multiplies that surround every rotation in the encoder:
//   y = post_mul[a] * H(x * pre_mul[a] / pre_div[a])
// (signed_block_hadamard, qsrt_coupled.py:108-126; the `W /= sv`, `W /= su`
// of regularize; the `H *= su` congruence; the `* su`, `* sv` of decode).
//
// Design: one 256-thread workgroup per 8192-element tile (block x 8192/block
// of the two axes; 16384 for block 512 along rows).  The tile is read with coalesced float4 loads into LDS,
// transformed in two in-register rounds (bits 0..4 of the transformed
// index, then the remaining bits), each thread owning one 32- or
// 2^(log2(block)-5)-point line per round, and written back with float4
// stores.  The kernel is HBM-bound: 8 bytes per element per call.

#include <cmath>

#include "common.h"
#include "qsrt_amd.h"

namespace {

constexpr int kThreads = 256;

// Elements per tile: B x (elements / B).  FP32 block 512 along rows gets twice the usual 8192 so that each row
// segment it reads and writes is 128 bytes (32 floats) rather than 64; float64 tiles stay at 8192 elements
// (64 KiB of LDS).
template <typename T, int NB, bool LEFT>
constexpr int tile_elems() {
    return (sizeof(T) == 4 && LEFT && NB == 9) ? 16384 : 8192;
}

// Four consecutive elements: one 16-byte access for FP32, two for float64.
__device__ __forceinline__ void load4(const float* p, float (&e)[4]) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    e[0] = v.x, e[1] = v.y, e[2] = v.z, e[3] = v.w;
}
__device__ __forceinline__ void load4(const double* p, double (&e)[4]) {
    const double2 u = *reinterpret_cast<const double2*>(p), v = *reinterpret_cast<const double2*>(p + 2);
    e[0] = u.x, e[1] = u.y, e[2] = v.x, e[3] = v.y;
}
__device__ __forceinline__ void store4(float* p, const float (&e)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(e[0], e[1], e[2], e[3]);
}
__device__ __forceinline__ void store4(double* p, const double (&e)[4]) {
    *reinterpret_cast<double2*>(p) = make_double2(e[0], e[1]);
    *reinterpret_cast<double2*>(p + 2) = make_double2(e[2], e[3]);
}

template <typename T, int NB>
__device__ __forceinline__ void fwht(T (&v)[1 << NB]) {
#pragma unroll
    for (int h = 1; h < (1 << NB); h <<= 1) {
#pragma unroll
        for (int i = 0; i < (1 << NB); ++i) {
            if (i & h) continue;
            const T a = v[i], b = v[i + h];
            v[i] = a + b;
            v[i + h] = a - b;
        }
    }
}

// One round over bits [LO, LO + NBITS) of the transformed index a, for every
// line (other-axis index b, remaining bits of a) of the tile.
template <typename T, int NB, int LO, int NBITS, int S, int O>
__device__ __forceinline__ void lds_round(T* lds, int t) {
    constexpr int V = 1 << NBITS;
    constexpr int kLines = (O << NB) / V;  // tile elements / V
    static_assert(kLines % kThreads == 0, "line count must fill the workgroup");
#pragma unroll
    for (int k = 0; k < kLines / kThreads; ++k) {
        const int line = t + kThreads * k;
        const int b = line % O;
        const int h = line / O;
        const int base = (h & ((1 << LO) - 1)) | ((h >> LO) << (LO + NBITS));
        T v[V];
#pragma unroll
        for (int j = 0; j < V; ++j) v[j] = lds[(base | (j << LO)) * S + b];
        fwht<T, NBITS>(v);
#pragma unroll
        for (int j = 0; j < V; ++j) lds[(base | (j << LO)) * S + b] = v[j];
    }
}

template <typename T, int NB, bool LEFT>
__global__ __launch_bounds__(kThreads) void hadamard_kernel(T* __restrict__ x, int64_t rows, int64_t cols,
                                                            int64_t ld, int64_t tiles_b,
                                                            const T* __restrict__ pre_mul,
                                                            const T* __restrict__ pre_div,
                                                            const T* __restrict__ post_mul, T norm) {
    constexpr int kTileElems = tile_elems<T, NB, LEFT>();
    constexpr int B = 1 << NB;        // transformed extent of one tile
    constexpr int O = kTileElems / B;  // other-axis extent of one tile
    constexpr int S = O + 1;           // LDS stride per transformed index (odd: spreads banks)
    __shared__ T lds[B * S];

    const int t = threadIdx.x;
    const int64_t tile = blockIdx.x;
    const int64_t a0 = (tile / tiles_b) * B;
    const int64_t b0 = (tile % tiles_b) * O;
    const int64_t ext_b = LEFT ? cols : rows;

    // Column rotations: a thread's four transformed indices a0 + 4 aq + i are
    // the same in every load and store iteration (kThreads is a multiple of
    // B / 4), so its multipliers are read once.
    constexpr int AQ = B / 4;
    static_assert(kThreads % AQ == 0, "column tiles need fixed transformed indices per thread");
    T col_pre[4] = {1, 1, 1, 1}, col_div[4] = {1, 1, 1, 1};
    T col_post[4] = {norm, norm, norm, norm};
    if constexpr (!LEFT) {
        const int64_t a = a0 + 4 * (t % AQ);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (pre_mul) col_pre[i] = pre_mul[a + i];
            if (pre_div) col_div[i] = pre_div[a + i];
            if (post_mul) col_post[i] = norm * post_mul[a + i];
        }
    }

    // ---- load (16 or 32 bytes along the contiguous axis), pre-scale, into LDS[a][b]
#pragma unroll
    for (int k = 0; k < kTileElems / 4 / kThreads; ++k) {
        const int f = t + kThreads * k;
        if constexpr (LEFT) {
            const int a = f / (O / 4), bq = f % (O / 4);
            const int64_t col = b0 + 4 * bq;
            T e[4] = {0, 0, 0, 0};
            if (col < ext_b) load4(x + (a0 + a) * ld + col, e);
            const T m = pre_mul ? pre_mul[a0 + a] : T(1);
            const T dv = pre_div ? pre_div[a0 + a] : T(1);
            T* d = lds + a * S + 4 * bq;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (pre_mul) e[i] *= m;
                if (pre_div) e[i] /= dv;
                d[i] = e[i];
            }
        } else {
            const int b = f / AQ, aq = f % AQ;
            const int64_t row = b0 + b;
            T e[4] = {0, 0, 0, 0};
            if (row < ext_b) load4(x + row * ld + a0 + 4 * aq, e);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (pre_mul) e[i] *= col_pre[i];
                if (pre_div) e[i] /= col_div[i];
                lds[(4 * aq + i) * S + b] = e[i];
            }
        }
    }
    __syncthreads();
    lds_round<T, NB, 0, 5, S, O>(lds, t);
    __syncthreads();
    lds_round<T, NB, 5, NB - 5, S, O>(lds, t);
    __syncthreads();

    // ---- store: normalise, post-scale, 16 or 32 bytes along the contiguous axis
#pragma unroll
    for (int k = 0; k < kTileElems / 4 / kThreads; ++k) {
        const int f = t + kThreads * k;
        if constexpr (LEFT) {
            const int a = f / (O / 4), bq = f % (O / 4);
            const int64_t col = b0 + 4 * bq;
            if (col >= ext_b) continue;
            T s = norm;
            if (post_mul) s *= post_mul[a0 + a];
            const T* d = lds + a * S + 4 * bq;
            const T e[4] = {d[0] * s, d[1] * s, d[2] * s, d[3] * s};
            store4(x + (a0 + a) * ld + col, e);
        } else {
            const int b = f / AQ, aq = f % AQ;
            const int64_t row = b0 + b;
            if (row >= ext_b) continue;
            T e[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) e[i] = lds[(4 * aq + i) * S + b] * col_post[i];
            store4(x + row * ld + a0 + 4 * aq, e);
        }
    }
}

template <typename T, int NB>
int launch(T* x, int64_t rows, int64_t cols, int64_t ld, int side, const T* pre_mul, const T* pre_div,
           const T* post_mul, hipStream_t stream) {
    constexpr int B = 1 << NB;
    const int O = (side == 0 ? tile_elems<T, NB, true>() : tile_elems<T, NB, false>()) / B;
    const int64_t ext_a = side == 0 ? rows : cols;
    const int64_t ext_b = side == 0 ? cols : rows;
    const int64_t tiles_b = (ext_b + O - 1) / O;
    const int64_t tiles = (ext_a / B) * tiles_b;
    if (tiles > 0x7fffffff) return qsrt::fail(qsrt::kBadArgument, "matrix too large for one launch");
    const T norm = T(1) / std::sqrt(static_cast<T>(B));
    if (side == 0)
        hipLaunchKernelGGL((hadamard_kernel<T, NB, true>), dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0,
                           stream, x, rows, cols, ld, tiles_b, pre_mul, pre_div, post_mul, norm);
    else
        hipLaunchKernelGGL((hadamard_kernel<T, NB, false>), dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0,
                           stream, x, rows, cols, ld, tiles_b, pre_mul, pre_div, post_mul, norm);
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

template <typename T>
int rotate(T* x, int64_t rows, int64_t cols, int64_t ld, int block, int side, const T* pre_mul, const T* pre_div,
           const T* post_mul, void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (side != 0 && side != 1) return qsrt::fail(qsrt::kBadArgument, "side must be 0 (rows) or 1 (columns)");
    if (rows < 0 || cols < 0) return qsrt::fail(qsrt::kBadArgument, "negative matrix extent");
    if (rows == 0 || cols == 0) return qsrt::kOk;
    if (!x) return qsrt::fail(qsrt::kBadArgument, "null matrix pointer");
    if (ld < cols) return qsrt::fail(qsrt::kBadArgument, "leading dimension %lld < columns %lld", (long long)ld,
                                     (long long)cols);
    if (ld % 4 || cols % 4 || reinterpret_cast<uintptr_t>(x) % 16)
        return qsrt::fail(qsrt::kBadArgument, "matrix must be 16-byte aligned with columns and ld multiples of 4");
    const int64_t ext_a = side == 0 ? rows : cols;
    if (ext_a % block)
        return qsrt::fail(qsrt::kBadArgument, "Hadamard axis (%lld) must be divisible by block %d", (long long)ext_a,
                          block);
    switch (block) {
        case 64: return launch<T, 6>(x, rows, cols, ld, side, pre_mul, pre_div, post_mul, stream);
        case 128: return launch<T, 7>(x, rows, cols, ld, side, pre_mul, pre_div, post_mul, stream);
        case 256: return launch<T, 8>(x, rows, cols, ld, side, pre_mul, pre_div, post_mul, stream);
        case 512: return launch<T, 9>(x, rows, cols, ld, side, pre_mul, pre_div, post_mul, stream);
        default: return qsrt::fail(qsrt::kBadArgument, "Hadamard block %d not supported (64, 128, 256, 512)", block);
    }
}

}  // namespace

extern "C" {

int qsrt_hadamard(float* x, int64_t rows, int64_t cols, int64_t ld, int block, int side, const float* pre_mul,
                  const float* pre_div, const float* post_mul, void* stream_handle) {
    return rotate<float>(x, rows, cols, ld, block, side, pre_mul, pre_div, post_mul, stream_handle);
}

int qsrt_hadamard_f64(double* x, int64_t rows, int64_t cols, int64_t ld, int block, int side, const double* pre_mul,
                      const double* pre_div, const double* post_mul, void* stream_handle) {
    return rotate<double>(x, rows, cols, ld, block, side, pre_mul, pre_div, post_mul, stream_handle);
}

}  // extern "C"
