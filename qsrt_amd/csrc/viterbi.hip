// Tail-biting L16 tile Viterbi for CDNA4 (gfx950).
//
// Replaces the reference's tile quantizer kernels
// (qsrt/csrc/qsrt_quantize_tiles_kernel.cuh:26-500 and
// qsrt/csrc/qsrt_quantize_tiles_k2_kernel.cuh:47-366) with an FP32 design:
//
//   * one 256-weight tile per workgroup of 1024 threads (16 wave64s), one
//     workgroup per CU, persistent over a strided tile range;
//   * FP32 path metrics ping-pong in LDS (2 * 2^(16-K) floats: 128 KiB at
//     K2, 64 KiB at K3, 32 KiB at K4);
//   * each thread owns 64 trellis edges for the whole kernel: the 2^K
//     predecessors of a few states, whose E4M3 labels are widened to FP32
//     once and kept in VGPRs;
//   * 2^K states sharing one predecessor set are evaluated together, so
//     every LDS cost read serves 2^K edges;
//   * per state: d = label - x, c = fma(d, d, cost[pred]), value = min3
//     chain, decision = lowest k with c == value (lowest-index ties);
//   * decisions are packed (2 bits at K2, a nibble at K3/K4) into one
//     coalesced store per thread per step, in a per-workgroup HBM buffer;
//   * the boundary argmin is a wave64 shuffle reduction with lowest-index
//     ties; tracebacks run on one lane with agent-scope loads.
//
// Arithmetic contract (bit-exact with oracle/viterbi_ref.c): see that file.

#include "common.h"
#include "qsrt_amd.h"

namespace {

constexpr int kTile = 256;
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

template <int K>
struct Geo;

// K2: 16384 states, groups of 4 states with predecessors q + 4096 k.
// Thread t owns groups q = t + 1024 j (j < 4).
template <>
struct Geo<2> {
    static constexpr int S = 1 << 14, P = 4, NG = 4, NS = 4, kPredStride = 1 << 12;
    static constexpr int kRowBytes = kThreads * 4, kDecBits = 2;
    __device__ static int group(int t, int j) { return t + kThreads * j; }
    __device__ static int first_state(int t, int j) { return 4 * group(t, j); }
    // field f = 4 j + e sits at bits [2 (15 - f), +2)
    __device__ static int decision(const uint8_t* row, int s) {
        const int q = s >> 2;
        const uint32_t w = __hip_atomic_load(reinterpret_cast<const uint32_t*>(row) + (q & (kThreads - 1)),
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return (w >> (2 * (15 - (4 * (q >> 10) + (s & 3))))) & 3;
    }
};

// K3: 8192 states, groups of 8 states with predecessors q + 1024 k.
// Thread t owns group q = t; decisions are nibbles.
template <>
struct Geo<3> {
    static constexpr int S = 1 << 13, P = 8, NG = 1, NS = 8, kPredStride = 1 << 10;
    static constexpr int kRowBytes = kThreads * 4, kDecBits = 4;
    __device__ static int group(int t, int) { return t; }
    __device__ static int first_state(int t, int) { return 8 * t; }
    // state 8 t + e sits at bits [4 (7 - e), +4)
    __device__ static int decision(const uint8_t* row, int s) {
        const uint32_t w = __hip_atomic_load(reinterpret_cast<const uint32_t*>(row) + (s >> 3),
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return (w >> (4 * (7 - (s & 7)))) & 7;
    }
};

// K4: 4096 states, groups of 16 states with predecessors q + 256 k.
// Thread t owns states 4t .. 4t+3 (group q = t >> 2); 16 decision bits.
template <>
struct Geo<4> {
    static constexpr int S = 1 << 12, P = 16, NG = 1, NS = 4, kPredStride = 1 << 8;
    static constexpr int kRowBytes = kThreads * 2, kDecBits = 4;
    __device__ static int group(int t, int) { return t >> 2; }
    __device__ static int first_state(int t, int) { return 4 * t; }
    // thread t's 16-bit field holds state 4 t + e at bits [4 (3 - e), +4);
    // little-endian: even threads in the low half of each dword.
    __device__ static int decision(const uint8_t* row, int s) {
        const uint32_t w = __hip_atomic_load(reinterpret_cast<const uint32_t*>(row) + (s >> 3),
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return (w >> (16 * ((s >> 2) & 1) + 4 * (3 - (s & 3)))) & 15;
    }
};

template <int K>
struct Labels {
    float v[Geo<K>::NG][Geo<K>::NS][Geo<K>::P];
};

__device__ __forceinline__ float fmin2(float a, float b) { return __builtin_fminf(a, b); }

// One trellis step over all states.  FIRST: no predecessor costs (the
// reference's step 0); CONSTRAINED: only predecessor `pre_state` is
// admissible at step 0; RECORD: pack and store decisions for this row.
template <int K, bool FIRST, bool CONSTRAINED, bool RECORD>
__device__ __forceinline__ void trellis_step(const Labels<K>& lab, const float* __restrict__ prev,
                                             float* __restrict__ next, float x, int pre_state,
                                             uint8_t* __restrict__ dec_row, int t, uint32_t dec_bits) {
    using G = Geo<K>;
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < G::NG; ++j) {
        const int q = G::group(t, j);
        float p[G::P];
        if constexpr (!FIRST) {
#pragma unroll
            for (int k = 0; k < G::P; ++k) p[k] = prev[q + k * G::kPredStride];
        }
        float best[G::NS];
#pragma unroll
        for (int e = 0; e < G::NS; ++e) {
            float c[G::P];
#pragma unroll
            for (int k = 0; k < G::P; ++k) {
                const float d = lab.v[j][e][k] - x;
                if constexpr (FIRST) {
                    c[k] = __builtin_fmaf(d, d, 0.0f);
                    if constexpr (CONSTRAINED) {
                        if (q + k * G::kPredStride != pre_state) c[k] = __builtin_inff();
                    }
                } else {
                    c[k] = __builtin_fmaf(d, d, p[k]);
                }
            }
            float m = c[0];
#pragma unroll
            for (int k = 1; k < G::P; ++k) m = fmin2(m, c[k]);
            best[e] = m;
            if constexpr (RECORD) {
                int arg = G::P - 1;
#pragma unroll
                for (int k = G::P - 2; k >= 0; --k) arg = (c[k] == m) ? k : arg;
                word = (word << dec_bits) | static_cast<uint32_t>(arg);
            }
        }
        float* dst = next + G::first_state(t, j);
#pragma unroll
        for (int e = 0; e < G::NS; e += 4)
            *reinterpret_cast<float4*>(dst + e) = make_float4(best[e], best[e + 1], best[e + 2], best[e + 3]);
    }
    if constexpr (RECORD) {
        if constexpr (K == 4)
            reinterpret_cast<uint16_t*>(dec_row)[t] = static_cast<uint16_t>(word);
        else
            reinterpret_cast<uint32_t*>(dec_row)[t] = word;
    }
}

// Lowest-index argmin of `cost` over all states; result valid in thread 0.
template <int K>
__device__ int boundary_argmin(const float* cost, float* red_v, int* red_i, int t) {
    using G = Geo<K>;
    float bv = __builtin_inff();
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < G::NG; ++j) {
#pragma unroll
        for (int e = 0; e < G::NS; ++e) {
            const int s = G::first_state(t, j) + e;
            const float v = cost[s];
            if (v < bv || (v == bv && s < bi)) { bv = v; bi = s; }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (ov < bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if ((t & 63) == 0) { red_v[t >> 6] = bv; red_i[t >> 6] = bi; }
    __syncthreads();
    if (t == 0) {
        bv = red_v[0]; bi = red_i[0];
        for (int w = 1; w < kWaves; ++w)
            if (red_v[w] < bv || (red_v[w] == bv && red_i[w] < bi)) { bv = red_v[w]; bi = red_i[w]; }
    }
    return bi;
}

// Single-lane traceback over `steps` rows ending at `edge` (the state after
// the last step).  With `out_states` null it stops after position 0 and
// returns the state before it; otherwise it emits codewords and labels.
template <int K>
__device__ int traceback(const uint8_t* dec, int roll, int steps, int edge, uint16_t* out_states,
                         float* out_recon, const uint8_t* __restrict__ lut) {
    using G = Geo<K>;
    for (int i = steps - 1; i >= 0; --i) {
        const int pos = (i + roll) & (kTile - 1);
        const int k = G::decision(dec + static_cast<size_t>(pos) * G::kRowBytes, edge);
        const int prev = (k << (16 - 2 * K)) | (edge >> K);
        if (out_states) {
            const int word = (prev << K) | edge;
            out_states[pos] = static_cast<uint16_t>(word);
            out_recon[pos] = qsrt::e4m3_to_float(lut[word]);
        } else if (pos == 0) {
            return prev;
        }
        edge = prev;
    }
    return edge;
}

template <int K>
__device__ __forceinline__ void forward_pass(const Labels<K>& lab, const float* sx, float*& prev, float*& next, int roll,
                             int steps, int pre_state, int trace_start, uint8_t* dec, int t,
                                             uint32_t dec_bits) {
    using G = Geo<K>;
    {
        const int pos = roll & (kTile - 1);
        uint8_t* row = dec + static_cast<size_t>(pos) * G::kRowBytes;
        if (pre_state >= 0)
            trellis_step<K, true, true, true>(lab, prev, next, sx[pos], pre_state, row, t, dec_bits);
        else if (trace_start == 0)
            trellis_step<K, true, false, true>(lab, prev, next, sx[pos], -1, row, t, dec_bits);
        else
            trellis_step<K, true, false, false>(lab, prev, next, sx[pos], -1, row, t, dec_bits);
        __syncthreads();
        float* tmp = prev; prev = next; next = tmp;
    }
    for (int i = 1; i < steps; ++i) {
        const int pos = (i + roll) & (kTile - 1);
        uint8_t* row = dec + static_cast<size_t>(pos) * G::kRowBytes;
        if (i >= trace_start)
            trellis_step<K, false, false, true>(lab, prev, next, sx[pos], -1, row, t, dec_bits);
        else
            trellis_step<K, false, false, false>(lab, prev, next, sx[pos], -1, row, t, dec_bits);
        __syncthreads();
        float* tmp = prev; prev = next; next = tmp;
    }
}

template <int K>
__global__ __launch_bounds__(kThreads, 1) void viterbi_tiles_kernel(
    const float* __restrict__ tiles, float* __restrict__ recon, uint16_t* __restrict__ states,
    int64_t n_tiles, int context, const uint8_t* __restrict__ lut, int boundary_lag,
    uint8_t* __restrict__ dec_ws, uint32_t dec_bits) {
    // dec_bits == Geo<K>::kDecBits, passed at run time on purpose: with a
    // compile-time shift the compiler folds the shifts into the argmin
    // selects and materialises ~30 pre-shifted constants in VGPRs.
    using G = Geo<K>;
    __shared__ __align__(16) float cost_a[G::S];
    __shared__ __align__(16) float cost_b[G::S];
    __shared__ float sx[kTile];
    __shared__ float red_v[kWaves];
    __shared__ int red_i[kWaves];
    __shared__ int bcast;

    const int t = threadIdx.x;
    uint8_t* dec = dec_ws + static_cast<size_t>(blockIdx.x) * kTile * G::kRowBytes;

    Labels<K> lab;
#pragma unroll
    for (int j = 0; j < G::NG; ++j)
#pragma unroll
        for (int e = 0; e < G::NS; ++e)
#pragma unroll
            for (int k = 0; k < G::P; ++k)
                lab.v[j][e][k] = qsrt::e4m3_to_float(lut[(k << (16 - K)) | (G::first_state(t, j) + e)]);

    for (int64_t tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        if (t < kTile) sx[t] = tiles[tile * kTile + t];
        __syncthreads();

        float* prev = cost_a;
        float* next = cost_b;
        // Primer over positions 256-C .. 255, 0 .. C-1; decisions kept for 0 .. C-1.
        forward_pass<K>(lab, sx, prev, next, kTile - context, 2 * context, -1, context, dec, t, dec_bits);
        __threadfence();
        const int start = boundary_argmin<K>(boundary_lag ? next : prev, red_v, red_i, t);
        if (t == 0) bcast = traceback<K>(dec, kTile - context, 2 * context, start, nullptr, nullptr, lut);
        __syncthreads();
        const int end_state = bcast;

        // Constrained pass from end_state, then the emitting traceback.
        prev = cost_a;
        next = cost_b;
        forward_pass<K>(lab, sx, prev, next, 0, kTile, end_state, 0, dec, t, dec_bits);
        __threadfence();
        __syncthreads();
        if (t == 0)
            traceback<K>(dec, 0, kTile, end_state, states + tile * kTile, recon + tile * kTile, lut);
        __syncthreads();
    }
}

template <int K>
size_t row_bytes() { return static_cast<size_t>(Geo<K>::kRowBytes); }

size_t workgroup_dec_bytes(int K) {
    switch (K) {
        case 2: return kTile * row_bytes<2>();
        case 3: return kTile * row_bytes<3>();
        case 4: return kTile * row_bytes<4>();
        default: return 0;
    }
}

int launch_workgroups(int64_t n_tiles, int cu_count) {
    const int64_t g = n_tiles < cu_count ? n_tiles : cu_count;
    return static_cast<int>(g);
}

}  // namespace

extern "C" {

size_t qsrt_viterbi_workspace_bytes(int K, int64_t n_tiles) {
    int cus = 0;
    if (qsrt::current_cu_count(&cus) != 0 || n_tiles <= 0) return 0;
    return workgroup_dec_bytes(K) * static_cast<size_t>(launch_workgroups(n_tiles, cus));
}

int qsrt_viterbi_tiles(const float* tiles, float* recon, uint16_t* states, int64_t n_tiles, int K,
                       int tailbite_context, const uint8_t* lut_e4m3, int boundary_lag, void* workspace,
                       size_t workspace_bytes, void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (K < 2 || K > 4)
        return qsrt::fail(qsrt::kBadArgument, "K%d is not supported by the MI355X tile kernel (K2..K4)", K);
    if (tailbite_context < 1 || tailbite_context > 128)
        return qsrt::fail(qsrt::kBadArgument, "tailbite_context must be in 1..128");
    if (boundary_lag != 0 && boundary_lag != 1)
        return qsrt::fail(qsrt::kBadArgument, "boundary_lag must be 0 or 1");
    if (n_tiles < 0) return qsrt::fail(qsrt::kBadArgument, "n_tiles must be non-negative");
    if (n_tiles == 0) return qsrt::kOk;
    if (!tiles || !recon || !states || !lut_e4m3 || !workspace)
        return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    int cus = 0;
    if (int rc = qsrt::current_cu_count(&cus)) return rc;
    const int grid = launch_workgroups(n_tiles, cus);
    const size_t need = workgroup_dec_bytes(K) * static_cast<size_t>(grid);
    if (workspace_bytes < need)
        return qsrt::fail(qsrt::kWorkspaceTooSmall, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
    auto* ws = static_cast<uint8_t*>(workspace);
    switch (K) {
        case 2:
            hipLaunchKernelGGL(viterbi_tiles_kernel<2>, dim3(grid), dim3(kThreads), 0, stream, tiles, recon, states,
                               n_tiles, tailbite_context, lut_e4m3, boundary_lag, ws, static_cast<uint32_t>(Geo<2>::kDecBits));
            break;
        case 3:
            hipLaunchKernelGGL(viterbi_tiles_kernel<3>, dim3(grid), dim3(kThreads), 0, stream, tiles, recon, states,
                               n_tiles, tailbite_context, lut_e4m3, boundary_lag, ws, static_cast<uint32_t>(Geo<3>::kDecBits));
            break;
        default:
            hipLaunchKernelGGL(viterbi_tiles_kernel<4>, dim3(grid), dim3(kThreads), 0, stream, tiles, recon, states,
                               n_tiles, tailbite_context, lut_e4m3, boundary_lag, ws, static_cast<uint32_t>(Geo<4>::kDecBits));
            break;
    }
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

}  // extern "C"
