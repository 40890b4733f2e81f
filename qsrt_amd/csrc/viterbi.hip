// Tail-biting L16 tile Viterbi for CDNA4 (gfx950).
//
// Replaces the reference's tile quantizer kernels
// (qsrt/csrc/qsrt_quantize_tiles_kernel.cuh:26-500 and
// qsrt/csrc/qsrt_quantize_tiles_k2_kernel.cuh:47-366) with an FP32 design:
//
//   * one 256-weight tile per workgroup of 1024 threads (16 wave64s), one
//     workgroup per CU, persistent over a strided tile range;
//   * FP32 path metrics ping-pong in LDS (2 * 2^(16-K) floats: 128 KiB at
//     K2, 64 KiB at K3, 32 KiB at K4, down to 8 KiB at K6); K1's 2^15
//     states use one 128 KiB array updated in place;
//   * each thread owns 64 trellis edges for the whole kernel: the 2^K
//     predecessors of a few states, whose E4M3 labels are widened to FP32
//     once and kept in VGPRs;
//   * 2^K states sharing one predecessor set are evaluated together, so
//     every LDS cost read serves 2^K edges;
//   * per state: d = label - x, c = fma(d, d, cost[pred]), value = min3
//     chain, decision = lowest k with c == value (lowest-index ties), read
//     off a tournament over the minimum's own tree on the recorded steps
//     (K2..K4; K1 uses wave ballots);
//   * K5 / K6 (32 / 64 predecessors per state) stream the predecessors
//     through a running minimum instead of holding them in registers;
//   * decisions are packed (K bits per state, 1..32 bits per thread) into
//     one coalesced store per thread per step, in a per-workgroup HBM buffer;
//   * the boundary argmin is a wave64 shuffle reduction with lowest-index
//     ties;
//   * passes are pipelined over two tiles per workgroup (P0, P1, F0, P2,
//     F1, ...): each traceback runs on one lane, one position per step of
//     the next pass, its dependent decision loads hidden behind the step;
//     a traceback with nothing to hide behind runs speculatively on wave 0.
//
// Arithmetic contract (bit-exact with oracle/viterbi_ref.c): see that file.

#include <cmath>

#include "common.h"
#include "qsrt_amd.h"

namespace {

constexpr int kTile = 256;
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

template <int K>
struct Geo;

// K1: 32768 states, groups of 2 states with predecessors q + 16384 k.
// Thread t owns groups q = t + 1024 j (j < 16); 32 one-bit decisions.  Two
// FP32 cost arrays would need 256 KiB of LDS, so K1 updates one array in
// place (every predecessor cost is read into registers before a barrier,
// then the new costs are written).
template <>
struct Geo<1> {
    static constexpr int S = 1 << 15, P = 2, NG = 16, NS = 2, kPredStride = 1 << 14;
    static constexpr int kRowBytes = kThreads * 4;
    __device__ static int group(int t, int j) { return t + kThreads * j; }
    __device__ static int first_state(int t, int j) { return 2 * group(t, j); }
    // field f = 2 j + e sits at bit 31 - f
    __device__ static int word_index(int s) { return (s >> 1) & (kThreads - 1); }
    __device__ static int extract(uint32_t w, int s) { return (w >> (31 - (2 * (s >> 11) + (s & 1)))) & 1; }
};

// K2: 16384 states, groups of 4 states with predecessors q + 4096 k.
// Thread t owns groups q = t + 1024 j (j < 4).
template <>
struct Geo<2> {
    static constexpr int S = 1 << 14, P = 4, NG = 4, NS = 4, kPredStride = 1 << 12;
    static constexpr int kRowBytes = kThreads * 4;
    __device__ static int group(int t, int j) { return t + kThreads * j; }
    __device__ static int first_state(int t, int j) { return 4 * group(t, j); }
    // field f = 4 j + e sits at bits [2 (15 - f), +2)
    __device__ static int word_index(int s) { return (s >> 2) & (kThreads - 1); }
    __device__ static int extract(uint32_t w, int s) { return (w >> (2 * (15 - (4 * (s >> 12) + (s & 3))))) & 3; }
};

// K3: 8192 states, groups of 8 states with predecessors q + 1024 k.
// Thread t owns group q = t; 3-bit decisions, 24 bits used per dword.
template <>
struct Geo<3> {
    static constexpr int S = 1 << 13, P = 8, NG = 1, NS = 8, kPredStride = 1 << 10;
    static constexpr int kRowBytes = kThreads * 4;
    __device__ static int group(int t, int) { return t; }
    __device__ static int first_state(int t, int) { return 8 * t; }
    // state 8 t + e sits at bits [3 (7 - e), +3)
    __device__ static int word_index(int s) { return s >> 3; }
    __device__ static int extract(uint32_t w, int s) { return (w >> (3 * (7 - (s & 7)))) & 7; }
};

// K4: 4096 states, groups of 16 states with predecessors q + 256 k.
// Thread t owns states 4t .. 4t+3 (group q = t >> 2); 16 decision bits.
template <>
struct Geo<4> {
    static constexpr int S = 1 << 12, P = 16, NG = 1, NS = 4, kPredStride = 1 << 8;
    static constexpr int kRowBytes = kThreads * 2;
    __device__ static int group(int t, int) { return t >> 2; }
    __device__ static int first_state(int t, int) { return 4 * t; }
    // thread t's 16-bit field holds state 4 t + e at bits [4 (3 - e), +4);
    // little-endian: even threads in the low half of each dword.
    __device__ static int word_index(int s) { return s >> 3; }
    __device__ static int extract(uint32_t w, int s) { return (w >> (16 * ((s >> 2) & 1) + 4 * (3 - (s & 3)))) & 15; }
};

// K5: 2048 states, groups of 32 states with predecessors q + 64 k.
// Thread t owns states 2t, 2t+1 (group q = t >> 4); 10 decision bits in a
// 16-bit field, state 2 t + e at bits [5 (1 - e), +5).
template <>
struct Geo<5> {
    static constexpr int S = 1 << 11, P = 32, NG = 1, NS = 2, kPredStride = 1 << 6;
    static constexpr int kRowBytes = kThreads * 2;
    __device__ static int group(int t, int) { return t >> 4; }
    __device__ static int first_state(int t, int) { return 2 * t; }
    __device__ static int word_index(int s) { return s >> 2; }
    __device__ static int extract(uint32_t w, int s) { return (w >> (16 * ((s >> 1) & 1) + 5 * (1 - (s & 1)))) & 31; }
};

// K6: 1024 states, groups of 64 states with predecessors q + 16 k.
// Thread t owns state t (group q = t >> 6, uniform over a wave); one byte
// per thread holds its 6-bit decision.
template <>
struct Geo<6> {
    static constexpr int S = 1 << 10, P = 64, NG = 1, NS = 1, kPredStride = 1 << 4;
    static constexpr int kRowBytes = kThreads;
    __device__ static int group(int t, int) { return t >> 6; }
    __device__ static int first_state(int t, int) { return t; }
    __device__ static int word_index(int s) { return s >> 2; }
    __device__ static int extract(uint32_t w, int s) { return (w >> (8 * (s & 3))) & 63; }
};

// Cost arrays in LDS: ping-pong pairs, except K1 (in place).
template <int K>
constexpr int kCostArrays = K == 1 ? 1 : 2;

// Decision word holding state s at tile position `pos` (workgroup-scope:
// the writers are this workgroup's other waves, fenced before a barrier).
template <int K>
__device__ __forceinline__ uint32_t load_decisions(const uint8_t* dec, int pos, int s) {
    const uint32_t* row = reinterpret_cast<const uint32_t*>(dec + static_cast<size_t>(pos) * Geo<K>::kRowBytes);
    return __hip_atomic_load(row + Geo<K>::word_index(s), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <int K>
struct Labels {
    float v[Geo<K>::NG][Geo<K>::NS][Geo<K>::P];
};

// K1 keeps its labels as fp16 pairs (E4M3 values are exact in fp16): its 32
// predecessor costs must sit in registers across the in-place barrier too.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <>
struct Labels<1> {
    f16x2 v[Geo<1>::NG][Geo<1>::NS];
};

__device__ __forceinline__ float fmin2(float a, float b) { return __builtin_fminf(a, b); }

// word = 2 * word + (lane's bit of `mask`): one v_addc_co_u32 with the lane
// mask as carry-in, instead of select-then-shift-or.
__device__ __forceinline__ uint32_t push_bit(uint32_t word, uint64_t mask) {
    uint32_t out;
    uint64_t carry_out;
    asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(out), "=s"(carry_out) : "v"(word), "s"(mask));
    return out;
}

// Pack the lowest-index argmin of c[0..P) (value m) into `word`, K bits, MSB
// first.  The P-1 equality tests are wave ballots (SGPR lane masks); the
// prefix masks ge[k] = "argmin >= k" and the bit masks are scalar-unit
// algebra, leaving K VALU ops for the insertion.
template <int K>
__device__ __forceinline__ uint32_t push_argmin(uint32_t word, const float (&c)[1 << K], float m) {
    constexpr int P = 1 << K;
    uint64_t ge[P + 1];
    ge[0] = ~0ull;
#pragma unroll
    for (int k = 0; k < P - 1; ++k) ge[k + 1] = ge[k] & ~__builtin_amdgcn_ballot_w64(c[k] == m);
    ge[P] = 0;
#pragma unroll
    for (int b = K - 1; b >= 0; --b) {
        uint64_t bit = 0;
#pragma unroll
        for (int lo = 1 << b; lo < P; lo += 2 << b) bit |= ge[lo] & ~ge[lo + (1 << b)];
        word = push_bit(word, bit);
    }
    return word;
}

// Minimum of c[0..P) and its lowest index pushed into `word` (K bits, MSB
// first) as a tournament whose levels are read off the minimum's own tree:
// bit K-1 says whether the lower half's minimum misses the overall one, the
// next bit the same of the first quarter of the chosen half, and so on down to
// the chosen pair's first element.  The minimum is exact whatever the order,
// so it equals the plain min3 chain; "equal to the minimum" at each level
// keeps the lowest index, so the bits equal a lowest-index scan.  At K3/K4
// the root is a compare (right half strictly smaller) and a select, which
// gives the top bit and the minimum in one compare.  K3: 4 min/min3 + 3
// compares + 5 selects + 3 pushes = 15 VALU per state (a scan with P - 1
// compares and selects takes 19); K4: 10 + 4 + 12 + 4 = 30 (39).  On gfx950 a
// select issues in half the cycles of a min, a compare or an FMA.
template <int K>
__device__ __forceinline__ float min_push_argmin(uint32_t& word, const float (&c)[1 << K]) {
    if constexpr (K == 2) {
        const float p0 = fmin2(c[0], c[1]);
        const float m = fmin2(p0, fmin2(c[2], c[3]));
        const bool b1 = p0 != m;
        const float e = b1 ? c[2] : c[0];
        const bool b0 = e != m;
        word = push_bit(word, __builtin_amdgcn_ballot_w64(b1));
        word = push_bit(word, __builtin_amdgcn_ballot_w64(b0));
        return m;
    } else if constexpr (K == 3) {
        const float p0 = fmin2(c[0], c[1]), p2 = fmin2(c[4], c[5]);
        const float h0 = fmin2(p0, fmin2(c[2], c[3])), h1 = fmin2(p2, fmin2(c[6], c[7]));
        const bool b2 = h1 < h0;  // the root as compare-and-select: the compare is needed anyway
        const float m = b2 ? h1 : h0;
        const float q = b2 ? p2 : p0;
        const bool b1 = q != m;
        const float e = b2 ? (b1 ? c[6] : c[4]) : (b1 ? c[2] : c[0]);
        const bool b0 = e != m;
        word = push_bit(word, __builtin_amdgcn_ballot_w64(b2));
        word = push_bit(word, __builtin_amdgcn_ballot_w64(b1));
        word = push_bit(word, __builtin_amdgcn_ballot_w64(b0));
        return m;
    } else {
        static_assert(K == 4, "tournament argmin is written for K2..K4");
        const float p0 = fmin2(c[0], c[1]), p2 = fmin2(c[4], c[5]), p4 = fmin2(c[8], c[9]),
                    p6 = fmin2(c[12], c[13]);
        const float q0 = fmin2(p0, fmin2(c[2], c[3])), q1 = fmin2(p2, fmin2(c[6], c[7]));
        const float q2 = fmin2(p4, fmin2(c[10], c[11])), q3 = fmin2(p6, fmin2(c[14], c[15]));
        const float h0 = fmin2(q0, q1), h1 = fmin2(q2, q3);
        const bool b3 = h1 < h0;
        const float m = b3 ? h1 : h0;
        const float q = b3 ? q2 : q0;
        const bool b2 = q != m;
        const float p = b3 ? (b2 ? p6 : p4) : (b2 ? p2 : p0);
        const bool b1 = p != m;
        const float s0 = b1 ? c[2] : c[0], s1 = b1 ? c[6] : c[4], s2 = b1 ? c[10] : c[8], s3 = b1 ? c[14] : c[12];
        const float t0 = b2 ? s1 : s0, t1 = b2 ? s3 : s2;
        const float e = b3 ? t1 : t0;
        const bool b0 = e != m;
        word = push_bit(word, __builtin_amdgcn_ballot_w64(b3));
        word = push_bit(word, __builtin_amdgcn_ballot_w64(b2));
        word = push_bit(word, __builtin_amdgcn_ballot_w64(b1));
        word = push_bit(word, __builtin_amdgcn_ballot_w64(b0));
        return m;
    }
}

// Predecessor cost of the first step of a pass: 0 for every predecessor, or,
// in the constrained pass, 0 for `pre_state` and +inf for the others
// (fma(d, d, 0) == d * d and fma(d, d, inf) == inf, so this is exactly the
// reference's step-0 rule).
__device__ __forceinline__ float first_cost(int pred, int pre_state) {
    return (pre_state < 0 || pred == pre_state) ? 0.0f : __builtin_inff();
}

// K1 step on the single in-place cost array: the thread's 32 predecessor
// costs are read into registers, a barrier orders every read before any
// write, then the 32 new costs are written over them.
template <bool RECORD, bool FIRST>
__device__ __forceinline__ void trellis_step_k1(const Labels<1>& lab, float* cost, float x, int pre_state,
                                                uint8_t* __restrict__ dec_row, int t) {
    using G = Geo<1>;
    float p[G::NG][G::P];
#pragma unroll
    for (int j = 0; j < G::NG; ++j)
#pragma unroll
        for (int k = 0; k < G::P; ++k) {
            const int pred = G::group(t, j) + k * G::kPredStride;
            p[j][k] = FIRST ? first_cost(pred, pre_state) : cost[pred];
        }
    if constexpr (!FIRST) __syncthreads();
    // Widen the fp16 labels here, per step: hoisted out of the pass loop,
    // 64 FP32 copies would not fit beside the predecessor costs.
    f16x2 h[G::NG][G::NS];
#pragma unroll
    for (int j = 0; j < G::NG; ++j)
#pragma unroll
        for (int e = 0; e < G::NS; ++e) {
            h[j][e] = lab.v[j][e];
            asm volatile("" : "+v"(h[j][e]));
        }
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < G::NG; ++j) {
        float best[G::NS];
#pragma unroll
        for (int e = 0; e < G::NS; ++e) {
            float c[G::P];
#pragma unroll
            for (int k = 0; k < G::P; ++k) {
                const float d = static_cast<float>(h[j][e][k]) - x;
                c[k] = __builtin_fmaf(d, d, p[j][k]);
            }
            best[e] = fmin2(c[0], c[1]);
            if constexpr (RECORD) word = push_argmin<1>(word, c, best[e]);
        }
        *reinterpret_cast<float2*>(cost + G::first_state(t, j)) = make_float2(best[0], best[1]);
    }
    if constexpr (RECORD) reinterpret_cast<uint32_t*>(dec_row)[t] = word;
}

// K5 / K6 step: 32 or 64 predecessors per state, streamed one at a time
// with a running minimum and its lowest index (strict less-than while k
// increases), so neither the predecessor costs nor the candidate costs have
// to sit in registers together with the thread's 64 labels.
template <int K, bool RECORD, bool FIRST>
__device__ __forceinline__ void trellis_step_wide(const Labels<K>& lab, const float* __restrict__ prev,
                                                  float* __restrict__ next, float x, int pre_state,
                                                  uint8_t* __restrict__ dec_row, int t) {
    using G = Geo<K>;
    const int q = G::group(t, 0);
    float m[G::NS];
    int arg[G::NS];
#pragma unroll
    for (int k = 0; k < G::P; ++k) {
        const int pred = q + k * G::kPredStride;
        const float p = FIRST ? first_cost(pred, pre_state) : prev[pred];
#pragma unroll
        for (int e = 0; e < G::NS; ++e) {
            const float d = lab.v[0][e][k] - x;
            const float c = __builtin_fmaf(d, d, p);
            if (k == 0) {
                m[e] = c;
                arg[e] = 0;
            } else {
                const bool lt = c < m[e];
                m[e] = lt ? c : m[e];
                arg[e] = lt ? k : arg[e];
            }
        }
    }
    if constexpr (G::NS == 2) {
        *reinterpret_cast<float2*>(next + G::first_state(t, 0)) = make_float2(m[0], m[1]);
        if constexpr (RECORD) reinterpret_cast<uint16_t*>(dec_row)[t] = static_cast<uint16_t>((arg[0] << K) | arg[1]);
    } else {
        next[G::first_state(t, 0)] = m[0];
        if constexpr (RECORD) dec_row[t] = static_cast<uint8_t>(arg[0]);
    }
}

// One trellis step over all states.  FIRST: the pass's first step (see
// first_cost).  RECORD: pack and store this row's decisions.
template <int K, bool RECORD, bool FIRST>
__device__ __forceinline__ void trellis_step(const Labels<K>& lab, const float* __restrict__ prev,
                                             float* __restrict__ next, float x, int pre_state,
                                             uint8_t* __restrict__ dec_row, int t) {
    using G = Geo<K>;
    if constexpr (K == 1) {
        trellis_step_k1<RECORD, FIRST>(lab, next, x, pre_state, dec_row, t);  // prev == next
    } else if constexpr (K >= 5) {
        trellis_step_wide<K, RECORD, FIRST>(lab, prev, next, x, pre_state, dec_row, t);
    } else {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < G::NG; ++j) {
        const int q = G::group(t, j);
        float p[G::P];
        if constexpr (FIRST) {
#pragma unroll
            for (int k = 0; k < G::P; ++k) p[k] = first_cost(q + k * G::kPredStride, pre_state);
        } else {
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
                c[k] = __builtin_fmaf(d, d, p[k]);
            }
            if constexpr (RECORD) {
                best[e] = min_push_argmin<K>(word, c);
            } else {
                float m = c[0];
#pragma unroll
                for (int k = 1; k < G::P; ++k) m = fmin2(m, c[k]);
                best[e] = m;
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
    }  // K2..K4
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

// Traceback on wave 0 alone, for tracebacks with no pass to hide behind.
// Positions top, top-1, ..., 0 are resolved from `edge` (the state after
// position `top`), D = floor(6 / K) per memory round trip: lane l guesses
// the next D branch choices (its base-2^K digits), loads the D decisions of
// its candidate states independently, and the one lane whose guesses all
// match the stored decisions supplies the state D steps back (ballot +
// shuffle, no barrier).  Codewords go to `words` when it is non-null.
// Returns the state before position 0 (uniform across wave 0).
template <int K>
__device__ int traceback_wave(const uint8_t* dec, int top, int edge, uint16_t* words, int lane) {
    constexpr int P = 1 << K;
    constexpr int D = 6 / K;
    int pos = top;
    while (pos >= 0) {
        const int d = pos + 1 < D ? pos + 1 : D;
        int state[D + 1];
        state[0] = edge;
        bool ok = lane < (1 << (K * d));
#pragma unroll
        for (int j = 1; j <= D; ++j) {
            if (j <= d) {
                const int k = (lane >> (K * (j - 1))) & (P - 1);
                const uint32_t w = load_decisions<K>(dec, pos - j + 1, state[j - 1]);
                ok = ok & (Geo<K>::extract(w, state[j - 1]) == k);
                state[j] = (k << (16 - 2 * K)) | (state[j - 1] >> K);
            }
        }
        const uint64_t hit = __builtin_amdgcn_ballot_w64(ok);
        const int src = __builtin_ctzll(hit);
        int back = state[1];
#pragma unroll
        for (int j = 2; j <= D; ++j)
            if (j == d) back = state[j];
        if (words && lane == src) {
#pragma unroll
            for (int j = 1; j <= D; ++j)
                if (j <= d) words[pos - j + 1] = static_cast<uint16_t>((state[j] << K) | state[j - 1]);
        }
        edge = __shfl(back, src, 64);
        pos -= d;
    }
    return edge;
}

// One traceback position, executed by lane 0 inside another pass's step
// loop: consume the decision word loaded one step earlier (its latency is
// hidden behind the step), record the codeword, load the next word.
template <int K>
__device__ __forceinline__ void trace_advance(const uint8_t* dec, uint16_t* words, int& pos, int& edge,
                                              uint32_t& pending) {
    const int k = Geo<K>::extract(pending, edge);
    const int prev = (k << (16 - 2 * K)) | (edge >> K);
    if (words) words[pos] = static_cast<uint16_t>((prev << K) | edge);
    edge = prev;
    --pos;
    if (pos >= 0) pending = load_decisions<K>(dec, pos, edge);
}

// A traceback being overlapped with the next forward pass.  `kind` and the
// pointers are uniform; pos / edge / pending are meaningful in lane 0 only.
struct TraceJob {
    int kind = 0;  // 0 none, 1 primer (yields end_state), 2 final (yields codewords)
    int tile = -1;
    const uint8_t* dec = nullptr;
    uint16_t* words = nullptr;
    int pos = -1, edge = 0;
    uint32_t pending = 0;
};

// One forward pass of `steps` steps over positions roll, roll+1, ... (mod
// 256), recording decisions from step `trace_start` on, with the pending
// traceback `job` advanced one position per step by lane 0.  `fresh`: the
// first step starts the pass (first_cost); otherwise the pass continues
// from the costs already in LDS.
template <int K>
__device__ __forceinline__ void forward_pass(const Labels<K>& lab, const float* sx, float*& prev, float*& next, int roll,
                                             int steps, int pre_state, int trace_start, uint8_t* dec, int t,
                                             TraceJob& job, bool fresh = true) {
    int i = 0;
    if (fresh) {
        const int pos = roll & (kTile - 1);
        uint8_t* row = dec + static_cast<size_t>(pos) * Geo<K>::kRowBytes;
        if (trace_start == 0)
            trellis_step<K, true, true>(lab, prev, next, sx[pos], pre_state, row, t);
        else
            trellis_step<K, false, true>(lab, prev, next, sx[pos], pre_state, row, t);
        if (job.kind && t == 0 && job.pos >= 0) trace_advance<K>(job.dec, job.words, job.pos, job.edge, job.pending);
        __syncthreads();
        float* tmp = prev; prev = next; next = tmp;
        i = 1;
    }
    for (; i < steps; ++i) {
        const int pos = (i + roll) & (kTile - 1);
        uint8_t* row = dec + static_cast<size_t>(pos) * Geo<K>::kRowBytes;
        if (i >= trace_start)
            trellis_step<K, true, false>(lab, prev, next, sx[pos], -1, row, t);
        else
            trellis_step<K, false, false>(lab, prev, next, sx[pos], -1, row, t);
        if (job.kind && t == 0 && job.pos >= 0) trace_advance<K>(job.dec, job.words, job.pos, job.edge, job.pending);
        __syncthreads();
        float* tmp = prev; prev = next; next = tmp;
    }
}

// Resolve whatever is left of `job` on wave 0 (lane 0 hands over its
// position).  Every thread must call it; returns after a barrier.  For a
// primer job the state before position 0 is stored to *end_state.
template <int K>
__device__ void finish_job(TraceJob& job, int* end_state, int t) {
    if (t < 64) {
        const int pos = __shfl(job.pos, 0, 64);
        const int edge = __shfl(job.edge, 0, 64);
        const int result = traceback_wave<K>(job.dec, pos, edge, job.words, t);
        if (t == 0 && job.kind == 1) *end_state = result;
    }
    __syncthreads();
}

// Start a traceback of the pass that just ended; the caller has fenced the
// pass's decision stores and passed a barrier.
template <int K>
__device__ __forceinline__ void start_job(TraceJob& job, int kind, int tile, const uint8_t* dec, uint16_t* words,
                                          int top, int edge, int t) {
    job.kind = kind;
    job.tile = tile;
    job.dec = dec;
    job.words = words;
    if (t == 0) {
        job.pos = top;
        job.edge = edge;
        job.pending = load_decisions<K>(dec, top, edge);
    }
}

template <int K>
__global__ __launch_bounds__(kThreads, 1) void viterbi_tiles_kernel(
    const float* __restrict__ tiles, float* __restrict__ recon, uint16_t* __restrict__ states,
    int64_t n_tiles, int context, const uint8_t* __restrict__ lut, int boundary_lag,
    uint8_t* __restrict__ dec_ws) {
    using G = Geo<K>;
    __shared__ __align__(16) float costs[kCostArrays<K> * G::S];
    __shared__ float sx[2][kTile];
    __shared__ uint16_t words[2][kTile];
    __shared__ int end_state[2];
    __shared__ float red_v[kWaves];
    __shared__ int red_i[kWaves];
    __shared__ int bcast;

    const int t = threadIdx.x;
    constexpr size_t kBufBytes = static_cast<size_t>(kTile) * G::kRowBytes;
    uint8_t* dec_base = dec_ws + static_cast<size_t>(blockIdx.x) * 2 * kBufBytes;

    Labels<K> lab;
#pragma unroll
    for (int j = 0; j < G::NG; ++j)
#pragma unroll
        for (int e = 0; e < G::NS; ++e)
#pragma unroll
            for (int k = 0; k < G::P; ++k)
                lab.v[j][e][k] = static_cast<decltype(+lab.v[j][e][k])>(
                    qsrt::e4m3_to_float(lut[(k << (16 - K)) | (G::first_state(t, j) + e)]));

    // This workgroup's tiles are first + i * stride, i < m.  Passes run in
    // the order P0, P1, F0, P2, F1, ..., F(m-1) (primer of tile i+1 before
    // the constrained pass of tile i) so that every traceback can hide
    // behind the pass after the one that produced it.  Pass n writes
    // decision buffer n & 1; tile i lives in LDS slot i & 1.
    const int64_t first = blockIdx.x, stride = gridDim.x;
    const int m = first < n_tiles ? static_cast<int>((n_tiles - first + stride - 1) / stride) : 0;

    auto finalize = [&](int i) {  // codewords of tile i are complete in words[i & 1]
        if (t < kTile) {
            const int64_t tile = first + static_cast<int64_t>(i) * stride;
            const uint32_t w = words[i & 1][t];
            states[tile * kTile + t] = static_cast<uint16_t>(w);
            recon[tile * kTile + t] = qsrt::e4m3_to_float(lut[w]);
        }
    };

    TraceJob job;
    int next_p = 0, next_f = 0;
    for (int n = 0; next_f < m; ++n) {
        const bool primer = next_p < m && next_p <= next_f + 1;
        const int i = primer ? next_p : next_f;
        const int slot = i & 1;
        uint8_t* dec = dec_base + static_cast<size_t>(n & 1) * kBufBytes;
        if (primer) {
            if (t < kTile) sx[slot][t] = tiles[(first + static_cast<int64_t>(i) * stride) * kTile + t];
        } else if (job.kind == 1 && job.tile == i) {
            // Nothing ran between this tile's primer and its constrained
            // pass: resolve the boundary now.
            finish_job<K>(job, &end_state[slot], t);
            job.kind = 0;
        }
        __syncthreads();

        // Primer: positions 256-C .. 255, 0 .. C-1, decisions kept for 0 .. C-1.
        // Constrained pass: positions 0 .. 255 from the boundary state.
        float* prev = costs;
        float* next = costs + (kCostArrays<K> - 1) * G::S;
        int start_in_place = 0;  // K1, boundary lag 1: argmin of the penultimate primer costs (thread 0)
        if (kCostArrays<K> == 1 && primer && boundary_lag) {
            // The single array still holds the penultimate costs after 2C - 1
            // steps: take their argmin there, then run the last, recorded step.
            forward_pass<K>(lab, sx[slot], prev, next, kTile - context, 2 * context - 1, -1, context, dec, t, job);
            start_in_place = boundary_argmin<K>(prev, red_v, red_i, t);  // has a barrier
            forward_pass<K>(lab, sx[slot], prev, next, kTile + context - 1, 1, -1, 0, dec, t, job, false);
        } else {
            forward_pass<K>(lab, sx[slot], prev, next, primer ? kTile - context : 0, primer ? 2 * context : kTile,
                            primer ? -1 : end_state[slot], primer ? context : 0, dec, t, job);
        }

        // Close the traceback that ran alongside this pass.
        if (job.kind) {
            const int jt = job.tile;
            const int kind = job.kind;
            finish_job<K>(job, &end_state[jt & 1], t);
            if (kind == 2) finalize(jt);
            job.kind = 0;
        }
        // This pass's decisions must be complete before any load of them;
        // writer and readers share one CU, so workgroup scope suffices.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (primer) {
            const int start = (kCostArrays<K> == 1 && boundary_lag)
                                  ? start_in_place
                                  : boundary_argmin<K>(boundary_lag ? next : prev, red_v, red_i, t);  // has a barrier
            if (t == 0) bcast = start;
            __syncthreads();
            start_job<K>(job, 1, i, dec, nullptr, context - 1, bcast, t);
            ++next_p;
        } else {
            __syncthreads();
            start_job<K>(job, 2, i, dec, words[slot], kTile - 1, end_state[slot], t);
            ++next_f;
        }
    }
    if (job.kind) {
        const int jt = job.tile;
        finish_job<K>(job, &end_state[jt & 1], t);
        finalize(jt);
    }
}

template <int K>
size_t row_bytes() { return static_cast<size_t>(Geo<K>::kRowBytes); }

size_t workgroup_dec_bytes(int K) {
    switch (K) {
        case 1: return 2 * kTile * row_bytes<1>();
        case 2: return 2 * kTile * row_bytes<2>();
        case 3: return 2 * kTile * row_bytes<3>();
        case 4: return 2 * kTile * row_bytes<4>();
        case 5: return 2 * kTile * row_bytes<5>();
        case 6: return 2 * kTile * row_bytes<6>();
        default: return 0;
    }
}

int launch_workgroups(int64_t n_tiles, int cu_count) {
    const int64_t g = n_tiles < cu_count ? n_tiles : cu_count;
    return static_cast<int>(g);
}

// The reference hands its kernels the K2..K4 codebook as [out-edge pair][predecessor][2] bytes
// (qsrt/sqg_quantizer.py:612-633 transposes the state-indexed [predecessor][out-edge pair][2] table so that a
// CUDA thread fetches all its predecessors' labels in one vector load).  This kernel writes the state-indexed
// table back: state s = (p << (16 - K)) | (2 e + b) sits at transposed byte (e * 2^K + p) * 2 + b.
__global__ __launch_bounds__(256) void untranspose_codebook_kernel(const uint8_t* __restrict__ transposed,
                                                                   uint8_t* __restrict__ state_indexed, int K) {
    const int s = blockIdx.x * 256 + threadIdx.x;
    const int p = s >> (16 - K), rest = s & ((1 << (16 - K)) - 1);
    const int e = rest >> 1, b = rest & 1;
    state_indexed[s] = transposed[((e << K) + p) * 2 + b];
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
    return qsrt_viterbi_tiles_ex(tiles, recon, states, n_tiles, K, tailbite_context, lut_e4m3, boundary_lag, 0,
                                 workspace, workspace_bytes, stream_handle);
}

int qsrt_viterbi_tiles_ex(const float* tiles, float* recon, uint16_t* states, int64_t n_tiles, int K,
                          int tailbite_context, const uint8_t* lut_e4m3, int boundary_lag, int max_workgroups,
                          void* workspace, size_t workspace_bytes, void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (max_workgroups < 0) return qsrt::fail(qsrt::kBadArgument, "max_workgroups must be non-negative");
    if (K < 1 || K > 6)
        return qsrt::fail(qsrt::kBadArgument, "K%d is not supported by the MI355X tile kernel (K1..K6)", K);
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
    const int grid = launch_workgroups(n_tiles, max_workgroups > 0 && max_workgroups < cus ? max_workgroups : cus);
    const size_t need = workgroup_dec_bytes(K) * static_cast<size_t>(grid);
    if (workspace_bytes < need)
        return qsrt::fail(qsrt::kWorkspaceTooSmall, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
    auto* ws = static_cast<uint8_t*>(workspace);
#define QSRT_LAUNCH_VITERBI(KK)                                                                                  \
    case KK:                                                                                                     \
        hipLaunchKernelGGL(viterbi_tiles_kernel<KK>, dim3(grid), dim3(kThreads), 0, stream, tiles, recon, states, \
                           n_tiles, tailbite_context, lut_e4m3, boundary_lag, ws);                             \
        break;
    switch (K) {
        QSRT_LAUNCH_VITERBI(1)
        QSRT_LAUNCH_VITERBI(2)
        QSRT_LAUNCH_VITERBI(3)
        QSRT_LAUNCH_VITERBI(4)
        QSRT_LAUNCH_VITERBI(5)
        QSRT_LAUNCH_VITERBI(6)
    }
#undef QSRT_LAUNCH_VITERBI
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

int qsrt_quantize_tiles_sqg(const float* input_tiles, float* output_tiles, int16_t* output_indices, int64_t n_tiles,
                            void* temp_costs, size_t temp_costs_bytes, uint8_t* temp_edges, size_t temp_edges_bytes,
                            const uint8_t* codebook, int K, int tailbite_context, double lut_abs_max,
                            void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (K < 1 || K > 6) return qsrt::fail(qsrt::kBadArgument, "SQG validation kernel supports K1--K6");
    if (tailbite_context < 1 || tailbite_context > 128)
        return qsrt::fail(qsrt::kBadArgument, "tailbite_context must be in 1..128");
    if (n_tiles < 0) return qsrt::fail(qsrt::kBadArgument, "n_tiles must be non-negative");
    if (n_tiles == 0) return qsrt::kOk;
    if (!input_tiles || !output_tiles || !output_indices || !temp_costs || !temp_edges || !codebook)
        return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    // the reference's K2 fast kernel (chosen for finite label bounds in (0, 16]) scores the last primer step,
    // its generic kernel the one before (qsrt/csrc/sqg_quantize.cu:730-749)
    const int lag = (K == 2 && std::isfinite(lut_abs_max) && lut_abs_max > 0.0 && lut_abs_max <= 16.0) ? 0 : 1;
    const uint8_t* lut = codebook;
    if (K >= 2 && K <= 4) {
        // the FP16 cost buffer is not needed (costs live in LDS): its first 64 KiB hold the state-indexed table
        if (temp_costs_bytes < 65536)
            return qsrt::fail(qsrt::kWorkspaceTooSmall, "temp_costs must hold at least 65536 bytes");
        uint8_t* table = static_cast<uint8_t*>(temp_costs);
        hipLaunchKernelGGL(untranspose_codebook_kernel, dim3(256), dim3(256), 0, stream, codebook, table, K);
        QSRT_HIP_TRY(hipGetLastError());
        lut = table;
    }
    // the traceback buffer bounds how many workgroups run at once
    const size_t per = workgroup_dec_bytes(K);
    if (temp_edges_bytes < per)
        return qsrt::fail(qsrt::kWorkspaceTooSmall, "temp_edges too small: %zu < %zu bytes", temp_edges_bytes, per);
    const size_t fit = temp_edges_bytes / per;
    const int cap = fit > 0x7fffffff ? 0x7fffffff : static_cast<int>(fit);
    return qsrt_viterbi_tiles_ex(input_tiles, output_tiles, reinterpret_cast<uint16_t*>(output_indices), n_tiles, K,
                                 tailbite_context, lut, lag, cap, temp_edges, temp_edges_bytes, stream_handle);
}


}  // extern "C"
