// Trellis payload codec kernels: EXL word packing and cyclic-state unpacking.
//
// Payload format (reference qsrt/qsrt.py:861-913, the EXL pack_trellis word
// order): per 256-symbol tile, the low K bits of each symbol form one
// MSB-first bitstream of 256 K bits, cut into 16 K big-endian 16-bit words;
// adjacent words are then swapped (word w is stored at w ^ 1).
// A state is the low 16 bits of (previous state << K) | edge, cyclic over
// the tile, so state i = OR_{lag < ceil(16/K)} edge[i - lag] << (lag K).

#include "common.h"
#include "qsrt_amd.h"

namespace {

constexpr int kTile = 256;

// One thread per 16-symbol span: 16 K bits -> K words, emitted as soon as
// 16 bits have accumulated (the accumulator never holds more than 15 + K).
template <int K>
__global__ __launch_bounds__(256) void pack_edges_kernel(const uint16_t* __restrict__ states, int64_t n_spans,
                                                        uint16_t* __restrict__ words) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= n_spans) return;
    const uint4* src = reinterpret_cast<const uint4*>(states + g * 16);
    const uint4 a = src[0], b = src[1];
    const uint32_t halves[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    const int64_t tile = g >> 4;
    const int span = static_cast<int>(g & 15);
    uint16_t* out = words + tile * (16 * K);
    uint32_t acc = 0;
    int held = 0, w = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t sym = (halves[i >> 1] >> (16 * (i & 1))) & ((1u << K) - 1);
        acc = (acc << K) | sym;
        held += K;
        if (held >= 16) {
            held -= 16;
            out[(span * K + w) ^ 1] = static_cast<uint16_t>(acc >> held);
            acc &= (1u << held) - 1;
            ++w;
        }
    }
}

// One workgroup per tile: symbol i from the bitstream, then its cyclic state.
template <int K>
__global__ __launch_bounds__(kTile) void unpack_states_kernel(const uint16_t* __restrict__ words, int64_t n_tiles,
                                                             uint16_t* __restrict__ states) {
    __shared__ uint16_t w[16 * K];
    __shared__ uint16_t e[kTile];
    const int t = threadIdx.x;
    const int64_t tile = blockIdx.x;
    if (t < 16 * K) w[t ^ 1] = words[tile * (16 * K) + t];
    __syncthreads();
    // bits [t K, t K + K) of the stream; the field may straddle two words
    const int bit = t * K;
    const uint32_t pair = (static_cast<uint32_t>(w[bit >> 4]) << 16) |
                          ((bit >> 4) + 1 < 16 * K ? w[(bit >> 4) + 1] : 0u);
    e[t] = static_cast<uint16_t>((pair >> (32 - (bit & 15) - K)) & ((1u << K) - 1));
    __syncthreads();
    uint32_t s = 0;
#pragma unroll
    for (int lag = 0; lag < (16 + K - 1) / K; ++lag) s |= static_cast<uint32_t>(e[(t - lag) & (kTile - 1)]) << (lag * K);
    states[tile * kTile + t] = static_cast<uint16_t>(s);
}

}  // namespace

extern "C" {

int qsrt_pack_edges(const uint16_t* states, int64_t n_tiles, int K, int16_t* words, void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (K < 1 || K > 6) return qsrt::fail(qsrt::kBadArgument, "K%d packing is not supported (K1..K6)", K);
    if (n_tiles < 0) return qsrt::fail(qsrt::kBadArgument, "n_tiles must be non-negative");
    if (n_tiles == 0) return qsrt::kOk;
    if (!states || !words) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (reinterpret_cast<uintptr_t>(states) % 16)
        return qsrt::fail(qsrt::kBadArgument, "states must be 16-byte aligned");
    const int64_t spans = n_tiles * 16;
    const dim3 grid(static_cast<unsigned>((spans + 255) / 256));
    auto* out = reinterpret_cast<uint16_t*>(words);
#define QSRT_PACK(KK) \
    case KK: hipLaunchKernelGGL(pack_edges_kernel<KK>, grid, dim3(256), 0, stream, states, spans, out); break;
    switch (K) { QSRT_PACK(1) QSRT_PACK(2) QSRT_PACK(3) QSRT_PACK(4) QSRT_PACK(5) QSRT_PACK(6) }
#undef QSRT_PACK
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

int qsrt_unpack_states(const int16_t* words, int64_t n_tiles, int K, uint16_t* states, void* stream_handle) {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (K < 1 || K > 6) return qsrt::fail(qsrt::kBadArgument, "K%d unpacking is not supported (K1..K6)", K);
    if (n_tiles < 0) return qsrt::fail(qsrt::kBadArgument, "n_tiles must be non-negative");
    if (n_tiles == 0) return qsrt::kOk;
    if (!states || !words) return qsrt::fail(qsrt::kBadArgument, "null pointer argument");
    if (n_tiles > 0x7fffffff) return qsrt::fail(qsrt::kBadArgument, "too many tiles for one launch");
    const auto* in = reinterpret_cast<const uint16_t*>(words);
    const dim3 grid(static_cast<unsigned>(n_tiles));
#define QSRT_UNPACK(KK) \
    case KK: hipLaunchKernelGGL(unpack_states_kernel<KK>, grid, dim3(kTile), 0, stream, in, n_tiles, states); break;
    switch (K) { QSRT_UNPACK(1) QSRT_UNPACK(2) QSRT_UNPACK(3) QSRT_UNPACK(4) QSRT_UNPACK(5) QSRT_UNPACK(6) }
#undef QSRT_UNPACK
    QSRT_HIP_TRY(hipGetLastError());
    return qsrt::kOk;
}

}  // extern "C"
