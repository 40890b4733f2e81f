// Shared helpers for the QSRT MI355X kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

namespace qsrt {

// Thread-local last-error message returned by qsrt_last_error().
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

#define QSRT_HIP_TRY(expr)                                                       \
    do {                                                                         \
        hipError_t qsrt_err__ = (expr);                                          \
        if (qsrt_err__ != hipSuccess)                                            \
            return ::qsrt::fail(-3, "%s failed: %s", #expr,                      \
                                hipGetErrorString(qsrt_err__));                  \
    } while (0)

enum : int {
    kOk = 0,
    kBadArgument = -1,
    kWorkspaceTooSmall = -2,
    kHipError = -3,
};

// Exact E4M3 (fn) byte -> float.  0x7F / 0xFF decode to NaN.
__host__ __device__ inline float e4m3_to_float(uint32_t byte) {
    const uint32_t mag = byte & 0x7Fu;
    const uint32_t e = mag >> 3, m = mag & 7u;
    float v;
    if (mag == 0x7Fu) {
        v = __builtin_nanf("");
    } else if (e == 0) {
        v = (float)m * (1.0f / 512.0f);
    } else {
        // (8 + m) * 2^(e - 10), built from the bit pattern of 2^(e-7) * (1 + m/8)
        union { uint32_t u; float f; } bits;
        bits.u = ((e + 120u) << 23) | (m << 20);
        v = bits.f;
    }
    return (byte & 0x80u) ? -v : v;
}

int current_cu_count(int* out);

}  // namespace qsrt
