// Error reporting and device queries shared by every C-ABI entry point.
#include "common.h"
#include "qsrt_amd.h"

#include <string.h>

namespace qsrt {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int current_cu_count(int* out) {
    static int cached[64] = {0};
    int dev = 0;
    QSRT_HIP_TRY(hipGetDevice(&dev));
    if (dev >= 0 && dev < 64 && cached[dev] > 0) {
        *out = cached[dev];
        return kOk;
    }
    int cus = 0;
    QSRT_HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    if (cus <= 0) return fail(kHipError, "device %d reports %d compute units", dev, cus);
    if (dev >= 0 && dev < 64) cached[dev] = cus;
    *out = cus;
    return kOk;
}

}  // namespace qsrt

extern "C" const char* qsrt_last_error(void) { return qsrt::g_last_error; }

extern "C" int qsrt_abi_version(void) { return 2; }
