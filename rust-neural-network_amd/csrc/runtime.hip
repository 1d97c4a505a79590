// runtime.hip -- error reporting and device queries shared by every entry point.
#include "common.hpp"

namespace rnn {

static thread_local char g_err[512] = "";

int set_error(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return status;
}

void clear_error() { g_err[0] = '\0'; }

int device_cu_count() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

}  // namespace rnn

extern "C" int rnn_abi_version(void) { return RNN_HIP_ABI_VERSION; }

extern "C" const char *rnn_last_error(void) { return rnn::g_err; }
