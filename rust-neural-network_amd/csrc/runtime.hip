// runtime.hip -- error reporting and device queries shared by every entry point.
#include <atomic>

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

// Per-device CU counts, filled on first use. Relaxed atomics: racing threads
// compute and store the same value, so no ordering is needed beyond the store
// itself being whole.
static std::atomic<int> g_cu_count[64];

int device_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = g_cu_count[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        g_cu_count[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

}  // namespace rnn

extern "C" int rnn_abi_version(void) { return RNN_HIP_ABI_VERSION; }

extern "C" const char *rnn_last_error(void) { return rnn::g_err; }
