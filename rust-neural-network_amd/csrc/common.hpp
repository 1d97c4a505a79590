// common.hpp -- shared helpers for the gfx950 kernels behind rnn_hip.h:
// per-thread error state, argument checks, launch checking, MFMA vector types.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>

#include "../../include/rnn_hip.h"

// The kernels are written for gfx950 only. Beyond the MFMA and LDS-DMA forms,
// two split-merge hand-offs (the split-K GEMV partials of qformat.hip and the
// sequence-split attention states of rqattn.hip) rely on gfx9 memory
// behaviour: device-scope atomic stores write through the XCD's L2 to the
// coherence point, and `s_waitcnt vmcnt(0)` waits for stores as well as
// loads, so a relaxed counter increment issued after it is ordered behind the
// partials. A target that counts stores separately (vscnt) would race there.
#if defined(__HIP_DEVICE_COMPILE__) && !(defined(__gfx950__) && defined(__GFX9__))
#error "librnn_hip is built for gfx950 only (gfx9 store counting is assumed by the split merges)"
#endif

namespace rnn {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Records the message for rnn_last_error() and returns the status.
int set_error(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Checks the launch that just happened on this thread.
inline int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(RNN_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return RNN_OK;
}

inline int check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess)
        return set_error(e == hipErrorOutOfMemory ? RNN_ERR_OUT_OF_MEMORY : RNN_ERR_HIP,
                         "%s: %s", what, hipGetErrorString(e));
    return RNN_OK;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Number of workgroups that fills the device a few times over for
// grid-stride kernels (256 CUs on MI355X).
int device_cu_count();

}  // namespace rnn

#define RNN_REQUIRE(cond, ...)                                          \
    do {                                                                \
        if (!(cond)) return ::rnn::set_error(RNN_ERR_INVALID_ARG, __VA_ARGS__); \
    } while (0)

// First statement of every status-returning entry point: a call that succeeds
// leaves rnn_last_error() empty, so the message always belongs to the calling
// thread's most recent call.
#define RNN_ENTRY() ::rnn::clear_error()

#define RNN_TRY(expr)                   \
    do {                                \
        int _rc = (expr);               \
        if (_rc != RNN_OK) return _rc;  \
    } while (0)
