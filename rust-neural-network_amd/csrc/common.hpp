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
