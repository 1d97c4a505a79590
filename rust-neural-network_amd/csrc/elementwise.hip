// elementwise.hip -- the f32 pieces a Sequential of mixed layers needs around
// the GEMMs: Tensor::relu, the fused bias + ReLU of Tensor::linear_layer, and
// linear_layer itself (x . W^T through rnn_sgemm, then bias + activation).
// HBM-bound streaming kernels, 16-byte vectorised when the rows allow it.
#include "common.hpp"

namespace rnn {

constexpr int kEwBlock = 256;

// The activation of linear_layer's fused path (src/tensor.rs:776-779):
// v > 0 ? v : 0, so NaN and -0 both become +0.
__device__ __forceinline__ float relu_fused(float v) { return v > 0.0f ? v : 0.0f; }

// Tensor::relu (src/tensor.rs:2025-2032): x.max(0.0). Rust's f32::max returns
// the non-NaN operand, as fmaxf does, so NaN becomes 0.
__global__ __launch_bounds__(kEwBlock) void relu_kernel(const float *__restrict__ x, int64_t n,
                                                      float *__restrict__ y) {
    const int64_t stride = (int64_t)gridDim.x * kEwBlock;
    const int64_t n4 = (((uintptr_t)x | (uintptr_t)y) & 15) == 0 ? n / 4 : 0;
    for (int64_t i = blockIdx.x * (int64_t)kEwBlock + threadIdx.x; i < n4; i += stride) {
        float4 v = reinterpret_cast<const float4 *>(x)[i];
        v.x = fmaxf(v.x, 0.0f);
        v.y = fmaxf(v.y, 0.0f);
        v.z = fmaxf(v.z, 0.0f);
        v.w = fmaxf(v.w, 0.0f);
        reinterpret_cast<float4 *>(y)[i] = v;
    }
    for (int64_t i = 4 * n4 + blockIdx.x * (int64_t)kEwBlock + threadIdx.x; i < n; i += stride)
        y[i] = fmaxf(x[i], 0.0f);
}

// y[r, c] = y[r, c] + bias[c] (bias may be null), then relu_fused when RELU:
// the loop of src/tensor.rs:771-786, one rounding per add.
template <bool RELU>
__global__ __launch_bounds__(kEwBlock) void bias_act_kernel(float *__restrict__ y,
                                                          const float *__restrict__ bias,
                                                          int64_t rows, int64_t cols) {
    const int64_t total = rows * cols;
    const int64_t stride = (int64_t)gridDim.x * kEwBlock;
    const bool vec = cols % 4 == 0 && (((uintptr_t)y | (uintptr_t)bias) & 15) == 0;
    const int64_t n4 = vec ? total / 4 : 0;
    for (int64_t i = blockIdx.x * (int64_t)kEwBlock + threadIdx.x; i < n4; i += stride) {
        float4 v = reinterpret_cast<float4 *>(y)[i];
        if (bias) {
            const float4 b = reinterpret_cast<const float4 *>(bias)[i % (cols / 4)];
            v.x = v.x + b.x;
            v.y = v.y + b.y;
            v.z = v.z + b.z;
            v.w = v.w + b.w;
        }
        if (RELU) {
            v.x = relu_fused(v.x);
            v.y = relu_fused(v.y);
            v.z = relu_fused(v.z);
            v.w = relu_fused(v.w);
        }
        reinterpret_cast<float4 *>(y)[i] = v;
    }
    for (int64_t i = 4 * n4 + blockIdx.x * (int64_t)kEwBlock + threadIdx.x; i < total; i += stride) {
        float v = y[i];
        if (bias) v = v + bias[i % cols];
        if (RELU) v = relu_fused(v);
        y[i] = v;
    }
}

static unsigned ew_blocks(int64_t n) {
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 4 * kEwBlock),
                                                            8 * device_cu_count()));
}

}  // namespace rnn

using namespace rnn;

extern "C" int rnn_relu(const float *x, int64_t n, float *y, void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_relu";
    RNN_REQUIRE(n >= 0, "%s: negative size", name);
    if (n == 0) return RNN_OK;
    RNN_REQUIRE(x && y, "%s: null pointer", name);
    relu_kernel<<<ew_blocks(n), kEwBlock, 0, as_stream(stream)>>>(x, n, y);
    return check_launch(name);
}

extern "C" int rnn_bias_act(float *y, const float *bias, int64_t rows, int64_t cols, int relu,
                            void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_bias_act";
    RNN_REQUIRE(rows >= 0 && cols >= 0, "%s: negative size", name);
    RNN_REQUIRE(relu == 0 || relu == 1, "%s: relu must be 0 or 1", name);
    if (rows == 0 || cols == 0 || (!bias && !relu)) return RNN_OK;
    RNN_REQUIRE(y != nullptr, "%s: null y", name);
    const unsigned g = ew_blocks(rows * cols);
    if (relu)
        bias_act_kernel<true><<<g, kEwBlock, 0, as_stream(stream)>>>(y, bias, rows, cols);
    else
        bias_act_kernel<false><<<g, kEwBlock, 0, as_stream(stream)>>>(y, bias, rows, cols);
    return check_launch(name);
}

extern "C" int rnn_linear_layer(const float *x, int64_t batch, int64_t in_f, const float *w,
                                int64_t out_f, const float *bias, int relu, float *y,
                                void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_linear_layer";
    RNN_REQUIRE(batch >= 0 && in_f >= 0 && out_f >= 0, "%s: negative size", name);
    RNN_REQUIRE(relu == 0 || relu == 1, "%s: relu must be 0 or 1", name);
    if (batch == 0 || out_f == 0) return RNN_OK;
    RNN_REQUIRE(y != nullptr && (in_f == 0 || (x && w)), "%s: null pointer", name);
    // y = x . W^T with W stored [out, in] (transb = 1, ldb = in), beta = 0
    RNN_TRY(rnn_sgemm(0, 1, batch, out_f, in_f, 1.0f, x, in_f, w, in_f, 0.0f, y, out_f, stream));
    return rnn_bias_act(y, bias, batch, out_f, relu, stream);
}
