// ternary.hip -- 2-bit ternary packing, quantization (reference per-row rule
// and the per-tensor absmean rule), dequantization and the reference-semantics
// TernaryLinear::forward (f32 shift-and-add, sequential in k: bit-exact).
#include <algorithm>

#include "common.hpp"
#include "numerics.hpp"

namespace rnn {

__device__ __forceinline__ uint32_t ternary_code(int8_t v) {
    return v == 0 ? 0u : (v > 0 ? 1u : 2u);  // src/ternary.rs:50-56
}

__device__ __forceinline__ int ternary_value(uint32_t code) {
    return code == 1u ? 1 : (code == 2u ? -1 : 0);  // src/ternary.rs:67-72
}

static unsigned grid_for(int64_t work, int threads) {
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(work, threads),
                                                            16 * device_cu_count()));
}

// One thread per packed word (16 codes, LSB first).
__global__ void ternary_pack_kernel(const int8_t *__restrict__ t, int64_t count,
                                    uint32_t *__restrict__ packed) {
    const int64_t words = (count + 15) / 16;
    for (int64_t w = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; w < words;
         w += (int64_t)gridDim.x * blockDim.x) {
        uint32_t word = 0;
        const int64_t base = w * 16;
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (base + j < count) word |= ternary_code(t[base + j]) << (2 * j);
        packed[w] = word;
    }
}

__global__ void ternary_unpack_kernel(const uint32_t *__restrict__ packed, int64_t count,
                                      int8_t *__restrict__ t) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * blockDim.x)
        t[i] = (int8_t)ternary_value((packed[i / 16] >> (2 * (i % 16))) & 3u);
}

// Per-row sum of |w| in k order (f32, exactly the reference's
// `row.iter().map(|v| v.abs()).sum::<f32>()`, src/ternary.rs:114), one thread
// per row. MEAN divides by cols (the reference's mean_abs).
template <bool MEAN>
__global__ void row_abs_sum_kernel(const float *__restrict__ w, int64_t rows, int64_t cols,
                                   float *__restrict__ out) {
    const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const float *row = w + r * cols;
    float s = 0.0f;
    for (int64_t j = 0; j < cols; ++j) s = s + fabsf(row[j]);
    out[r] = MEAN ? s / (float)(cols > 0 ? cols : 1) : s;
}

// gamma = max((float)(sum_r (double)rowsum[r] / numel), 1e-8), added in row
// order by one thread, then broadcast into scales[0..rows).
__global__ void absmean_gamma_kernel(float *__restrict__ scales, int64_t rows, int64_t numel) {
    __shared__ float g;
    if (threadIdx.x == 0) {
        double total = 0.0;
        for (int64_t r = 0; r < rows; ++r) total = total + (double)scales[r];
        float gamma = (float)(total / (double)(numel > 0 ? numel : 1));
        g = fmaxf(gamma, 1e-8f);
    }
    __syncthreads();
    for (int64_t r = threadIdx.x; r < rows; r += blockDim.x) scales[r] = g;
}

// Quantize + pack, one thread per packed word. ROWS mode reads the row's
// mean|w| from `stat` (threshold 0.7*mean, src/ternary.rs:115-127);
// ABSMEAN mode reads gamma and uses round(w/gamma).clamp(-1,1).
template <bool ABSMEAN>
__global__ void ternary_quant_pack_kernel(const float *__restrict__ w, int64_t numel, int64_t cols,
                                          const float *__restrict__ stat,
                                          uint32_t *__restrict__ packed) {
    const int64_t words = (numel + 15) / 16;
    for (int64_t wd = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; wd < words;
         wd += (int64_t)gridDim.x * blockDim.x) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int64_t i = wd * 16 + j;
            if (i >= numel) break;
            const float v = w[i];
            int8_t t;
            if (ABSMEAN) {
                t = to_i8_rs(clamp_rs(roundf(v / stat[i / cols]), -1.0f, 1.0f));
            } else {
                const float thr = 0.7f * stat[i / cols];
                t = fabsf(v) < thr ? 0 : (v > 0.0f ? 1 : -1);
            }
            word |= ternary_code(t) << (2 * j);
        }
        packed[wd] = word;
    }
}

// scale = mean.max(1e-8) (src/ternary.rs:116), in place.
__global__ void finalize_row_scales_kernel(float *__restrict__ scales, int64_t rows) {
    const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (r < rows) scales[r] = fmaxf(scales[r], 1e-8f);
}

__global__ void ternary_dequant_kernel(const uint32_t *__restrict__ packed, int64_t numel,
                                       const float *__restrict__ scales, int64_t n_scales,
                                       int64_t cols, float *__restrict__ w) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < numel;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = std::min<int64_t>(i / cols, n_scales - 1);
        w[i] = (float)ternary_value((packed[i / 16] >> (2 * (i % 16))) & 3u) * scales[r];
    }
}

// Reference TernaryLinear::forward: one thread per (b, o), f32 add/subtract
// in k order (src/ternary.rs:250-264), then acc * scale[o] (+ bias[o]).
template <bool BIAS>
__global__ __launch_bounds__(256) void ternary_linear_ref_kernel(
    const float *__restrict__ x, int64_t in_f, const uint32_t *__restrict__ packed,
    const float *__restrict__ scales, int64_t out_f, const float *__restrict__ bias,
    float *__restrict__ y) {
    const int64_t b = blockIdx.y;
    const int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (o >= out_f) return;
    const float *xr = x + b * in_f;
    float acc = 0.0f;
    int64_t idx = o * in_f;
    uint32_t word = in_f > 0 ? packed[idx / 16] >> (2 * (idx % 16)) : 0u;
    for (int64_t i = 0; i < in_f; ++i, ++idx) {
        if (idx % 16 == 0) word = packed[idx / 16];
        const uint32_t code = word & 3u;
        word >>= 2;
        const float xv = xr[i];
        if (code == 1u) acc = acc + xv;
        else if (code == 2u) acc = acc - xv;
    }
    float v = acc * scales[o];
    if (BIAS) v = v + bias[o];
    y[b * out_f + o] = v;
}

}  // namespace rnn

using namespace rnn;

extern "C" int rnn_ternary_pack(const int8_t *t, int64_t count, uint32_t *packed, void *stream) {
    RNN_ENTRY();
    RNN_REQUIRE(count >= 0, "rnn_ternary_pack: negative count");
    if (count == 0) return RNN_OK;
    RNN_REQUIRE(t && packed, "rnn_ternary_pack: null pointer");
    ternary_pack_kernel<<<grid_for((count + 15) / 16, 256), 256, 0, as_stream(stream)>>>(t, count,
                                                                                         packed);
    return check_launch("rnn_ternary_pack");
}

extern "C" int rnn_ternary_unpack(const uint32_t *packed, int64_t count, int8_t *t, void *stream) {
    RNN_ENTRY();
    RNN_REQUIRE(count >= 0, "rnn_ternary_unpack: negative count");
    if (count == 0) return RNN_OK;
    RNN_REQUIRE(t && packed, "rnn_ternary_unpack: null pointer");
    ternary_unpack_kernel<<<grid_for(count, 256), 256, 0, as_stream(stream)>>>(packed, count, t);
    return check_launch("rnn_ternary_unpack");
}

extern "C" int rnn_ternary_quantize(const float *w, int64_t rows, int64_t cols, int mode,
                                    uint32_t *packed, float *scales, void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_ternary_quantize";
    RNN_REQUIRE(rows >= 0 && cols >= 0, "%s: negative size", name);
    RNN_REQUIRE(mode == RNN_TERNARY_ROWS || mode == RNN_TERNARY_ABSMEAN, "%s: bad mode %d", name,
                mode);
    if (rows == 0) return RNN_OK;
    RNN_REQUIRE(scales && (cols == 0 || (w && packed)), "%s: null pointer", name);
    hipStream_t st = as_stream(stream);
    const int64_t numel = rows * cols;
    const unsigned rblocks = (unsigned)ceil_div(rows, 64);
    if (mode == RNN_TERNARY_ROWS) {
        row_abs_sum_kernel<true><<<rblocks, 64, 0, st>>>(w, rows, cols, scales);
        RNN_TRY(check_launch(name));
        if (numel > 0) {
            ternary_quant_pack_kernel<false>
                <<<grid_for((numel + 15) / 16, 256), 256, 0, st>>>(w, numel, cols, scales, packed);
            RNN_TRY(check_launch(name));
        }
        finalize_row_scales_kernel<<<(unsigned)ceil_div(rows, 256), 256, 0, st>>>(scales, rows);
        return check_launch(name);
    }
    row_abs_sum_kernel<false><<<rblocks, 64, 0, st>>>(w, rows, cols, scales);
    RNN_TRY(check_launch(name));
    absmean_gamma_kernel<<<1, 256, 0, st>>>(scales, rows, numel);
    RNN_TRY(check_launch(name));
    if (numel > 0) {
        ternary_quant_pack_kernel<true>
            <<<grid_for((numel + 15) / 16, 256), 256, 0, st>>>(w, numel, cols, scales, packed);
        RNN_TRY(check_launch(name));
    }
    return RNN_OK;
}

extern "C" int rnn_ternary_dequantize(const uint32_t *packed, int64_t numel, const float *scales,
                                      int64_t n_scales, int64_t cols, float *w, void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_ternary_dequantize";
    RNN_REQUIRE(numel >= 0 && cols > 0 && n_scales > 0, "%s: bad size", name);
    if (numel == 0) return RNN_OK;
    RNN_REQUIRE(packed && scales && w, "%s: null pointer", name);
    ternary_dequant_kernel<<<grid_for(numel, 256), 256, 0, as_stream(stream)>>>(
        packed, numel, scales, n_scales, cols, w);
    return check_launch(name);
}

extern "C" int rnn_ternary_linear_forward(const float *x, int64_t batch, int64_t in_f,
                                          const uint32_t *packed, const float *scales,
                                          int64_t out_f, const float *bias, float *y,
                                          void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_ternary_linear_forward";
    RNN_REQUIRE(batch >= 0 && in_f >= 0 && out_f >= 0, "%s: negative size", name);
    RNN_REQUIRE(batch <= 65535, "%s: batch > 65535 unsupported", name);
    if (batch == 0 || out_f == 0) return RNN_OK;
    RNN_REQUIRE(scales && y && (in_f == 0 || (x && packed)), "%s: null pointer", name);
    dim3 grid((unsigned)ceil_div(out_f, 256), (unsigned)batch);
    hipStream_t st = as_stream(stream);
    if (bias)
        ternary_linear_ref_kernel<true><<<grid, 256, 0, st>>>(x, in_f, packed, scales, out_f, bias, y);
    else
        ternary_linear_ref_kernel<false><<<grid, 256, 0, st>>>(x, in_f, packed, scales, out_f,
                                                               nullptr, y);
    return check_launch(name);
}
