// quant.hip -- per-row symmetric int8 quantization (weights and activations),
// int8 dequantization, and the reference-semantics Int8Linear::forward /
// Int8Weights::matmul_f32 kernels (VALU; parity path, not the perf path).
#include "common.hpp"
#include "numerics.hpp"

namespace rnn {

constexpr int kQuantBlock = 256;

// One workgroup per row. Pass 1: max|x| (max is order-independent, so the
// tree reduction equals the reference's sequential fold, src/int8.rs:36).
// Pass 2: q = (x/scale).round().clamp(-128,127) (src/int8.rs:42), re-reading
// the row from L2. Rows are 16-byte vectorised when cols % 4 == 0.
template <bool VEC4>
__global__ __launch_bounds__(kQuantBlock) void quant_rows_kernel(
    const float *__restrict__ x, int64_t cols, int8_t *__restrict__ q,
    float *__restrict__ scale) {
    const int64_t r = blockIdx.x;
    const float *row = x + r * cols;
    int8_t *qrow = q + r * cols;
    float m = 0.0f;
    if (VEC4) {
        const float4 *row4 = reinterpret_cast<const float4 *>(row);
        for (int64_t j = threadIdx.x; j < cols / 4; j += kQuantBlock) {
            float4 v = row4[j];
            m = fmaxf(m, fabsf(v.x));
            m = fmaxf(m, fabsf(v.y));
            m = fmaxf(m, fabsf(v.z));
            m = fmaxf(m, fabsf(v.w));
        }
    } else {
        for (int64_t j = threadIdx.x; j < cols; j += kQuantBlock) m = fmaxf(m, fabsf(row[j]));
    }
    __shared__ float red[kQuantBlock / 64];
    m = block_max<kQuantBlock>(m, red);
    const float s = m > 0.0f ? m / 127.0f : 1.0f;
    if (threadIdx.x == 0) scale[r] = s;
    if (VEC4) {
        const float4 *row4 = reinterpret_cast<const float4 *>(row);
        uint32_t *q4 = reinterpret_cast<uint32_t *>(qrow);
        for (int64_t j = threadIdx.x; j < cols / 4; j += kQuantBlock) {
            float4 v = row4[j];
            uint32_t b0 = (uint8_t)quant_i8(v.x, s), b1 = (uint8_t)quant_i8(v.y, s),
                     b2 = (uint8_t)quant_i8(v.z, s), b3 = (uint8_t)quant_i8(v.w, s);
            q4[j] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
        }
    } else {
        for (int64_t j = threadIdx.x; j < cols; j += kQuantBlock) qrow[j] = quant_i8(row[j], s);
    }
}

// The same rule with the row held in registers (cols % 4 == 0, 16-byte
// aligned x, cols <= 1024 R): each thread loads its R float4 at once, so a
// row is one round trip instead of a strided loop and a second pass over L2,
// and the quotient is a multiply by 1/scale (round_quotient: rint of it
// wherever that provably equals the rounded IEEE quotient, the division
// itself near a half-integer). The scale itself is the IEEE m / 127.
template <int R>
__global__ __launch_bounds__(kQuantBlock) void quant_rows_reg_kernel(
    const float *__restrict__ x, int64_t cols, int8_t *__restrict__ q,
    float *__restrict__ scale) {
    const int64_t r = blockIdx.x;
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 *row4 = reinterpret_cast<const f32x4 *>(x + r * cols);
    uint32_t *q4 = reinterpret_cast<uint32_t *>(q + r * cols);
    const int64_t n4 = cols / 4;
    f32x4 v[R];
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int64_t j = threadIdx.x + (int64_t)u * kQuantBlock;
        v[u] = j < n4 ? __builtin_nontemporal_load(row4 + j) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float m = 0.0f;
#pragma unroll
    for (int u = 0; u < R; ++u) {
        m = fmaxf(m, fabsf(v[u].x));
        m = fmaxf(m, fabsf(v[u].y));
        m = fmaxf(m, fabsf(v[u].z));
        m = fmaxf(m, fabsf(v[u].w));
    }
    __shared__ float red[kQuantBlock / 64];
    m = block_max<kQuantBlock>(m, red);
    const float s = m > 0.0f ? m / 127.0f : 1.0f;
    const float inv = __builtin_amdgcn_rcpf(s);
    if (threadIdx.x == 0) scale[r] = s;
    auto code = [&](float e) -> uint32_t {
        return (uint8_t)to_i8_rs(clamp_rs(round_quotient(e, s, inv), -128.0f, 127.0f));
    };
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int64_t j = threadIdx.x + (int64_t)u * kQuantBlock;
        if (j < n4)
            q4[j] = code(v[u].x) | (code(v[u].y) << 8) | (code(v[u].z) << 16) | (code(v[u].w) << 24);
    }
}

__global__ void int8_dequant_kernel(const int8_t *__restrict__ q, const float *__restrict__ s,
                                    int64_t rows, int64_t cols, float *__restrict__ w) {
    const int64_t total = rows * cols;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x)
        w[i] = (float)q[i] * s[i / cols];
}

// Reference Int8Linear::forward / matmul_f32: one thread per (b, o); the
// activation is re-quantized with the weight's channel scale for every MAC
// (src/int8.rs:152-158, :78-83). INV selects matmul_f32's x * (1/s) form.
template <bool INV, bool BIAS>
__global__ __launch_bounds__(256) void int8_linear_ref_kernel(
    const float *__restrict__ x, int64_t in_f, const int8_t *__restrict__ wq,
    const float *__restrict__ ws, int64_t out_f, const float *__restrict__ bias,
    float *__restrict__ y) {
    const int64_t b = blockIdx.y;
    const int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (o >= out_f) return;
    const float s = ws[o];
    const float *xr = x + b * in_f;
    const int8_t *wr = wq + o * in_f;
    uint32_t acc = 0;
    for (int64_t k = 0; k < in_f; ++k) {
        const float xv = xr[k];
        const float t = INV ? xv * (1.0f / s) : xv / s;
        acc += (uint32_t)((int32_t)quant_i8_from_ratio(t) * (int32_t)wr[k]);
    }
    float v = (float)(int32_t)acc * s * s;
    if (BIAS) v = v + bias[o];
    y[b * out_f + o] = v;
}

}  // namespace rnn

using namespace rnn;

extern "C" int rnn_quant_rows_i8(const float *x, int64_t rows, int64_t cols, int8_t *q,
                                 float *scale, void *stream) {
    RNN_ENTRY();
    RNN_REQUIRE(rows >= 0 && cols >= 0, "rnn_quant_rows_i8: negative size");
    RNN_REQUIRE(rows <= 0x7fffffff, "rnn_quant_rows_i8: rows too large");
    if (rows == 0) return RNN_OK;
    RNN_REQUIRE(scale != nullptr, "rnn_quant_rows_i8: null scale");
    RNN_REQUIRE(cols == 0 || (x != nullptr && q != nullptr), "rnn_quant_rows_i8: null pointer");
    const bool vec = cols % 4 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)q % 4) == 0;
    hipStream_t st = as_stream(stream);
    const unsigned g = (unsigned)rows;
    if (vec && cols <= 1024)
        quant_rows_reg_kernel<1><<<g, kQuantBlock, 0, st>>>(x, cols, q, scale);
    else if (vec && cols <= 2048)
        quant_rows_reg_kernel<2><<<g, kQuantBlock, 0, st>>>(x, cols, q, scale);
    else if (vec && cols <= 4096)
        quant_rows_reg_kernel<4><<<g, kQuantBlock, 0, st>>>(x, cols, q, scale);
    else if (vec && cols <= 8192)
        quant_rows_reg_kernel<8><<<g, kQuantBlock, 0, st>>>(x, cols, q, scale);
    else if (vec)
        quant_rows_kernel<true><<<(unsigned)rows, kQuantBlock, 0, as_stream(stream)>>>(x, cols, q, scale);
    else
        quant_rows_kernel<false><<<(unsigned)rows, kQuantBlock, 0, as_stream(stream)>>>(x, cols, q, scale);
    return check_launch("rnn_quant_rows_i8");
}

extern "C" int rnn_int8_dequantize(const int8_t *q, const float *scale, int64_t rows,
                                   int64_t cols, float *w, void *stream) {
    RNN_ENTRY();
    RNN_REQUIRE(rows >= 0 && cols >= 0, "rnn_int8_dequantize: negative size");
    if (rows == 0 || cols == 0) return RNN_OK;
    RNN_REQUIRE(q && scale && w, "rnn_int8_dequantize: null pointer");
    const int64_t total = rows * cols;
    const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), 8 * device_cu_count());
    int8_dequant_kernel<<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(q, scale, rows, cols, w);
    return check_launch("rnn_int8_dequantize");
}

static int launch_int8_ref(bool inv, const float *x, int64_t batch, int64_t in_f,
                           const int8_t *wq, const float *ws, int64_t out_f, const float *bias,
                           float *y, void *stream, const char *name) {
    RNN_REQUIRE(batch >= 0 && in_f >= 0 && out_f >= 0, "%s: negative size", name);
    RNN_REQUIRE(batch <= 65535, "%s: batch > 65535 unsupported", name);
    if (batch == 0 || out_f == 0) return RNN_OK;
    RNN_REQUIRE(ws && y && (in_f == 0 || (x && wq)), "%s: null pointer", name);
    dim3 grid((unsigned)ceil_div(out_f, 256), (unsigned)batch);
    hipStream_t st = as_stream(stream);
    if (inv)
        int8_linear_ref_kernel<true, false><<<grid, 256, 0, st>>>(x, in_f, wq, ws, out_f, nullptr, y);
    else if (bias)
        int8_linear_ref_kernel<false, true><<<grid, 256, 0, st>>>(x, in_f, wq, ws, out_f, bias, y);
    else
        int8_linear_ref_kernel<false, false><<<grid, 256, 0, st>>>(x, in_f, wq, ws, out_f, nullptr, y);
    return check_launch(name);
}

extern "C" int rnn_int8_matmul_f32(const int8_t *wq, const float *ws, int64_t out_f, int64_t in_f,
                                   const float *x, int64_t m, float *y, void *stream) {
    RNN_ENTRY();
    return launch_int8_ref(true, x, m, in_f, wq, ws, out_f, nullptr, y, stream,
                           "rnn_int8_matmul_f32");
}

extern "C" int rnn_int8_linear_forward(const float *x, int64_t batch, int64_t in_f,
                                       const int8_t *wq, const float *ws, int64_t out_f,
                                       const float *bias, float *y, void *stream) {
    RNN_ENTRY();
    return launch_int8_ref(false, x, batch, in_f, wq, ws, out_f, bias, y, stream,
                           "rnn_int8_linear_forward");
}
