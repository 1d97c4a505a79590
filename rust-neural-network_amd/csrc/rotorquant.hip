// rotorquant.hip -- RotorQuant (block Cl(3,0) rotor decorrelation + per-group
// symmetric scalar quantization) for KV-cache rows, streaming and HBM-bound.
//
// Each persistent workgroup first builds the 3x3 rotation matrix of every
// group from its rotor with the reference's sandwich expressions
// (src/quant.rs:70-113) into LDS, then streams tiles of whole vectors:
// 16-byte global loads -> LDS tile -> one thread per (vector, 3-group) does
// rotate / max / divide / round / clamp / rescale / inverse-rotate in
// registers -> LDS -> 16-byte global stores.
#include <algorithm>

#include "common.hpp"
#include "numerics.hpp"

namespace rnn {

constexpr int kRqThreads = 256;
constexpr int kRqTileFloats = 8192;  // 32 KiB of LDS per tile
constexpr int kRqMaxGroups = 896;    // dim <= 2688: 32 KiB tile + 31.5 KiB rotations <= 64 KiB

// rotor * x on a multivector [1,e1,e2,e3,e12,e13,e23,e123] (src/quant.rs:70-81)
__device__ __forceinline__ void rotor_apply(const float *x, float s, float p12, float p13,
                                            float p23, float *o) {
    o[0] = s * x[0] - p12 * x[4] - p13 * x[5] - p23 * x[6];
    o[1] = s * x[1] + p12 * x[2] + p13 * x[3] + p23 * x[7];
    o[2] = s * x[2] - p12 * x[1] + p23 * x[3] - p13 * x[7];
    o[3] = s * x[3] - p13 * x[1] - p23 * x[2] + p12 * x[7];
    o[4] = s * x[4] + p12 * x[0];
    o[5] = s * x[5] + p13 * x[0];
    o[6] = s * x[6] + p23 * x[0];
    o[7] = s * x[7] - p23 * x[1] + p13 * x[2] - p12 * x[3];
}

// Rotor::rotation_matrix: column j is the vector part of R e_j R~
// (src/quant.rs:84-89, :101-113). rot is row-major 3x3.
__device__ __forceinline__ void rotation_matrix(const float *r, float *rot) {
    for (int j = 0; j < 3; ++j) {
        float e[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        e[1 + j] = 1.0f;
        float t[8], o[8];
        rotor_apply(e, r[0], r[1], r[2], r[3], t);
        rotor_apply(t, r[0], -r[1], -r[2], -r[3], o);
        rot[0 * 3 + j] = o[1];
        rot[1 * 3 + j] = o[2];
        rot[2 * 3 + j] = o[3];
    }
}

__global__ void rotation_matrices_kernel(const float *__restrict__ rotors, int64_t n,
                                         float *__restrict__ rot9) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) {
        float m[9];
        rotation_matrix(rotors + 4 * i, m);
        for (int e = 0; e < 9; ++e) rot9[9 * i + e] = m[e];
    }
}

// quantize_vec for one group (src/quant.rs:178-205). Returns false for a
// group skipped by the max_abs < 1e-12 rule (its values stay untouched).
__device__ __forceinline__ bool rq_group(const float *R, float qmax, float &x0, float &x1,
                                         float &x2, float &scale, float q[3]) {
    float rv0 = R[0] * x0 + R[1] * x1 + R[2] * x2;
    float rv1 = R[3] * x0 + R[4] * x1 + R[5] * x2;
    float rv2 = R[6] * x0 + R[7] * x1 + R[8] * x2;
    float m = 0.0f;
    m = fmaxf(m, fabsf(rv0));
    m = fmaxf(m, fabsf(rv1));
    m = fmaxf(m, fabsf(rv2));
    if (m < 1e-12f) return false;
    scale = m / qmax;
    q[0] = clamp_rs(roundf(rv0 / scale), -qmax, qmax);
    q[1] = clamp_rs(roundf(rv1 / scale), -qmax, qmax);
    q[2] = clamp_rs(roundf(rv2 / scale), -qmax, qmax);
    rv0 = q[0] * scale;
    rv1 = q[1] * scale;
    rv2 = q[2] * scale;
    x0 = R[0] * rv0 + R[3] * rv1 + R[6] * rv2;
    x1 = R[1] * rv0 + R[4] * rv1 + R[7] * rv2;
    x2 = R[2] * rv0 + R[5] * rv1 + R[8] * rv2;
    return true;
}

template <bool VEC4>
__global__ __launch_bounds__(kRqThreads) void rotorquant_kernel(
    const float *__restrict__ x, int64_t rows, int dim, int ng, int vpt, float qmax,
    uint32_t ng_magic, const float *__restrict__ rotors, float *__restrict__ y,
    int8_t *__restrict__ codes, float *__restrict__ scales) {
    __shared__ __attribute__((aligned(16))) float tile[kRqTileFloats];
    extern __shared__ float rot[];  // ng * 9 floats (dynamic)
    const int tid = threadIdx.x;
    for (int g = tid; g < ng; g += kRqThreads) rotation_matrix(rotors + 4 * g, rot + 9 * g);
    const int padded = ng * 3;
    const int64_t ntiles = (rows + vpt - 1) / vpt;
    __syncthreads();
    for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
        const int64_t r0 = t * vpt;
        const int nv = (int)std::min<int64_t>(vpt, rows - r0);
        const int nf = nv * dim;
        const float *src = x + r0 * dim;
        if (VEC4) {
            for (int i = tid; i < nf / 4; i += kRqThreads)
                reinterpret_cast<float4 *>(tile)[i] = reinterpret_cast<const float4 *>(src)[i];
        } else {
            for (int i = tid; i < nf; i += kRqThreads) tile[i] = src[i];
        }
        __syncthreads();
        const int work = nv * ng;
        for (int f = tid; f < work; f += kRqThreads) {
            // ng == 1 has no 32-bit magic (2^32 overflows): v = f directly
            int v = ng == 1 ? f : (int)__umulhi((uint32_t)f, ng_magic);
            int g = f - v * ng;
            if (g >= ng) { g -= ng; ++v; }
            if (g < 0) { g += ng; --v; }
            const int e = 3 * g;
            float *p = tile + v * dim + e;
            float x0 = p[0];
            float x1 = e + 1 < dim ? p[1] : 0.0f;
            float x2 = e + 2 < dim ? p[2] : 0.0f;
            float scale = 0.0f, q[3] = {0.0f, 0.0f, 0.0f};
            const bool done = rq_group(rot + 9 * g, qmax, x0, x1, x2, scale, q);
            const int64_t row = r0 + v;
            if (codes) {
                int8_t *c = codes + row * padded + e;
                c[0] = to_i8_rs(q[0]);
                c[1] = to_i8_rs(q[1]);
                c[2] = to_i8_rs(q[2]);
            }
            if (scales) scales[row * ng + g] = scale;
            if (y && done) {
                p[0] = x0;
                if (e + 1 < dim) p[1] = x1;
                if (e + 2 < dim) p[2] = x2;
            }
        }
        __syncthreads();
        if (y) {
            float *dst = y + r0 * dim;
            if (VEC4) {
                for (int i = tid; i < nf / 4; i += kRqThreads)
                    reinterpret_cast<float4 *>(dst)[i] = reinterpret_cast<const float4 *>(tile)[i];
            } else {
                for (int i = tid; i < nf; i += kRqThreads) dst[i] = tile[i];
            }
        }
        __syncthreads();
    }
}

// Reconstruction from codes: one thread per (row, group).
__global__ __launch_bounds__(kRqThreads) void rotorquant_dequant_kernel(
    const int8_t *__restrict__ codes, const float *__restrict__ scales, int64_t rows, int dim,
    int ng, const float *__restrict__ rotors, float *__restrict__ y) {
    extern __shared__ float rot[];  // ng * 9 floats (dynamic)
    for (int g = threadIdx.x; g < ng; g += kRqThreads) rotation_matrix(rotors + 4 * g, rot + 9 * g);
    __syncthreads();
    const int padded = 3 * ng;
    const int64_t work = rows * ng;
    for (int64_t f = blockIdx.x * (int64_t)kRqThreads + threadIdx.x; f < work;
         f += (int64_t)gridDim.x * kRqThreads) {
        const int64_t row = f / ng;
        const int g = (int)(f - row * ng);
        const float *R = rot + 9 * g;
        const float s = scales[f];
        const int8_t *c = codes + row * padded + 3 * g;
        const float rv0 = (float)c[0] * s, rv1 = (float)c[1] * s, rv2 = (float)c[2] * s;
        float *o = y + row * dim + 3 * g;
        o[0] = R[0] * rv0 + R[3] * rv1 + R[6] * rv2;
        if (3 * g + 1 < dim) o[1] = R[1] * rv0 + R[4] * rv1 + R[7] * rv2;
        if (3 * g + 2 < dim) o[2] = R[2] * rv0 + R[5] * rv1 + R[8] * rv2;
    }
}

}  // namespace rnn

using namespace rnn;

extern "C" int rnn_rotor_rotation_matrices(const float *rotors, int64_t n, float *rot9,
                                           void *stream) {
    RNN_REQUIRE(n >= 0, "rnn_rotor_rotation_matrices: negative n");
    if (n == 0) return RNN_OK;
    RNN_REQUIRE(rotors && rot9, "rnn_rotor_rotation_matrices: null pointer");
    rotation_matrices_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, as_stream(stream)>>>(rotors, n,
                                                                                        rot9);
    return check_launch("rnn_rotor_rotation_matrices");
}

extern "C" int rnn_rotorquant_quantize(const float *x, int64_t rows, int64_t dim, int bits,
                                       const float *rotors, float *y, int8_t *codes,
                                       float *scales, void *stream) {
    const char *name = "rnn_rotorquant_quantize";
    RNN_REQUIRE(rows >= 0, "%s: negative rows", name);
    RNN_REQUIRE(dim > 0, "%s: dim must be positive (RotorQuant dim %lld)", name, (long long)dim);
    RNN_REQUIRE(bits >= 2, "%s: RotorQuant needs at least 2 bits", name);
    RNN_REQUIRE(bits <= (codes ? 8 : 32), "%s: bits %d out of range", name, bits);
    const int64_t ng = (dim + 2) / 3;
    if (ng > kRqMaxGroups || dim > kRqTileFloats)
        return set_error(RNN_ERR_UNSUPPORTED, "%s: dim %lld > %d unsupported", name,
                         (long long)dim, 3 * kRqMaxGroups);
    if (rows == 0) return RNN_OK;
    RNN_REQUIRE(x && rotors, "%s: null input", name);
    RNN_REQUIRE(y || codes || scales, "%s: no output requested", name);
    RNN_REQUIRE(rows * ng < 0x7fffffffLL * 16, "%s: too many rows", name);
    const int vpt = std::max<int>(1, kRqTileFloats / (int)dim);
    const float qmax = (float)((1u << (bits - 1)) - 1u);
    const uint32_t magic = ng > 1 ? (uint32_t)((0x100000000ULL + ng - 1) / ng) : 0u;
    const int64_t ntiles = ceil_div(rows, vpt);
    const unsigned grid = (unsigned)std::min<int64_t>(ntiles, 4 * device_cu_count());
    const bool vec = dim % 4 == 0 && ((uintptr_t)x % 16) == 0 && (!y || ((uintptr_t)y % 16) == 0);
    hipStream_t st = as_stream(stream);
    const size_t smem = (size_t)ng * 9 * sizeof(float);
    if (vec)
        rotorquant_kernel<true><<<grid, kRqThreads, smem, st>>>(x, rows, (int)dim, (int)ng, vpt, qmax,
                                                             magic, rotors, y, codes, scales);
    else
        rotorquant_kernel<false><<<grid, kRqThreads, smem, st>>>(x, rows, (int)dim, (int)ng, vpt, qmax,
                                                              magic, rotors, y, codes, scales);
    return check_launch(name);
}

extern "C" int rnn_rotorquant_dequantize(const int8_t *codes, const float *scales, int64_t rows,
                                         int64_t dim, const float *rotors, float *y,
                                         void *stream) {
    const char *name = "rnn_rotorquant_dequantize";
    RNN_REQUIRE(rows >= 0 && dim > 0, "%s: bad size", name);
    const int64_t ng = (dim + 2) / 3;
    if (ng > kRqMaxGroups)
        return set_error(RNN_ERR_UNSUPPORTED, "%s: dim %lld unsupported", name, (long long)dim);
    if (rows == 0) return RNN_OK;
    RNN_REQUIRE(codes && scales && rotors && y, "%s: null pointer", name);
    const int64_t work = rows * ng;
    const unsigned grid =
        (unsigned)std::min<int64_t>(ceil_div(work, kRqThreads), 8 * device_cu_count());
    rotorquant_dequant_kernel<<<grid, kRqThreads, (size_t)ng * 9 * sizeof(float),
                                as_stream(stream)>>>(codes, scales, rows,
                                                                          (int)dim, (int)ng, rotors, y);
    return check_launch(name);
}
