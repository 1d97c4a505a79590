// qformat.hip -- QuantizedTensor (src/quantize.rs): quantize / dequantize of
// every QuantFormat, and QuantizedLinear::forward with the weights decoded on
// the fly.
//
// Storage follows QuantizedTensor::{data, scales, group_size} byte for byte:
// 8-bit codes one per byte, 4-bit codes packed per group (low nibble first),
// f16/bf16 as little-endian u16 pairs, f32 scales per group (GGUF: per block
// of min(group, 32)). Codes, scales and dequantized values are bit-exact with
// the reference; the linear forward sums in f32 in its own order.
#include "common.hpp"
#include "numerics.hpp"

namespace rnn {

// Code kinds of the fused GEMV: signed 4-bit, int8, f16, bf16, and 4-bit
// indices into a 16-entry table (NF4, E2M1).
enum QKind { KIND_I4 = 0, KIND_I8 = 1, KIND_F16 = 2, KIND_BF16 = 3, KIND_NF4 = 4, KIND_E2M1 = 5 };

__host__ __device__ constexpr bool kind4(int k) { return k == KIND_I4 || k == KIND_NF4 || k == KIND_E2M1; }

__host__ __device__ inline bool qf_is4(int f) {
    return f == RNN_QF_INT4 || f == RNN_QF_NF4 || f == RNN_QF_NVFP4 || f == RNN_QF_GGUF_Q4 ||
           f == RNN_QF_GGUF_Q4K;
}
__host__ __device__ inline bool qf_is_gguf(int f) {
    return f == RNN_QF_GGUF_Q4 || f == RNN_QF_GGUF_Q4K || f == RNN_QF_GGUF_Q8;
}

// src/quantize.rs:96-114 and :138-144 (index 8 of the E2M1 table is -0.0).
__constant__ float kNF4[16] = {-1.0f, -0.6961928f, -0.52507305f, -0.3949175f,
                               -0.28444138f, -0.18477343f, -0.091050036f, 0.0f,
                               0.0795803f, 0.1609302f, 0.2461123f, 0.33791524f,
                               0.44070983f, 0.562617f, 0.72295684f, 1.0f};
__constant__ float kE2M1[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

// Scale of a group from its max|x| (src/quantize.rs:307, :345, :408, :466,
// :174-176, :567).
__device__ inline float group_scale(int f, float max_abs) {
    switch (f) {
    case RNN_QF_INT8: case RNN_QF_GGUF_Q8: return max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
    case RNN_QF_INT4: return max_abs > 0.0f ? max_abs / 7.0f : 1.0f;
    case RNN_QF_NF4: return max_abs > 0.0f ? max_abs : 1.0f;
    case RNN_QF_NVFP4: return max_abs > 0.0f ? max_abs / 6.0f : 1.0f;
    default: {
        const float s = max_abs / -8.0f;  // Q4_0: signed range [-8, 7]
        return s == 0.0f ? 1.0f : s;
    }
    }
}

// Code of one value (src/quantize.rs:117-129, :146-161, :181-186, :350-353).
__device__ inline uint8_t code4(int f, float v, float s) {
    const float t = v / s;
    if (f == RNN_QF_NF4) {
        uint8_t best = 0;
        float bd = INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float d = fabsf(kNF4[i] - t);
            if (d < bd) { bd = d; best = (uint8_t)i; }
        }
        return best;
    }
    if (f == RNN_QF_NVFP4) {
        const float a = fabsf(t);
        uint8_t best = 0;
        float bd = INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float d = fabsf(kE2M1[i] - a);
            if (d < bd) { bd = d; best = (uint8_t)i; }
        }
        return (uint8_t)((t < 0.0f ? 8 : 0) | best);
    }
    return (uint8_t)(to_i8_rs(clamp_rs(roundf(t), -8.0f, 7.0f)) & 0xF);
}

// src/quantize.rs:639-666 (truncating f32 -> f16).
__device__ inline uint16_t f32_to_f16_rs(float f) {
    const uint32_t bits = __float_as_uint(f);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
    const uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 0xFF) return sign | 0x7C00u | (mant != 0 ? 0x200u : 0u);
    const int32_t ne = exp - 127 + 15;
    if (ne >= 31) return sign | 0x7C00u;
    if (ne <= 0) {
        if (14 - ne >= 24) return sign;
        return sign | (uint16_t)((mant | 0x800000u) >> (uint32_t)(14 - ne));
    }
    return sign | (uint16_t)((uint32_t)ne << 10) | (uint16_t)(mant >> 13);
}

// src/quantize.rs:668-695 with release integer semantics: a subnormal with
// s leading zeros below bit 10 gets exponent 113 - s.
__device__ inline float f16_to_f32_rs(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t mant = h & 0x3FFu;
    uint32_t v;
    if (exp == 0) {
        if (mant == 0) {
            v = sign;
        } else {
            const int s = __clz(mant) - 21;  // shifts until bit 10 is set
            v = sign | ((uint32_t)(113 - s) << 23) | (((mant << s) & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        v = sign | 0x7F800000u | (mant << 13);
    } else {
        v = sign | ((exp + 112) << 23) | (mant << 13);
    }
    return __uint_as_float(v);
}

// src/quantize.rs:697-703 (wrapping add, as release Rust).
__device__ inline uint16_t f32_to_bf16_rs(float f) {
    const uint32_t b = __float_as_uint(f);
    return (uint16_t)((b + ((b >> 16) & 1u) + 0x7FFFu) >> 16);
}

// ------------------------------------------------------------ quantize

__global__ void qt_half_quant_kernel(int f, const float *__restrict__ x, int64_t n,
                                     uint16_t *__restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = f == RNN_QF_FP16 ? f32_to_f16_rs(x[i]) : f32_to_bf16_rs(x[i]);
}

// Stores the codes of elements [start, end) of one group with scale s: one
// byte per element, or one byte per pair for 4-bit formats at byte offset
// `off` (each group packed on its own, src/quantize.rs:355-365).
__device__ inline void emit_codes(int f, const float *__restrict__ x, int64_t start, int64_t end,
                                  float s, int64_t off, uint8_t *__restrict__ data, int64_t t0,
                                  int64_t stride) {
    if (!qf_is4(f)) {
        for (int64_t i = start + t0; i < end; i += stride) data[i] = (uint8_t)quant_i8(x[i], s);
        return;
    }
    const int64_t nb = (end - start + 1) / 2;
    for (int64_t b = t0; b < nb; b += stride) {
        const int64_t i = start + 2 * b;
        const uint8_t lo = code4(f, x[i], s);
        const uint8_t hi = i + 1 < end ? code4(f, x[i + 1], s) : (uint8_t)0;
        data[off + b] = (uint8_t)(lo | (hi << 4));
    }
}

// Groups of up to kSmallGroup elements: one wave per group finds max|x|
// (order-free, equal to the reference's sequential fold), then writes the
// scale and the codes.
constexpr int64_t kSmallGroup = 8192;

__global__ __launch_bounds__(256) void qt_quant_group_kernel(
    int f, const float *__restrict__ x, int64_t n, int64_t g, int64_t ng,
    uint8_t *__restrict__ data, float *__restrict__ scales) {
    const int64_t gi = blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if (gi >= ng) return;
    const int64_t start = gi * g, end = start + g < n ? start + g : n;
    float m = 0.0f;
    for (int64_t i = start + lane; i < end; i += 64) m = fmaxf(m, fabsf(x[i]));
    m = wave_max(m);
    const float s = group_scale(f, m);
    if (lane == 0) scales[gi] = s;
    emit_codes(f, x, start, end, s, gi * ((g + 1) / 2), data, lane, 64);
}

// Larger groups: max|x| per group through an atomic max on the bit patterns
// of non-negative floats (kept in `scales`, zeroed first), then codes, then
// max -> scale in place.
constexpr int64_t kChunk = 4096;

__global__ void qt_zero_kernel(uint32_t *__restrict__ p, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

__global__ __launch_bounds__(256) void qt_group_max_kernel(const float *__restrict__ x, int64_t n,
                                                           int64_t g, int64_t chunks_per_group,
                                                           uint32_t *__restrict__ maxbits) {
    const int64_t gi = blockIdx.x / chunks_per_group, c = blockIdx.x % chunks_per_group;
    const int64_t gend = gi * g + g < n ? gi * g + g : n;
    const int64_t start = gi * g + c * kChunk;
    const int64_t end = start + kChunk < gend ? start + kChunk : gend;
    float m = 0.0f;
    for (int64_t i = start + threadIdx.x; i < end; i += 256) m = fmaxf(m, fabsf(x[i]));
    __shared__ float red[4];
    m = block_max<256>(m, red);  // NaN inputs drop out here, as in f32::max
    if (threadIdx.x == 0 && start < end) atomicMax(maxbits + gi, __float_as_uint(m));
}

__global__ __launch_bounds__(256) void qt_big_codes_kernel(int f, const float *__restrict__ x,
                                                           int64_t n, int64_t g,
                                                           int64_t chunks_per_group,
                                                           const float *__restrict__ maxv,
                                                           uint8_t *__restrict__ data) {
    const int64_t gi = blockIdx.x / chunks_per_group, c = blockIdx.x % chunks_per_group;
    const int64_t gstart = gi * g, gend = gstart + g < n ? gstart + g : n;
    const int64_t start = gstart + c * kChunk;  // kChunk is even: pairs stay whole
    const int64_t end = start + kChunk < gend ? start + kChunk : gend;
    if (start >= end) return;
    const float s = group_scale(f, maxv[gi]);
    emit_codes(f, x, start, end, s, gi * ((g + 1) / 2) + c * (kChunk / 2), data, threadIdx.x, 256);
}

__global__ void qt_finish_scales_kernel(int f, float *__restrict__ scales, int64_t ng) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < ng;
         i += (int64_t)gridDim.x * blockDim.x)
        scales[i] = group_scale(f, scales[i]);
}

// ------------------------------------------------------------ dequantize

// One element per thread: src/quantize.rs:324-332, :377-396, :440-454,
// :498-512 (data[i/2], scales[min(i/group, ns-1)]), :538-554 (GGUF Q4_0 block
// offsets), :604-610, :627-632.
__global__ void qt_dequant_kernel(int f, const uint8_t *__restrict__ data,
                                  const float *__restrict__ scales, int64_t ns, int64_t g,
                                  int64_t n, float *__restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        float v;
        if (f == RNN_QF_FP16 || f == RNN_QF_BF16) {
            const uint32_t h = (uint32_t)data[2 * i] | ((uint32_t)data[2 * i + 1] << 8);
            v = f == RNN_QF_FP16 ? f16_to_f32_rs(h) : __uint_as_float(h << 16);
        } else if (f == RNN_QF_GGUF_Q4 || f == RNN_QF_GGUF_Q4K) {
            const int64_t b = i / g, j = i - b * g;
            const uint8_t byte = data[b * ((g + 1) / 2) + j / 2];
            const int nib = (j & 1) ? (byte >> 4) : (byte & 0xF);
            v = (float)((nib ^ 8) - 8) * scales[b];
        } else {
            const int64_t gi = i / g;
            const float s = scales[gi < ns - 1 ? gi : ns - 1];
            if (f == RNN_QF_INT8 || f == RNN_QF_GGUF_Q8) {
                v = (float)(int8_t)data[i] * s;
            } else {
                const uint8_t byte = data[i / 2];
                const int nib = (i & 1) ? (byte >> 4) : (byte & 0xF);
                if (f == RNN_QF_INT4) v = (float)((nib ^ 8) - 8) * s;
                else if (f == RNN_QF_NF4) v = kNF4[nib] * s;
                else v = kE2M1[nib] * s;
            }
        }
        out[i] = v;
    }
}

// Eight elements per thread, for n and the group multiples of 8 with the
// codes and out aligned to their vector width: one group index and one scale
// per eight elements (a shift for a power-of-two group), the codes in one 4-,
// 8- or 16-byte load, the values in two 16-byte stores, each value the
// one-element kernel's. For groups of whole bytes GGUF Q4_0's block offset
// b*(g/2) + j/2 is i/2, as for INT4.
template <int F, bool POW2>
__global__ __launch_bounds__(256) void qt_dequant8_kernel(const uint8_t *__restrict__ data,
                                                          const float *__restrict__ scales,
                                                          int64_t ns, int64_t g, int gshift,
                                                          int64_t n8, float *__restrict__ out) {
    constexpr bool TABLE = F == RNN_QF_NF4 || F == RNN_QF_NVFP4;
    __shared__ float lut[16];
    if (TABLE) {
        if (threadIdx.x < 16) lut[threadIdx.x] = F == RNN_QF_NF4 ? kNF4[threadIdx.x] : kE2M1[threadIdx.x];
        __syncthreads();
    }
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < n8;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = 8 * t;
        float v[8];
        if constexpr (F == RNN_QF_FP16 || F == RNN_QF_BF16) {
            const uint4 h = reinterpret_cast<const uint4 *>(data)[t];
            const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t u = (hw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
                v[e] = F == RNN_QF_FP16 ? f16_to_f32_rs(u) : __uint_as_float(u << 16);
            }
        } else {
            int64_t gi = POW2 ? (i >> gshift) : i / g;
            if (F != RNN_QF_GGUF_Q4 && F != RNN_QF_GGUF_Q4K) gi = gi < ns - 1 ? gi : ns - 1;
            const float sc = scales[gi];
            if constexpr (F == RNN_QF_INT8 || F == RNN_QF_GGUF_Q8) {
                const uint2 c = reinterpret_cast<const uint2 *>(data)[t];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    v[e] = (float)(int8_t)((e < 4 ? c.x : c.y) >> (8 * (e & 3))) * sc;
            } else {
                const uint32_t w = reinterpret_cast<const uint32_t *>(data)[t];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int nib = (int)((w >> (4 * e)) & 0xFu);
                    v[e] = TABLE ? lut[nib] * sc : (float)((nib ^ 8) - 8) * sc;
                }
            }
        }
        float4 *o = reinterpret_cast<float4 *>(out + i);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// ------------------------------------------------------------ fused GEMV

// QuantizedLinear::forward (src/quantize.rs:744-754) for few rows of x:
// y[m, o] = sum_k x[m, k] * W[o, k] + bias[o] with W decoded from its codes
// in registers.
//
// A workgroup of 4 waves owns 4R consecutive output rows, a wave R of them.
// K is walked in slices of 2048 elements. In a slice each lane takes NV
// 16-byte pieces of every row: piece j at byte j*1024 + 16*lane of the
// slice, so one load instruction reads 1 KiB of whole cache lines
// (non-temporal: each weight byte is read once). The slice of x (MT rows) is
// staged once per workgroup in a double-buffered LDS ring, and the next
// slice's weights are in flight while the current slice is computed. The EP
// products of a piece are summed first and scaled once by the group's scale
// (a piece never spans two groups: group % EP == 0). At the end the wave
// reduces its R*MT partial sums with a halving butterfly.
template <int KIND>
struct Fmt {
    static constexpr int NV = kind4(KIND) ? 1 : (KIND == KIND_I8 ? 2 : 4);  // pieces per lane
    static constexpr int EP = 32 / NV;               // elements per 16-byte piece
    static constexpr int PIECE_STRIDE = 1024 * EP / 16;  // elements between a lane's pieces
};

constexpr int kSlice = 2048;  // elements of K per slice (64 lanes x 32)
typedef float f4v __attribute__((ext_vector_type(4)));

// Decodes one 16-byte piece into EP floats. INT4 nibbles go through
// v_cvt_off_f32_i4, which reads the low 4 bits of its (byte-selected) source
// as a signed nibble q and returns exactly q/16; the caller multiplies the
// piece's sum by 16. NF4 and
// E2M1 nibbles index a 16-float table in LDS (the 16 entries sit in 16
// different banks, so a wave's lookups never conflict).
template <int KIND>
__device__ __attribute__((always_inline)) inline void decode_piece(const v4i raw, float *v,
                                                                   const float *lut) {
    if (KIND == KIND_NF4 || KIND == KIND_E2M1) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t w = (uint32_t)raw[d];
#pragma unroll
            for (int b = 0; b < 8; ++b) v[8 * d + b] = lut[(w >> (4 * b)) & 0xFu];
        }
    } else if (KIND == KIND_I4) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t w = (uint32_t)raw[d];
            uint32_t h = w >> 4;
            // keeps h a register of its own, so each conversion below reads
            // a byte of w or of h through a byte select instead of a
            // separate bit-field extract per high nibble
            asm("" : "+v"(h));
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                v[8 * d + 2 * b] = __builtin_amdgcn_cvt_off_f32_i4((int)((w >> (8 * b)) & 0xFFu));
                v[8 * d + 2 * b + 1] = __builtin_amdgcn_cvt_off_f32_i4((int)((h >> (8 * b)) & 0xFFu));
            }
        }
    } else if (KIND == KIND_I8) {
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int b = 0; b < 4; ++b) v[4 * d + b] = (float)(int8_t)((uint32_t)raw[d] >> (8 * b));
    } else if (KIND == KIND_F16) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t w = (uint32_t)raw[d];
            v[2 * d] = (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xFFFFu));
            v[2 * d + 1] = (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
        }
    } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t w = (uint32_t)raw[d];
            v[2 * d] = __uint_as_float(w << 16);
            v[2 * d + 1] = __uint_as_float(w & 0xFFFF0000u);
        }
    }
}

// Register state of one slice: the pieces of R rows and their scales.
template <int KIND, int R>
struct SliceRegs {
    v4i raw[R][Fmt<KIND>::NV];
    float sc[R][Fmt<KIND>::NV];
};

// Group index of element e of a row: rows hold whole groups (K % g == 0,
// gbase = row * (K / g), per-piece term e / g) or groups hold whole rows
// (g % K == 0, gbase = row / (g / K), per-piece term 0). Both avoid a 64-bit
// division per load.
template <int KIND, int R, bool SCALED>
__device__ __attribute__((always_inline)) inline void load_slice(SliceRegs<KIND, R> &s, const uint8_t *__restrict__ data,
                                  const float *__restrict__ scales, int64_t ns,
                                  const int64_t (&gbase)[R], uint32_t g, bool rows_hold_groups,
                                  int64_t K, int64_t N, int64_t r0, int64_t kb, int lane) {
    using F = Fmt<KIND>;
#pragma unroll
    for (int j = 0; j < F::NV; ++j) {
        int64_t e = kb + j * F::PIECE_STRIDE + lane * F::EP;
        e = e < K ? e : kb;  // pieces past K (last slice) re-read a valid one
        const uint32_t ge = SCALED && rows_hold_groups ? (uint32_t)e / g : 0u;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t row = r0 + r < N ? r0 + r : N - 1;
            const int64_t flat = row * K + e;
            s.raw[r][j] = __builtin_nontemporal_load(
                reinterpret_cast<const v4i *>(data + flat * 16 / F::EP));
            if (SCALED) {
                const int64_t gi = gbase[r] + ge;
                s.sc[r][j] = scales[gi < ns - 1 ? gi : ns - 1];
            }
        }
    }
}

// LDS layout of an x slice: the EP floats that lane l reads for piece j
// start at j * PIECE_STRIDE + l * EP, and their float4 number q is stored at
// slot q ^ swz(l), which spreads the lanes of one LDS pass over all banks
// (lane strides of 128, 64 or 32 bytes would otherwise collide 8, 4 or 2
// ways).
template <int KIND>
__device__ __attribute__((always_inline)) inline int x_swz(int lane) {
    constexpr int EP = Fmt<KIND>::EP;
    return (lane * EP / 64) & (EP / 4 - 1);
}

// Slot in the swizzled slice of the float4 holding slice elements [4p, 4p+4).
template <int KIND>
__device__ __attribute__((always_inline)) inline int x_slot(int p) {
    using F = Fmt<KIND>;
    const int o = 4 * p;
    const int j = o / F::PIECE_STRIDE, w = o % F::PIECE_STRIDE;
    const int lane = w / F::EP, q = (w % F::EP) / 4;
    return j * F::PIECE_STRIDE + lane * F::EP + 4 * (q ^ x_swz<KIND>(lane));
}

// x[:, kb .. kb + 2048) of MT rows for an LDS buffer, 16 bytes per thread
// per row of x.
template <int MT>
__device__ __attribute__((always_inline)) inline void stage_x_load(f4v (&t)[MT], const float *__restrict__ x, int mrows,
                                    int64_t K, int64_t kb) {
    const int64_t e = kb + 4 * (int64_t)threadIdx.x;  // 256 threads x 4 = 1024 ... x2 below
    // Past K the load re-reads a valid address (no branch around it); those
    // values reach only pieces whose sums compute_slice discards.
    const int64_t ec = e < K ? e : 0;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int mr = m < mrows ? m : 0;
        t[m] = *reinterpret_cast<const f4v *>(x + (int64_t)mr * K + ec);
    }
}

template <int KIND, int MT, int R, bool SCALED>
__device__ __attribute__((always_inline)) inline void compute_slice(const SliceRegs<KIND, R> &s, const float *__restrict__ xs,
                                     int64_t K, int64_t kb, int lane, float (&acc)[R][MT],
                                     const float *lut) {
    using F = Fmt<KIND>;
#pragma unroll
    for (int j = 0; j < F::NV; ++j) {
        const int off = j * F::PIECE_STRIDE + lane * F::EP;
        const bool act = kb + off < K;
        float xr[MT][F::EP];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int q = 0; q < F::EP / 4; ++q) {
                const f4v t = *reinterpret_cast<const f4v *>(
                    xs + m * kSlice + off + 4 * (q ^ x_swz<KIND>(lane)));
                xr[m][4 * q] = t.x, xr[m][4 * q + 1] = t.y, xr[m][4 * q + 2] = t.z,
                xr[m][4 * q + 3] = t.w;
            }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // one row at a time: without the barrier the scheduler decodes
            // every row up front and the values of all rows stay live
            __builtin_amdgcn_sched_barrier(0);
            float v[F::EP];
            decode_piece<KIND>(s.raw[r][j], v, lut);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                float p = xr[m][0] * v[0];
#pragma unroll
                for (int e = 1; e < F::EP; ++e) p = __builtin_fmaf(xr[m][e], v[e], p);
                if (KIND == KIND_I4) p = p * 16.0f;  // the codes were read as q/16
                p = act ? p : 0.0f;
                acc[r][m] = SCALED ? __builtin_fmaf(s.sc[r][j], p, acc[r][m]) : acc[r][m] + p;
            }
        }
    }
}

// SFIX = 1 or 2: K takes exactly that many slices and the body is straight
// line; 0: any K, slices walked two at a time in a loop.
template <int KIND, int MT, int R, bool SCALED, bool BIAS, int SFIX>
__global__ __launch_bounds__(256) void qt_gemv_kernel(
    const float *__restrict__ x, int mrows, int64_t K, const uint8_t *__restrict__ data,
    const float *__restrict__ scales, int64_t ns, uint32_t g, uint32_t kg, uint32_t rpg, int64_t N,
    const float *__restrict__ bias, float *__restrict__ y) {
    // g: the group size; kg = K / g when rows hold whole groups, else 0 and
    // rpg = g / K rows per group (both computed on the host)
    constexpr int V = R * MT;
    static_assert((V & (V - 1)) == 0 && V <= 64, "R*MT must be a power of two <= 64");
    __shared__ __attribute__((aligned(16))) float xs[2][MT * kSlice];
    __shared__ float lut[16];  // NF4 / E2M1 values (src/quantize.rs:96-114, :138-144)
    if ((KIND == KIND_NF4 || KIND == KIND_E2M1) && threadIdx.x < 16)
        lut[threadIdx.x] = KIND == KIND_NF4 ? kNF4[threadIdx.x] : kE2M1[threadIdx.x];
    // (published by the barrier after the first x slice is staged)
    const int lane = threadIdx.x % 64;
    const int64_t r0 = (blockIdx.x * 4 + threadIdx.x / 64) * (int64_t)R;  // rows past N: clamped
    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

    const int64_t S = (K + kSlice - 1) / kSlice;
    const int slot0 = x_slot<KIND>(threadIdx.x), slot1 = x_slot<KIND>(threadIdx.x + 256);
    const bool rows_hold_groups = kg != 0;
    int64_t gbase[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = (uint32_t)(r0 + r < N ? r0 + r : N - 1);
        gbase[r] = !SCALED ? 0 : (rows_hold_groups ? (int64_t)row * kg : (int64_t)(row / rpg));
    }
    // Two slices in flight: slices s and s+1 sit in register sets A and B
    // and LDS buffers 0 and 1. While A is computed, the loads of slice s+2
    // go out; while B is computed, those of slice s+3. x is always issued
    // before weights, so waiting for x (to write it to LDS) never waits for
    // weight loads: the memory counter completes in issue order.
    SliceRegs<KIND, R> A, B;
    f4v tx[2][2][MT];
    auto ld = [&](SliceRegs<KIND, R> &w, int64_t kb) {
        load_slice<KIND, R, SCALED>(w, data, scales, ns, gbase, g, rows_hold_groups, K, N, r0, kb,
                                    lane);
    };
    auto stx = [&](int b, f4v (&t)[2][MT]) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            *reinterpret_cast<f4v *>(&xs[b][m * kSlice + slot0]) = t[0][m];
            *reinterpret_cast<f4v *>(&xs[b][m * kSlice + slot1]) = t[1][m];
        }
    };
    stage_x_load<MT>(tx[0][0], x, mrows, K, 0);
    stage_x_load<MT>(tx[0][1], x, mrows, K, 1024);
    if (SFIX != 1) {
        stage_x_load<MT>(tx[1][0], x, mrows, K, kSlice);
        stage_x_load<MT>(tx[1][1], x, mrows, K, kSlice + 1024);
    }
    ld(A, 0);
    if (SFIX != 1) ld(B, kSlice);
    stx(0, tx[0]);
    if (SFIX != 1) stx(1, tx[1]);
    __syncthreads();
    if (SFIX != 0) {
        // Straight line (the slice count is a template constant): the
        // compiler waits for exactly the loads each row needs. Where loads
        // are conditional or sit behind a loop back-edge it waits for every
        // outstanding load first, so slice 0 would wait for slice 1's data.
        compute_slice<KIND, MT, R, SCALED>(A, xs[0], K, 0, lane, acc, lut);
        if (SFIX == 2) compute_slice<KIND, MT, R, SCALED>(B, xs[1], K, kSlice, lane, acc, lut);
    } else
    for (int64_t s = 0; s < S; s += 2) {
        const int64_t kb = s * kSlice;
        compute_slice<KIND, MT, R, SCALED>(A, xs[0], K, kb, lane, acc, lut);
        const bool n2 = s + 2 < S, n3 = s + 3 < S;
        if (n2) {
            stage_x_load<MT>(tx[0][0], x, mrows, K, kb + 2 * kSlice);
            stage_x_load<MT>(tx[0][1], x, mrows, K, kb + 2 * kSlice + 1024);
        }
        if (n3) {
            stage_x_load<MT>(tx[1][0], x, mrows, K, kb + 3 * kSlice);
            stage_x_load<MT>(tx[1][1], x, mrows, K, kb + 3 * kSlice + 1024);
        }
        if (n2) ld(A, kb + 2 * kSlice);
        if (s + 1 < S) compute_slice<KIND, MT, R, SCALED>(B, xs[1], K, kb + kSlice, lane, acc, lut);
        if (n3) ld(B, kb + 3 * kSlice);
        if (!n2) break;
        __syncthreads();  // every wave is done reading both buffers
        stx(0, tx[0]);
        if (n3) stx(1, tx[1]);
        __syncthreads();
    }

    // Halving butterfly: at distance d, the lanes with bit d set keep the
    // upper half of their values and the others the lower half, each adding
    // the partner's copy; once one value is left the remaining steps sum it.
    // Lane l ends with value index l >> (6 - log2 V).
    float v[V];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) v[r * MT + m] = acc[r][m];
#pragma unroll
    for (int d = 32, cnt = V; d >= 1; d >>= 1) {
        if (cnt > 1) {
            const int half = cnt / 2;
            const bool up = (lane & d) != 0;
#pragma unroll
            for (int i = 0; i < half; ++i) {
                const float keep = up ? v[half + i] : v[i];
                const float send = up ? v[i] : v[half + i];
                v[i] = keep + __shfl_xor(send, d, 64);
            }
            cnt = half;
        } else {
            v[0] += __shfl_xor(v[0], d, 64);
        }
    }
    constexpr int LOG_V = V == 1 ? 0 : (V == 2 ? 1 : (V == 4 ? 2 : (V == 8 ? 3 : (V == 16 ? 4 : (V == 32 ? 5 : 6)))));
    if ((lane & ((64 >> LOG_V) - 1)) == 0) {
        const int idx = lane >> (6 - LOG_V);
        const int r = idx / MT, m = idx % MT;
        const int64_t row = r0 + r;
        if (row < N && m < mrows) {
            float o = v[0];
            if (BIAS) o = o + bias[row];
            y[(int64_t)m * N + row] = o;
        }
    }
}

// ------------------------------------------------------------ MFMA GEMV (m up to 16)

// QuantizedLinear::forward for 5..16 rows of x on v_mfma_f32_16x16x4f32, all
// rows at once (the VALU GEMV above re-reads the weights for every 4 rows).
// A workgroup of 4 waves owns 16*NT output columns (weight rows); wave w takes
// the w-th quarter of K. (4 waves and one 16-column tile per workgroup: 23 /
// 25 us at m = 8 / 16 over 4096 x 11008 INT4, against 29-33 for 8 waves or
// two tiles, which hold fewer workgroups per CU.) Lane l = 16*k4 + i provides, per MFMA, the A value
// x[i][k] and the B value W[n0 + i][k] for the same k: both walk the lane's
// 16-byte weight piece (EP codes of row i at k = kc + k4*EP + t, MFMA t). The
// codes are decoded and scaled in registers -- the value is exactly the
// reference's dequantized q*s (for INT4, 16q * (s/16)) -- so the MFMA sums
// x * W as QuantizedLinear::forward does, in its own order. Rows of x past m
// read row m-1 and their outputs are dropped. Partial 16x16 tiles of the 8
// waves are summed through LDS.
constexpr int kMfmaWaves = 4;

template <int KIND, int NT, bool SCALED, bool BIAS>
__global__ __launch_bounds__(kMfmaWaves * 64) void qt_gemv_mfma_kernel(
    const float *__restrict__ x, int mrows, int64_t K, const uint8_t *__restrict__ data,
    const float *__restrict__ scales, int64_t ns, uint32_t g, uint32_t kg, uint32_t rpg, int64_t N,
    const float *__restrict__ bias, float *__restrict__ y) {
    using F = Fmt<KIND>;
    constexpr int EP = F::EP;  // elements per 16-byte piece
    typedef float f4 __attribute__((ext_vector_type(4)));
    __shared__ float part[kMfmaWaves][NT][16][17];
    // per wave, the x chunk (16 rows x 4*EP floats, row pitch 4*EP + 4: the
    // lanes' 16-byte reads of one pass fall in different banks)
    constexpr int XP = 4 * EP + 4;
    __shared__ __attribute__((aligned(16))) float xsh[kMfmaWaves][16 * XP];
    __shared__ float lut[16];
    if ((KIND == KIND_NF4 || KIND == KIND_E2M1) && threadIdx.x < 16)
        lut[threadIdx.x] = KIND == KIND_NF4 ? kNF4[threadIdx.x] : kE2M1[threadIdx.x];
    __syncthreads();
    const int wid = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int i = lane % 16, k4 = lane / 16;
    const int64_t n0 = (int64_t)blockIdx.x * 16 * NT;
    const int64_t kw = K / kMfmaWaves, k0 = wid * kw;  // kw % (4 * EP) == 0 (host check)
    // x staging: load instruction q covers rows 2q' .. (EP/4 instructions of
    // 64 lanes x 16 bytes = the 16 x 4*EP chunk, each row contiguous)
    constexpr int LPR = EP;  // lanes per x row of the chunk (4*EP floats / 4)
    const int sr0 = lane / LPR, sc4 = lane % LPR;
    const uint8_t *wrow[NT];
    int64_t gbase[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int64_t n = n0 + 16 * nt + i < N ? n0 + 16 * nt + i : N - 1;
        wrow[nt] = data + (n * K) * 16 / EP;  // row start (EP codes per 16 bytes)
        gbase[nt] = !SCALED ? 0 : (kg ? n * (int64_t)kg : (int64_t)((uint32_t)n / rpg));
    }
    f4 acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = f4{0.f, 0.f, 0.f, 0.f};
    // One K chunk (4*EP) of this lane: EP values of x and one piece per tile.
    struct Chunk {
        f4 xt[EP / 4];  // this lane's share of the x chunk, before it goes to LDS
        v4i raw[NT];
        float sc[NT];
    };
    auto load = [&](Chunk &c, int64_t kc) {
        const int64_t e = kc + k4 * EP;
#pragma unroll
        for (int q = 0; q < EP / 4; ++q) {
            const int r = sr0 + q * (64 / LPR);
            const float *xr = x + (int64_t)(r < mrows ? r : mrows - 1) * K;
            c.xt[q] = *reinterpret_cast<const f4 *>(xr + kc + 4 * sc4);
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            c.raw[nt] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(wrow[nt] + e * 16 / EP));
            if (SCALED) {
                const int64_t gi = gbase[nt] + (kg ? (int64_t)((uint32_t)e / g) : 0);
                c.sc[nt] = scales[gi < ns - 1 ? gi : ns - 1];
            }
        }
    };
    auto compute = [&](const Chunk &c) {
        float *xs = xsh[wid];
#pragma unroll
        for (int q = 0; q < EP / 4; ++q)
            *reinterpret_cast<f4 *>(&xs[(sr0 + q * (64 / LPR)) * XP + 4 * sc4]) = c.xt[q];
        __builtin_amdgcn_wave_barrier();  // one wave's LDS operations complete in order
        float xv[EP];
#pragma unroll
        for (int q = 0; q < EP / 4; ++q) {
            const f4 t = *reinterpret_cast<const f4 *>(&xs[i * XP + k4 * EP + 4 * q]);
            xv[4 * q] = t.x, xv[4 * q + 1] = t.y, xv[4 * q + 2] = t.z, xv[4 * q + 3] = t.w;
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            float v[EP];
            decode_piece<KIND>(c.raw[nt], v, lut);
            const float s = SCALED ? (KIND == KIND_I4 ? c.sc[nt] * 16.0f : c.sc[nt]) : 1.0f;
#pragma unroll
            for (int t = 0; t < EP; ++t) {
                const float w = SCALED ? v[t] * s : v[t];
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[t], w, acc[nt], 0, 0, 0);
            }
        }
    };
    // Two chunks in flight (register sets A and B alternate, two chunks per
    // iteration); loads past the wave's range re-read its last chunk so that
    // every load is unconditional and the compiler's waits stay exact.
    const int64_t nch = kw / (4 * EP), lastk = k0 + (nch - 1) * 4 * EP;
    auto kof = [&](int64_t c) { const int64_t k = k0 + c * 4 * EP; return k < lastk ? k : lastk; };
    Chunk A, B;
    load(A, kof(0));
    load(B, kof(1));
    for (int64_t c = 0; c < nch; c += 2) {
        compute(A);
        load(A, kof(c + 2));
        if (c + 1 < nch) compute(B);
        load(B, kof(c + 3));
    }
    // lane holds D[m = 4*k4 + r][n = i] of each tile
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) part[wid][nt][4 * k4 + r][i] = acc[nt][r];
    __syncthreads();
    for (int t = threadIdx.x; t < NT * 256; t += kMfmaWaves * 64) {
        const int nt = t / 256, m = (t / 16) % 16, n = t % 16;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kMfmaWaves; ++w) s += part[w][nt][m][n];
        const int64_t col = n0 + 16 * nt + n;
        if (m < mrows && col < N) {
            if (BIAS) s = s + bias[col];
            y[(int64_t)m * N + col] = s;
        }
    }
}

// ------------------------------------------------------------ bf16 MFMA GEMV (m up to 16)

// QuantizedLinear::forward for up to 16 rows of x on v_mfma_f32_16x16x32_bf16.
// Integer codes (INT4 as 16q, INT8) and bf16 weights are exact in bf16, and
// x = h + m + l splits exactly into three bf16 parts (h = x with the low 16
// bits cleared, m likewise of x - h, l = x - h - m, which has at most 8
// significant bits), so each product is exact and the MFMA sums in f32; the
// sum of a group's products enters the tile's total in one fused multiply-add
// by the group's scale (INT4's factor 16 is applied once to the total). This is the
// reference's sum of x * (q*s) reassociated, within the same f32 GEMM
// rounding bound, at 16x the f32 MFMA's rate per MFMA (three of them per
// product).
//
// Each workgroup splits the x it reads in registers. At m = 16, 4 bytes of x
// per element against half a byte per INT4 weight mean that a CU taking
// whole rows of W over all of K would read 2.9x as many x bytes as weight
// bytes (4096 x 11008) and split every element of x. So K is also split, S
// ways: workgroup (range r, part s) takes the row range r (of R balanced
// ranges, up to TPW 16-row tiles) over the s-th K part, with 8 waves each
// taking CPW chunks (4*EP elements) of it (all loads of a one-chunk wave
// issued up front). Per chunk a lane (q, i) loads, for each tile, the 16-byte
// piece of its row i at k = c*4EP + q*EP (the EP codes of MFMA steps j = 0..
// EP/8-1, 8 each) and x[i][the same EP elements] (rows past m read zero
// through the buffer descriptor), splits x into the A fragments of the
// chunk's steps, which serve every tile. A chunk's 4*EP elements lie in one
// group (the host admits groups that are multiples of 4*EP, or whole rows):
// the chunk's MFMAs sum into a fresh accumulator, which is scaled and added
// to the tile's total. The 8 waves' totals are summed through LDS; with
// S > 1 each workgroup stores its partial tile in the workspace and counts
// itself in, and the last of a range's S workgroups sums the S partials in
// part order (deterministic) and writes y, then resets the counter to zero.
// No workgroup waits for another.
constexpr int kSplitParts = 3;

__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
    // high halves of two floats -> packed bf16 (lo in bits 0-15)
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// x = h + m + l exactly: h and m are x and x - h with the low 16 bits
// cleared, l = x - h - m has at most 8 significant bits. Infinities stay
// whole in h (r = 0 when h == x); a NaN whose payload sits only in the low
// 16 bits becomes an infinity in h, but then r = x - h is NaN, so the sum
// stays NaN as the reference's product does.
__device__ __forceinline__ void split3(float x, float &h, float &m, float &l) {
    h = __uint_as_float(__float_as_uint(x) & 0xFFFF0000u);
    const float r = h == x ? 0.0f : x - h;
    m = __uint_as_float(__float_as_uint(r) & 0xFFFF0000u);
    l = r - m;
}

// split3 for finite x (x - h is then exact, and 0 when h == x): the same
// parts without the guard's compare and select.
__device__ __forceinline__ void split3_finite(float x, float &h, float &m, float &l) {
    h = __uint_as_float(__float_as_uint(x) & 0xFFFF0000u);
    const float r = x - h;
    m = __uint_as_float(__float_as_uint(r) & 0xFFFF0000u);
    l = r - m;
}

constexpr int kBf16Waves = 8, kBf16MaxParts = 8;

// (waves_per_eu: the launch has one workgroup of 8 waves per CU, so the
// register budget is that of 2 waves per SIMD; without it the compiler
// trades the up-front loads for a higher occupancy that is never used.)
//
// SC: 0 unscaled (BF16), 1 one scale per chunk (groups of whole chunks or
// rows), 2 groups of 32 elements inside a chunk (GGUF Q4_0 / Q8_0 blocks):
// every MFMA step then takes one group. A step sums 8 elements from each of
// the 4 lane groups q (lanes 16q .. 16q+15), so after the 16-byte loads the
// lanes trade dwords: int8 pieces swap halves between lane groups q and q+2
// (elements 8q' .. of group j land in step j), 4-bit pieces (one whole group
// per lane group) are transposed 4 x 4 across the lane groups; both through
// the gfx950 lane-swap instructions, or (weights staged in LDS) by reading
// those dwords from the staged rows. x is read in the matching order.
template <int KIND, int TPW, bool ONE, int SC, bool BIAS, bool LN = false>
__global__ __launch_bounds__(kBf16Waves * 64) __attribute__((amdgpu_waves_per_eu(1, 2)))
void qt_gemv_bf16_kernel(
    const float *__restrict__ x, int mrows, int64_t K, const uint8_t *__restrict__ data,
    const float *__restrict__ scales, int64_t ns, uint32_t cpg, uint32_t kg, uint32_t rpg,
    int64_t N, int S, uint32_t cpw, float *__restrict__ wpart, uint32_t *__restrict__ counters,
    const float *__restrict__ bias, float *__restrict__ y) {
    constexpr int EP = Fmt<KIND>::EP;  // elements per 16-byte piece
    constexpr int JS = EP / 8;         // MFMA steps per chunk
    constexpr int NW = kBf16Waves;
    constexpr bool SCALED = SC != 0, G32 = SC == 2;
    static_assert(!G32 || KIND == KIND_I4 || KIND == KIND_I8, "32-element groups: 4- or 8-bit codes");
    constexpr int NSC = G32 ? JS : 1;  // scales per tile and chunk
    // Several chunks per wave (!ONE): x is loaded in whole-row runs (a load
    // instruction reads 1 KiB of consecutive bytes: 64/EP rows of the chunk)
    // and regrouped into the fragment layout through the wave's LDS slice.
    // The fragment layout itself (each lane reads 4 EP consecutive bytes of
    // its row, so one instruction touches 64 different lines 16 bytes at a
    // time) measured 19.3 against 15.2 us at m = 16 over all of K.
    constexpr bool STAGE = !ONE;
    constexpr int XP = 4 * EP + 4;     // floats per staged row (16-byte pad: no bank conflicts)
    constexpr int XRPL = 64 / EP;      // rows per whole-row load instruction
    typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
    // LINES: several chunks per wave also read the weights of two chunks at
    // a time as whole 128-byte lines (a load instruction: 8 rows x 128
    // bytes), which the wave stores in its LDS slice of the pool and reads
    // back in the fragment layout; the 8 waves' partial tiles reuse the pool
    // after the loop. Measured at 4096 x 11008 against one chunk's 64 bytes
    // per row (16 rows x 64 bytes per load instruction, half lines): GGUF
    // Q8_0 m = 16 / 8 19.7 / 18.5 against 22.7 / 21.2 us, GGUF Q4_0 m = 16
    // 17.1 against 18.4 us; INT4 in groups of whole chunks, whose time is
    // the decode and split work, measured 15.4 / 15.1 / 14.9 / 14.5 against
    // 15.8 / 15.3 / 14.7 / 13.8 us at m = 16 / 12 / 9 / 4: LN, which the host
    // sets from 12 rows of x on (more x bytes per chunk), selects whole lines
    // for it.
    constexpr bool LINES = STAGE && (LN || !(KIND == KIND_I4 && SC == 1));
    constexpr int WSLICE = TPW * 16 * 128;  // bytes of a wave's weight slice
    constexpr int PART_BYTES = NW * TPW * 16 * 17 * 4;
    constexpr int POOL = LINES && NW * WSLICE > PART_BYTES ? NW * WSLICE : PART_BYTES;
    __shared__ __attribute__((aligned(16))) uint8_t pool[POOL];
    float (*const part)[TPW][16][17] = reinterpret_cast<float (*)[TPW][16][17]>(pool);
    __shared__ __attribute__((aligned(16))) float xs[STAGE ? NW * 16 * XP : 4];
    __shared__ uint32_t last;
    // (the wave index through readfirstlane: uniform to the compiler, so the
    // chunk offsets are scalar and the buffer loads take them as soffset)
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const int i = lane % 16, q = lane / 16;
    const uint32_t R = gridDim.x / S, rg = blockIdx.x / S, sp = blockIdx.x % S;
    // (32-bit: the launch keeps N * R < 2^32 and 64 rows < 2^31 bytes)
    const uint32_t r0 = rg * (uint32_t)N / R;
    const int nrows = (int)((rg + 1) * (uint32_t)N / R - r0);
    const uint32_t rowbytes = (uint32_t)(K * 16 / EP);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(data + (int64_t)r0 * rowbytes), 0, (int)(nrows * rowbytes), 0x00020000);
    // x: rows past mrows read zero (the launch keeps 16 K floats < 2^31 bytes)
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(x), 0, (int)(mrows * K * 4), 0x00020000);
    // (the row is always in the per-lane offset, which the descriptor's
    // range check covers: rows past mrows read zero)
    const uint32_t xoff = STAGE ? (uint32_t)(((lane / EP) * K + (lane % EP) * 4) * 4)
                                : (uint32_t)((i * K + q * EP) * 4);
    // element offset in the chunk of the lane's x float4 u (steps j = u / 2)
    auto xfo = [&](int u) -> int {
        if constexpr (G32)
            return 32 * (u / 2) + (EP == 16 ? 16 * (q & 1) + 8 * (q >> 1) : 8 * q) + 4 * (u % 2);
        else
            return q * EP + 4 * u;
    };
    const uint32_t c0 = (sp * NW + wid) * cpw;  // this wave's first chunk
    // per tile: the lane's byte offset within the range (row 16t + i, piece
    // q of a chunk) and its row's first scale index
    uint32_t voff[TPW];
    int64_t gbase[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        voff[t] = (16 * t + i) * rowbytes + 16 * q;
        const int64_t n = r0 + std::min(16 * t + i, nrows - 1);
        gbase[t] = !SCALED ? 0 : (kg ? n * (int64_t)kg : (int64_t)((uint32_t)n / rpg));
        // (G32: the row's first scale, which keeps the chunk's vector load aligned)
        if (SCALED) gbase[t] = std::min<int64_t>(gbase[t], G32 ? ns - kg : ns - 1);
    }
    struct Chunk {
        f4v xf[EP / 4];  // x[i][c*4EP + q*EP ..+ EP), or (staged) whole-row runs
        v4i w[TPW];
        float sc[TPW][NSC];
    };
    auto load = [&](Chunk &ch, uint32_t c) {
#pragma unroll
        for (int u = 0; u < EP / 4; ++u)
            ch.xf[u] = __builtin_bit_cast(
                f4v, STAGE ? __builtin_amdgcn_raw_buffer_load_b128(
                                 xr, xoff + (uint32_t)(u * XRPL * K * 4), c * (4 * EP * 4), 0)
                           : __builtin_amdgcn_raw_buffer_load_b128(
                                 xr, G32 ? (uint32_t)((i * K + xfo(u)) * 4) : xoff + 16 * u,
                                 c * (4 * EP * 4), 0));
        // chunk c starts 64 bytes per chunk into every row (4 pieces); the
        // group of a chunk is uniform (groups hold whole chunks or rows), or
        // (G32) the chunk holds the row's groups JS c .. JS c + JS - 1
        const uint32_t grp = G32 ? c * JS : (kg ? c / cpg : 0u);
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            if constexpr (!LINES)
                ch.w[t] = __builtin_bit_cast(
                    v4i, __builtin_amdgcn_raw_buffer_load_b128(wr, voff[t], c * 64u, 2 /* nt */));
            if constexpr (G32) {
                // (a row's scales start at a multiple of kg, itself a multiple
                // of 16: the JS-float load is aligned)
                typedef float fjv __attribute__((ext_vector_type(JS)));
                const fjv sv = *reinterpret_cast<const fjv *>(scales + gbase[t] + grp);
#pragma unroll
                for (int j = 0; j < JS; ++j) ch.sc[t][j] = sv[j];
            } else if (SCALED) {
                const int64_t gi = gbase[t] + grp;  // (a row's groups are in range)
                ch.sc[t][0] = scales[gi];
            }
        }
    };
    // (LINES) The weights of chunks c and c + 1: per tile two loads, the
    // lane's 16 bytes at row 16t + 8h + lane/8, piece lane%8 of the 128 bytes
    // from byte 64c of the row. In the wave's slice the piece of tile row rr
    // sits at (16t + rr) * 128 + 16 * (piece ^ wswz(rr)): the 16 rows of a
    // fragment read then fall on 16 different 16-byte bank groups. (The rows
    // of a range are 16-byte aligned and lie in the range's descriptor, so a
    // pair that runs past the row or the range reads the next row or zeros,
    // which no MFMA of this wave uses.)
    v4i wl[LINES ? TPW : 1][2];
    uint8_t *const wsl = pool + (LINES ? wid * WSLICE : 0);
    auto wswz = [](int rr) { return (rr >> 1) & 7; };
    auto load_w = [&](uint32_t c) {
        if constexpr (LINES) {
#pragma unroll
            for (int t = 0; t < TPW; ++t)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    wl[t][h] = __builtin_bit_cast(
                        v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                 wr, (uint32_t)(16 * t + 8 * h + lane / 8) * rowbytes + 16 * (lane % 8),
                                 c * 64u, 2 /* nt */));
        }
    };
    auto stage_w = [&]() {
        if constexpr (LINES) {
#pragma unroll
            for (int t = 0; t < TPW; ++t)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int rr = 8 * h + lane / 8;
                    *reinterpret_cast<v4i *>(wsl + (16 * t + rr) * 128 + 16 * ((lane % 8) ^ wswz(rr))) =
                        wl[t][h];
                }
        }
    };
    // Lane (q, i)'s 16 bytes of tile t for the pair's chunk h, in the layout
    // the MFMA steps take: piece q of the chunk, or (G32) the dwords a step
    // of one 32-element group needs (int8: bytes 8g .. 8g+7 and 32+8g ..
    // 32+8g+7 with g = 2(q%2) + q/2; 4-bit: dword q of each of the 4 pieces).
    auto lds_w = [&](int t, int h) -> v4i {
        const uint8_t *row = wsl + (16 * t + i) * 128;
        auto piece = [&](int p) { return row + 16 * ((4 * h + p) ^ wswz(i)); };
        if constexpr (G32 && EP == 16) {
            typedef int v2i __attribute__((ext_vector_type(2)));
            const v2i a = *reinterpret_cast<const v2i *>(piece(q & 1) + 8 * (q >> 1));
            const v2i b = *reinterpret_cast<const v2i *>(piece(2 + (q & 1)) + 8 * (q >> 1));
            return v4i{a[0], a[1], b[0], b[1]};
        } else if constexpr (G32) {
            v4i w;
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = *reinterpret_cast<const int *>(piece(j) + 4 * q);
            return w;
        } else {
            return *reinterpret_cast<const v4i *>(piece(q));
        }
    };
    f4v tot[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) tot[t] = f4v{0.f, 0.f, 0.f, 0.f};
    // (h: the chunk's half of the pair staged in the wave's slice)
    auto compute = [&](const Chunk &ch, int h) {
        // (staged: the whole-row runs into the wave's LDS slice, then the
        // lane's fragment, x[i][q EP .. q EP + EP), back; one wave's LDS
        // operations complete in order)
        f4v xfr[EP / 4];
        if constexpr (STAGE) {
            float *xw = xs + wid * 16 * XP;
#pragma unroll
            for (int u = 0; u < EP / 4; ++u)
                *reinterpret_cast<f4v *>(xw + (u * XRPL + lane / EP) * XP + (lane % EP) * 4) = ch.xf[u];
#pragma unroll
            for (int u = 0; u < EP / 4; ++u)
                xfr[u] = *reinterpret_cast<const f4v *>(xw + i * XP + xfo(u));
        } else {
#pragma unroll
            for (int u = 0; u < EP / 4; ++u) xfr[u] = ch.xf[u];
        }
        // the chunk's A fragments: step j takes elements 8j .. 8j+7. The
        // wave takes the guarded split only when a lane's x holds an
        // infinity or a NaN (x * 0 + ... is then NaN): the same parts, one
        // compare and select fewer per element otherwise (measured, INT4 and
        // GGUF Q8_0 4096 x 11008: 0.2-0.5 us faster, bit-identical).
        v4i a[JS][kSplitParts];
        auto split_chunk = [&](auto guarded) {
#pragma unroll
            for (int j = 0; j < JS; ++j)
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const f4v &v4 = xfr[2 * j + d / 2];
                    float h0, m0, l0, h1, m1, l1;
                    if constexpr (decltype(guarded)::value) {
                        split3(v4[2 * (d % 2)], h0, m0, l0);
                        split3(v4[2 * (d % 2) + 1], h1, m1, l1);
                    } else {
                        split3_finite(v4[2 * (d % 2)], h0, m0, l0);
                        split3_finite(v4[2 * (d % 2) + 1], h1, m1, l1);
                    }
                    a[j][0][d] = (int)bf16_pair(h0, h1);
                    a[j][1][d] = (int)bf16_pair(m0, m1);
                    a[j][2][d] = (int)bf16_pair(l0, l1);
                }
        };
        float probe = 0.0f;
#pragma unroll
        for (int u = 0; u < EP / 4; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) probe = __builtin_fmaf(xfr[u][e], 0.0f, probe);
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(probe != probe) != 0, 0))
            split_chunk(std::true_type{});
        else
            split_chunk(std::false_type{});
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            float v[EP];
            v4i w;
            if constexpr (LINES) {
                w = lds_w(t, h);
            } else if constexpr (G32) {
                w = ch.w[t];
                // lane group q's dwords to the steps of their groups: swap the
                // upper 32 lanes of one register with the lower 32 of another
                // (lane groups 2, 3 <-> 0, 1), then (4-bit) odd rows of 16
                // lanes of one with even rows of the other
                const auto s02 = __builtin_amdgcn_permlane32_swap((uint32_t)w[0], (uint32_t)w[2], false, false);
                const auto s13 = __builtin_amdgcn_permlane32_swap((uint32_t)w[1], (uint32_t)w[3], false, false);
                w = v4i{(int)s02[0], (int)s13[0], (int)s02[1], (int)s13[1]};
                if constexpr (EP == 32) {
                    const auto s01 = __builtin_amdgcn_permlane16_swap((uint32_t)w[0], (uint32_t)w[1], false, false);
                    const auto s23 = __builtin_amdgcn_permlane16_swap((uint32_t)w[2], (uint32_t)w[3], false, false);
                    w = v4i{(int)s01[0], (int)s01[1], (int)s23[0], (int)s23[1]};
                }
            } else {
                w = ch.w[t];
            }
            if (KIND != KIND_BF16) decode_piece<KIND>(w, v, nullptr);
            f4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < JS; ++j) {
                v4i b;
                if (KIND == KIND_BF16) {
                    b = w;  // already 8 bf16
                } else {
#pragma unroll
                    for (int d = 0; d < 4; ++d) b[d] = (int)bf16_pair(v[8 * j + 2 * d], v[8 * j + 2 * d + 1]);
                }
                if constexpr (G32) {  // a step is one group: its own sum and scale
                    f4v aj = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int p = 0; p < kSplitParts; ++p)
                        aj = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a[j][p]),
                                                                    __builtin_bit_cast(bf8, b), aj, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) tot[t][r] = __builtin_fmaf(aj[r], ch.sc[t][j], tot[t][r]);
                } else {
#pragma unroll
                    for (int p = 0; p < kSplitParts; ++p)
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a[j][p]),
                                                                     __builtin_bit_cast(bf8, b), acc, 0, 0, 0);
                }
            }
            if constexpr (G32) {
            } else if (SCALED) {
#pragma unroll
                for (int r = 0; r < 4; ++r) tot[t][r] = __builtin_fmaf(acc[r], ch.sc[t][0], tot[t][r]);
            } else {
                tot[t] = tot[t] + acc;
            }
        }
    };
    if constexpr (ONE) {  // one chunk per wave: every load up front
        Chunk A;
        load(A, c0);
        __builtin_amdgcn_sched_barrier(0);
        compute(A, 0);
    } else if constexpr (LINES) {
        // x one chunk ahead of the one being computed, the weights one pair
        // ahead of the pair being computed, each pair's loads issued before
        // its chunks' x (the memory counter completes in order: the wait for
        // a chunk's x then also covers its weights). Past the wave's last
        // chunk the loads repeat the last chunk or pair.
        Chunk A, B;
        const uint32_t last_pair = (cpw - 1) & ~1u;
        load_w(c0);
        load(A, c0);
        load(B, c0 + 1);
        for (uint32_t c = 0; c < cpw; c += 2) {
            stage_w();
            load_w(c0 + std::min(c + 2, last_pair));
            compute(A, 0);
            load(A, c0 + std::min(c + 2, cpw - 1));
            if (c + 1 < cpw) compute(B, 1);
            load(B, c0 + std::min(c + 3, cpw - 1));
        }
        __syncthreads();  // every wave's slice read before the pool takes the partials
    } else {  // one chunk in flight ahead of the one being computed
        Chunk A, B;
        load(A, c0);
        for (uint32_t c = 0; c < cpw; c += 2) {
            load(B, c0 + std::min(c + 1, cpw - 1));
            compute(A, 0);
            load(A, c0 + std::min(c + 2, cpw - 1));
            if (c + 1 < cpw) compute(B, 0);
        }
    }
    // lane holds D[m = 4q + r][n = i] of each tile (INT4 codes entered as
    // q/16: the factor 16, exact, once here)
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            part[wid][t][4 * q + r][i] = KIND == KIND_I4 ? tot[t][r] * 16.0f : tot[t][r];
    __syncthreads();
    // outputs of this workgroup: (tile t, row m, column n), m < mrows
    if (S == 1) {
        for (int u = threadIdx.x; u < TPW * 256; u += NW * 64) {
            const int t = u / 256, m = (u / 16) % 16, n = u % 16;
            if (m >= mrows || 16 * t + n >= nrows) continue;
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) sum += part[w][t][m][n];
            const int64_t col = r0 + 16 * t + n;
            if (BIAS) sum = sum + bias[col];
            y[(int64_t)m * N + col] = sum;
        }
        return;
    }
    // S > 1: this part's sums into the workspace, [S][16][N]
    for (int u = threadIdx.x; u < TPW * 256; u += NW * 64) {
        const int t = u / 256, m = (u / 16) % 16, n = u % 16;
        if (m >= mrows || 16 * t + n >= nrows) continue;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) sum += part[w][t][m][n];
        __hip_atomic_store(&wpart[((int64_t)sp * 16 + m) * N + r0 + 16 * t + n], sum,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // The partials are device-scope atomic stores, which write through this
    // XCD's L2 to the device's coherence point; once this workgroup's stores
    // have completed (vmcnt 0), it counts itself in. The last workgroup
    // reads the partials with device-scope atomic loads, from that point.
    // (A release/acquire fence pair would write back and invalidate the
    // whole L2 once per workgroup: 6x slower for the whole GEMV.)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(&counters[rg], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (uint32_t)S - 1;
    __syncthreads();
    if (!last) return;
    for (int u = threadIdx.x; u < TPW * 256; u += NW * 64) {
        const int t = u / 256, m = (u / 16) % 16, n = u % 16;
        if (m >= mrows || 16 * t + n >= nrows) continue;
        const int64_t col = r0 + 16 * t + n;
        // all S loads in flight, then summed in part order
        float pv[kBf16MaxParts];
#pragma unroll
        for (int sq = 0; sq < kBf16MaxParts; ++sq)
            pv[sq] = sq < S ? __hip_atomic_load(&wpart[((int64_t)sq * 16 + m) * N + col],
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                            : 0.0f;
        float sum = pv[0];
#pragma unroll
        for (int sq = 1; sq < kBf16MaxParts; ++sq)
            if (sq < S) sum += pv[sq];
        if (BIAS) sum = sum + bias[col];
        y[(int64_t)m * N + col] = sum;
    }
    if (threadIdx.x == 0)  // ready for the next call
        __hip_atomic_store(&counters[rg], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void qt_bias_kernel(float *__restrict__ y, int64_t m, int64_t n,
                               const float *__restrict__ bias) {
    const int64_t total = m * n;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] = y[i] + bias[i % n];
}

int grid_for(int64_t work, int per_block) {
    return (int)std::max<int64_t>(1, std::min<int64_t>(ceil_div(work, per_block),
                                                       (int64_t)8 * device_cu_count()));
}

}  // namespace rnn

using namespace rnn;

extern "C" int rnn_qt_layout(int format, int64_t n, int64_t group_size, int64_t *data_bytes,
                             int64_t *n_scales, int64_t *stored_group) {
    RNN_ENTRY();
    RNN_REQUIRE(format >= RNN_QF_FP16 && format <= RNN_QF_GGUF_Q8, "rnn_qt_layout: bad format %d",
                format);
    RNN_REQUIRE(n >= 0 && group_size >= 0, "rnn_qt_layout: negative size");
    RNN_REQUIRE(data_bytes && n_scales && stored_group, "rnn_qt_layout: null pointer");
    if (format == RNN_QF_FP16 || format == RNN_QF_BF16) {
        *data_bytes = 2 * n, *n_scales = 0, *stored_group = 0;
        return RNN_OK;
    }
    int64_t g = group_size == 0 ? n : group_size;
    if (qf_is_gguf(format)) g = std::min<int64_t>(g, 32);
    // group_size 0 on an empty tensor divides by zero in the reference
    // (n.div_ceil(0), src/quantize.rs:298)
    RNN_REQUIRE(g > 0, "rnn_qt_layout: group size 0 with n = 0");
    const int64_t ng = ceil_div(n, g);
    *stored_group = g, *n_scales = ng;
    if (!qf_is4(format)) *data_bytes = n;
    else *data_bytes = ng == 0 ? 0 : (ng - 1) * ((g + 1) / 2) + (n - (ng - 1) * g + 1) / 2;
    return RNN_OK;
}

extern "C" int rnn_qt_quantize(int format, const float *x, int64_t n, int64_t group_size,
                               uint8_t *data, float *scales, void *stream) {
    RNN_ENTRY();
    int64_t nb, ng, g;
    RNN_TRY(rnn_qt_layout(format, n, group_size, &nb, &ng, &g));
    if (n == 0) return RNN_OK;
    RNN_REQUIRE(x && data, "rnn_qt_quantize: null pointer");
    hipStream_t st = as_stream(stream);
    if (format == RNN_QF_FP16 || format == RNN_QF_BF16) {
        qt_half_quant_kernel<<<grid_for(n, 256), 256, 0, st>>>(format, x, n,
                                                               reinterpret_cast<uint16_t *>(data));
        return check_launch("rnn_qt_quantize");
    }
    RNN_REQUIRE(scales != nullptr, "rnn_qt_quantize: null scales");
    if (g <= kSmallGroup) {
        RNN_REQUIRE(ceil_div(ng, 4) <= 0x7fffffff, "rnn_qt_quantize: too many groups");
        qt_quant_group_kernel<<<(unsigned)ceil_div(ng, 4), 256, 0, st>>>(format, x, n, g, ng, data,
                                                                        scales);
        return check_launch("rnn_qt_quantize");
    }
    const int64_t cpg = ceil_div(g, kChunk);
    RNN_REQUIRE(ng * cpg <= 0x7fffffff, "rnn_qt_quantize: tensor too large");
    qt_zero_kernel<<<grid_for(ng, 256), 256, 0, st>>>(reinterpret_cast<uint32_t *>(scales), ng);
    qt_group_max_kernel<<<(unsigned)(ng * cpg), 256, 0, st>>>(
        x, n, g, cpg, reinterpret_cast<uint32_t *>(scales));
    qt_big_codes_kernel<<<(unsigned)(ng * cpg), 256, 0, st>>>(format, x, n, g, cpg, scales, data);
    qt_finish_scales_kernel<<<grid_for(ng, 256), 256, 0, st>>>(format, scales, ng);
    return check_launch("rnn_qt_quantize");
}

static int check_tensor(const char *name, int format, const uint8_t *data, int64_t data_bytes,
                        const float *scales, int64_t n_scales, int64_t group, int64_t n) {
    RNN_REQUIRE(format >= RNN_QF_FP16 && format <= RNN_QF_GGUF_Q8, "%s: bad format %d", name,
                format);
    RNN_REQUIRE(n >= 0 && data_bytes >= 0 && n_scales >= 0 && group >= 0, "%s: negative size",
                name);
    if (n == 0) return RNN_OK;
    RNN_REQUIRE(data != nullptr, "%s: null data", name);
    if (format == RNN_QF_FP16 || format == RNN_QF_BF16) {
        RNN_REQUIRE(data_bytes >= 2 * n, "%s: data holds %lld bytes, needs %lld", name,
                    (long long)data_bytes, (long long)(2 * n));
        return RNN_OK;
    }
    // the reference indexes scales[] and data[] without checks and panics on
    // a short array; here the same conditions are errors
    RNN_REQUIRE(group > 0, "%s: group size 0", name);
    RNN_REQUIRE(scales != nullptr && n_scales > 0, "%s: no scales", name);
    int64_t need;
    if (format == RNN_QF_GGUF_Q4 || format == RNN_QF_GGUF_Q4K) {
        RNN_REQUIRE(n_scales >= ceil_div(n, group), "%s: %lld scales for %lld blocks", name,
                    (long long)n_scales, (long long)ceil_div(n, group));
        const int64_t nbk = ceil_div(n, group);
        need = (nbk - 1) * ((group + 1) / 2) + (n - (nbk - 1) * group + 1) / 2;
    } else {
        need = qf_is4(format) ? (n + 1) / 2 : n;
    }
    RNN_REQUIRE(data_bytes >= need, "%s: data holds %lld bytes, needs %lld", name,
                (long long)data_bytes, (long long)need);
    return RNN_OK;
}

extern "C" int rnn_qt_dequantize(int format, const uint8_t *data, int64_t data_bytes,
                                 const float *scales, int64_t n_scales, int64_t group, int64_t n,
                                 float *out, void *stream) {
    RNN_ENTRY();
    RNN_TRY(check_tensor("rnn_qt_dequantize", format, data, data_bytes, scales, n_scales, group, n));
    if (n == 0) return RNN_OK;
    RNN_REQUIRE(out != nullptr, "rnn_qt_dequantize: null out");
    hipStream_t st = as_stream(stream);
    const bool grouped = format != RNN_QF_FP16 && format != RNN_QF_BF16;
    // bytes of codes per eight elements
    const int vec = format == RNN_QF_INT8 || format == RNN_QF_GGUF_Q8 ? 8 : grouped ? 4 : 16;
    if (n % 8 == 0 && (!grouped || group % 8 == 0) && (uintptr_t)data % vec == 0 &&
        (uintptr_t)out % 16 == 0) {
        const bool pow2 = grouped && (group & (group - 1)) == 0;
        const int gshift = pow2 ? __builtin_ctzll((unsigned long long)group) : 0;
        const int blocks = grid_for(n / 8, 256);
#define RNN_DQ8(F)                                                                             \
    do {                                                                                       \
        if (pow2)                                                                              \
            qt_dequant8_kernel<F, true><<<blocks, 256, 0, st>>>(data, scales, n_scales, group,  \
                                                                gshift, n / 8, out);           \
        else                                                                                   \
            qt_dequant8_kernel<F, false><<<blocks, 256, 0, st>>>(data, scales, n_scales, group, \
                                                                 gshift, n / 8, out);          \
    } while (0)
        switch (format) {
        case RNN_QF_FP16: RNN_DQ8(RNN_QF_FP16); break;
        case RNN_QF_BF16: RNN_DQ8(RNN_QF_BF16); break;
        case RNN_QF_INT8: RNN_DQ8(RNN_QF_INT8); break;
        case RNN_QF_GGUF_Q8: RNN_DQ8(RNN_QF_GGUF_Q8); break;
        case RNN_QF_INT4: RNN_DQ8(RNN_QF_INT4); break;
        case RNN_QF_NF4: RNN_DQ8(RNN_QF_NF4); break;
        case RNN_QF_NVFP4: RNN_DQ8(RNN_QF_NVFP4); break;
        default: RNN_DQ8(RNN_QF_GGUF_Q4); break;  // Q4_0 and Q4_K (stored as Q4_0)
        }
#undef RNN_DQ8
    } else {
        qt_dequant_kernel<<<grid_for(n, 256), 256, 0, st>>>(format, data, scales, n_scales, group,
                                                            n, out);
    }
    return check_launch("rnn_qt_dequantize");
}

template <int KIND, int MT, int R, bool SCALED, bool BIAS>
static void launch_gemv_b(unsigned blocks, const float *x, int mrows, int64_t K,
                          const uint8_t *data, const float *scales, int64_t ns, uint32_t g,
                          uint32_t kg, uint32_t rpg, int64_t N, const float *bias, float *y,
                          hipStream_t st) {
    if (K <= kSlice)
        qt_gemv_kernel<KIND, MT, R, SCALED, BIAS, 1><<<blocks, 256, 0, st>>>(
            x, mrows, K, data, scales, ns, g, kg, rpg, N, bias, y);
    else if (K <= 2 * kSlice)
        qt_gemv_kernel<KIND, MT, R, SCALED, BIAS, 2><<<blocks, 256, 0, st>>>(
            x, mrows, K, data, scales, ns, g, kg, rpg, N, bias, y);
    else
        qt_gemv_kernel<KIND, MT, R, SCALED, BIAS, 0><<<blocks, 256, 0, st>>>(
            x, mrows, K, data, scales, ns, g, kg, rpg, N, bias, y);
}

template <int KIND, int MT, int R, bool SCALED>
static void launch_gemv(const float *x, int mrows, int64_t K, const uint8_t *data,
                        const float *scales, int64_t ns, int64_t g, int64_t N, const float *bias,
                        float *y, hipStream_t st) {
    const unsigned blocks = (unsigned)ceil_div(ceil_div(N, R), 4);
    const uint32_t kg = K % g == 0 ? (uint32_t)(K / g) : 0u;
    const uint32_t rpg = kg ? 1u : (uint32_t)(g / K);
    if (bias)
        launch_gemv_b<KIND, MT, R, SCALED, true>(blocks, x, mrows, K, data, scales, ns,
                                                 (uint32_t)g, kg, rpg, N, bias, y, st);
    else
        launch_gemv_b<KIND, MT, R, SCALED, false>(blocks, x, mrows, K, data, scales, ns,
                                                  (uint32_t)g, kg, rpg, N, bias, y, st);
}

template <int KIND, bool SCALED>
static void gemv_chunk(int mt, const float *x, int64_t K, const uint8_t *data, const float *scales,
                       int64_t ns, int64_t g, int64_t N, const float *bias, float *y,
                       hipStream_t st) {
    constexpr int R = kind4(KIND) ? 4 : 2;  // rows per wave (wider pieces hold more registers)
    if (mt == 1) launch_gemv<KIND, 1, R, SCALED>(x, 1, K, data, scales, ns, g, N, bias, y, st);
    else if (mt == 2) launch_gemv<KIND, 2, R, SCALED>(x, 2, K, data, scales, ns, g, N, bias, y, st);
    else launch_gemv<KIND, 4, 2, SCALED>(x, mt, K, data, scales, ns, g, N, bias, y, st);
}

template <int KIND, bool SCALED>
static void launch_mfma(const float *x, int mrows, int64_t K, const uint8_t *data,
                        const float *scales, int64_t ns, int64_t g, int64_t N, const float *bias,
                        float *y, hipStream_t st) {
    constexpr int NT = 1;  // 16 columns per workgroup: more workgroups in flight
    const unsigned blocks = (unsigned)ceil_div(N, 16 * NT);
    const uint32_t kg = K % g == 0 ? (uint32_t)(K / g) : 0u;
    const uint32_t rpg = kg ? 1u : (uint32_t)(g / K);
    if (bias)
        qt_gemv_mfma_kernel<KIND, NT, SCALED, true><<<blocks, kMfmaWaves * 64, 0, st>>>(
            x, mrows, K, data, scales, ns, (uint32_t)g, kg, rpg, N, bias, y);
    else
        qt_gemv_mfma_kernel<KIND, NT, SCALED, false><<<blocks, kMfmaWaves * 64, 0, st>>>(
            x, mrows, K, data, scales, ns, (uint32_t)g, kg, rpg, N, bias, y);
}

static void launch_mfma_kind(int kind, const float *x, int mrows, int64_t K, const uint8_t *data,
                             const float *scales, int64_t ns, int64_t g, int64_t N,
                             const float *bias, float *y, hipStream_t st) {
    switch (kind) {
    case KIND_I4: launch_mfma<KIND_I4, true>(x, mrows, K, data, scales, ns, g, N, bias, y, st); break;
    case KIND_NF4: launch_mfma<KIND_NF4, true>(x, mrows, K, data, scales, ns, g, N, bias, y, st); break;
    case KIND_E2M1: launch_mfma<KIND_E2M1, true>(x, mrows, K, data, scales, ns, g, N, bias, y, st); break;
    case KIND_I8: launch_mfma<KIND_I8, true>(x, mrows, K, data, scales, ns, g, N, bias, y, st); break;
    case KIND_F16: launch_mfma<KIND_F16, false>(x, mrows, K, data, scales, ns, 1, N, bias, y, st); break;
    default: launch_mfma<KIND_BF16, false>(x, mrows, K, data, scales, ns, 1, N, bias, y, st); break;
    }
}

// Shape of the bf16 GEMV launch: S K parts, R row ranges, TPW tiles per
// range, CPW chunks per wave.
struct Bf16Plan {
    int S, R, TPW;
    uint32_t cpw;
};
constexpr int kBf16MaxTilesOne = 12, kBf16MaxTiles = 4;

// The K split S (1, 2, 4 or 8) with the lowest estimated time among those
// that give every wave whole chunks and keep the tiles per range within the
// register budget; S = 0 if none does. The estimate, per workgroup, from
// rates measured on this kernel (MI355X, m = 8 and 16, K = 4096 to 14336,
// INT4 and INT8): 5.75 us + x bytes at 77 GB/s (rows past m are not
// fetched) + weight bytes at 13 GB/s + 4.5 us for the partial sums' round
// trip when S > 1, times the rounds of workgroups over the CUs. Splitting K
// cuts the x bytes every CU reads (all of its K range, for 16 rows) at the
// cost of that round trip. Measured (us, S = 1 against the split chosen
// before by size alone): INT4 m = 16 4096 x 11008 15.9 against 18.1 (S = 4),
// 8192 x 8192 22.5 against 33.3 (S = 8, 344 workgroups); 14336 x 4096 26.4
// against 23.5 (S = 2, which the estimate keeps); INT8 m = 16 4096 x 11008
// 22.7 against 33.8 (S = 8).
static Bf16Plan bf16_plan(int64_t M, int64_t K, int64_t N, int ep) {
    const int64_t nch = K / (4 * ep), cus = device_cu_count();
    const double wbytes = 16.0 / ep;  // weight bytes per element
    Bf16Plan best = {0, 0, 0, 0};
    double best_us = 0.0;
    for (int S = kBf16MaxParts; S >= 1; S /= 2) {
        if (nch % (S * kBf16Waves) != 0) continue;
        const uint32_t cpw = (uint32_t)(nch / (S * kBf16Waves));
        const int tmax = cpw == 1 ? kBf16MaxTilesOne : kBf16MaxTiles;
        const int64_t R = std::max<int64_t>(std::min<int64_t>(ceil_div(N, 16), std::max<int64_t>(1, cus / S)),
                                            ceil_div(N, 16 * tmax));
        const int64_t tpw = ceil_div(ceil_div(N, R), 16);
        if (tpw > tmax || N * R >= (int64_t(1) << 32) || R * S > 0x7fffffffLL) continue;
        const double kpart = (double)K / S;
        const double x_bytes = 4.0 * std::min<int64_t>(M, 16) * kpart;
        const double w_bytes = (double)ceil_div(N, R) * kpart * wbytes;
        const double us = (5.75 + x_bytes / 77e3 + w_bytes / 13e3 + (S > 1 ? 4.5 : 0.0)) *
                          (double)ceil_div(R * S, cus);
        if (best.S == 0 || us < best_us) best = {S, (int)R, (int)tpw, cpw}, best_us = us;
    }
    return best;
}

// Workspace (split K): one counter per range, then the parts' sums
// [S][16][N] -- bounded for any device.
static size_t bf16_workspace(int64_t N) {
    return 4 * (size_t)ceil_div(N, 16) + 256 + (size_t)kBf16MaxParts * 16 * N * 4;
}
static size_t bf16_counter_bytes(int64_t N) { return 4 * (size_t)ceil_div(N, 16) + 256; }

template <int KIND, int TPW, bool ONE, int SC>
static void launch_bf16_t(const float *xs, int mrows, int64_t K, const uint8_t *data,
                          const float *scales, int64_t ns, int64_t g, int64_t N, const float *bias,
                          float *y, const Bf16Plan &pl, float *wpart, uint32_t *cnt, hipStream_t st) {
    constexpr int EP = Fmt<KIND>::EP;
    constexpr bool SCALED = SC != 0;
    const uint32_t kg = !SCALED ? 0u : (K % g == 0 ? (uint32_t)(K / g) : 0u);
    const uint32_t rpg = !SCALED ? 1u : (kg ? 1u : (uint32_t)(g / K));
    const uint32_t cpg = kg && SC == 1 ? (uint32_t)(g / (4 * EP)) : 1u;  // chunks per group
    const unsigned grid = (unsigned)(pl.R * pl.S);
    // whole-line weights for INT4 in groups of whole chunks from 12 rows of x on
    constexpr bool LN_OK = KIND == KIND_I4 && SC == 1 && !ONE;
    const bool ln = LN_OK && mrows >= 12;
#define RNN_BF16_GO(B, L)                                                                    \
    qt_gemv_bf16_kernel<KIND, TPW, ONE, SC, B, L><<<grid, kBf16Waves * 64, 0, st>>>(        \
        xs, mrows, K, data, scales, ns, cpg, kg, rpg, N, pl.S, pl.cpw, wpart, cnt, bias, y)
    if (bias) {
        if (ln) RNN_BF16_GO(true, LN_OK);
        else RNN_BF16_GO(true, false);
    } else {
        if (ln) RNN_BF16_GO(false, LN_OK);
        else RNN_BF16_GO(false, false);
    }
#undef RNN_BF16_GO
}

template <int KIND, int SC>
static void launch_bf16_tpw(const float *xs, int mrows, int64_t K, const uint8_t *data,
                            const float *scales, int64_t ns, int64_t g, int64_t N, const float *bias,
                            float *y, const Bf16Plan &pl, float *wp, uint32_t *cnt, hipStream_t st) {
#define RNN_BF16_T(T, O) launch_bf16_t<KIND, T, O, SC>(xs, mrows, K, data, scales, ns, g, N, bias, y, pl, wp, cnt, st)
    if (pl.cpw != 1) {
        switch (pl.TPW) {
        case 1: RNN_BF16_T(1, false); break;
        case 2: RNN_BF16_T(2, false); break;
        case 3: RNN_BF16_T(3, false); break;
        default: RNN_BF16_T(4, false); break;
        }
        return;
    }
    switch (pl.TPW) {
    case 1: RNN_BF16_T(1, true); break;
    case 2: RNN_BF16_T(2, true); break;
    case 3: RNN_BF16_T(3, true); break;
    case 4: RNN_BF16_T(4, true); break;
    case 5: RNN_BF16_T(5, true); break;
    case 6: RNN_BF16_T(6, true); break;
    case 7: RNN_BF16_T(7, true); break;
    case 8: RNN_BF16_T(8, true); break;
    case 9: RNN_BF16_T(9, true); break;
    case 10: RNN_BF16_T(10, true); break;
    case 11: RNN_BF16_T(11, true); break;
    default: RNN_BF16_T(12, true); break;
    }
#undef RNN_BF16_T
}

template <int KIND, bool SCALED>
static int launch_bf16(const float *x, int mrows, int64_t K, const uint8_t *data,
                       const float *scales, int64_t ns, int64_t g, int64_t N, const float *bias,
                       float *y, void *workspace, hipStream_t st, const char *name) {
    constexpr int EP = Fmt<KIND>::EP;
    const Bf16Plan pl = bf16_plan(mrows, K, N, EP);
    void *ws = workspace;
    if (!ws && pl.S > 1) {
        // stream-ordered scratch, its counters zeroed (a caller's workspace
        // starts zeroed and every call leaves its counters at zero)
        RNN_TRY(check_hip(hipMallocAsync(&ws, bf16_workspace(N), st), name));
        qt_zero_kernel<<<grid_for(pl.R, 256), 256, 0, st>>>(static_cast<uint32_t *>(ws), pl.R);
    }
    uint8_t *base = static_cast<uint8_t *>(ws);
    uint32_t *cnt = reinterpret_cast<uint32_t *>(base);
    float *wpart = base ? reinterpret_cast<float *>(base + bf16_counter_bytes(N)) : nullptr;
    // groups of 32 inside a chunk (GGUF blocks): a scale per MFMA step
    if (SCALED && 4 * EP > 32 && g == 32)
        launch_bf16_tpw<KIND, KIND == KIND_BF16 ? 0 : 2>(x, mrows, K, data, scales, ns, g, N, bias, y, pl,
                                                         wpart, cnt, st);
    else
        launch_bf16_tpw<KIND, SCALED ? 1 : 0>(x, mrows, K, data, scales, ns, g, N, bias, y, pl, wpart,
                                              cnt, st);
    const int rc = check_launch(name);
    if (workspace || !ws) return rc;
    const int rf = check_hip(hipFreeAsync(ws, st), name);
    return rc != RNN_OK ? rc : rf;
}

static int piece_elems(int kind) { return kind4(kind) ? 32 : (kind == KIND_I8 ? 16 : 8); }

// The fused path takes every format: K a multiple of 32, 16-byte aligned x
// and data, and (for scaled formats) a group that is a multiple of the
// piece length (32 for 4-bit codes, 16 for int8) and divides or is divided
// by K.
static int gemv_kind(int format) {
    switch (format) {
    case RNN_QF_INT4: case RNN_QF_GGUF_Q4: case RNN_QF_GGUF_Q4K: return KIND_I4;
    case RNN_QF_INT8: case RNN_QF_GGUF_Q8: return KIND_I8;
    case RNN_QF_FP16: return KIND_F16;
    case RNN_QF_BF16: return KIND_BF16;
    case RNN_QF_NF4: return KIND_NF4;
    case RNN_QF_NVFP4: return KIND_E2M1;
    default: return -1;
    }
}

extern "C" size_t rnn_qt_linear_workspace_size(int64_t in_f, int64_t out_f) {
    return in_f > 0 && out_f > 0 ? bf16_workspace(out_f) : 0;
}

extern "C" int rnn_qt_linear_forward_ws(int format, const float *x, int64_t m, int64_t in_f,
                                        const uint8_t *data, int64_t data_bytes,
                                        const float *scales, int64_t n_scales, int64_t group,
                                        int64_t out_f, const float *bias, float *y,
                                        void *workspace, size_t workspace_bytes, unsigned flags,
                                        void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_qt_linear_forward";
    RNN_REQUIRE(!workspace || (workspace_bytes >= rnn_qt_linear_workspace_size(in_f, out_f) &&
                               ((uintptr_t)workspace % 16) == 0),
                "%s: workspace of %zu bytes (or misaligned), %zu needed", name, workspace_bytes,
                rnn_qt_linear_workspace_size(in_f, out_f));
    RNN_REQUIRE(m >= 0 && in_f >= 0 && out_f >= 0, "%s: negative size", name);
    RNN_TRY(check_tensor(name, format, data, data_bytes, scales, n_scales, group, out_f * in_f));
    const unsigned algo = flags & RNN_ALGO_MASK;
    RNN_REQUIRE(algo == RNN_ALGO_AUTO || algo == RNN_ALGO_GEMV || algo == RNN_ALGO_TILED ||
                    algo == RNN_ALGO_GEMV_MFMA || algo == RNN_ALGO_GEMV_BF16,
                "%s: bad algo 0x%x", name, algo);
    if (m == 0 || out_f == 0) return RNN_OK;
    RNN_REQUIRE(y != nullptr && (in_f == 0 || x != nullptr), "%s: null pointer", name);
    hipStream_t st = as_stream(stream);
    if (in_f == 0) {  // empty sum: y = 0 (+ bias)
        qt_zero_kernel<<<grid_for(m * out_f, 256), 256, 0, st>>>(reinterpret_cast<uint32_t *>(y),
                                                                   m * out_f);
        if (bias) qt_bias_kernel<<<grid_for(m * out_f, 256), 256, 0, st>>>(y, m, out_f, bias);
        return check_launch(name);
    }
    const int kind = gemv_kind(format);
    const bool scaled = format != RNN_QF_FP16 && format != RNN_QF_BF16;
    const bool fits = kind >= 0 && in_f % 32 == 0 &&
                      (!scaled || (group % (kind4(kind) ? 32 : 16) == 0 && group <= 0xffffffffLL &&
                                   (in_f % group == 0 || group % in_f == 0))) &&
                      ((uintptr_t)x % 16) == 0 && ((uintptr_t)data % 16) == 0 &&
                      out_f <= 0x7fffffffLL;
    // the MFMA GEMV takes all m <= 16 rows at once; its 4 waves split K in
    // whole chunks of 4 pieces
    const bool fits_mfma = fits && m <= 16 && in_f % (kMfmaWaves * 4 * piece_elems(kind)) == 0;
    // the bf16 MFMA GEMV: integer codes and bf16 weights, whole chunks of
    // 4 pieces per group
    const int ep = kind >= 0 ? piece_elems(kind) : 32;
    auto bf16_fits = [&](int64_t rows) {
        return fits && rows <= 16 && (kind == KIND_I4 || kind == KIND_I8 || kind == KIND_BF16) &&
        in_f % (kBf16Waves * 4 * ep) == 0 &&
        (!scaled || (group % (4 * ep) == 0 && in_f % group == 0) || group % in_f == 0 ||
         // (groups of 32: a chunk's scales come in one vector load)
         (group == 32 && kind != KIND_BF16 && ((uintptr_t)scales % 16) == 0)) &&
        // (a scale for every group: the kernel reads a row's scales from the
        // row's first without the per-index clamp of a shortened array)
        (!scaled || n_scales >= ceil_div(out_f * in_f, group)) &&
        bf16_plan(rows, in_f, out_f, ep).S > 0 && 64 * in_f * 16 / ep < (int64_t(1) << 31) &&
        16 * in_f * 4 < (int64_t(1) << 31);
    };
    const bool fits_bf16 = bf16_fits(m);
    // m > 16: the GEMVs run on 16-row slices of x and y, one after the other,
    // each slice reading the weights again. A forced GEMV does so for every
    // m; AUTO does so while the slices beat dequantize + f32 GEMM (measured,
    // 4096 x 11008, slices against the latter: bf16 GEMV INT4 g128 m = 32
    // 29.9 us against 182, m = 512 467 against 554; GGUF Q8_0 m = 192 232
    // against 327, m = 256 316 against 306; BF16 m = 192 249 against 341,
    // m = 256 305 against 291; f32 MFMA GEMV NF4 g64 m = 96 157 against 178,
    // m = 128 208 against 194)
    if (m > 16 && algo != RNN_ALGO_TILED) {
        const int64_t lim = bf16_fits(16) ? (kind == KIND_I4 ? 512 : 192)
                            : fits && in_f % (kMfmaWaves * 4 * ep) == 0 ? 96
                                                                        : 32;
        if (algo != RNN_ALGO_AUTO || (fits && m <= lim)) {
            for (int64_t m0 = 0; m0 < m; m0 += 16)
                RNN_TRY(rnn_qt_linear_forward_ws(format, x + m0 * in_f, std::min<int64_t>(16, m - m0), in_f,
                                                 data, data_bytes, scales, n_scales, group, out_f,
                                                 bias, y + m0 * out_f, workspace, workspace_bytes,
                                                 flags, stream));
            return RNN_OK;
        }
    }
    // AUTO takes it for m >= 5, and for 4- and 8-bit codes at m = 3, 4 when
    // every CU gets at least two row tiles (measured, 4096 x 11008, m = 4:
    // INT4 g128 14.0 us against 16.3 for the VALU GEMV, GGUF Q4_0 15.8 against
    // 16.3, GGUF Q8_0 17.7 against 19.8, INT8 g64 16.7 against 19.8; at
    // N = 4096, one tile per CU, INT4 9.0 against 7.5, GGUF Q8_0 10.7 against
    // 9.1)
    const bool bf16_auto =
        fits_bf16 && (m >= 5 || (m >= 3 && (kind == KIND_I4 || kind == KIND_I8) &&
                                 bf16_plan(m, in_f, out_f, ep).TPW >= 2));
    if (algo == RNN_ALGO_GEMV_BF16 || (algo == RNN_ALGO_AUTO && bf16_auto)) {
        RNN_REQUIRE(fits_bf16, "%s: the bf16 MFMA GEMV needs INT4/Q4/INT8/Q8/BF16 weights, m <= 16, "
                    "in_f a multiple of %d, a group that is a multiple of %d dividing in_f (or a "
                    "multiple of in_f, or 32 for 4- and 8-bit codes with 16-byte aligned scales), a "
                    "scale for every group, and 16-byte aligned x and data", name, kBf16Waves * 4 * ep, 4 * ep);
        switch (kind) {
        case KIND_I4:
            return launch_bf16<KIND_I4, true>(x, (int)m, in_f, data, scales, n_scales, group, out_f,
                                              bias, y, workspace, st, name);
        case KIND_I8:
            return launch_bf16<KIND_I8, true>(x, (int)m, in_f, data, scales, n_scales, group, out_f,
                                              bias, y, workspace, st, name);
        default:
            return launch_bf16<KIND_BF16, false>(x, (int)m, in_f, data, scales, n_scales, 1, out_f,
                                                 bias, y, workspace, st, name);
        }
    }
    if (algo == RNN_ALGO_GEMV_MFMA || (algo == RNN_ALGO_AUTO && m >= 5 && fits_mfma)) {
        RNN_REQUIRE(fits_mfma, "%s: the MFMA GEMV needs m <= 16, the fused GEMV's conditions and "
                    "in_f a multiple of %d", name, kMfmaWaves * 4 * (kind >= 0 ? piece_elems(kind) : 32));
        launch_mfma_kind(kind, x, (int)m, in_f, data, scales, n_scales, group, out_f, bias, y, st);
        return check_launch(name);
    }
    const bool gemv = algo == RNN_ALGO_GEMV || (algo == RNN_ALGO_AUTO && m <= 16 && fits);
    if (gemv) {
        RNN_REQUIRE(fits, "%s: the fused GEMV needs in_f %% 32 == 0, a group that is a multiple of "
                    "32 (4-bit formats) or 16 (INT8, Q8) and divides or is divided by in_f, and "
                    "16-byte aligned x and data", name);
        for (int64_t m0 = 0; m0 < m; m0 += 4) {
            const int mt = (int)std::min<int64_t>(4, m - m0);
            const float *xs = x + m0 * in_f;
            float *ys = y + m0 * out_f;
            switch (kind) {
            case KIND_I4:
                gemv_chunk<KIND_I4, true>(mt, xs, in_f, data, scales, n_scales, group, out_f, bias,
                                          ys, st);
                break;
            case KIND_NF4:
                gemv_chunk<KIND_NF4, true>(mt, xs, in_f, data, scales, n_scales, group, out_f, bias,
                                           ys, st);
                break;
            case KIND_E2M1:
                gemv_chunk<KIND_E2M1, true>(mt, xs, in_f, data, scales, n_scales, group, out_f,
                                            bias, ys, st);
                break;
            case KIND_I8:
                gemv_chunk<KIND_I8, true>(mt, xs, in_f, data, scales, n_scales, group, out_f, bias,
                                          ys, st);
                break;
            case KIND_F16:
                gemv_chunk<KIND_F16, false>(mt, xs, in_f, data, scales, n_scales, 1, out_f, bias,
                                            ys, st);
                break;
            default:
                gemv_chunk<KIND_BF16, false>(mt, xs, in_f, data, scales, n_scales, 1, out_f, bias,
                                             ys, st);
                break;
            }
            RNN_TRY(check_launch(name));
        }
        return RNN_OK;
    }
    // Otherwise: W = dequantize() into stream-ordered scratch, y = x . W^T on
    // the f32 MFMA GEMM, then + bias -- the reference's own three steps.
    void *w = nullptr;
    RNN_TRY(check_hip(hipMallocAsync(&w, sizeof(float) * out_f * in_f, st), name));
    int rc = rnn_qt_dequantize(format, data, data_bytes, scales, n_scales, group, out_f * in_f,
                               static_cast<float *>(w), stream);
    if (rc == RNN_OK)
        rc = rnn_sgemm(0, 1, m, out_f, in_f, 1.0f, x, in_f, static_cast<const float *>(w), in_f,
                       0.0f, y, out_f, stream);
    if (rc == RNN_OK && bias) {
        qt_bias_kernel<<<grid_for(m * out_f, 256), 256, 0, st>>>(y, m, out_f, bias);
        rc = check_launch(name);
    }
    const int rf = check_hip(hipFreeAsync(w, st), name);
    return rc != RNN_OK ? rc : rf;
}

extern "C" int rnn_qt_linear_forward(int format, const float *x, int64_t m, int64_t in_f,
                                     const uint8_t *data, int64_t data_bytes, const float *scales,
                                     int64_t n_scales, int64_t group, int64_t out_f,
                                     const float *bias, float *y, unsigned flags, void *stream) {
    return rnn_qt_linear_forward_ws(format, x, m, in_f, data, data_bytes, scales, n_scales, group,
                                    out_f, bias, y, nullptr, 0, flags, stream);
}
