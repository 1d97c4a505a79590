// numerics.hpp -- device arithmetic that must round exactly like the Rust
// reference (every translation unit is compiled with -ffp-contract=off and
// correctly rounded fp32 division).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rnn {

// f32::clamp: NaN passes through.
__device__ __forceinline__ float clamp_rs(float x, float lo, float hi) {
    return x < lo ? lo : (x > hi ? hi : x);
}

// `f32 as i8` of a value already clamped to [-128, 127]; NaN -> 0.
__device__ __forceinline__ int8_t to_i8_rs(float v) {
    return v != v ? (int8_t)0 : (int8_t)(int)v;
}

// (t).round().clamp(-128.0, 127.0) as i8  -- roundf is half away from zero,
// like f32::round.
__device__ __forceinline__ int8_t quant_i8_from_ratio(float t) {
    return to_i8_rs(clamp_rs(roundf(t), -128.0f, 127.0f));
}

// (v / s).round().clamp(-128.0, 127.0) as i8 with an IEEE division.
__device__ __forceinline__ int8_t quant_i8(float v, float s) {
    return quant_i8_from_ratio(v / s);
}

// round(rv / scale) with the reference's rounding (IEEE-rounded quotient, then
// f32::round = half away from zero) from a multiply by inv ~= 1/scale
// (v_rcp_f32, 1 ulp): t = rv * inv is within 3 * 2^-23 |t| of the rounded
// quotient, so whenever t is farther than 4e-6 * (1 + |t|) from a
// half-integer both round to the same integer, and rint(t) is that integer
// (rint and round differ only at exact halves). Near a half-integer the exact
// division decides.
__device__ __forceinline__ float round_quotient(float rv, float scale, float inv) {
    const float t = rv * inv;
    const float r = rintf(t);
    if (__builtin_expect(fabsf(fabsf(t - r) - 0.5f) > __builtin_fmaf(fabsf(t), 4.0e-6f, 4.0e-6f), 1))
        return r;
    return roundf(rv / scale);
}

// Max over the (whole, active) wave of non-negative, non-NaN floats -- every
// caller folds |x| with fmaxf, which drops NaN as f32::max does. Such floats
// order as their bit patterns do as unsigned integers, so the reduction runs
// on DPP lane moves instead of six LDS permute round trips.
__device__ __forceinline__ float wave_max(float v) {
    return __uint_as_float(__reduce_max_sync(~0ull, __float_as_uint(v)));
}

// Block-wide max of non-negative values; `red` holds BLOCK/64 floats.
template <int BLOCK>
__device__ __forceinline__ float block_max(float v, float *red) {
    v = wave_max(v);
    const int wid = threadIdx.x / 64, lane = threadIdx.x % 64;
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < BLOCK / 64; ++i) m = fmaxf(m, red[i]);
    return m;
}

}  // namespace rnn
