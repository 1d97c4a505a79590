// rqattn.hip -- RotorQuant codes as a KV-cache format, and attention that
// reads that cache directly (Tensor::flash_attention, src/tensor.rs:618-672,
// over K and V stored by RotorQuant, src/quant.rs:116-239).
//
// Page layout. Per (batch*head) sequence the cache holds T = ceil(S/64) tiles
// of 64 positions. Inside a tile, position j = 4*q4 + r (q4 in 0..15, r in
// 0..3) of group g sits at ((tile*16 + q4)*ng + g)*4 + r, in two arrays:
//   codes  u16: the group's three codes as 4-bit two's complement nibbles
//          (c0 | c1 << 4 | c2 << 8), bits <= 4 only;
//   scales f32: the group's scale.
// A lane that owns group g reads four positions with one 16-byte (scales) and
// one 8-byte (codes) load, and the lanes of a wave read consecutive bytes.
// That is 258 bytes per vector at head_dim 128 (43 groups), against 512 in
// f32. Positions past S hold zero codes and scales and are masked.
//
// Attention without reconstructing K or V. RotorQuant reconstructs a group
// as K_g = R_g^T (c_g * s_g) (R_g the group's rotation). Then
//   q . K = sum_g s_g ((R_g q_g) . c_g),
//   sum_j p_j V_j = blockdiag(R_g^T) (sum_j p_j s_{j,g} c_{j,g}),
// so each query is rotated once, scores come straight from codes and
// scales, V is accumulated in the rotated domain and rotated back once at the
// end. Lane g of a wave owns group g: its rotated query and its three
// accumulators stay in registers. Per tile the 64 scores are summed over
// groups through LDS (a transpose), the softmax runs online per tile (as
// src/tensor.rs:640-654 does per key), and the probabilities go back through
// LDS to the group lanes. The waves of a workgroup take tiles round-robin and
// merge their (max, sum, accumulators) at the end.
#include "common.hpp"
#include "rotor.hpp"

namespace rnn {

constexpr int kTile = 64;
constexpr int kAttnWaves = 4;

__host__ __device__ inline int64_t rq_page_index(int64_t bh, int64_t T, int64_t ng, int64_t pos,
                                                 int64_t g) {
    const int64_t t = pos / kTile, j = pos % kTile;
    return (((bh * T + t) * 16 + j / 4) * ng + g) * 4 + (j % 4);
}

// One thread per (sequence, tile position, group).
__global__ void rq_kv_pack_kernel(const int8_t *__restrict__ codes, const float *__restrict__ scales,
                                  int64_t BH, int64_t S, int64_t ng, int64_t T,
                                  uint16_t *__restrict__ pc, float *__restrict__ ps) {
    const int64_t total = BH * T * kTile * ng;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t g = i % ng, pos = (i / ng) % (T * kTile), bh = i / (ng * T * kTile);
        const int64_t dst = rq_page_index(bh, T, ng, pos, g);
        uint16_t w = 0;
        float s = 0.0f;
        if (pos < S) {
            const int64_t row = bh * S + pos;
            const int8_t *c = codes + row * 3 * ng + 3 * g;
            w = (uint16_t)((c[0] & 15) | ((c[1] & 15) << 4) | ((c[2] & 15) << 8));
            s = scales[row * ng + g];
        }
        pc[dst] = w;
        ps[dst] = s;
    }
}

typedef float f4v __attribute__((ext_vector_type(4)));
typedef unsigned int u2v __attribute__((ext_vector_type(2)));

// code c (0..2) of a packed group word, sign-extended
__device__ __forceinline__ float rq_code(uint32_t w, int c) {
    return (float)(((int32_t)(w << (28 - 4 * c))) >> 28);
}

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// One tile's codes and scales for this lane's group: 16 quads of 4 positions.
struct RqTile {
    f4v s[16];
    u2v c[16];
};

__device__ __forceinline__ void rq_load_tile(RqTile &t, const uint16_t *__restrict__ pc,
                                             const float *__restrict__ ps, int64_t base,
                                             int64_t ng, int g) {
#pragma unroll
    for (int q4 = 0; q4 < 16; ++q4) {
        const int64_t idx = base + ((int64_t)q4 * ng + g) * 4;
        t.s[q4] = *reinterpret_cast<const f4v *>(ps + idx);
        t.c[q4] = *reinterpret_cast<const u2v *>(pc + idx);
    }
}

__device__ __forceinline__ uint32_t quad_word(const u2v c, int r) {
    const uint32_t w = r < 2 ? c.x : c.y;
    return (r & 1) ? (w >> 16) : (w & 0xFFFFu);
}

// grid: BH * nq workgroups of kAttnWaves waves; dim <= 192 (ng <= 64).
__global__ __launch_bounds__(kAttnWaves * 64) void rq_kv_attn_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const float *__restrict__ ks,
    const uint16_t *__restrict__ vc, const float *__restrict__ vs, const float *__restrict__ krot,
    const float *__restrict__ vrot, int64_t nq, int64_t S, int64_t dim, int64_t ng, int64_t T,
    float scale, float *__restrict__ out) {
    // red: per wave, 64 score terms per group, the slot of position j in row
    // g swizzled to j ^ 4*(g & 15) (conflict-free 16-byte writes by group
    // lanes and 4-byte reads by position lanes); pb: the tile's probabilities.
    __shared__ __attribute__((aligned(16))) float red[kAttnWaves][64 * 64];
    __shared__ __attribute__((aligned(16))) float pb[kAttnWaves][64];
    __shared__ float mrg[kAttnWaves][2 + 3 * 64];
    const int wid = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int64_t bh = blockIdx.x / nq, qi = blockIdx.x % nq;
    const int g = lane < ng ? lane : (int)ng - 1;  // lanes past the groups mirror the last one
    const bool gact = lane < ng;

    // rotated query of this lane's group: q'_g = R_g q_g (zero past dim)
    float qr[3];
    {
        float R[9];
        rotation_matrix(krot + 4 * g, R);
        const float *qrow = q + (bh * nq + qi) * dim;
        float x[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {  // unconditional load (index clamped), zero past dim
            const int64_t d = 3 * g + c;
            const float v = qrow[d < dim ? d : dim - 1];
            x[c] = d < dim ? v : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 3; ++i) qr[i] = R[3 * i] * x[0] + R[3 * i + 1] * x[1] + R[3 * i + 2] * x[2];
    }
    float m = -INFINITY, l = 0.0f, a0 = 0.0f, a1 = 0.0f, a2 = 0.0f;
    float *rw = red[wid];
    const int sw = 4 * (g & 15);

    RqTile K, V;
    int t = wid;
    const int64_t seq = bh * T;
    if (t < T) {
        rq_load_tile(K, kc, ks, (seq + t) * 16 * ng * 4, ng, g);
        rq_load_tile(V, vc, vs, (seq + t) * 16 * ng * 4, ng, g);
    }
    for (; t < T; t += kAttnWaves) {
        // the next tile, or this one again at the end (an L2 hit): the loads
        // stay unconditional so that the compiler's waits stay exact
        const int tn = t + kAttnWaves < T ? t + kAttnWaves : t;
        // score terms of the 64 positions for this group
#pragma unroll
        for (int q4 = 0; q4 < 16; ++q4) {
            f4v term;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t w = quad_word(K.c[q4], r);
                const float d = qr[0] * rq_code(w, 0) + qr[1] * rq_code(w, 1) + qr[2] * rq_code(w, 2);
                term[r] = K.s[q4][r] * d;
            }
            if (gact) *reinterpret_cast<f4v *>(&rw[g * 64 + ((4 * q4) ^ sw)]) = term;
        }
        rq_load_tile(K, kc, ks, (seq + tn) * 16 * ng * 4, ng, g);
        __builtin_amdgcn_wave_barrier();
        // lane = position: sum over groups, scale, mask, online softmax
        float sc = 0.0f;
        for (int gg = 0; gg < ng; ++gg) sc += rw[gg * 64 + (lane ^ (4 * (gg & 15)))];
        sc *= scale;
        if ((int64_t)t * kTile + lane >= S) sc = -INFINITY;
        const float mt = wave_max_f(sc);
        const float mn = fmaxf(m, mt);
        const float corr = expf(m - mn);  // 0 on the first tile (m = -inf)
        const float p = expf(sc - mn);    // 0 for masked positions
        l = l * corr + p;
        m = mn;
        pb[wid][lane] = p;
        __builtin_amdgcn_wave_barrier();
        // V in the rotated domain: acc_g = acc_g * corr + sum_j p_j s_jg c_jg
        a0 *= corr, a1 *= corr, a2 *= corr;
#pragma unroll
        for (int q4 = 0; q4 < 16; ++q4) {
            const f4v p4 = *reinterpret_cast<const f4v *>(&pb[wid][4 * q4]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t w = quad_word(V.c[q4], r);
                const float ws = p4[r] * V.s[q4][r];
                a0 = __builtin_fmaf(ws, rq_code(w, 0), a0);
                a1 = __builtin_fmaf(ws, rq_code(w, 1), a1);
                a2 = __builtin_fmaf(ws, rq_code(w, 2), a2);
            }
        }
        rq_load_tile(V, vc, vs, (seq + tn) * 16 * ng * 4, ng, g);
        __builtin_amdgcn_wave_barrier();
    }
    // merge the waves: M = max m_w, L = sum l_w e^(m_w - M), A = sum a_w e^(m_w - M)
    l = wave_sum_f(l);
    if (lane == 0) mrg[wid][0] = m, mrg[wid][1] = l;
    mrg[wid][2 + 3 * lane] = a0, mrg[wid][3 + 3 * lane] = a1, mrg[wid][4 + 3 * lane] = a2;
    __syncthreads();
    if (wid != 0) return;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, mrg[w][0]);
    float L = 0.0f, A0 = 0.0f, A1 = 0.0f, A2 = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            const float mw = mrg[w][0];
            const float f = mw == -INFINITY ? 0.0f : expf(mw - M);
            L = L + f * mrg[w][1];
            A0 = A0 + f * mrg[w][2 + 3 * lane];
            A1 = A1 + f * mrg[w][3 + 3 * lane];
            A2 = A2 + f * mrg[w][4 + 3 * lane];
        }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;  // src/tensor.rs:657
    if (!gact) return;
    float R[9];
    rotation_matrix(vrot + 4 * g, R);
    float *orow = out + (bh * nq + qi) * dim;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float o = (R[c] * A0 + R[3 + c] * A1 + R[6 + c] * A2) * inv;  // R^T A, then * inv
        if (3 * g + c < dim) orow[3 * g + c] = o;
    }
}

}  // namespace rnn

using namespace rnn;

extern "C" int rnn_rotorquant_kv_page_elems(int64_t bh, int64_t seq, int64_t dim, int64_t *elems) {
    RNN_REQUIRE(bh >= 0 && seq >= 0 && dim > 0 && elems, "rnn_rotorquant_kv_page_elems: bad argument");
    *elems = bh * ceil_div(seq, kTile) * kTile * ceil_div(dim, 3);
    return RNN_OK;
}

extern "C" int rnn_rotorquant_kv_pack(const int8_t *codes, const float *scales, int64_t bh,
                                      int64_t seq, int64_t dim, int bits, uint16_t *page_codes,
                                      float *page_scales, void *stream) {
    const char *name = "rnn_rotorquant_kv_pack";
    RNN_REQUIRE(bh >= 0 && seq >= 0 && dim > 0, "%s: bad size", name);
    RNN_REQUIRE(bits >= 2 && bits <= 4, "%s: the page stores 4-bit codes (bits 2..4), got %d", name,
                bits);
    if (bh == 0 || seq == 0) return RNN_OK;
    RNN_REQUIRE(codes && scales && page_codes && page_scales, "%s: null pointer", name);
    const int64_t ng = ceil_div(dim, 3), T = ceil_div(seq, kTile);
    const int64_t total = bh * T * kTile * ng;
    const int blocks = (int)std::min<int64_t>(ceil_div(total, 256), 8 * (int64_t)device_cu_count());
    rq_kv_pack_kernel<<<blocks, 256, 0, as_stream(stream)>>>(codes, scales, bh, seq, ng, T,
                                                             page_codes, page_scales);
    return check_launch(name);
}

extern "C" int rnn_rotorquant_kv_attention(const float *q, int64_t bh, int64_t nq,
                                           const uint16_t *k_codes, const float *k_scales,
                                           const uint16_t *v_codes, const float *v_scales,
                                           const float *k_rotors, const float *v_rotors,
                                           int64_t seq, int64_t dim, float scale, float *out,
                                           void *stream) {
    const char *name = "rnn_rotorquant_kv_attention";
    RNN_REQUIRE(bh >= 0 && nq >= 0 && seq >= 0 && dim > 0, "%s: bad size", name);
    RNN_REQUIRE(dim <= 192, "%s: head dim %lld > 192 (at most 64 groups per wave)", name,
                (long long)dim);
    if (bh == 0 || nq == 0) return RNN_OK;
    RNN_REQUIRE(q && out && k_rotors && v_rotors, "%s: null pointer", name);
    RNN_REQUIRE(seq == 0 || (k_codes && k_scales && v_codes && v_scales), "%s: null page", name);
    RNN_REQUIRE(((uintptr_t)k_scales % 16) == 0 && ((uintptr_t)v_scales % 16) == 0 &&
                    ((uintptr_t)k_codes % 8) == 0 && ((uintptr_t)v_codes % 8) == 0,
                "%s: pages must be 16-byte (scales) and 8-byte (codes) aligned", name);
    RNN_REQUIRE(bh * nq <= 0x7fffffffLL, "%s: too many queries", name);
    const int64_t ng = ceil_div(dim, 3), T = ceil_div(seq, kTile);
    rq_kv_attn_kernel<<<(unsigned)(bh * nq), kAttnWaves * 64, 0, as_stream(stream)>>>(
        q, k_codes, k_scales, v_codes, v_scales, k_rotors, v_rotors, nq, seq, dim, ng, T, scale, out);
    return check_launch(name);
}
