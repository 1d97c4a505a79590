// rqattn.hip -- RotorQuant codes as a KV-cache format, and attention that
// reads that cache directly (Tensor::flash_attention, src/tensor.rs:618-672,
// over K and V stored by RotorQuant, src/quant.rs:116-239).
//
// Page layout. Per (batch*head) sequence the cache holds T = ceil(S/64) tiles
// of 64 positions, in two arrays: codes, a u16 per position and group holding
// the group's three codes as 4-bit two's complement nibbles (c0 | c1 << 4 |
// c2 << 8, bits <= 4 only), and scales, an f32 per position and group. The
// order inside a tile depends on which lanes read it:
//   K pages (a lane per position): scales of groups 4a..4a+3 of position j
//     side by side at ((tile*ng4 + a)*64 + j)*4, codes of groups 8b..8b+7 at
//     ((tile*ng8 + b)*64 + j)*8 (ng4 = ceil(ng/4), ng8 = ceil(ng/8); the
//     groups past ng are padding).
//   V pages (a lane per group): the scale of position j = 4*q4 + r, group g
//     at ((tile*16 + q4)*ng + g)*4 + r; its code at ((tile*8 + j/8)*ng + g)*8
//     + j%8.
// Every load instruction reads 16 consecutive bytes per lane, consecutive
// across the lanes; a wave's tile takes 17 loads for K and 24 for V, within
// the 63 a wave can have in flight. 6 bytes per position and group (plus
// the K padding): 272 bytes per K vector and 258 per V vector at head_dim 128
// (43 groups), against 512 in f32. Positions past S hold zero codes and
// scales and are masked.
//
// Attention without reconstructing K or V. RotorQuant reconstructs a group
// as K_g = R_g^T (c_g * s_g) (R_g the group's rotation). Then
//   q . K = sum_g s_g ((R_g q_g) . c_g),
//   sum_j p_j V_j = blockdiag(R_g^T) (sum_j p_j s_{j,g} c_{j,g}),
// so each query is rotated once, scores come straight from codes and
// scales, V is accumulated in the rotated domain and rotated back once at the
// end. Scores: a lane per position (all 64 busy), the rotated query read from
// LDS by broadcast. V: a lane per group, which keeps its three rotated
// accumulators in registers; the tile's probabilities reach it through LDS.
// The softmax runs online per tile (as src/tensor.rs:640-654 does per key).
// The waves of a workgroup take tiles round-robin and merge their (max, sum,
// accumulators) at the end.
#include "common.hpp"
#include "rotor.hpp"

#include <atomic>

namespace rnn {

constexpr int kTile = 64;
constexpr int kAttnWaves = 4;
// Sequence splits: at most kMaxSplits, each of at least kAttnWaves tiles.
constexpr int kMaxSplits = 16;

enum { RQ_PAGE_K = 0, RQ_PAGE_V = 1 };

// Indices of (sequence sq, position pos, group g) in the code (u16) and scale
// arrays of a page of the given kind; T tiles per sequence.
__host__ __device__ inline void rq_page_pos(int kind, int64_t sq, int64_t T, int64_t ng,
                                            int64_t pos, int64_t g, int64_t &ci, int64_t &si) {
    const int64_t t = sq * T + pos / kTile, j = pos % kTile;
    if (kind == RQ_PAGE_K) {
        const int64_t ng4 = (ng + 3) / 4, ng8 = (ng + 7) / 8;
        si = ((t * ng4 + g / 4) * 64 + j) * 4 + (g % 4);
        ci = ((t * ng8 + g / 8) * 64 + j) * 8 + (g % 8);
    } else {
        si = ((t * 16 + j / 4) * ng + g) * 4 + (j % 4);
        ci = ((t * 8 + j / 8) * ng + g) * 8 + (j % 8);
    }
}

// One thread per (sequence, tile position, group incl. the K padding).
__global__ void rq_kv_pack_kernel(int kind, const int8_t *__restrict__ codes,
                                  const float *__restrict__ scales, int64_t BH, int64_t S,
                                  int64_t ng, int64_t T, uint16_t *__restrict__ pc,
                                  float *__restrict__ ps) {
    const int64_t ngw = kind == RQ_PAGE_K ? 8 * ((ng + 7) / 8) : ng;
    const int64_t total = BH * T * kTile * ngw;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t g = i % ngw, pos = (i / ngw) % (T * kTile), sq = i / (ngw * T * kTile);
        int64_t ci, si;
        rq_page_pos(kind, sq, T, ng, pos, g, ci, si);
        uint16_t w = 0;
        float sc = 0.0f;
        if (pos < S && g < ng) {
            const int64_t row = sq * S + pos;
            const int8_t *c = codes + row * 3 * ng + 3 * g;
            w = (uint16_t)((c[0] & 15) | ((c[1] & 15) << 4) | ((c[2] & 15) << 8));
            sc = scales[row * ng + g];
        }
        pc[ci] = w;
        if (kind == RQ_PAGE_V ? g < ng : g < 4 * ((ng + 3) / 4)) ps[si] = sc;
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

// A V tile for this lane's group: 16 quads of 4 positions.
struct RqTileV {
    f4v s[16];
    v4i c[8];
};

__device__ __forceinline__ void rq_load_v(RqTileV &t, const uint16_t *__restrict__ pc,
                                          const float *__restrict__ ps, int64_t tile, int64_t ng,
                                          int g) {
#pragma unroll
    for (int q4 = 0; q4 < 16; ++q4)
        t.s[q4] = *reinterpret_cast<const f4v *>(ps + ((tile * 16 + q4) * ng + g) * 4);
#pragma unroll
    for (int q8 = 0; q8 < 8; ++q8)
        t.c[q8] = *reinterpret_cast<const v4i *>(pc + ((tile * 8 + q8) * ng + g) * 8);
}

// A K tile for this lane's position: the scales of NG4 x 4 groups and the
// codes of NG8 x 8 groups (groups past ng are padding; their terms are
// dropped). Blocks past the page's own count re-read its last one.
template <int NG4, int NG8>
struct RqTileK {
    f4v s[NG4];
    v4i c[NG8];
};

template <int NG4, int NG8>
__device__ __forceinline__ void rq_load_k(RqTileK<NG4, NG8> &t, const uint16_t *__restrict__ pc,
                                          const float *__restrict__ ps, int64_t tile, int64_t ng,
                                          int lane) {
    const int64_t ng4 = (ng + 3) / 4, ng8 = (ng + 7) / 8;
#pragma unroll
    for (int a = 0; a < NG4; ++a)
        t.s[a] = *reinterpret_cast<const f4v *>(ps + ((tile * ng4 + (a < ng4 ? a : ng4 - 1)) * 64 + lane) * 4);
#pragma unroll
    for (int b = 0; b < NG8; ++b) {
        const uint16_t *p = pc + ((tile * ng8 + (b < ng8 ? b : ng8 - 1)) * 64 + lane) * 8;
        if (b == NG8 - 1 && 4 * NG4 <= 8 * b + 4) {
            // only the block's first 4 groups are scored: an 8-byte load, so
            // that no register of the tile is dead (the compiler would reuse
            // it and wait for every outstanding load before the write)
            const u2v h = *reinterpret_cast<const u2v *>(p);
            t.c[b] = v4i{(int)h.x, (int)h.y, 0, 0};
        } else {
            t.c[b] = *reinterpret_cast<const v4i *>(p);
        }
    }
}


// grid: (BH * nq, splits) workgroups of kAttnWaves waves; ng <= 4 * NG4 <= 8
// * NG8 <= 64. Split y takes tiles [y * tps, min(T, (y + 1) * tps)). With
// several splits (part != null) each writes its unnormalised state (max,
// sum, rotated accumulators) to part and counts itself in at cnt[query];
// the last of a query's splits merges the states in split order (M = max
// m_s, L = sum l_s e^(m_s - M), A = sum a_s e^(m_s - M)), writes the output
// and resets the count.
// The states are device-scope atomic stores, written through the XCD's L2
// to the device's coherence point and complete (vmcnt 0) before the count;
// the last split reads them with device-scope atomic loads. No workgroup
// waits for another.
template <int NG4, int NG8>
__global__ __launch_bounds__(kAttnWaves * 64) void rq_kv_attn_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const float *__restrict__ ks,
    const uint16_t *__restrict__ vc, const float *__restrict__ vs, const float *__restrict__ krot,
    const float *__restrict__ vrot, int64_t nq, int64_t S, int64_t dim, int64_t ng, int64_t T,
    int64_t tps, float scale, float *__restrict__ out, float *__restrict__ part,
    uint32_t *__restrict__ cnt) {
    __shared__ __attribute__((aligned(16))) float qs[4 * 64];  // rotated query, 4 floats per group
    __shared__ __attribute__((aligned(16))) float pb[kAttnWaves][64];
    __shared__ float mrg[kAttnWaves][2 + 3 * 64];
    const int wid = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int64_t bh = blockIdx.x / nq, qi = blockIdx.x % nq;
    const int g = lane < ng ? lane : (int)ng - 1;  // group lanes past ng mirror the last one
    const bool gact = lane < ng;

    const int64_t seq = bh * T;
    // this split's tiles [tb, te); the waves take them round-robin. The first
    // tile's loads are issued before the query is rotated.
    const int64_t tb = blockIdx.y * tps, te = tb + tps < T ? tb + tps : T;
    const int64_t nt = wid < te - tb ? (te - tb - wid + kAttnWaves - 1) / kAttnWaves : 0;
    const int64_t last = tb + wid + (nt - 1) * kAttnWaves;
    RqTileK<NG4, NG8> K;
    RqTileV V;
    if (nt > 0) {
        rq_load_k<NG4, NG8>(K, kc, ks, seq + tb + wid, ng, lane);
        rq_load_v(V, vc, vs, seq + tb + wid, ng, g);
    }

    // rotated query q'_g = R_g q_g (zero past dim), published in LDS
    if (wid == 0) {
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
        f4v qv;
#pragma unroll
        for (int i = 0; i < 3; ++i)
            qv[i] = gact ? R[3 * i] * x[0] + R[3 * i + 1] * x[1] + R[3 * i + 2] * x[2] : 0.0f;
        qv[3] = 0.0f;
        *reinterpret_cast<f4v *>(&qs[4 * lane]) = qv;
    }
    // a barrier over LDS only: the tile loads stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    float m = -INFINITY, l = 0.0f, a0 = 0.0f, a1 = 0.0f, a2 = 0.0f;
    for (int64_t i = 0; i < nt; ++i) {
        const int64_t t = tb + wid + i * kAttnWaves;
        // the next tile, or this one again at the end (an L2 hit): the loads
        // stay unconditional so that the compiler's waits stay exact
        const int64_t tn = t + kAttnWaves <= last ? t + kAttnWaves : t;
        // lane = position: score = scale * sum_g s_g (q'_g . c_g)
        float sc = 0.0f;
#pragma unroll
        for (int gg = 0; gg < 4 * NG4; ++gg) {
            const f4v qv = *reinterpret_cast<const f4v *>(&qs[4 * (gg < ng ? gg : 0)]);
            const uint32_t word = (uint32_t)K.c[gg / 8][(gg % 8) / 2];
            const uint32_t w = (gg & 1) ? (word >> 16) : word;
            float d = qv[0] * rq_code(w, 0);
            d = __builtin_fmaf(qv[1], rq_code(w, 1), d);
            d = __builtin_fmaf(qv[2], rq_code(w, 2), d);
            const float sg = gg < ng ? K.s[gg / 4][gg % 4] : 0.0f;
            sc = __builtin_fmaf(sg, d, sc);
        }
        rq_load_k<NG4, NG8>(K, kc, ks, seq + tn, ng, lane);
        sc *= scale;
        if (t * kTile + lane >= S) sc = -INFINITY;
        const float mt = wave_max_f(sc);
        const float mn = fmaxf(m, mt);
        const float corr = expf(m - mn);  // 0 on the first tile (m = -inf)
        const float p = expf(sc - mn);    // 0 for masked positions
        l = l * corr + p;
        m = mn;
        pb[wid][lane] = p;
        __builtin_amdgcn_wave_barrier();  // one wave's LDS operations complete in order
        // lane = group: acc_g = acc_g * corr + sum_j p_j s_jg c_jg (rotated domain)
        a0 *= corr, a1 *= corr, a2 *= corr;
#pragma unroll
        for (int q4 = 0; q4 < 16; ++q4) {
            const f4v p4 = *reinterpret_cast<const f4v *>(&pb[wid][4 * q4]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t word = (uint32_t)V.c[q4 / 2][2 * (q4 & 1) + r / 2];
                const uint32_t w = (r & 1) ? (word >> 16) : (word & 0xFFFFu);
                const float ws = p4[r] * V.s[q4][r];
                a0 = __builtin_fmaf(ws, rq_code(w, 0), a0);
                a1 = __builtin_fmaf(ws, rq_code(w, 1), a1);
                a2 = __builtin_fmaf(ws, rq_code(w, 2), a2);
            }
        }
        rq_load_v(V, vc, vs, seq + tn, ng, g);
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
    if (part) {
        const int64_t qrow = bh * nq + qi, stride = 2 + 3 * ng;
        const int ns = (int)gridDim.y;
        float *pp = part + (qrow * ns + blockIdx.y) * stride;
        if (lane == 0) {
            __hip_atomic_store(pp, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pp + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (gact) {
            __hip_atomic_store(pp + 2 + 3 * g, A0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pp + 3 + 3 * g, A1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pp + 4 + 3 * g, A2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        uint32_t old = 0;
        if (lane == 0)
            old = __hip_atomic_fetch_add(&cnt[qrow], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__shfl(old, 0, 64) != (uint32_t)ns - 1) return;
        // the last split: every state's loads in flight, then merged in split order
        float mv[kMaxSplits], lv[kMaxSplits], av[kMaxSplits][3];
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s) {
            const float *ps = part + (qrow * ns + (s < ns ? s : ns - 1)) * stride;
            mv[s] = __hip_atomic_load(ps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            lv[s] = __hip_atomic_load(ps + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int c = 0; c < 3; ++c)
                av[s][c] = __hip_atomic_load(ps + 2 + 3 * g + c, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        }
        if (lane == 0)  // ready for the next call
            __hip_atomic_store(&cnt[qrow], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        M = -INFINITY;
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s)
            if (s < ns) M = fmaxf(M, mv[s]);
        L = 0.0f, A0 = 0.0f, A1 = 0.0f, A2 = 0.0f;
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s)
            if (s < ns) {
                const float f = (M == -INFINITY || mv[s] == -INFINITY) ? 0.0f : expf(mv[s] - M);
                L = L + f * lv[s];
                A0 = A0 + f * av[s][0];
                A1 = A1 + f * av[s][1];
                A2 = A2 + f * av[s][2];
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

// Head dims past 192 (more than 64 groups). The same online softmax; the
// scores loop over the K page's 8-group blocks with the rotated query in LDS
// (16 bytes per group), and V takes the workgroup's range of at most
// kWideRange groups 64 at a time, a lane per group, each wave's accumulators
// kept in LDS between tiles. grid: (BH * nq, ceil(ng / kWideRange), splits);
// every workgroup of a query scores all groups and accumulates its own range
// over its split's tiles (as rq_kv_attn_kernel, part != null: the split's
// state, the first range writing the max and sum).
constexpr int kWideRange = 256;

__global__ __launch_bounds__(kAttnWaves * 64) void rq_kv_attn_wide_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const float *__restrict__ ks,
    const uint16_t *__restrict__ vc, const float *__restrict__ vs, const float *__restrict__ krot,
    const float *__restrict__ vrot, int64_t nq, int64_t S, int64_t dim, int64_t ng, int64_t T,
    int64_t tps, float scale, float *__restrict__ out, float *__restrict__ part,
    uint32_t *__restrict__ cnt) {
    extern __shared__ __attribute__((aligned(16))) float dyn[];
    __shared__ __attribute__((aligned(16))) float pb[kAttnWaves][64];
    __shared__ float mrg[kAttnWaves][2];
    __shared__ float sml[2][kMaxSplits];
    __shared__ uint32_t last;
    const int64_t ng4 = (ng + 3) / 4, ng8 = (ng + 7) / 8;
    float *qs = dyn;               // rotated query: 4 floats per group, 8 * ng8 groups, zero past ng
    float *acc = dyn + 32 * ng8;   // [kAttnWaves][3 * kWideRange]
    const int wid = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int64_t bh = blockIdx.x / nq, qi = blockIdx.x % nq;
    const int64_t g0 = (int64_t)blockIdx.y * kWideRange;
    const int nr = (int)(ng - g0 < kWideRange ? ng - g0 : kWideRange);  // groups of this range
    const float *qrow = q + (bh * nq + qi) * dim;
    for (int64_t g = threadIdx.x; g < 8 * ng8; g += kAttnWaves * 64) {
        f4v qv = {0.0f, 0.0f, 0.0f, 0.0f};
        if (g < ng) {
            float R[9];
            rotation_matrix(krot + 4 * g, R);
            float x[3];
#pragma unroll
            for (int c = 0; c < 3; ++c) x[c] = 3 * g + c < dim ? qrow[3 * g + c] : 0.0f;
#pragma unroll
            for (int i = 0; i < 3; ++i) qv[i] = R[3 * i] * x[0] + R[3 * i + 1] * x[1] + R[3 * i + 2] * x[2];
        }
        *reinterpret_cast<f4v *>(&qs[4 * g]) = qv;
    }
    for (int i = threadIdx.x; i < kAttnWaves * 3 * kWideRange; i += kAttnWaves * 64) acc[i] = 0.0f;
    __syncthreads();
    float *aw = acc + wid * 3 * kWideRange;
    float m = -INFINITY, l = 0.0f;
    const int64_t tb = blockIdx.z * tps, te = tb + tps < T ? tb + tps : T;
    for (int64_t t = tb + wid; t < te; t += kAttnWaves) {
        const int64_t tile = bh * T + t;
        // lane = position: score = scale * sum_g s_g (q'_g . c_g), 8 groups a block
        const uint16_t *pcb = kc + (tile * ng8 * 64 + lane) * 8;
        const float *psb = ks + (tile * ng4 * 64 + lane) * 4;
        float sc = 0.0f;
        for (int64_t b = 0; b < ng8; ++b) {
            const v4i c = *reinterpret_cast<const v4i *>(pcb + b * 64 * 8);
            const bool two = 2 * b + 1 < ng4;  // the block's second 4 scales exist
            const f4v s0 = *reinterpret_cast<const f4v *>(psb + 2 * b * 64 * 4);
            const f4v s1 = *reinterpret_cast<const f4v *>(psb + (two ? 2 * b + 1 : 2 * b) * 64 * 4);
#pragma unroll
            for (int gg = 0; gg < 8; ++gg) {
                const f4v qv = *reinterpret_cast<const f4v *>(&qs[4 * (8 * b + gg)]);
                const uint32_t word = (uint32_t)c[gg / 2];
                const uint32_t w = (gg & 1) ? (word >> 16) : word;
                float d = qv[0] * rq_code(w, 0);
                d = __builtin_fmaf(qv[1], rq_code(w, 1), d);
                d = __builtin_fmaf(qv[2], rq_code(w, 2), d);
                const float sg = 8 * b + gg < ng ? (gg < 4 ? s0[gg] : s1[gg - 4]) : 0.0f;
                sc = __builtin_fmaf(sg, d, sc);
            }
        }
        sc *= scale;
        if (t * kTile + lane >= S) sc = -INFINITY;
        const float mt = wave_max_f(sc);
        const float mn = fmaxf(m, mt);
        const float corr = expf(m - mn);  // 0 on the first tile (m = -inf)
        const float p = expf(sc - mn);    // 0 for masked positions
        l = l * corr + p;
        m = mn;
        pb[wid][lane] = p;
        __builtin_amdgcn_wave_barrier();  // one wave's LDS operations complete in order
        // lane = group of the range: acc_g = acc_g * corr + sum_j p_j s_jg c_jg
        for (int c0 = 0; c0 < nr; c0 += 64) {
            const int gl = c0 + lane;
            if (gl < nr) {
                RqTileV V;
                rq_load_v(V, vc, vs, tile, ng, (int)(g0 + gl));
                float a0 = aw[3 * gl] * corr, a1 = aw[3 * gl + 1] * corr, a2 = aw[3 * gl + 2] * corr;
#pragma unroll
                for (int q4 = 0; q4 < 16; ++q4) {
                    const f4v p4 = *reinterpret_cast<const f4v *>(&pb[wid][4 * q4]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint32_t word = (uint32_t)V.c[q4 / 2][2 * (q4 & 1) + r / 2];
                        const uint32_t w = (r & 1) ? (word >> 16) : (word & 0xFFFFu);
                        const float ws = p4[r] * V.s[q4][r];
                        a0 = __builtin_fmaf(ws, rq_code(w, 0), a0);
                        a1 = __builtin_fmaf(ws, rq_code(w, 1), a1);
                        a2 = __builtin_fmaf(ws, rq_code(w, 2), a2);
                    }
                }
                aw[3 * gl] = a0, aw[3 * gl + 1] = a1, aw[3 * gl + 2] = a2;
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    // merge the waves: M = max m_w, L = sum l_w e^(m_w - M), A = sum a_w e^(m_w - M)
    l = wave_sum_f(l);
    if (lane == 0) mrg[wid][0] = m, mrg[wid][1] = l;
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, mrg[w][0]);
    float f[kAttnWaves], L = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
        const float mw = mrg[w][0];
        f[w] = (M == -INFINITY || mw == -INFINITY) ? 0.0f : expf(mw - M);
        L = L + f[w] * mrg[w][1];
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;  // src/tensor.rs:657
    float *orow = out + (bh * nq + qi) * dim;
    if (part) {
        // this split's state (every range writes the same max and sum: the
        // scores are computed alike), counted in per (query, range); the
        // last split of the range merges them, as in rq_kv_attn_kernel
        const int64_t qrow = bh * nq + qi, stride = 2 + 3 * ng;
        const int ns = (int)gridDim.z;
        float *pp = part + (qrow * ns + blockIdx.z) * stride;
        if (threadIdx.x == 0) {
            __hip_atomic_store(pp, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pp + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        for (int gl = threadIdx.x; gl < nr; gl += kAttnWaves * 64) {
            float A[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w = 0; w < kAttnWaves; ++w)
#pragma unroll
                for (int c = 0; c < 3; ++c) A[c] = A[c] + f[w] * acc[w * 3 * kWideRange + 3 * gl + c];
#pragma unroll
            for (int c = 0; c < 3; ++c)
                __hip_atomic_store(pp + 2 + 3 * (g0 + gl) + c, A[c], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        uint32_t *cq = cnt + qrow * gridDim.y + blockIdx.y;
        if (threadIdx.x == 0)
            last = __hip_atomic_fetch_add(cq, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (uint32_t)ns - 1;
        __syncthreads();
        if (!last) return;
        if (threadIdx.x < kMaxSplits) {
            const float *ps = part + (qrow * ns + (threadIdx.x < ns ? threadIdx.x : ns - 1)) * stride;
            sml[0][threadIdx.x] = __hip_atomic_load(ps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sml[1][threadIdx.x] = __hip_atomic_load(ps + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (threadIdx.x == 0)  // ready for the next call
            __hip_atomic_store(cq, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        float Ms = -INFINITY;
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s)
            if (s < ns) Ms = fmaxf(Ms, sml[0][s]);
        float fs[kMaxSplits], Ls = 0.0f;
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s) {
            fs[s] = 0.0f;
            if (s < ns) {
                fs[s] = (Ms == -INFINITY || sml[0][s] == -INFINITY) ? 0.0f : expf(sml[0][s] - Ms);
                Ls = Ls + fs[s] * sml[1][s];
            }
        }
        const float invs = Ls > 0.0f ? 1.0f / Ls : 0.0f;  // src/tensor.rs:657
        for (int gl = threadIdx.x; gl < nr; gl += kAttnWaves * 64) {
            const int64_t g = g0 + gl;
            float av[kMaxSplits][3];
#pragma unroll
            for (int s = 0; s < kMaxSplits; ++s)
#pragma unroll
                for (int c = 0; c < 3; ++c)
                    av[s][c] = __hip_atomic_load(part + (qrow * ns + (s < ns ? s : ns - 1)) * stride +
                                                     2 + 3 * g + c,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            float A0 = 0.0f, A1 = 0.0f, A2 = 0.0f;
#pragma unroll
            for (int s = 0; s < kMaxSplits; ++s)
                if (s < ns) {
                    A0 = A0 + fs[s] * av[s][0];
                    A1 = A1 + fs[s] * av[s][1];
                    A2 = A2 + fs[s] * av[s][2];
                }
            float R[9];
            rotation_matrix(vrot + 4 * g, R);
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const float o = (R[c] * A0 + R[3 + c] * A1 + R[6 + c] * A2) * invs;
                if (3 * g + c < dim) orow[3 * g + c] = o;
            }
        }
        return;
    }
    for (int gl = threadIdx.x; gl < nr; gl += kAttnWaves * 64) {
        float A0 = 0.0f, A1 = 0.0f, A2 = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            A0 = A0 + f[w] * acc[w * 3 * kWideRange + 3 * gl];
            A1 = A1 + f[w] * acc[w * 3 * kWideRange + 3 * gl + 1];
            A2 = A2 + f[w] * acc[w * 3 * kWideRange + 3 * gl + 2];
        }
        const int64_t g = g0 + gl;
        float R[9];
        rotation_matrix(vrot + 4 * g, R);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const float o = (R[c] * A0 + R[3 + c] * A1 + R[6 + c] * A2) * inv;  // R^T A, then * inv
            if (3 * g + c < dim) orow[3 * g + c] = o;
        }
    }
}


// Splits of each query's tiles: enough workgroups for the given number per
// CU, at least kAttnWaves tiles per split, one split when the queries alone
// fill the device. tps = tiles per split.
constexpr int kNarrowWgsPerCu = 1, kWideWgsPerCu = 2;

static void attn_splits(int64_t wgs, int64_t T, bool wide, int64_t &ns, int64_t &tps) {
    const int64_t want = (int64_t)(wide ? kWideWgsPerCu : kNarrowWgsPerCu) * device_cu_count();
    ns = 1;
    if (wgs < want && T >= 2 * kAttnWaves)
        ns = std::min<int64_t>({ceil_div(want, wgs), T / kAttnWaves, kMaxSplits});
    tps = ceil_div(T, ns);
    ns = T > 0 ? ceil_div(T, tps) : 1;  // no empty split
}

// Split workspace: a count per query and range (the first bytes, rounded up
// to 256), then the splits' states [query][split][2 + 3 ng].
static size_t attn_count_bytes(int64_t queries) {
    return (size_t)ceil_div(4 * queries, 256) * 256;
}
static size_t attn_split_bytes(int64_t queries, int64_t ns, int64_t ng) {
    const int64_t ranges = ng > 64 ? ceil_div(ng, kWideRange) : 1;  // a count per range
    return ns > 1 ? attn_count_bytes(queries * ranges) +
                        (size_t)(queries * ns * (2 + 3 * ng)) * sizeof(float)
                  : 0;
}

static size_t attn_workspace_bytes(int64_t bh, int64_t nq, int64_t seq, int64_t dim) {
    const int64_t ng = ceil_div(dim, 3), T = ceil_div(seq, kTile);
    const int64_t wgs = bh * nq * (ng > 64 ? ceil_div(ng, kWideRange) : 1);
    int64_t ns, tps;
    attn_splits(wgs, T, ng > 64, ns, tps);
    return attn_split_bytes(bh * nq, ns, ng);
}

__global__ void rq_zero_kernel(uint32_t *__restrict__ p, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// Largest LDS a workgroup may use on the current device (cached per device).
static int device_max_lds() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
            n <= 0)
            n = 65536;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

}  // namespace rnn

using namespace rnn;

extern "C" int rnn_rotorquant_kv_page_elems(int64_t bh, int64_t seq, int64_t dim,
                                            int64_t *code_elems, int64_t *scale_elems) {
    RNN_ENTRY();
    RNN_REQUIRE(bh >= 0 && seq >= 0 && dim > 0 && code_elems && scale_elems,
                "rnn_rotorquant_kv_page_elems: bad argument");
    const int64_t ng = ceil_div(dim, 3), pos = bh * ceil_div(seq, kTile) * kTile;
    *code_elems = pos * 8 * ceil_div(ng, 8);   // K pages pad to 8 groups, V pages use ng
    *scale_elems = pos * 4 * ceil_div(ng, 4);  // K pages pad to 4 groups
    return RNN_OK;
}

extern "C" int rnn_rotorquant_kv_pack(const int8_t *codes, const float *scales, int64_t bh,
                                      int64_t seq, int64_t dim, int bits, int kind,
                                      uint16_t *page_codes, float *page_scales, void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_rotorquant_kv_pack";
    RNN_REQUIRE(bh >= 0 && seq >= 0 && dim > 0, "%s: bad size", name);
    RNN_REQUIRE(bits >= 2 && bits <= 4, "%s: the page stores 4-bit codes (bits 2..4), got %d", name,
                bits);
    RNN_REQUIRE(kind == RQ_PAGE_K || kind == RQ_PAGE_V, "%s: kind must be K (0) or V (1)", name);
    if (bh == 0 || seq == 0) return RNN_OK;
    RNN_REQUIRE(codes && scales && page_codes && page_scales, "%s: null pointer", name);
    const int64_t ng = ceil_div(dim, 3), T = ceil_div(seq, kTile);
    const int64_t total = bh * T * kTile * (kind == RQ_PAGE_K ? 8 * ceil_div(ng, 8) : ng);
    const int blocks = (int)std::min<int64_t>(ceil_div(total, 256), 8 * (int64_t)device_cu_count());
    rq_kv_pack_kernel<<<blocks, 256, 0, as_stream(stream)>>>(kind, codes, scales, bh, seq, ng, T,
                                                             page_codes, page_scales);
    return check_launch(name);
}

extern "C" size_t rnn_rotorquant_kv_attention_workspace_size(int64_t bh, int64_t nq, int64_t seq,
                                                             int64_t dim) {
    if (bh <= 0 || nq <= 0 || seq <= 0 || dim <= 0) return 0;
    return attn_workspace_bytes(bh, nq, seq, dim);
}

extern "C" int rnn_rotorquant_kv_attention_ws(const float *q, int64_t bh, int64_t nq,
                                              const uint16_t *k_codes, const float *k_scales,
                                              const uint16_t *v_codes, const float *v_scales,
                                              const float *k_rotors, const float *v_rotors,
                                              int64_t seq, int64_t dim, float scale, float *out,
                                              void *workspace, size_t workspace_bytes,
                                              void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_rotorquant_kv_attention";
    RNN_REQUIRE(bh >= 0 && nq >= 0 && seq >= 0 && dim > 0, "%s: bad size", name);
    // the split counts and states are updated with 4-byte atomics
    RNN_REQUIRE(((uintptr_t)workspace % 16) == 0, "%s: workspace must be 16-byte aligned", name);
    const int64_t ngw = ceil_div(dim, 3);
    // the wide kernel's LDS: the rotated query (16 bytes per group, 8-group
    // blocks), the accumulators, and the static probabilities and merge rows
    const int64_t wide_lds = (32 * ceil_div(ngw, 8) + kAttnWaves * 3 * kWideRange) * 4;
    const int64_t wide_static = kAttnWaves * (64 + 2) * 4;
    RNN_REQUIRE(ngw <= 64 || wide_lds + wide_static <= device_max_lds(),
                "%s: head dim %lld needs %lld bytes of LDS (the device has %d)", name,
                (long long)dim, (long long)(wide_lds + wide_static), device_max_lds());
    if (bh == 0 || nq == 0) return RNN_OK;
    RNN_REQUIRE(q && out && k_rotors && v_rotors, "%s: null pointer", name);
    RNN_REQUIRE(seq == 0 || (k_codes && k_scales && v_codes && v_scales), "%s: null page", name);
    RNN_REQUIRE(((uintptr_t)v_scales % 16) == 0 && ((uintptr_t)v_codes % 16) == 0 &&
                    ((uintptr_t)k_scales % 16) == 0 && ((uintptr_t)k_codes % 16) == 0,
                "%s: pages must be 16-byte aligned", name);
    RNN_REQUIRE(bh * nq <= 0x7fffffffLL, "%s: too many queries", name);
    const int64_t ng = ceil_div(dim, 3), T = ceil_div(seq, kTile);
    const unsigned grid = (unsigned)(bh * nq);
    const int64_t nranges = ng > 64 ? ceil_div(ng, kWideRange) : 1;
    int64_t ns, tps;
    attn_splits(bh * nq * nranges, T, ng > 64, ns, tps);
    hipStream_t st = as_stream(stream);
    // ns > 1: the splits' states go to the workspace (or stream-ordered
    // scratch, its counts zeroed); the last split of each query (and range)
    // merges them
    const size_t need = attn_split_bytes(bh * nq, ns, ng);
    RNN_REQUIRE(!workspace || workspace_bytes >= need,
                "%s: workspace of %zu bytes, %zu needed (rnn_rotorquant_kv_attention_workspace_size)",
                name, workspace_bytes, need);
    if (ng > 64 && wide_lds > 65536)
        RNN_REQUIRE(hipFuncSetAttribute((const void *)rq_kv_attn_wide_kernel,
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)wide_lds) == hipSuccess,
                    "%s: %lld bytes of dynamic LDS refused", name, (long long)wide_lds);
    void *ws = need ? workspace : nullptr;
    if (need && !ws) {
        RNN_TRY(check_hip(hipMallocAsync(&ws, need, st), name));
        rq_zero_kernel<<<(unsigned)std::min<int64_t>(ceil_div(bh * nq * nranges, 256), 1024), 256,
                         0, st>>>(static_cast<uint32_t *>(ws), bh * nq * nranges);
    }
    uint32_t *cnt = static_cast<uint32_t *>(ws);
    float *part = ws ? reinterpret_cast<float *>(static_cast<uint8_t *>(ws) +
                                                 attn_count_bytes(bh * nq * nranges))
                     : nullptr;
    if (ng > 64) {
        rq_kv_attn_wide_kernel<<<dim3(grid, (unsigned)nranges, (unsigned)ns), kAttnWaves * 64,
                                 (size_t)wide_lds, st>>>(q, k_codes, k_scales, v_codes, v_scales,
                                                         k_rotors, v_rotors, nq, seq, dim, ng, T,
                                                         tps, scale, out, part, cnt);
    } else if (ng <= 44) {
        rq_kv_attn_kernel<11, 6><<<dim3(grid, (unsigned)ns), kAttnWaves * 64, 0, st>>>(
            q, k_codes, k_scales, v_codes, v_scales, k_rotors, v_rotors, nq, seq, dim, ng, T, tps,
            scale, out, part, cnt);
    } else {
        rq_kv_attn_kernel<16, 8><<<dim3(grid, (unsigned)ns), kAttnWaves * 64, 0, st>>>(
            q, k_codes, k_scales, v_codes, v_scales, k_rotors, v_rotors, nq, seq, dim, ng, T, tps,
            scale, out, part, cnt);
    }
    int rc = check_launch(name);
    if (ws && ws != workspace) {
        const int rf = check_hip(hipFreeAsync(ws, st), name);
        if (rc == RNN_OK) rc = rf;
    }
    return rc;
}

extern "C" int rnn_rotorquant_kv_attention(const float *q, int64_t bh, int64_t nq,
                                           const uint16_t *k_codes, const float *k_scales,
                                           const uint16_t *v_codes, const float *v_scales,
                                           const float *k_rotors, const float *v_rotors,
                                           int64_t seq, int64_t dim, float scale, float *out,
                                           void *stream) {
    return rnn_rotorquant_kv_attention_ws(q, bh, nq, k_codes, k_scales, v_codes, v_scales,
                                          k_rotors, v_rotors, seq, dim, scale, out, nullptr, 0,
                                          stream);
}
