// rotorquant.hip -- RotorQuant (block Cl(3,0) rotor decorrelation + per-group
// symmetric scalar quantization) for KV-cache rows, streaming and HBM-bound.
//
// Each workgroup first builds the 3x3 rotation matrix of every group from its
// rotor with the reference's sandwich expressions (src/quant.rs:70-113) into
// LDS, then streams (vector, 3-group) items grid-stride: 12-byte loads ->
// rotate / max / divide / round / clamp / rescale / inverse-rotate in
// registers -> 12-byte stores (+ codes and scales when requested).
#include <algorithm>

#include "common.hpp"
#include "numerics.hpp"
#include "rotor.hpp"

namespace rnn {

constexpr int kRqThreads = 256;
constexpr int kRqMaxGroups = 896;  // dim <= 2688: 42 KiB of rotation matrices in LDS (larger
                                   // dims rebuild them per item)

__global__ void rotation_matrices_kernel(const float *__restrict__ rotors, int64_t n,
                                         float *__restrict__ rot9) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) {
        float m[9];
        rotation_matrix(rotors + 4 * i, m);
        for (int e = 0; e < 9; ++e) rot9[9 * i + e] = m[e];
    }
}

// m / qmax correctly rounded, for qmax = 2^(bits-1) - 1 with bits in [2, 8]
// and y = RN(1/qmax): q0 = RN(m*y), r = m - q0*qmax (exact in one FMA),
// q1 = RN(q0 + r*y) (Markstein's correction). Checked equal to the IEEE
// quotient for every normal m and each of those qmax; m = inf (r is NaN)
// keeps q0 = inf, the IEEE result.
__device__ __forceinline__ float div_qmax(float m, float qmax, float y) {
    const float q0 = m * y;
    const float r = __builtin_fmaf(-q0, qmax, m);
    const float q1 = __builtin_fmaf(r, y, q0);
    return r == r ? q1 : q0;
}

// quantize_vec for one group (src/quant.rs:178-205). Returns false for a
// group skipped by the max_abs < 1e-12 rule (its values stay untouched).
// Expression order follows the reference (no contraction: rv = R v row by
// row, left to right; scale = max/qmax; rv = q * scale; x = R^T rv). R holds
// the row-major 3x3 rotation; y_qmax is RN(1/qmax), or 0 to divide exactly.
__device__ __forceinline__ bool rq_group(const float *R, float qmax, float y_qmax, float &x0,
                                         float &x1, float &x2, float &scale, float q[3]) {
    float rv0 = R[0] * x0 + R[1] * x1 + R[2] * x2;
    float rv1 = R[3] * x0 + R[4] * x1 + R[5] * x2;
    float rv2 = R[6] * x0 + R[7] * x1 + R[8] * x2;
    float m = 0.0f;
    m = fmaxf(m, fabsf(rv0));
    m = fmaxf(m, fabsf(rv1));
    m = fmaxf(m, fabsf(rv2));
    if (m < 1e-12f) return false;
    scale = y_qmax != 0.0f ? div_qmax(m, qmax, y_qmax) : m / qmax;
    const float inv = __builtin_amdgcn_rcpf(scale);
    q[0] = clamp_rs(round_quotient(rv0, scale, inv), -qmax, qmax);
    q[1] = clamp_rs(round_quotient(rv1, scale, inv), -qmax, qmax);
    q[2] = clamp_rs(round_quotient(rv2, scale, inv), -qmax, qmax);
    rv0 = q[0] * scale;
    rv1 = q[1] * scale;
    rv2 = q[2] * scale;
    x0 = R[0] * rv0 + R[3] * rv1 + R[6] * rv2;
    x1 = R[1] * rv0 + R[4] * rv1 + R[7] * rv2;
    x2 = R[2] * rv0 + R[5] * rv1 + R[8] * rv2;
    return true;
}

// Streaming round trip: one thread per (row, 3-group) item f = row * ng + g,
// grid-stride, kRqU independent items in flight per thread. A wave's items
// are consecutive groups, so its 12-byte loads and stores cover one
// contiguous run of the row-major tensor, and the scales output [rows, ng] is
// indexed by f itself. The rotation matrices sit in LDS at a 48-byte stride
// (three conflict-free 16-byte reads per group); nothing else is staged.
// IDX is the element-offset type: uint32_t when rows * padded < 2^32 (item
// split by a magic multiply), int64_t otherwise. LDSROT = false (dims past
// the LDS table, 3 * kRqMaxGroups): each item rebuilds its group's matrix from
// the rotor (the same expressions, so the same bits; the rotors stay in L2).
constexpr int kRqU = 4;
constexpr int kRotStride = 12;  // floats per rotation matrix in LDS (9 used)

template <typename IDX, bool LDSROT = true>
__global__ __launch_bounds__(kRqThreads) void rotorquant_kernel(
    const float *__restrict__ x, int64_t rows, int dim, int ng, float qmax, float y_qmax,
    uint32_t ng_magic, const float *__restrict__ rotors, float *__restrict__ y,
    int8_t *__restrict__ codes, float *__restrict__ scales) {
    extern __shared__ __attribute__((aligned(16))) float rot[];  // ng * kRotStride floats
    if (LDSROT) {
        for (int g = threadIdx.x; g < ng; g += kRqThreads)
            rotation_matrix(rotors + 4 * g, rot + kRotStride * g);
        __syncthreads();
    }
    const IDX padded = (IDX)ng * 3;
    const IDX total = (IDX)rows * (IDX)ng;
    const IDX stride = (IDX)gridDim.x * kRqThreads;
    for (IDX f0 = (IDX)blockIdx.x * kRqThreads + threadIdx.x; f0 < total; f0 += stride * kRqU) {
        float v[kRqU][3];
        IDX row[kRqU];
        int grp[kRqU];
        bool live[kRqU];
#pragma unroll
        for (int u = 0; u < kRqU; ++u) {
            const IDX f = f0 + (IDX)u * stride;
            live[u] = f < total;
            IDX r;
            if (sizeof(IDX) == 4 && ng > 1) {  // floor(f / ng) or one more, then fix
                r = __umulhi((uint32_t)f, ng_magic);
                if (r * (IDX)ng > f) --r;
            } else {
                r = f / (IDX)ng;
            }
            row[u] = r;
            grp[u] = (int)(f - r * (IDX)ng);
            v[u][0] = v[u][1] = v[u][2] = 0.0f;
            if (live[u]) {
                const int e = 3 * grp[u];
                const float *p = x + (r * (IDX)dim + (IDX)e);
                v[u][0] = p[0];
                if (e + 1 < dim) v[u][1] = p[1];
                if (e + 2 < dim) v[u][2] = p[2];
            }
        }
#pragma unroll
        for (int u = 0; u < kRqU; ++u) {
            if (!live[u]) continue;
            const int g = grp[u], e = 3 * g;
            float R[12];
            if (LDSROT) {
                *reinterpret_cast<float4 *>(R + 0) = *reinterpret_cast<const float4 *>(rot + kRotStride * g);
                *reinterpret_cast<float4 *>(R + 4) = *reinterpret_cast<const float4 *>(rot + kRotStride * g + 4);
                *reinterpret_cast<float4 *>(R + 8) = *reinterpret_cast<const float4 *>(rot + kRotStride * g + 8);
            } else {
                rotation_matrix(rotors + 4 * g, R);
            }
            float scale = 0.0f, q[3] = {0.0f, 0.0f, 0.0f};
            rq_group(R, qmax, y_qmax, v[u][0], v[u][1], v[u][2], scale, q);
            if (codes) {
                int8_t *c = codes + (row[u] * padded + (IDX)e);
                c[0] = to_i8_rs(q[0]);
                c[1] = to_i8_rs(q[1]);
                c[2] = to_i8_rs(q[2]);
            }
            if (scales) scales[row[u] * (IDX)ng + (IDX)g] = scale;
            if (y) {  // a skipped group is written back unchanged
                float *o = y + (row[u] * (IDX)dim + (IDX)e);
                o[0] = v[u][0];
                if (e + 1 < dim) o[1] = v[u][1];
                if (e + 2 < dim) o[2] = v[u][2];
            }
        }
    }
}

// Tiled round trip for head_dim DIM in {64, 128, 256} (16-byte aligned
// tensors): each wave owns an LDS slice of kRqTileV*256 floats = RPC whole rows
// (a "chunk", 4 KiB). Per chunk: kRqTileV coalesced 16-byte loads per lane
// (issued one chunk ahead into registers) -> LDS -> the wave's lanes take the
// chunk's RPC*NG (row, group) items in passes of 64 (12-byte group reads at a
// 12-byte lane stride: conflict-free) and write the reconstruction back in
// place -> coalesced 16-byte stores. No block barriers after the rotation
// setup. The pad element of a row's last group (beyond DIM) is read as 0 and
// never written back.
typedef float f4v __attribute__((ext_vector_type(4)));  // 16-byte vector for nt accesses
constexpr int kRqTileV = 4;                      // float4 per lane per chunk
constexpr int kRqChunk = kRqTileV * 256;         // floats per chunk (4 KiB)

template <int DIM>
__global__ __launch_bounds__(kRqThreads) void rotorquant_tile_kernel(
    const float *__restrict__ x, int64_t rows, float qmax, float y_qmax,
    const float *__restrict__ rotors, float *__restrict__ y, int8_t *__restrict__ codes,
    float *__restrict__ scales) {
    constexpr int NG = (DIM + 2) / 3, PADDED = 3 * NG;
    constexpr int RPC = kRqChunk / DIM;           // rows per chunk
    constexpr int ITEMS = RPC * NG, PASSES = (ITEMS + 63) / 64;
    static_assert(kRqChunk % DIM == 0, "a chunk holds whole rows");
    __shared__ __attribute__((aligned(16))) float rot[NG * kRotStride];
    __shared__ __attribute__((aligned(16))) float tile[kRqThreads / 64][kRqChunk];
    for (int g = threadIdx.x; g < NG; g += kRqThreads)
        rotation_matrix(rotors + 4 * g, rot + kRotStride * g);
    __syncthreads();
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    float *t = tile[wid];
    const int64_t nchunks = (rows + RPC - 1) / RPC;
    const int64_t wstride = (int64_t)gridDim.x * (kRqThreads / 64);
    int64_t c = (int64_t)blockIdx.x * (kRqThreads / 64) + wid;

    // float4 i of a chunk (lane + 64 v) is row i / (DIM/4) of the chunk. Loads
    // and stores are non-temporal: every byte is touched once, and keeping the
    // stream out of the caches measured ~8% faster than plain accesses.
    auto load_chunk = [&](int64_t ch, f4v (&r)[kRqTileV]) {
        const f4v *src = reinterpret_cast<const f4v *>(x + ch * kRqChunk);
        const int64_t valid4 = (rows - ch * RPC) * (DIM / 4);  // float4s inside the tensor
#pragma unroll
        for (int v = 0; v < kRqTileV; ++v) {
            const int i = lane + 64 * v;
            r[v] = f4v{0.f, 0.f, 0.f, 0.f};
            if (ch < nchunks && i < valid4) r[v] = __builtin_nontemporal_load(src + i);
        }
    };
    f4v cur[kRqTileV], nxt[kRqTileV];
    load_chunk(c, cur);
    for (; c < nchunks; c += wstride) {
        load_chunk(c + wstride, nxt);
#pragma unroll
        for (int v = 0; v < kRqTileV; ++v) reinterpret_cast<f4v *>(t)[lane + 64 * v] = cur[v];
        const int64_t row0 = c * RPC;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int q = lane + 64 * p;
            const int rr = q / NG, g = q - rr * NG, e = 3 * g;
            const int64_t row = row0 + rr;
            if (q < ITEMS && row < rows) {
                float *pv = t + rr * DIM + e;
                float x0 = pv[0];
                float x1 = e + 1 < DIM ? pv[1] : 0.0f;
                float x2 = e + 2 < DIM ? pv[2] : 0.0f;
                float R[12];
                *reinterpret_cast<float4 *>(R + 0) = *reinterpret_cast<const float4 *>(rot + kRotStride * g);
                *reinterpret_cast<float4 *>(R + 4) = *reinterpret_cast<const float4 *>(rot + kRotStride * g + 4);
                *reinterpret_cast<float4 *>(R + 8) = *reinterpret_cast<const float4 *>(rot + kRotStride * g + 8);
                float scale = 0.0f, qv[3] = {0.0f, 0.0f, 0.0f};
                rq_group(R, qmax, y_qmax, x0, x1, x2, scale, qv);
                if (codes) {
                    int8_t *cp = codes + row * PADDED + e;
                    cp[0] = to_i8_rs(qv[0]);
                    cp[1] = to_i8_rs(qv[1]);
                    cp[2] = to_i8_rs(qv[2]);
                }
                if (scales) scales[row * NG + g] = scale;
                pv[0] = x0;
                if (e + 1 < DIM) pv[1] = x1;
                if (e + 2 < DIM) pv[2] = x2;
            }
        }
        if (y) {
            f4v *dst = reinterpret_cast<f4v *>(y + c * kRqChunk);
            const int64_t valid4 = (rows - row0) * (DIM / 4);
#pragma unroll
            for (int v = 0; v < kRqTileV; ++v) {
                const int i = lane + 64 * v;
                if (i < valid4)
                    __builtin_nontemporal_store(reinterpret_cast<const f4v *>(t)[i], dst + i);
            }
        }
#pragma unroll
        for (int v = 0; v < kRqTileV; ++v) cur[v] = nxt[v];
    }
}

// Reconstruction from codes: one thread per (row, group); LDSROT as in
// rotorquant_kernel.
template <bool LDSROT = true>
__global__ __launch_bounds__(kRqThreads) void rotorquant_dequant_kernel(
    const int8_t *__restrict__ codes, const float *__restrict__ scales, int64_t rows, int dim,
    int ng, const float *__restrict__ rotors, float *__restrict__ y) {
    extern __shared__ float rot[];  // ng * 9 floats (dynamic)
    if (LDSROT) {
        for (int g = threadIdx.x; g < ng; g += kRqThreads) rotation_matrix(rotors + 4 * g, rot + 9 * g);
        __syncthreads();
    }
    const int padded = 3 * ng;
    const int64_t work = rows * ng;
    for (int64_t f = blockIdx.x * (int64_t)kRqThreads + threadIdx.x; f < work;
         f += (int64_t)gridDim.x * kRqThreads) {
        const int64_t row = f / ng;
        const int g = (int)(f - row * ng);
        float Rg[9];
        if (!LDSROT) rotation_matrix(rotors + 4 * g, Rg);
        const float *R = LDSROT ? rot + 9 * g : Rg;
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
    RNN_ENTRY();
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
    RNN_ENTRY();
    const char *name = "rnn_rotorquant_quantize";
    RNN_REQUIRE(rows >= 0, "%s: negative rows", name);
    RNN_REQUIRE(dim > 0, "%s: dim must be positive (RotorQuant dim %lld)", name, (long long)dim);
    RNN_REQUIRE(bits >= 2, "%s: RotorQuant needs at least 2 bits", name);
    RNN_REQUIRE(bits <= (codes ? 8 : 32), "%s: bits %d out of range", name, bits);
    const int64_t ng = (dim + 2) / 3;
    RNN_REQUIRE(ng <= 0x7fffffff / 3, "%s: dim %lld too large", name, (long long)dim);
    if (rows == 0) return RNN_OK;
    RNN_REQUIRE(x && rotors, "%s: null input", name);
    RNN_REQUIRE(y || codes || scales, "%s: no output requested", name);
    RNN_REQUIRE(rows <= INT64_MAX / ng, "%s: too many rows", name);
    const float qmax = (float)((1u << (bits - 1)) - 1u);
    const float y_qmax = bits <= 8 ? 1.0f / qmax : 0.0f;  // 0: divide m / qmax exactly
    const int64_t total = rows * ng;
    hipStream_t st = as_stream(stream);
    const bool al16 = ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0;
    if (al16 && (dim == 64 || dim == 128 || dim == 256)) {
        const int64_t nchunks = ceil_div(rows * dim, kRqChunk);
        const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(nchunks, kRqThreads / 64),
                                                          8 * device_cu_count());
        if (dim == 64)
            rotorquant_tile_kernel<64><<<grid, kRqThreads, 0, st>>>(x, rows, qmax, y_qmax, rotors,
                                                                    y, codes, scales);
        else if (dim == 128)
            rotorquant_tile_kernel<128><<<grid, kRqThreads, 0, st>>>(x, rows, qmax, y_qmax, rotors,
                                                                     y, codes, scales);
        else
            rotorquant_tile_kernel<256><<<grid, kRqThreads, 0, st>>>(x, rows, qmax, y_qmax, rotors,
                                                                     y, codes, scales);
        return check_launch(name);
    }
    const bool narrow = rows <= (int64_t)0xffffffffLL / (3 * ng);
    const uint32_t magic = ng > 1 ? (uint32_t)((0x100000000ULL + ng - 1) / ng) : 0u;
    // Grid-stride: enough resident waves for the loads in flight that HBM
    // needs, and the per-block rotation-matrix setup amortised over many items.
    const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(total, kRqThreads * kRqU),
                                                      8 * device_cu_count());
    if (ng > kRqMaxGroups) {  // matrices rebuilt per item, no LDS table
        if (narrow)
            rotorquant_kernel<uint32_t, false><<<grid, kRqThreads, 0, st>>>(
                x, rows, (int)dim, (int)ng, qmax, y_qmax, magic, rotors, y, codes, scales);
        else
            rotorquant_kernel<int64_t, false><<<grid, kRqThreads, 0, st>>>(
                x, rows, (int)dim, (int)ng, qmax, y_qmax, magic, rotors, y, codes, scales);
        return check_launch(name);
    }
    const size_t smem = (size_t)ng * kRotStride * sizeof(float);
    if (narrow)
        rotorquant_kernel<uint32_t><<<grid, kRqThreads, smem, st>>>(
            x, rows, (int)dim, (int)ng, qmax, y_qmax, magic, rotors, y, codes, scales);
    else
        rotorquant_kernel<int64_t><<<grid, kRqThreads, smem, st>>>(
            x, rows, (int)dim, (int)ng, qmax, y_qmax, magic, rotors, y, codes, scales);
    return check_launch(name);
}

extern "C" int rnn_rotorquant_dequantize(const int8_t *codes, const float *scales, int64_t rows,
                                         int64_t dim, const float *rotors, float *y,
                                         void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_rotorquant_dequantize";
    RNN_REQUIRE(rows >= 0 && dim > 0, "%s: bad size", name);
    const int64_t ng = (dim + 2) / 3;
    RNN_REQUIRE(ng <= 0x7fffffff / 3, "%s: dim %lld too large", name, (long long)dim);
    if (rows == 0) return RNN_OK;
    RNN_REQUIRE(codes && scales && rotors && y, "%s: null pointer", name);
    RNN_REQUIRE(rows <= INT64_MAX / ng, "%s: too many rows", name);
    const int64_t work = rows * ng;
    const unsigned grid =
        (unsigned)std::min<int64_t>(ceil_div(work, kRqThreads), 8 * device_cu_count());
    if (ng > kRqMaxGroups)  // matrices rebuilt per item, no LDS table
        rotorquant_dequant_kernel<false><<<grid, kRqThreads, 0, as_stream(stream)>>>(
            codes, scales, rows, (int)dim, (int)ng, rotors, y);
    else
        rotorquant_dequant_kernel<true><<<grid, kRqThreads, (size_t)ng * 9 * sizeof(float),
                                          as_stream(stream)>>>(codes, scales, rows, (int)dim,
                                                               (int)ng, rotors, y);
    return check_launch(name);
}
