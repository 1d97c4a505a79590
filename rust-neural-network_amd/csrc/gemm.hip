// gemm.hip -- int8 GEMM/GEMV on gfx950 MFMA (v_mfma_i32_16x16x64_i8).
//
//   acc[m,n] = sum_k A[m,k] * B[n,k]     A [M,K] int8, B [N,K] int8 (both
//                                        K-contiguous: the Int8Weights layout)
// Entry points: rnn_w8a8_linear (W8A8 with fused dequant epilogue), rnn_igemm
// (the reference's u8 x i8 [K,N] contract via a pack step + zero-point
// correction) and rnn_ternary_gemm (B = 2-bit codes decoded in the tile loader).
#include <algorithm>
#include <mutex>
#include <type_traits>
#include <utility>

#include "common.hpp"
#include "numerics.hpp"

namespace rnn {

// ------------------------------------------------------------------ epilogue
// Applied per output element. Float path (y != null):
//   v = ((float)acc * sa[m]) * sw[n]; v = v + bias[n]; v = max(v, 0)
// (the order of src/int8.rs:159-162 and src/tensor.rs:2025-2032).
// Raw path (acc_out != null): acc_out = acc (+ 128*colsum[n] for igemm).
// Zero words that stand in for absent epilogue operands, so that operand loads
// can be issued unconditionally.
__device__ const uint32_t kEpiZero[4] = {0u, 0u, 0u, 0u};

// One output's epilogue operands, loaded ahead of its accumulator.
struct EpiOps {
    float sa, sw, bias;
    uint32_t cs;
};

struct Epilogue {
    const float *sa;
    const float *sw;
    const float *bias;
    float *y;
    int32_t *acc_out;
    const int32_t *colsum;  // igemm zero-point correction, may be null
    int64_t M, N;
    int relu;

    __device__ __forceinline__ void store(int64_t m, int64_t n, int32_t acc) const {
        if (m >= M || n >= N) return;
        if (acc_out) {
            uint32_t v = (uint32_t)acc;
            if (colsum) v += 128u * (uint32_t)colsum[n];
            acc_out[m * N + n] = (int32_t)v;
        }
        if (y) {
            float v = (float)acc * sa[m] * sw[n];
            if (bias) v = v + bias[n];
            if (relu) v = fmaxf(v, 0.0f);
            y[m * N + n] = v;
        }
    }
    // The operands store() reads for output (m, n), loaded without branches
    // (indices clamped into range, absent operands read zero words).
    // (Explicitly global pointers: a select between an argument pointer and
    // kEpiZero's address would otherwise become a flat load, which the
    // compiler counts against both the vector-memory and the LDS counters.)
    __device__ __forceinline__ EpiOps load_ops(int64_t m, int64_t n) const {
        typedef const __attribute__((address_space(1))) float *gf;
        typedef const __attribute__((address_space(1))) uint32_t *gu;
        const int64_t mc = m < M ? m : M - 1, nc = n < N ? n : N - 1;
        const gu z = (gu)kEpiZero;
        EpiOps o;
        o.sa = *(sa ? (gf)(sa + mc) : (gf)z);
        o.sw = *(sw ? (gf)(sw + nc) : (gf)z);
        o.bias = *(bias ? (gf)(bias + nc) : (gf)z);
        o.cs = *(colsum ? (gu)(colsum + nc) : z);
        return o;
    }
    // store() with operands from load_ops(m, n): the same arithmetic.
    __device__ __forceinline__ void store_ops(int64_t m, int64_t n, int32_t acc, const EpiOps &o) const {
        if (m >= M || n >= N) return;
        if (acc_out) {
            uint32_t v = (uint32_t)acc;
            if (colsum) v += 128u * o.cs;
            acc_out[m * N + n] = (int32_t)v;
        }
        if (y) {
            float v = (float)acc * o.sa * o.sw;
            if (bias) v = v + o.bias;
            if (relu) v = fmaxf(v, 0.0f);
            y[m * N + n] = v;
        }
    }
};

// ---------------------------------------------------------- ternary decode
// Four 2-bit codes (00 -> 0, 01 -> +1, 10 -> -1, 11 -> 0; src/ternary.rs:9-14,
// :63-75) in the low byte of x -> four int8 lanes. Low code bits are spread
// to byte positions with one 24-bit multiply (bit 2j -> bit 8j); the bytes are
// then subtracted lane-wise (p - n), which maps code 11 to 0.
__device__ __forceinline__ uint32_t ternary_byte_to_i8x4(uint32_t x) {
    const uint32_t p = __umul24(x & 0x55u, 0x41041u) & 0x01010101u;
    const uint32_t n = __umul24((x >> 1) & 0x55u, 0x41041u) & 0x01010101u;
    return ((p | 0x80808080u) - n) ^ 0x80808080u;
}

__device__ __forceinline__ v4i ternary_word_to_i8x16(uint32_t w) {
    v4i r;
    r.x = (int)ternary_byte_to_i8x4(w & 0xffu);
    r.y = (int)ternary_byte_to_i8x4((w >> 8) & 0xffu);
    r.z = (int)ternary_byte_to_i8x4((w >> 16) & 0xffu);
    r.w = (int)ternary_byte_to_i8x4(w >> 24);
    return r;
}

// The MFMA layout of packed ternary codes (rnn_ternary_prepack): within each
// 32-bit word of 16 codes (k = k0 .. k0+15) the code of k0 + 4r + b sits at
// bits 8b + 2r, so (w >> 2r) & 0x03030303 holds the codes of k0+4r .. k0+4r+3
// one per byte, and one byte permute maps each code through a 4-entry table
// (00 -> 0, 01 -> +1, 10 -> -1, 11 -> 0, src/ternary.rs:9-14, :63-75) held in
// a constant: bytes {0x00, 0x01, 0xFF, 0x00}. Selector values 0-3 pick those
// bytes, so 16 codes decode with no LDS table.
// The codes at bits 2-3 of a byte are used in place, as selectors 0, 4, 8,
// 12: v_perm_b32 gives src1 byte 0 for 0, src0 byte 0 for 4, the sign of
// src1 byte 1 replicated for 8, and 0x00 for 12; with src0 = 0x01 and src1
// byte 1 = 0x80 that is the same table. So a word takes one shift, four
// masks and four permutes (9 VALU operations).
constexpr uint32_t kTerPermTable = 0x00FF0100u;
constexpr uint32_t kTerPermHi0 = 0x00000001u, kTerPermHi1 = 0x00008000u;
__device__ __forceinline__ v4i ternary_perm_decode(uint32_t w) {
    v4i r;
    const uint32_t w4 = w >> 4;
    r.x = (int)__builtin_amdgcn_perm(kTerPermTable, kTerPermTable, w & 0x03030303u);
    r.y = (int)__builtin_amdgcn_perm(kTerPermHi0, kTerPermHi1, w & 0x0C0C0C0Cu);
    r.z = (int)__builtin_amdgcn_perm(kTerPermTable, kTerPermTable, w4 & 0x03030303u);
    r.w = (int)__builtin_amdgcn_perm(kTerPermHi0, kTerPermHi1, w4 & 0x0C0C0C0Cu);
    return r;
}

// Reference word (code t at bits 2t) -> MFMA-layout word (code 4r + b at bits
// 8b + 2r): a fixed permutation of the 16 two-bit fields.
__host__ __device__ __forceinline__ uint32_t ternary_word_to_mfma_layout(uint32_t w) {
    uint32_t o = 0;
    for (int t = 0; t < 16; ++t) {
        const int r = t >> 2, b = t & 3;
        o |= ((w >> (2 * t)) & 3u) << (8 * b + 2 * r);
    }
    return o;
}

// ------------------------------------------------------------ tiled GEMM
// Block tile BM x BN, K step 64 (one MFMA K), (BM/WM) x (BN/WN) waves, each
// wave a WM x WN tile of 16x16 MFMA blocks. Operand tiles live in LDS as
// [rows][64 bytes] with the 16-byte chunk index XOR-swizzled by (r>>1) & 3,
// which keeps the ds_read_b128 fragment loads (16 rows x one chunk per
// quarter-wave) free of bank conflicts on gfx950. Global tiles are prefetched into registers one K step
// ahead (double-buffered LDS).
constexpr int kBK = 64;

__device__ __forceinline__ int swz(int r) { return (r >> 1) & 3; }

template <int BM, int BN, int WM, int WN, bool TERNARY>
struct TileGemm {
    static constexpr int WAVES = (BM / WM) * (BN / WN);
    static constexpr int NT = WAVES * 64;
    static constexpr int TI = WM / 16, TJ = WN / 16;
    static constexpr int A_CHUNKS = BM * kBK / 16 / NT;         // 16-B chunks/thread
    static constexpr int B_CHUNKS = TERNARY ? 0 : BN * kBK / 16 / NT;
    static constexpr int B_ROWS = TERNARY ? (BN + NT - 1) / NT : 0;  // packed rows/thread
    static_assert(BM * kBK / 16 % NT == 0, "A tile must split evenly");
    static_assert(TERNARY || BN * kBK / 16 % NT == 0, "B tile must split evenly");
};

// RAGGED: any K and any operand alignment (the igemm contract's "any K",
// src/int8.rs:288-296). Every chunk is assembled from byte loads (k >= K reads
// as 0), and ternary code words are gathered from arbitrary bit offsets of the
// flat row-major codes (a row of K codes starts at code n*K, so rows are not
// word aligned unless K % 16 == 0). Slower; used only for such shapes.
__device__ __forceinline__ v4i load16_ragged(const int8_t *row, int64_t k0, int64_t K) {
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t v = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int64_t k = k0 + 4 * q + b;
            v |= (k < K ? (uint32_t)(uint8_t)row[k] : 0u) << (8 * b);
        }
        w[q] = v;
    }
    return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

// The 16 codes of row n at k0 .. k0+15 (codes past the row's K read as 0) as
// one word in the packed layout (code t at bits 2t).
__device__ __forceinline__ uint32_t ternary_word_ragged(const uint32_t *Bp, int64_t n, int64_t k0,
                                                        int64_t N, int64_t K) {
    const int64_t left = K - k0;
    if (left <= 0) return 0u;
    const int64_t c0 = n * K + k0, w0 = c0 >> 4, words = (N * K + 15) / 16;
    const int sh = (int)(c0 & 15) * 2;
    const uint32_t lo = Bp[w0];
    const uint32_t hi = (sh != 0 && w0 + 1 < words) ? Bp[w0 + 1] : 0u;
    uint32_t v = sh ? (lo >> sh) | (hi << (32 - sh)) : lo;
    if (left < 16) v &= (1u << (2 * left)) - 1u;
    return v;
}

template <int BM, int BN, int WM, int WN, bool TERNARY, bool RAGGED = false, bool PERM = false>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_tiled_kernel(
    const int8_t *__restrict__ A, const void *__restrict__ Bv, int64_t M, int64_t N, int64_t K,
    Epilogue epi) {
    using C = TileGemm<BM, BN, WM, WN, TERNARY>;
    __shared__ __attribute__((aligned(16))) int8_t As[2][BM * kBK];
    __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * kBK];

    const int tid = threadIdx.x;
    const int wid = tid / 64, lane = tid % 64;
    const int wm0 = (wid / (BN / WN)) * WM, wn0 = (wid % (BN / WN)) * WN;
    const int64_t bm0 = (int64_t)blockIdx.y * BM, bn0 = (int64_t)blockIdx.x * BN;
    const int64_t nk = (K + kBK - 1) / kBK;

    const int8_t *B8 = static_cast<const int8_t *>(Bv);
    const uint32_t *Bp = static_cast<const uint32_t *>(Bv);
    const int64_t kwords = K / 16;  // packed words per ternary row

    v4i ra[C::A_CHUNKS];
    v4i rb[C::B_CHUNKS > 0 ? C::B_CHUNKS : 1];
    v4i rt[C::B_ROWS > 0 ? C::B_ROWS : 1];

    auto gload = [&](int64_t kt) {
        const int64_t k0 = kt * kBK;
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i) {
            const int c = tid + i * C::NT;
            const int r = c / 4, ch = c % 4;
            const int64_t gm = std::min<int64_t>(bm0 + r, M - 1);
            const int64_t gk = k0 + ch * 16;
            if constexpr (RAGGED)
                ra[i] = load16_ragged(A + gm * K, gk, K);
            else
                ra[i] = gk < K ? *reinterpret_cast<const v4i *>(A + gm * K + gk) : v4i{0, 0, 0, 0};
        }
        if constexpr (!TERNARY) {
#pragma unroll
            for (int i = 0; i < C::B_CHUNKS; ++i) {
                const int c = tid + i * C::NT;
                const int r = c / 4, ch = c % 4;
                const int64_t gn = std::min<int64_t>(bn0 + r, N - 1);
                const int64_t gk = k0 + ch * 16;
                if constexpr (RAGGED)
                    rb[i] = load16_ragged(B8 + gn * K, gk, K);
                else
                    rb[i] = gk < K ? *reinterpret_cast<const v4i *>(B8 + gn * K + gk)
                                   : v4i{0, 0, 0, 0};
            }
        } else if constexpr (RAGGED) {
#pragma unroll
            for (int i = 0; i < C::B_ROWS; ++i) {
                const int r = tid + i * C::NT;
                if (r < BN) {
                    const int64_t gn = std::min<int64_t>(bn0 + r, N - 1);
                    rt[i].x = (int)ternary_word_ragged(Bp, gn, k0, N, K);
                    rt[i].y = (int)ternary_word_ragged(Bp, gn, k0 + 16, N, K);
                    rt[i].z = (int)ternary_word_ragged(Bp, gn, k0 + 32, N, K);
                    rt[i].w = (int)ternary_word_ragged(Bp, gn, k0 + 48, N, K);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < C::B_ROWS; ++i) {
                const int r = tid + i * C::NT;
                if (r < BN) {
                    const int64_t gn = std::min<int64_t>(bn0 + r, N - 1);
                    const uint32_t *row = Bp + gn * kwords + k0 / 16;
                    const int64_t left = kwords - k0 / 16;  // words left in this row
                    if (left >= 4 && ((uintptr_t)row & 15) == 0) {
                        rt[i] = *reinterpret_cast<const v4i *>(row);
                    } else {
                        rt[i].x = left > 0 ? (int)row[0] : 0;
                        rt[i].y = left > 1 ? (int)row[1] : 0;
                        rt[i].z = left > 2 ? (int)row[2] : 0;
                        rt[i].w = left > 3 ? (int)row[3] : 0;
                    }
                }
            }
        }
    };

    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i) {
            const int c = tid + i * C::NT;
            const int r = c / 4, ch = c % 4;
            *reinterpret_cast<v4i *>(&As[buf][r * kBK + ((ch ^ swz(r)) * 16)]) = ra[i];
        }
        if constexpr (!TERNARY) {
#pragma unroll
            for (int i = 0; i < C::B_CHUNKS; ++i) {
                const int c = tid + i * C::NT;
                const int r = c / 4, ch = c % 4;
                *reinterpret_cast<v4i *>(&Bs[buf][r * kBK + ((ch ^ swz(r)) * 16)]) = rb[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < C::B_ROWS; ++i) {
                const int r = tid + i * C::NT;
                if (r < BN) {
                    const uint32_t w[4] = {(uint32_t)rt[i].x, (uint32_t)rt[i].y,
                                           (uint32_t)rt[i].z, (uint32_t)rt[i].w};
#pragma unroll
                    for (int ch = 0; ch < 4; ++ch)
                        *reinterpret_cast<v4i *>(&Bs[buf][r * kBK + ((ch ^ swz(r)) * 16)]) =
                            PERM ? ternary_perm_decode(w[ch]) : ternary_word_to_i8x16(w[ch]);
                }
            }
        }
    };

    v4i acc[C::TI][C::TJ];
#pragma unroll
    for (int i = 0; i < C::TI; ++i)
#pragma unroll
        for (int j = 0; j < C::TJ; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    const int fr = lane & 15, fq = lane >> 4;  // fragment row / k-chunk
    if (nk > 0) {
        gload(0);
        sstore(0);
    }
    __syncthreads();
    for (int64_t kt = 0; kt < nk; ++kt) {
        const int buf = (int)(kt & 1);
        if (kt + 1 < nk) gload(kt + 1);
        v4i af[C::TI], bf[C::TJ];
#pragma unroll
        for (int i = 0; i < C::TI; ++i) {
            const int r = wm0 + i * 16 + fr;
            af[i] = *reinterpret_cast<const v4i *>(&As[buf][r * kBK + ((fq ^ swz(r)) * 16)]);
        }
#pragma unroll
        for (int j = 0; j < C::TJ; ++j) {
            const int r = wn0 + j * 16 + fr;
            bf[j] = *reinterpret_cast<const v4i *>(&Bs[buf][r * kBK + ((fq ^ swz(r)) * 16)]);
        }
#pragma unroll
        for (int i = 0; i < C::TI; ++i)
#pragma unroll
            for (int j = 0; j < C::TJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // D layout of the 16x16 MFMA block: lane l, register e holds
    // row 4*(l/16) + e, column l%16.
#pragma unroll
    for (int i = 0; i < C::TI; ++i)
#pragma unroll
        for (int j = 0; j < C::TJ; ++j) {
            const int64_t n = bn0 + wn0 + j * 16 + (lane & 15);
            const int64_t mb = bm0 + wm0 + i * 16 + 4 * (lane >> 4);
            epi.store(mb + 0, n, acc[i][j].x);
            epi.store(mb + 1, n, acc[i][j].y);
            epi.store(mb + 2, n, acc[i][j].z);
            epi.store(mb + 3, n, acc[i][j].w);
        }
}

// ------------------------------------------------- LDS-DMA pipelined GEMM
// The large-shape kernel (prefill). Requires K % 64 == 0.
//
//  * Block tile BM x BN, WGM x WGN waves, each wave a (BM/WGM) x (BN/WGN)
//    register tile of 16x16x64 MFMA blocks whose int32 accumulators live in
//    the AGPR file.
//  * Operands go global -> LDS with global_load_lds_dwordx4 (no VGPR
//    staging, no ds_write): every wave instruction moves 1 KiB = 16 tile rows
//    x 64 B, lane l landing at byte 16*l. The 16-byte chunk order inside a
//    row is XOR-swizzled (lane l fetches logical chunk (l&3) ^ swz16(row)),
//    so the fragment reads (16 rows x one chunk per quarter-wave) hit 8
//    distinct bank groups per 8 lanes.
//  * STAGES LDS buffers, loads issued STAGES-1 K-steps ahead; each step waits
//    only for its own stage (s_waitcnt vmcnt(n)) before the block barrier.
//  * MFMA operand roles are swapped (A-operand = weight rows n, B-operand =
//    activation rows m), so a lane's 4 accumulator registers are 4
//    consecutive n of one m: the epilogue writes 16-byte float4 / int4.
//  * Tiles are ordered so that the blocks the hardware places on one XCD
//    (block id b goes to XCD b % 8) cover a compact range of tiles that
//    share A rows and B columns in that XCD's L2.
constexpr int kDmaBK = 64;

// Swizzle of the 16-byte chunk index by tile row (depends on row & 15 only,
// so a lane's swizzle is the same for every fragment it reads). With 64-byte
// rows, chunk ^ ((row >> 1) & 3) is the pattern that measured conflict-free
// for ds_read_b128 on gfx950's 256 B/clk LDS (231 B/clk/CU of fragment reads;
// adding a (row >> 3) term halves that).
__device__ __forceinline__ int swz16(int r) { return (r >> 1) & 3; }

// acc += a . b on v_mfma_i32_16x16x64_i8 with the accumulator tied to an
// AGPR quad. (Device pass only: the host pass parses but never emits kernel
// bodies, and "a" is not an AGPR constraint there.)
// ORDERED adds a memory clobber, so that the LDS reads and DMA issues placed
// between such MFMAs in the source stay interleaved with them.
template <bool ORDERED = false>
__device__ __forceinline__ void mfma_i8_acc(v4i &acc, const v4i &a, const v4i &b) {
#if defined(__HIP_DEVICE_COMPILE__)
    if (ORDERED)
        asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b) : "memory");
    else
        asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
#endif
}

// 16-byte global -> LDS DMA (global_load_lds_dwordx4): lane l's 16 bytes land
// at lds + 16*l; `lds` must be wave-uniform. (Device pass only: the host pass
// rejects the builtin with a const source and would silently drop the
// kernel's launch stub.)
__device__ __forceinline__ void dma16(const void *g, void *lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(const_cast<void *>(g),
                                     (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
#endif
}

// 16-byte buffer -> LDS DMA (buffer_load_dwordx4 ... offen lds): lane l's 16
// bytes at base + voff + soff land at lds + 16*l (`lds` wave-uniform). The
// descriptor covers `bytes` from `base`, so an offset past the operand reads
// zeros instead of faulting. voff is a per-lane VGPR that the caller keeps
// loop-invariant; soff (scalar) carries the per-stage advance. (Device pass
// only, as dma16.)
__device__ __forceinline__ void dma16_buf(const void *base, uint32_t bytes, uint32_t voff,
                                          uint32_t soff, void *lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    // word 3 of a gfx9 buffer descriptor: 32-bit data format, no swizzle
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                             voff, soff, 0, 0);
#endif
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// TER: B is 2-bit ternary codes (16 per u32, the TernaryTensor::packed layout),
// 16 bytes per row per 64-k step instead of 64.
template <int BM, int BN, int WGM, int WGN, int STAGES, bool TER = false>
struct DmaCfg {
    static constexpr int NW = WGM * WGN;
    static constexpr int NT = NW * 64;
    static constexpr int WM = BM / WGM, WN = BN / WGN;
    static constexpr int FM = WM / 16, FN = WN / 16;
    static constexpr int B_ROW = TER ? 16 : kDmaBK;  // bytes of a B row per K step
    static constexpr int A_INS = BM / 16;            // 1 KiB wave loads per stage
    static constexpr int B_INS = BN * B_ROW / 1024;
    static constexpr int INS = A_INS + B_INS;
    // Wave w issues the stage's loads j = w, w + NW, ... < INS: INS_HI of them
    // for w < INS % NW, else INS_LO (the two vmcnt thresholds of the loop).
    static constexpr int INS_PER_WAVE = (INS + NW - 1) / NW;
    static constexpr int INS_HI = INS_PER_WAVE, INS_LO = INS / NW;
    static constexpr int STAGE_BYTES = INS * 1024;
    static constexpr int LDS_BYTES = STAGES * STAGE_BYTES;
    static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile must be a multiple of 16");
    static_assert(BM % WGM == 0 && BN % WGN == 0, "waves must split the tile");
    static_assert(INS_LO >= 1 && STAGES >= 2, "pipeline shape");
    static_assert((STAGES - 1) * INS_HI < 64, "vmcnt range");
    static_assert(LDS_BYTES <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");
    static_assert(!TER || (BN % 64 == 0 && NT >= 256), "ternary B loads 64 rows per wave load");
};

// Ternary decode table: byte x holding four 2-bit codes (code i at bits
// 2i..2i+1; 00 -> 0, 01 -> +1, 10 -> -1, 11 -> 0, src/ternary.rs:9-14, :63-75)
// -> the four int8 values, byte i = code i. A u32 of 16 codes decodes with four
// lookups into the 16 int8 of an MFMA operand fragment.
__device__ __forceinline__ uint32_t ternary_lut_entry(uint32_t x) {
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) {
        const uint32_t c = (x >> (2 * i)) & 3u;
        r |= (c == 1u ? 0x01u : (c == 2u ? 0xffu : 0u)) << (8 * i);
    }
    return r;
}

// The same lookup in a table replicated R times (entry x of copy c at x*R + c)
// with lane l reading copy l % R: lanes that look up different entries fall in
// different LDS banks far more often than with a single 256-entry table.
template <int R>
__device__ __forceinline__ v4i ternary_lut_decode_rep(const uint32_t *lut_lane, uint32_t w) {
    v4i r;
    r.x = (int)lut_lane[(w & 0xffu) * R];
    r.y = (int)lut_lane[((w >> 8) & 0xffu) * R];
    r.z = (int)lut_lane[((w >> 16) & 0xffu) * R];
    r.w = (int)lut_lane[(w >> 24) * R];
    return r;
}

__device__ __forceinline__ v4i ternary_lut_decode(const uint32_t *lut, uint32_t w) {
    v4i r;
    r.x = (int)lut[w & 0xffu];
    r.y = (int)lut[(w >> 8) & 0xffu];
    r.z = (int)lut[(w >> 16) & 0xffu];
    r.w = (int)lut[w >> 24];
    return r;
}

// Tile coordinates of block b. When the tile count splits evenly over the 8
// XCDs, XCD x (blocks b with b % 8 == x) gets the contiguous tile range
// [x*T/8, (x+1)*T/8), walked with m fastest.
__device__ __forceinline__ void xcd_tile(int b, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int T = tiles_m * tiles_n;
    const int t = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
    tm = t % tiles_m;
    tn = t / tiles_m;
}

// Epilogue of a wave tile held as FN x FM 16x16 MFMA blocks with the operand
// roles swapped (D of block (i, j): lane l, register e = column n0 + 16i + e,
// row m0 + 16j, where m0 = tile row + l%16 and n0 = tile column + 4*(l/16)):
// a lane stores 4 consecutive columns of one row as one 16-byte float4 / int4.
// The host guarantees N % 4 == 0 and 16-byte aligned y / acc_out / sw / bias /
// colsum, so n..n+3 are in range whenever n is.
//  * Every operand (row and column scales, bias, colsum) is loaded before the
//    first store: stores count in vmcnt, so a wait for a load issued after
//    them would drain them too.
//  * Bias and ReLU are uniform selects and the bounds check exists only for
//    edge tiles (INTERIOR = false): a branch per store makes the compiler
//    merge its wait-count state at every join and drain the stores there.
//  * The arithmetic is the reference's: ((float)acc * sa[m]) * sw[n], then
//    + bias[n], then max(., 0) (src/int8.rs:159-162).
//  * WT (write-through): the stores are device-scope buffer stores (sc1),
//    which pass through the XCD's L2 instead of leaving the output dirty in
//    it. The prefill writes 117 MB of output in two chip-wide bursts; with
//    the lines left dirty the launch took 103.7-104.6 us against 101.1-102.8
//    with write-through (one process, bit-identical output); non-temporal
//    stores were slower (107 us). The host takes it only when y and acc_out
//    span less than 4 GiB (the buffer range).
// True when the wave tile at (m0, n0) (lane-adjusted as in tile_epilogue) lies
// inside M x N, so that every lane issues all of its FM * FN stores.
template <int FM, int FN>
__device__ __forceinline__ bool tile_interior(const Epilogue &epi, int64_t m0, int64_t n0) {
    return m0 - (m0 & 15) + 16 * FM <= epi.M && n0 - (n0 & 15) + 16 * FN <= epi.N;
}
template <int FM, int FN, bool OUT_Y, bool OUT_ACC, bool WT = false, int G = (FN < 4 ? FN : 4)>
__device__ __forceinline__ void tile_epilogue(const Epilogue &epi, const v4i (&acc)[FN][FM],
                                              int64_t m0, int64_t n0) {
    const bool has_bias = epi.bias != nullptr, relu = epi.relu != 0;
    // (WT only) buffer ranges of the outputs: byte offsets of whole rows
    const int out_bytes = WT ? (int)(epi.M * epi.N * 4) : 0;
    const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
        OUT_Y ? (void *)epi.y : (void *)epi.acc_out, 0, out_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
        OUT_ACC ? (void *)epi.acc_out : (void *)epi.y, 0, out_bytes, 0x00020000);
    auto put = [&](const __amdgpu_buffer_rsrc_t &r, void *base, int64_t idx, v4i v) {
        if constexpr (WT)
            __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)(idx * 4), 0, 16 /* sc1 */);
        else
            *reinterpret_cast<v4i *>(static_cast<int32_t *>(base) + idx) = v;
    };
    float sam[FM];
#pragma unroll
    for (int j = 0; j < FM; ++j)
        sam[j] = OUT_Y ? epi.sa[std::min<int64_t>(m0 + 16 * j, epi.M - 1)] : 0.0f;
    // the wave tile's corner: bounds checks are needed only past the edges
    const bool interior = tile_interior<FM, FN>(epi, m0, n0);

    // Column blocks in groups of G (the operand registers of a group stay
    // within a two-waves-per-SIMD budget): operand loads, then the stores.
#pragma unroll
    for (int g = 0; g < FN; g += G) {
        float4 swv[G], bv[G];
        v4i csv[G];
#pragma unroll
        for (int k = 0; k < G; ++k) {
            const int64_t n = std::min<int64_t>(n0 + 16 * std::min(g + k, FN - 1), epi.N - 4);
            swv[k] = float4{0.f, 0.f, 0.f, 0.f};
            bv[k] = float4{0.f, 0.f, 0.f, 0.f};
            csv[k] = v4i{0, 0, 0, 0};
            if (OUT_Y) {
                swv[k] = *reinterpret_cast<const float4 *>(epi.sw + n);
                if (has_bias) bv[k] = *reinterpret_cast<const float4 *>(epi.bias + n);
            }
            if (OUT_ACC && epi.colsum) csv[k] = *reinterpret_cast<const v4i *>(epi.colsum + n);
        }
        auto store = [&](int k, int j, bool guard) {
            const int i = g + k;
            const int64_t m = m0 + 16 * j, n = n0 + 16 * i;
            if (guard && (m >= epi.M || n >= epi.N)) return;
            const v4i &a = acc[i][j];
            if (OUT_ACC) {
                v4i o;
                o.x = (int)((uint32_t)a.x + 128u * (uint32_t)csv[k].x);
                o.y = (int)((uint32_t)a.y + 128u * (uint32_t)csv[k].y);
                o.z = (int)((uint32_t)a.z + 128u * (uint32_t)csv[k].z);
                o.w = (int)((uint32_t)a.w + 128u * (uint32_t)csv[k].w);
                put(ar, epi.acc_out, m * epi.N + n, o);
            }
            if (OUT_Y) {
                float4 v;
                v.x = (float)a.x * sam[j] * swv[k].x;
                v.y = (float)a.y * sam[j] * swv[k].y;
                v.z = (float)a.z * sam[j] * swv[k].z;
                v.w = (float)a.w * sam[j] * swv[k].w;
                v.x = has_bias ? v.x + bv[k].x : v.x;
                v.y = has_bias ? v.y + bv[k].y : v.y;
                v.z = has_bias ? v.z + bv[k].z : v.z;
                v.w = has_bias ? v.w + bv[k].w : v.w;
                v.x = relu ? fmaxf(v.x, 0.0f) : v.x;
                v.y = relu ? fmaxf(v.y, 0.0f) : v.y;
                v.z = relu ? fmaxf(v.z, 0.0f) : v.z;
                v.w = relu ? fmaxf(v.w, 0.0f) : v.w;
                put(yr, epi.y, m * epi.N + n, __builtin_bit_cast(v4i, v));
            }
        };
        if (interior) {
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int k = 0; k < G; ++k)
                    if (g + k < FN) store(k, j, false);
        } else {
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int k = 0; k < G; ++k)
                    if (g + k < FN) store(k, j, true);
        }
    }
}

// Fragments of one K step held in registers: FM activation blocks, FN weight
// blocks (16 rows x 64 B each, one 16-byte chunk per lane); for ternary B the
// lane's 32-bit word of 16 codes (w) is read first and decoded into b.
template <int FM, int FN>
struct Frags {
    v4i a[FM];
    v4i b[FN];
    uint32_t w[FN];
};

// KS > 1 splits K inside the block: KS groups of WGM x WGN waves each run the
// pipeline below over K/KS with their own LDS stages, and the int32 partial
// sums are added through LDS before group 0's epilogue (exact: wrapping int32
// addition is associative). It gives a small tile more waves per CU.
template <int BM, int BN, int WGM, int WGN, int STAGES, bool OUT_Y, bool OUT_ACC, bool TER,
          int KS = 1>
__global__ __launch_bounds__(KS *WGM *WGN * 64)
__attribute__((amdgpu_waves_per_eu(KS * WGM * WGN / 4, KS * WGM * WGN / 4)))
void gemm_dma_kernel(const int8_t *__restrict__ A, const int8_t *__restrict__ B, int64_t M,
                     int64_t N, int64_t K, int tiles_m, int tiles_n, Epilogue epi) {
    using C = DmaCfg<BM, BN, WGM, WGN, STAGES, TER>;
    using F = Frags<C::FM, C::FN>;
    constexpr int PART = C::NW * C::FN * C::FM * 64 * 16;  // one group's partial sums
    static_assert(KS == 1 || (KS - 1) * PART <= KS * C::LDS_BYTES, "split-K partials fit in LDS");
    static_assert(KS * C::LDS_BYTES <= 159 * 1024, "gfx950 has 160 KiB of LDS per CU");
    // one LDS object (stages, then the ternary decode table): see gemm_l128_kernel
    __shared__ __attribute__((aligned(1024))) int8_t smem_all[KS * C::LDS_BYTES + (TER ? 1024 : 0)];
    uint32_t *const lut = reinterpret_cast<uint32_t *>(smem_all + KS * C::LDS_BYTES);
    if (TER) {
        for (int t = threadIdx.x; t < 256; t += KS * C::NT) lut[t] = ternary_lut_entry((uint32_t)t);
        __syncthreads();
    }

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = wave / C::NW, wid = wave % C::NW;  // K group, wave within the group
    int8_t *const smem = smem_all + kg * C::LDS_BYTES;
    int tm, tn;
    xcd_tile((int)blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t bm0 = (int64_t)tm * BM, bn0 = (int64_t)tn * BN;
    const int64_t kbase = kg * (K / KS);             // this group's K range
    const int nk = (int)(K / KS / kDmaBK);           // even, >= 2 (host-checked)

    // Global sources of this wave's DMA loads at k = 0, and how far each
    // advances per K step (64 bytes, or 16 for packed ternary rows).
    // Instruction j of a stage fills LDS bytes [1024 j, 1024 j + 1024):
    // A-tile rows for j < A_INS, then B-tile rows (a stage is [A | B]).
    const int8_t *src[C::INS_PER_WAVE];
    int kstep[C::INS_PER_WAVE];
    {
        const int rr = lane >> 2, pc = lane & 3;
#pragma unroll
        for (int i = 0; i < C::INS_PER_WAVE; ++i) {
            const int j = std::min(wid + i * C::NW, C::INS - 1);  // (clamped: slot unused when >= INS)
            kstep[i] = kDmaBK;
            if (j < C::A_INS) {
                const int r = 16 * j + rr;
                const int64_t g = std::min<int64_t>(bm0 + r, M - 1);
                src[i] = A + g * K + kbase + 16 * (pc ^ swz16(r));
            } else if (TER) {  // 64 packed rows x 16 bytes, lane = row
                const int r = 64 * (j - C::A_INS) + lane;
                const int64_t g = std::min<int64_t>(bn0 + r, N - 1);
                src[i] = B + g * (K / 4) + kbase / 4;
                kstep[i] = C::B_ROW;
            } else {
                const int r = 16 * (j - C::A_INS) + rr;
                const int64_t g = std::min<int64_t>(bn0 + r, N - 1);
                src[i] = B + g * K + kbase + 16 * (pc ^ swz16(r));
            }
        }
    }
    // DMA of K step ks into LDS buffer `buf`. Past the last step the loop
    // keeps issuing (ks clamped to nk-1) into a buffer that is never read
    // again, so every step has the same number of loads in flight and one
    // vmcnt threshold serves the whole loop.
    const bool hi = C::INS % C::NW == 0 || wid < C::INS % C::NW;  // wave-uniform
    auto issue = [&](int ks, int buf) {
        int8_t *stage = smem + buf * C::STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < C::INS_PER_WAVE; ++i) {
            const int j = wid + i * C::NW;
            if (i < C::INS_LO || hi) dma16(src[i] + (int64_t)ks * kstep[i], stage + 1024 * j);
        }
    };
    // Stage of step kt is in LDS (for every wave) once this wave has at most
    // the loads of the STAGES-2 later stages in flight and the block has met.
    auto wait_later = [&]() {
        if (hi)
            wait_vmcnt<(STAGES - 2) * C::INS_HI>();
        else
            wait_vmcnt<(STAGES - 2) * C::INS_LO>();
    };
    auto wait_stage = [&]() {
        wait_later();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    const int wm = wid / WGN, wn = wid % WGN;
    const int fr = lane & 15, fq = lane >> 4;
    const int chunk = 16 * (fq ^ swz16(fr));
    const int a_off = (wm * C::WM + fr) * kDmaBK + chunk;
    // B fragment i: 16 rows from b_off + i*16*B_ROW; packed ternary rows hold
    // 4 words (one 16-code word per lane: row fr, word fq, conflict-free).
    const int b_off = TER ? BM * kDmaBK + (wn * C::WN + fr) * C::B_ROW + 4 * fq
                          : BM * kDmaBK + (wn * C::WN + fr) * kDmaBK + chunk;
    auto read_b = [&](const int8_t *st, int i, F &f) {
        if (TER)
            f.w[i] = *reinterpret_cast<const uint32_t *>(st + b_off + i * 16 * C::B_ROW);
        else
            f.b[i] = *reinterpret_cast<const v4i *>(st + b_off + i * 16 * C::B_ROW);
    };
    auto read_frags = [&](int buf, F &f) {
        const int8_t *st = smem + buf * C::STAGE_BYTES;
#pragma unroll
        for (int j = 0; j < C::FM; ++j)
            f.a[j] = *reinterpret_cast<const v4i *>(st + a_off + j * 16 * kDmaBK);
#pragma unroll
        for (int i = 0; i < C::FN; ++i) read_b(st, i, f);
        if (TER) {
#pragma unroll
            for (int i = 0; i < C::FN; ++i) f.b[i] = ternary_lut_decode(lut, f.w[i]);
        }
    };

    v4i acc[C::FN][C::FM];
#pragma unroll
    for (int i = 0; i < C::FN; ++i)
#pragma unroll
        for (int j = 0; j < C::FM; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    // The MFMA is issued as inline asm with its accumulator tied to an AGPR
    // operand ("+a"): the builtin's untied form makes the register allocator
    // rotate 224-256 live accumulators through copies at this register
    // pressure. The compiler does not see these as MFMAs, so the wait states
    // it would insert after the AGPR zero-fill and before the epilogue reads
    // the accumulators are written out explicitly (s_nop below).
    auto mfma_rows = [&](const F &f, int i0, int i1) {
#pragma unroll
        for (int i = i0; i < i1; ++i)
#pragma unroll
            for (int j = 0; j < C::FM; ++j)
                mfma_i8_acc(acc[i][j], f.b[i], f.a[j]);
    };

    // One K step with fragments `cur` (step kt) in registers: the first half
    // of its MFMAs, then, while they run, the wait + barrier for step kt+1,
    // the DMA of step kt+STAGES into the buffer `cur` came from and the
    // fragment reads of step kt+1 into `nxt`; then the second half.
    // In the second half each MFMA is followed by one memory operation, in
    // the order they are needed: for ternary B first the FN code words, then
    // the FM activation fragment reads of step kt+1, the FN weight fragment
    // reads (ternary: the LUT decodes of the words), then the DMA issues of
    // step kt+STAGES.
    constexpr int H0 = C::FN / 2;
    constexpr int W0 = TER ? C::FN : 0;  // leading slots for ternary code words
    constexpr int NMEM = W0 + C::FM + C::FN + C::INS_PER_WAVE;
    constexpr int NMF = (C::FN - H0) * C::FM;
    constexpr int NSLOT = NMF > NMEM ? NMF : NMEM;
    auto step = [&](int kt, F &cur, F &nxt) {
        mfma_rows(cur, 0, H0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // cur fully read out of LDS
        wait_stage();
        const int8_t *rd = smem + ((kt + 1) % STAGES) * C::STAGE_BYTES;
        int8_t *wr = smem + (kt % STAGES) * C::STAGE_BYTES;
        const int64_t kn = std::min(kt + STAGES, nk - 1);
#pragma unroll
        for (int t = 0; t < NSLOT; ++t) {
            if (t < NMF) mfma_i8_acc<true>(acc[H0 + t / C::FM][t % C::FM], cur.b[H0 + t / C::FM],
                                           cur.a[t % C::FM]);
            if (t < W0) {
                read_b(rd, t, nxt);
            } else if (t < W0 + C::FM) {
                const int ja = t - W0;
                nxt.a[ja] = *reinterpret_cast<const v4i *>(rd + a_off + ja * 16 * kDmaBK);
            } else if (t < W0 + C::FM + C::FN) {
                const int ib = t - W0 - C::FM;
                if (TER)
                    nxt.b[ib] = ternary_lut_decode(lut, nxt.w[ib]);
                else
                    read_b(rd, ib, nxt);
            } else if (t < NMEM) {
                const int q = t - W0 - C::FM - C::FN;
                if (q < C::INS_LO || hi) dma16(src[q] + kn * kstep[q], wr + 1024 * (wid + q * C::NW));
            }
        }
    };

#pragma unroll
    for (int s = 0; s < STAGES; ++s) issue(std::min(s, nk - 1), s);
    if (hi)  // stage 0 of this wave landed
        wait_vmcnt<(STAGES - 1) * C::INS_HI>();
    else
        wait_vmcnt<(STAGES - 1) * C::INS_LO>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    asm volatile("s_nop 4" ::: "memory");  // AGPR writes of the zero-fill -> MFMA srcC
    F f0, f1;
    read_frags(0, f0);
    for (int kt = 0; kt < nk; kt += 2) {
        step(kt, f0, f1);
        step(kt + 1, f1, f0);
    }
    wait_vmcnt<0>();  // drain the trailing DMA before the block's LDS is released
    // last MFMA results -> accumulator reads (16-cycle MFMA: >= 18 wait states)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");

    if constexpr (KS > 1) {
        // groups 1..KS-1 park their partial sums in the (now idle) stage
        // buffers, lane-contiguous 16-byte slots; group 0 adds them
        __builtin_amdgcn_s_barrier();  // every group is done reading its stages
        constexpr int WPART = C::FN * C::FM * 64;  // v4i per wave
        v4i *red = reinterpret_cast<v4i *>(smem_all);
        if (kg > 0) {
            v4i *dst = red + ((kg - 1) * C::NW + wid) * WPART + lane;
#pragma unroll
            for (int i = 0; i < C::FN; ++i)
#pragma unroll
                for (int j = 0; j < C::FM; ++j) dst[(i * C::FM + j) * 64] = acc[i][j];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (kg > 0) return;
#pragma unroll
        for (int g = 1; g < KS; ++g) {
            const v4i *srcp = red + ((g - 1) * C::NW + wid) * WPART + lane;
#pragma unroll
            for (int i = 0; i < C::FN; ++i)
#pragma unroll
                for (int j = 0; j < C::FM; ++j) {
                    const v4i p = srcp[(i * C::FM + j) * 64];
                    acc[i][j].x = (int)((uint32_t)acc[i][j].x + (uint32_t)p.x);
                    acc[i][j].y = (int)((uint32_t)acc[i][j].y + (uint32_t)p.y);
                    acc[i][j].z = (int)((uint32_t)acc[i][j].z + (uint32_t)p.z);
                    acc[i][j].w = (int)((uint32_t)acc[i][j].w + (uint32_t)p.w);
                }
        }
    }
    tile_epilogue<C::FM, C::FN, OUT_Y, OUT_ACC>(epi, acc, bm0 + wm * C::WM + fr,
                                                bn0 + wn * C::WN + 4 * fq);
}

// --------------------------------------- prefill GEMM on 128-byte LDS rows
// The M > 128 kernel: block tile 256 x 224, WGM x WGN waves with int32
// accumulators in AGPRs, as gemm_dma_kernel, but staged in K steps of 128
// bytes so that every DMA instruction moves whole 128-byte cache lines (8 tile
// rows x 128 B). With 64-byte rows each instruction used half of each line it
// pulled from L2, and the DMA stream ran at ~60% of the full-line rate (14.6
// vs 24.5 TB/s L2 -> LDS on this tile order).
//
//  * LDS: activations in a ring of 3 stages (3 x 32 KiB), weights in a ring
//    of 2 (2 x 28 KiB): 152 KiB. A stage's activation loads are issued two
//    stages ahead, its weight loads one stage ahead (weights first, so that
//    one vmcnt threshold -- the activation loads of the stage after -- waits
//    for exactly what the next stage needs).
//  * Row layout: 128 B per tile row, 16-byte chunk c stored at c ^ swz8(row),
//    conflict-free for the fragment reads (16 rows x one chunk per quarter
//    wave).
//  * One barrier per stage, placed PRE MFMAs into the stage's second half
//    (64-K). After it, the DMA of the next stages is spread one instruction
//    per IL MFMAs (a burst of DMA issues stalls the issuing waves' MFMAs
//    behind the memory queue); the sequence runs into the next stage and is
//    complete before the next barrier.
//  * Fragment reads of the next half-stage are interleaved one per MFMA.
//  * The stage body is generated slot by slot at compile time (static_for),
//    so the 56-112 MFMA slots and their memory operations are straight-line
//    code whatever the unroller's thresholds.
constexpr int kL = 128;  // K bytes per stage
constexpr int kTerLutCopies = 16;  // ternary decode table copies (16 KiB)

// f(std::integral_constant<int, 0>{}), ..., f(std::integral_constant<int, N-1>{}):
// a loop unrolled by construction, whose body sees its index as a constant.
template <class Fn, int... Is>
__device__ __forceinline__ void static_for_impl(Fn &&f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class Fn>
__device__ __forceinline__ void static_for(Fn &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ int swz8(int r) { return (r >> 1) & 7; }

// BM x BN block tile of WGM x WGN waves per K group; PRE: MFMAs of a stage's
// second half before its barrier; IL: MFMAs per DMA issue; KS: K groups (K
// split inside the block, partial sums added in LDS); TER: the weights are
// packed 2-bit ternary codes (TernaryTensor::packed rows, 32 bytes per row per
// 128-K stage), decoded to int8 MFMA operands through an LDS table. DEC
// (ternary only, > 0): the early-word schedule -- the code words of both
// halves of the next stage are read right after the barrier, the next
// stage's first half is decoded DEC MFMAs after it and its second half at the
// start of that stage, so no table lookup sits just before the MFMAs that use
// it.
template <int BM_, int BN_, int WGM_, int WGN_, int PRE, int IL, int KS_ = 1, bool TER_ = false,
          int DEC_ = 0, bool PERM_ = false>
struct L128Cfg {
    static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, KS = KS_;
    static constexpr bool TER = TER_;
    // PERM (ternary only): the weights are in the MFMA layout of
    // rnn_ternary_prepack and decode by byte permutes, with no LDS table
    static constexpr bool PERM = PERM_;
    static constexpr int DEC = DEC_;
    static constexpr int NW = WGM * WGN, NT = NW * 64;          // per K group
    static constexpr int WM = BM / WGM, WN = BN / WGN, FM = WM / 16, FN = WN / 16;
    static constexpr int W_ROW = TER ? kL / 4 : kL;             // weight bytes per row per stage
    static constexpr int W_LPR = W_ROW / 16;                    // lanes per weight row in a load
    static constexpr int RA = 3, RW = 2;                        // ring stages
    static constexpr int A_SLOT = BM * kL, W_SLOT = BN * W_ROW;
    static constexpr int A_INS = A_SLOT / 1024, W_INS = W_SLOT / 1024;  // 1 KiB loads per stage
    static constexpr int APW = A_INS / NW;                      // per wave
    static constexpr int WPW = (W_INS + NW - 1) / NW;           // waves >= W_INS % NW: WPW - 1
    static constexpr bool W_EVEN = W_INS % NW == 0;             // every wave issues WPW
    static constexpr int NDMA = WPW + APW;                      // DMA slots per stage
    static constexpr int GROUP_LDS = RA * A_SLOT + RW * W_SLOT;
    static constexpr int LDS_BYTES = KS * GROUP_LDS;
    static constexpr int LUT_BYTES = TER && !PERM ? 1024 * kTerLutCopies : 0;  // decode table copies
    static constexpr int HALF = FM * FN;                        // MFMAs per 64-K half
    static constexpr int T0 = HALF + PRE;                       // barrier slot
    // fragment-read slots of a half: weight fragments (ternary: code words,
    // then table decodes) and activation fragments
    static constexpr int RD = TER ? 2 * FN + FM : FN + FM;
    static constexpr int PART = NW * FN * FM * 64 * 16;         // one group's partial sums
    static_assert(WM % 16 == 0 && WN % 16 == 0 && BM % WGM == 0 && BN % WGN == 0, "wave tiles");
    static_assert(A_SLOT % 1024 == 0 && W_SLOT % 1024 == 0, "whole 1 KiB loads");
    static_assert(A_INS % NW == 0 && (W_EVEN || W_INS / NW == WPW - 1), "load split");
    static_assert(LDS_BYTES + LUT_BYTES <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");
    static_assert(KS == 1 || (KS - 1) * PART <= LDS_BYTES, "split-K partials fit in LDS");
    static_assert(DEC > 0 || (RD <= HALF && T0 + RD <= 2 * HALF), "fragment-read slots");
    static_assert(!PERM || TER, "the MFMA code layout is a ternary layout");
    // the ternary weight-row DMA and the early-word schedule are written for
    // one row of waves per K group
    static_assert(!TER || WGM == 1, "ternary tiles: one row of waves");
    static_assert(DEC == 0 || (TER && FN + FM <= T0 && T0 + FM < 2 * HALF &&
                               DEC >= 1 && T0 + DEC + FN <= 2 * HALF),
                  "early-word slots: second-half decodes and activations before the barrier, "
                  "the next stage's activations and decodes after it");
    // DMA op q of the sequence started at the barrier of stage s sits after
    // MFMA slot pos(q) (counted from stage s's first MFMA): ops with
    // pos < 2*HALF ("head") are issued in stage s, the rest ("tail") at
    // pos - 2*HALF in stage s+1, all before the next barrier.
    static constexpr int pos(int q) { return T0 + IL * (q + 1) - 1; }
    static constexpr bool head(int q) { return pos(q) < 2 * HALF; }
    // head ops a wave issues (waves without the last W load skip op WPW-1)
    static constexpr int head_ops(bool w_hi) {
        int n = 0;
        for (int q = 0; q < NDMA; ++q) n += head(q) && (q != WPW - 1 || w_hi);
        return n;
    }
    static constexpr bool window_ok() { return pos(NDMA - 1) - 2 * HALF < T0; }
};
// The prefill geometry (run by gemm_pp_kernel, whose schedule does not use
// PRE / IL): 256 x 224 block tiles, 8 waves of 64 x 112 (two per SIMD). Four
// waves of 128 x 112 (one per SIMD) read 32% fewer LDS fragment bytes and run
// at a higher clock, but lose that to single-wave issue stalls: 1-2% slower
// on the prefill shape.
using PrefillCfg = L128Cfg<256, 224, 4, 2, 0, 1>;
// Ternary: 64 x 128 tiles (512 x 4096 is 256 tiles, one per CU) of two K
// groups of 4 waves (64 x 32 each): 8 waves per CU. Against 128 x 64 tiles a
// block moves a third fewer bytes into LDS (64 activation rows per stage
// instead of 128) and no weight word is decoded by two waves. The
// early-word schedule decodes the next stage's first half 3 MFMAs after the
// barrier. Measured on 512 x 4096 x 4096: 12.99 us against 13.63 us for
// 128 x 64 tiles with the plain schedule.
using L128Ter = L128Cfg<64, 128, 1, 4, 0, 3, 2, true, 3>;
static_assert(L128Ter::window_ok(), "DMA window");
// The same tiles and schedule on weights in the MFMA code layout. A sweep of
// the schedule parameters (write-through epilogue, one process): IL 3 / 5 with
// DEC 2-5 and PRE 0-2 all within 0.3 us of this one (10.87 us), none faster.
// The generated schedule is validated by the GPU tests only for the
// configurations instantiated here: IL = 4 with DEC = 3 passes window_ok()
// yet computed wrong sums in that sweep.
using L128TerPerm = L128Cfg<64, 128, 1, 4, 0, 5, 2, true, 3, true>;
static_assert(L128TerPerm::window_ok(), "DMA window");

template <class C, bool OUT_Y, bool OUT_ACC, bool WT = false>
__global__ __launch_bounds__(C::KS *C::NT)
__attribute__((amdgpu_waves_per_eu(C::KS * C::NW / 4, C::KS * C::NW / 4)))
void gemm_l128_kernel(const int8_t *__restrict__ A, const int8_t *__restrict__ B, int64_t M,
                      int64_t N, int64_t K, int tiles_m, int tiles_n, Epilogue epi) {
    using F = Frags<C::FM, C::FN>;
    // One LDS array (stage rings, then the ternary decode table): with a
    // second __shared__ object the compiler tags LDS accesses with per-object
    // alias scopes and then makes every fragment read that follows a DMA into
    // the same object wait for all outstanding loads.
    __shared__ __attribute__((aligned(1024))) int8_t smem_all[C::LDS_BYTES + C::LUT_BYTES];
    uint32_t *const lut = reinterpret_cast<uint32_t *>(smem_all + C::LDS_BYTES);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = wave / C::NW, wid = wave % C::NW;  // K group, wave within the group
    int8_t *const sa = smem_all + kg * C::GROUP_LDS;
    int8_t *const sw = sa + C::RA * C::A_SLOT;
    int tm, tn;
    xcd_tile((int)blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t bm0 = (int64_t)tm * C::BM, bn0 = (int64_t)tn * C::BN;
    const int64_t kbase = kg * (K / C::KS);  // this group's K range
    const int nk = (int)(K / C::KS / kL);    // >= 1 (host-checked)

    // DMA instruction j of a stage covers activation rows 8j..8j+7 (lane l:
    // row 8j + l/8, LDS chunk l%8 filled with the row's logical chunk
    // (l%8) ^ swz8(row)), or weight rows W_ROW/16-lanes each: int8 as the
    // activations; ternary 32 rows x 32 B (lane l: row 32j + l/2, LDS half l%2
    // filled with the row's logical half (l%2) ^ ((row >> 3) & 1)). Wave w
    // issues A loads j = w + NW*i and W loads j = w + NW*i < W_INS.
    // A lane's source is a loop-invariant 32-bit byte offset into the operand
    // (the host checks that the operands span less than 4 GiB) and the stage
    // advance is the load's scalar offset, so no address register is written
    // in the loop: the compiler makes a write to a register that an
    // outstanding load used as its address wait for every outstanding load.
    uint32_t oa[C::APW], ow[C::WPW];
    {
        const int rr = lane >> 3, pc = lane & 7;
#pragma unroll
        for (int i = 0; i < C::APW; ++i) {
            const int r = 8 * (wid + C::NW * i) + rr;
            oa[i] = (uint32_t)(std::min<int64_t>(bm0 + r, M - 1) * K + kbase + 16 * (pc ^ swz8(r)));
        }
        const int wr = lane / C::W_LPR, wc = lane % C::W_LPR;
#pragma unroll
        for (int i = 0; i < C::WPW; ++i) {
            const int r = (1024 / C::W_ROW) * std::min(wid + C::NW * i, C::W_INS - 1) + wr;
            const int64_t g = std::min<int64_t>(bn0 + r, N - 1);
            if constexpr (C::TER)
                ow[i] = (uint32_t)(g * (K / 4) + kbase / 4 + 16 * (wc ^ ((r >> 3) & 1)));
            else
                ow[i] = (uint32_t)(g * K + kbase + 16 * (wc ^ swz8(r)));
        }
    }
    const bool w_hi = C::W_EVEN || wid < C::W_INS % C::NW;  // issues the last W load
    // Loads of stage ks (clamped to the last stage: past the end the loop keeps
    // issuing into slots that are never read again, so every barrier waits for
    // the same count).
    const uint32_t a_bytes = (uint32_t)(M * K), w_bytes = (uint32_t)(N * (C::TER ? K / 4 : K));
    auto dma_w = [&](int i, int ks) {
        dma16_buf(B, w_bytes, ow[i], (uint32_t)(std::min(ks, nk - 1) * C::W_ROW),
                  sw + (ks & 1) * C::W_SLOT + 1024 * (wid + C::NW * i));
    };
    auto dma_a = [&](int i, int ks, int slot3) {
        dma16_buf(A, a_bytes, oa[i], (uint32_t)(std::min(ks, nk - 1) * kL),
                  sa + slot3 * C::A_SLOT + 1024 * (wid + C::NW * i));
    };
    // Op q of the DMA sequence that follows the barrier of stage s: W loads of
    // stage s+2, then A loads of stage s+3.
    auto dma_op = [&](int q, int s, int slot3_s) {
        if (q < C::WPW) {
            if (q < C::WPW - 1 || w_hi) dma_w(q, s + 2);
        } else {
            dma_a(q - C::WPW, s + 3, slot3_s);  // (s+3) % 3 == s % 3
        }
    };

    const int wm = wid / C::WGN, wn = wid % C::WGN;
    const int fr = lane & 15, fq = lane >> 4;
    const uint32_t *const lut_lane = lut + lane % kTerLutCopies;  // this lane's table copy
    // 2-bit codes -> the int8 MFMA operand: byte permutes (MFMA layout) or the
    // replicated LDS table (reference layout)
    auto decode = [&](uint32_t w) -> v4i {
        if constexpr (C::PERM)
            return ternary_perm_decode(w);
        else
            return ternary_lut_decode_rep<kTerLutCopies>(lut_lane, w);
    };
    // fragment rows start at multiples of 16, so the row swizzles depend on fr
    const int a_row = (wm * C::WM + fr) * kL, b_row = (wn * C::WN + fr) * C::W_ROW;
    const int ch0 = 16 * (fq ^ swz8(fr)), ch1 = 16 * ((4 + fq) ^ swz8(fr));
    // weight fragment of half h: int8 chunk 4h+fq; ternary code word 4h+fq of
    // the 32-byte row (16 codes), in the half h ^ ((fr >> 3) & 1)
    const int wb0 = C::TER ? 16 * ((fr >> 3) & 1) + 4 * fq : ch0;
    const int wb1 = C::TER ? 16 * (1 ^ ((fr >> 3) & 1)) + 4 * fq : ch1;
    auto read_w = [&](const int8_t *slot, int i, int wb, F &f) {
        if constexpr (C::TER)
            f.w[i] = *reinterpret_cast<const uint32_t *>(slot + b_row + i * 16 * C::W_ROW + wb);
        else
            f.b[i] = *reinterpret_cast<const v4i *>(slot + b_row + i * 16 * C::W_ROW + wb);
    };
    auto read_a = [&](const int8_t *slot, int j, int ch, F &f) {
        f.a[j] = *reinterpret_cast<const v4i *>(slot + a_row + j * 16 * kL + ch);
    };
    // the fragment-read slots of a half, starting at slot t0: weight words /
    // fragments, activation fragments, (ternary) decodes
    auto read_slot = [&](auto uc, const int8_t *aslot, const int8_t *wslot, int ch, int wb, F &f) {
        constexpr int u = decltype(uc)::value;
        if constexpr (u < C::FN) {
            read_w(wslot, u, wb, f);
        } else if constexpr (u < C::FN + C::FM) {
            read_a(aslot, u - C::FN, ch, f);
        } else if constexpr (C::TER && u < C::RD) {
            f.b[u - C::FN - C::FM] = decode(f.w[u - C::FN - C::FM]);
        }
    };

    v4i acc[C::FN][C::FM];
#pragma unroll
    for (int i = 0; i < C::FN; ++i)
#pragma unroll
        for (int j = 0; j < C::FM; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    // Prologue: A(0); the sequence of "stage -2" (W(0), A(1)); the head ops of
    // the sequence of "stage -1" (W(1), A(2)) -- its tail ops are issued by
    // the first loop iteration, as every iteration issues the previous
    // sequence's tail.
#pragma unroll
    for (int i = 0; i < C::APW; ++i) dma_a(i, 0, 0);
#pragma unroll
    for (int i = 0; i < C::WPW; ++i)
        if (i < C::WPW - 1 || w_hi) dma_w(i, 0);
#pragma unroll
    for (int i = 0; i < C::APW; ++i) dma_a(i, 1, 1);
#pragma unroll
    for (int q = 0; q < C::NDMA; ++q)
        if (C::head(q)) dma_op(q, -1, 2);
    // the decode table is built while the first loads are in flight (the
    // barrier below publishes it)
    if constexpr (C::TER && !C::PERM) {
        for (int t = threadIdx.x; t < 256 * kTerLutCopies; t += C::KS * C::NT)
            lut[t] = ternary_lut_entry((uint32_t)(t / kTerLutCopies));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    // A(0), W(0) of this wave landed: only A(1) and the head ops outstanding
    if (w_hi)
        wait_vmcnt<C::APW + C::head_ops(true)>();
    else
        wait_vmcnt<C::APW + C::head_ops(false)>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    asm volatile("s_nop 4" ::: "memory");  // AGPR writes of the zero-fill -> MFMA srcC

    F f0, f1;
    if constexpr (C::DEC > 0) {
        // stage 0: the code words of both halves, the first half's
        // activations and decodes (the second half decodes at its start)
#pragma unroll
        for (int i = 0; i < C::FN; ++i) read_w(sw, i, wb0, f0);
#pragma unroll
        for (int i = 0; i < C::FN; ++i) read_w(sw, i, wb1, f1);
#pragma unroll
        for (int j = 0; j < C::FM; ++j) read_a(sa, j, ch0, f0);
#pragma unroll
        for (int i = 0; i < C::FN; ++i) f0.b[i] = decode(f0.w[i]);
    } else {
        static_for<C::RD>([&](auto uc) { read_slot(uc, sa, sw, ch0, wb0, f0); });
    }

    int slot3 = 0;  // s % 3
    for (int s = 0; s < nk; ++s) {
        const int slot3n = slot3 == 2 ? 0 : slot3 + 1;            // (s+1) % 3
        const int slot3p = slot3 == 0 ? 2 : slot3 - 1;            // (s-1) % 3 == (s+2) % 3
        const int8_t *a_cur = sa + slot3 * C::A_SLOT, *w_cur = sw + (s & 1) * C::W_SLOT;
        const int8_t *a_nxt = sa + slot3n * C::A_SLOT, *w_nxt = sw + ((s + 1) & 1) * C::W_SLOT;
        // One MFMA slot t of the stage (t < HALF: first half on f0, else second
        // half on f1) and the memory operations that follow it, generated at
        // compile time for every t.
        static_for<2 * C::HALF>([&](auto tc) {
            constexpr int t = decltype(tc)::value;
            if constexpr (t == C::T0) {
                // fragments of this stage fully read; next stage's A and W in LDS
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                wait_vmcnt<C::APW>();
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
            }
            if constexpr (t < C::HALF) {
                mfma_i8_acc<true>(acc[t / C::FM][t % C::FM], f0.b[t / C::FM], f0.a[t % C::FM]);
            } else {
                constexpr int u = t - C::HALF;
                mfma_i8_acc<true>(acc[u / C::FM][u % C::FM], f1.b[u / C::FM], f1.a[u % C::FM]);
            }
            if constexpr (C::DEC > 0) {
                // early-word schedule: this stage's second half decodes its
                // words (read after the previous barrier), then reads its
                // activations; after the barrier, the next stage's words of
                // both halves, its first-half activations and, DEC MFMAs in,
                // its first-half decodes
                if constexpr (t < C::FN)
                    f1.b[t] = decode(f1.w[t]);
                else if constexpr (t < C::FN + C::FM)
                    read_a(a_cur, t - C::FN, ch1, f1);
                if constexpr (t == C::T0) {
#pragma unroll
                    for (int i = 0; i < C::FN; ++i) read_w(w_nxt, i, wb0, f0);
#pragma unroll
                    for (int i = 0; i < C::FN; ++i) read_w(w_nxt, i, wb1, f1);
                }
                if constexpr (t > C::T0 && t <= C::T0 + C::FM) read_a(a_nxt, t - C::T0 - 1, ch0, f0);
                if constexpr (t >= C::T0 + C::DEC && t < C::T0 + C::DEC + C::FN)
                    f0.b[t - C::T0 - C::DEC] =
                        decode(f0.w[t - C::T0 - C::DEC]);
            } else {
                // second half of this stage -> f1 (weight fragments first:
                // they were released earliest by the previous stage's MFMAs)
                if constexpr (t < C::RD)
                    read_slot(std::integral_constant<int, t>{}, a_cur, w_cur, ch1, wb1, f1);
                // first half of the next stage -> f0, after the barrier
                if constexpr (t >= C::T0 && t < C::T0 + C::RD)
                    read_slot(std::integral_constant<int, t - C::T0>{}, a_nxt, w_nxt, ch0, wb0, f0);
            }
            // DMA: the tail of the sequence started at the previous barrier,
            // then the head of this stage's
            static_for<C::NDMA>([&](auto qc) {
                constexpr int q = decltype(qc)::value;
                if constexpr (!C::head(q) && t == C::pos(q) - 2 * C::HALF) dma_op(q, s - 1, slot3p);
                if constexpr (C::head(q) && t == C::pos(q)) dma_op(q, s, slot3);
            });
        });
        slot3 = slot3n;
    }
    wait_vmcnt<0>();  // drain the trailing DMA before the block's LDS is released
    // last MFMA results -> accumulator reads (16-cycle MFMA: >= 18 wait states)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");

    if constexpr (C::KS == 2 && C::FM % 2 == 0) {
        // The two K groups exchange halves of their wave tiles through the
        // (now idle) stage buffers: group 0 keeps the first FM/2 row blocks
        // and hands over the rest, group 1 the reverse. Each adds the
        // partner's partial sums to the half it keeps (exact: wrapping int32
        // addition is associative) and writes that half of the output, so the
        // epilogue is split over all 8 waves.
        constexpr int HF = C::FM / 2;
        constexpr int WPART = C::FN * HF * 64;  // v4i per wave and group
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();  // every group is done with its stages
        v4i *red = reinterpret_cast<v4i *>(smem_all);
        auto finish = [&](auto gc) {
            constexpr int g = decltype(gc)::value;
            constexpr int give = g == 0 ? HF : 0, keep = g == 0 ? 0 : HF;
            v4i *dst = red + (g * C::NW + wid) * WPART + lane;
#pragma unroll
            for (int i = 0; i < C::FN; ++i)
#pragma unroll
                for (int j = 0; j < HF; ++j) dst[(i * HF + j) * 64] = acc[i][give + j];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            const v4i *srcp = red + ((1 - g) * C::NW + wid) * WPART + lane;
            v4i half[C::FN][HF];
#pragma unroll
            for (int i = 0; i < C::FN; ++i)
#pragma unroll
                for (int j = 0; j < HF; ++j) {
                    const v4i p = srcp[(i * HF + j) * 64];
                    const v4i a = acc[i][keep + j];
                    half[i][j].x = (int)((uint32_t)a.x + (uint32_t)p.x);
                    half[i][j].y = (int)((uint32_t)a.y + (uint32_t)p.y);
                    half[i][j].z = (int)((uint32_t)a.z + (uint32_t)p.z);
                    half[i][j].w = (int)((uint32_t)a.w + (uint32_t)p.w);
                }
            tile_epilogue<HF, C::FN, OUT_Y, OUT_ACC, WT>(epi, half, bm0 + wm * C::WM + fr + 16 * keep,
                                                     bn0 + wn * C::WN + 4 * fq);
        };
        if (kg == 0)
            finish(std::integral_constant<int, 0>{});
        else
            finish(std::integral_constant<int, 1>{});
        return;
    } else if constexpr (C::KS > 1) {
        // groups 1..KS-1 park their partial sums in the (now idle) stage
        // buffers, lane-contiguous 16-byte slots; group 0 adds them (exact:
        // wrapping int32 addition is associative)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();  // every group is done with its stages
        constexpr int WPART = C::FN * C::FM * 64;  // v4i per wave
        v4i *red = reinterpret_cast<v4i *>(smem_all);
        if (kg > 0) {
            v4i *dst = red + ((kg - 1) * C::NW + wid) * WPART + lane;
#pragma unroll
            for (int i = 0; i < C::FN; ++i)
#pragma unroll
                for (int j = 0; j < C::FM; ++j) dst[(i * C::FM + j) * 64] = acc[i][j];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (kg > 0) return;
#pragma unroll
        for (int g = 1; g < C::KS; ++g) {
            const v4i *srcp = red + ((g - 1) * C::NW + wid) * WPART + lane;
#pragma unroll
            for (int i = 0; i < C::FN; ++i)
#pragma unroll
                for (int j = 0; j < C::FM; ++j) {
                    const v4i p = srcp[(i * C::FM + j) * 64];
                    acc[i][j].x = (int)((uint32_t)acc[i][j].x + (uint32_t)p.x);
                    acc[i][j].y = (int)((uint32_t)acc[i][j].y + (uint32_t)p.y);
                    acc[i][j].z = (int)((uint32_t)acc[i][j].z + (uint32_t)p.z);
                    acc[i][j].w = (int)((uint32_t)acc[i][j].w + (uint32_t)p.w);
                }
        }
    }
    tile_epilogue<C::FM, C::FN, OUT_Y, OUT_ACC, WT>(epi, acc, bm0 + wm * C::WM + fr,
                                                    bn0 + wn * C::WN + 4 * fq);
}

// ------------------------------------------ prefill: ping-pong (8 waves)
// The tiles, LDS rings, DMA addressing and epilogue of gemm_l128_kernel, with
// the two waves of a SIMD taking turns instead of each interleaving reads and
// MFMAs: in each phase one group of 4 waves (one per SIMD) issues the 28 MFMAs
// of a half-stage back to back while the other group reads its next fragments
// and issues its share of the DMA; a barrier swaps the roles (1% faster than
// the interleaved schedule on the prefill shape). Four phases per 128-K stage s:
//   phase 4s   : G0 computes (s,0)      G1 reads (s,0), DMA
//   phase 4s+1 : G0 reads (s,1), DMA    G1 computes (s,0)
//   phase 4s+2 : G0 computes (s,1)      G1 reads (s,1), DMA
//   phase 4s+3 : G0 reads (s+1,0), DMA  G1 computes (s,1)
// Stage s is read in phases 4s-1 .. 4s+2, so its slots take the DMA of
// sequence s (W(s+2), then A(s+3)) from phase 4s+3 on; each wave issues its
// ops of a sequence in its two load phases of the window [4s+3, 4s+7), weight
// loads first. At the end of phase 4s+2 every wave waits until only its A
// loads of the latest sequence are in flight: stage s+1 has landed.
template <class C, bool OUT_Y, bool OUT_ACC, bool WT>
__global__ __launch_bounds__(C::NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_pp_kernel(const int8_t *__restrict__ A, const int8_t *__restrict__ B, int64_t M,
                    int64_t N, int64_t K, int tiles_m, int tiles_n, Epilogue epi) {
    static_assert(C::NW == 8 && C::KS == 1 && !C::TER, "two groups of four int8 waves");
    static_assert(C::NDMA % 2 == 0 && C::NDMA / 2 == C::WPW, "first half: W ops, second: A ops");
    using F = Frags<C::FM, C::FN>;
    __shared__ __attribute__((aligned(1024))) int8_t smem[C::LDS_BYTES];
    int8_t *const sa = smem;
    int8_t *const sw = smem + C::RA * C::A_SLOT;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wid >> 2;  // waves w and w+4 share SIMD w
    int tm, tn;
    xcd_tile((int)blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t bm0 = (int64_t)tm * C::BM, bn0 = (int64_t)tn * C::BN;
    const int nk = (int)(K / kL);

    uint32_t oa[C::APW], ow[C::WPW];
    {
        const int rr = lane >> 3, pc = lane & 7;
#pragma unroll
        for (int i = 0; i < C::APW; ++i) {
            const int r = 8 * (wid + C::NW * i) + rr;
            oa[i] = (uint32_t)(std::min<int64_t>(bm0 + r, M - 1) * K + 16 * (pc ^ swz8(r)));
        }
#pragma unroll
        for (int i = 0; i < C::WPW; ++i) {
            const int r = 8 * std::min(wid + C::NW * i, C::W_INS - 1) + rr;
            ow[i] = (uint32_t)(std::min<int64_t>(bn0 + r, N - 1) * K + 16 * (pc ^ swz8(r)));
        }
    }
    const bool w_hi = C::W_EVEN || wid < C::W_INS % C::NW;
    const uint32_t a_bytes = (uint32_t)(M * K), w_bytes = (uint32_t)(N * K);
    auto dma_w = [&](int i, int ks) {
        dma16_buf(B, w_bytes, ow[i], (uint32_t)(std::min(ks, nk - 1) * kL),
                  sw + (ks & 1) * C::W_SLOT + 1024 * (wid + C::NW * i));
    };
    auto dma_a = [&](int i, int ks, int slot3) {
        dma16_buf(A, a_bytes, oa[i], (uint32_t)(std::min(ks, nk - 1) * kL),
                  sa + slot3 * C::A_SLOT + 1024 * (wid + C::NW * i));
    };
    // the two halves of sequence s: its W loads (stage s+2), its A loads
    // (stage s+3, into slot s % 3)
    auto dma_w_half = [&](int s) {
#pragma unroll
        for (int i = 0; i < C::WPW; ++i)
            if (i < C::WPW - 1 || w_hi) dma_w(i, s + 2);
    };
    auto dma_a_half = [&](int s, int slot3_s) {
#pragma unroll
        for (int i = 0; i < C::APW; ++i) dma_a(i, s + 3, slot3_s);
    };

    const int wm = wid / C::WGN, wn = wid % C::WGN;
    const int fr = lane & 15, fq = lane >> 4;
    const int a_row = (wm * C::WM + fr) * kL, b_row = (wn * C::WN + fr) * kL;
    const int ch0 = 16 * (fq ^ swz8(fr)), ch1 = 16 * ((4 + fq) ^ swz8(fr));
    auto load = [&](const int8_t *aslot, const int8_t *wslot, int ch, F &f) {
#pragma unroll
        for (int j = 0; j < C::FM; ++j)
            f.a[j] = *reinterpret_cast<const v4i *>(aslot + a_row + j * 16 * kL + ch);
#pragma unroll
        for (int i = 0; i < C::FN; ++i)
            f.b[i] = *reinterpret_cast<const v4i *>(wslot + b_row + i * 16 * kL + ch);
    };
    v4i acc[C::FN][C::FM];
#pragma unroll
    for (int i = 0; i < C::FN; ++i)
#pragma unroll
        for (int j = 0; j < C::FM; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    auto compute = [&](const F &f) {
#pragma unroll
        for (int i = 0; i < C::FN; ++i)
#pragma unroll
            for (int j = 0; j < C::FM; ++j) mfma_i8_acc<true>(acc[i][j], f.b[i], f.a[j]);
    };
    auto barrier = [&]() {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    // Prologue: A(0), W(0), A(1); G0 also the first half of sequence -1
    // (W(1)), which the loop would have issued in phase -1.
#pragma unroll
    for (int i = 0; i < C::APW; ++i) dma_a(i, 0, 0);
#pragma unroll
    for (int i = 0; i < C::WPW; ++i)
        if (i < C::WPW - 1 || w_hi) dma_w(i, 0);
#pragma unroll
    for (int i = 0; i < C::APW; ++i) dma_a(i, 1, 1);
    F f;
    if (grp == 0) {
        dma_w_half(-1);
        // A(0), W(0) landed: A(1) and W(1) outstanding
        if (w_hi)
            wait_vmcnt<C::APW + C::WPW>();
        else
            wait_vmcnt<C::APW + C::WPW - 1>();
        barrier();
        asm volatile("s_nop 4" ::: "memory");  // AGPR writes of the zero-fill -> MFMA srcC
        load(sa, sw, ch0, f);                  // (0,0), phase -1
        barrier();
        int slot3 = 0;
        for (int s = 0; s < nk; ++s) {
            const int slot3n = slot3 == 2 ? 0 : slot3 + 1, slot3p = slot3 == 0 ? 2 : slot3 - 1;
            compute(f);                                                      // 4s: (s,0)
            barrier();
            load(sa + slot3 * C::A_SLOT, sw + (s & 1) * C::W_SLOT, ch1, f);  // 4s+1: (s,1)
            dma_a_half(s - 1, slot3p);
            barrier();
            compute(f);                                                      // 4s+2: (s,1)
            wait_vmcnt<C::APW>();
            barrier();
            load(sa + slot3n * C::A_SLOT, sw + ((s + 1) & 1) * C::W_SLOT, ch0, f);  // 4s+3: (s+1,0)
            dma_w_half(s);
            barrier();
            slot3 = slot3n;
        }
    } else {
        wait_vmcnt<C::APW>();  // A(0), W(0) landed: A(1) outstanding
        barrier();
        asm volatile("s_nop 4" ::: "memory");
        barrier();
        int slot3 = 0;
        for (int s = 0; s < nk; ++s) {
            const int slot3n = slot3 == 2 ? 0 : slot3 + 1, slot3p = slot3 == 0 ? 2 : slot3 - 1;
            load(sa + slot3 * C::A_SLOT, sw + (s & 1) * C::W_SLOT, ch0, f);  // 4s: (s,0)
            dma_w_half(s - 1);
            barrier();
            compute(f);                                                      // 4s+1: (s,0)
            barrier();
            load(sa + slot3 * C::A_SLOT, sw + (s & 1) * C::W_SLOT, ch1, f);  // 4s+2: (s,1)
            dma_a_half(s - 1, slot3p);
            wait_vmcnt<C::APW>();
            barrier();
            compute(f);                                                      // 4s+3: (s,1)
            barrier();
            slot3 = slot3n;
        }
    }
    wait_vmcnt<0>();  // drain the trailing DMA before the block's LDS is released
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    tile_epilogue<C::FM, C::FN, OUT_Y, OUT_ACC, WT>(epi, acc, bm0 + wm * C::WM + fr,
                                                    bn0 + wn * C::WN + 4 * fq);
}

// ------------------------------------------------------------ skinny GEMV
// M <= 16 (decode). One workgroup per 16 output columns; the WAVES waves of a
// workgroup split K, each streaming its K range of the 16 weight rows with
// 16-byte loads (KCH loads in flight per lane) into 16x16x64 MFMAs whose A
// operand is the (zero-padded) activation block. Partial 16x16 int32 tiles
// are summed in LDS (exact) and the epilogue runs once per output.
template <int WAVES, int KCH>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(
    const int8_t *__restrict__ A, const int8_t *__restrict__ W, int64_t M, int64_t N, int64_t K,
    Epilogue epi) {
    __shared__ int32_t part[WAVES][16][16];
    const int tid = threadIdx.x, wid = tid / 64, lane = tid % 64;
    const int row = lane & 15, q = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * 16;
    const int64_t nblk = (K + 63) / 64;               // 64-wide K blocks
    const int64_t per = (nblk + WAVES - 1) / WAVES;    // blocks per wave
    const int64_t kb0 = wid * per, kb1 = std::min<int64_t>(nblk, kb0 + per);
    const bool arow = row < M;
    const int64_t wn = std::min<int64_t>(n0 + row, N - 1);
    const int8_t *arp = A + (arow ? row : 0) * K;
    const int8_t *wrp = W + wn * K;

    v4i acc = {0, 0, 0, 0};
    for (int64_t kb = kb0; kb < kb1; kb += KCH) {
        v4i a[KCH], b[KCH];
#pragma unroll
        for (int c = 0; c < KCH; ++c) {
            const int64_t k = (kb + c) * 64 + q * 16;
            const bool ok = kb + c < kb1 && k < K;
            b[c] = ok ? *reinterpret_cast<const v4i *>(wrp + k) : v4i{0, 0, 0, 0};
            a[c] = ok && arow ? *reinterpret_cast<const v4i *>(arp + k) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int c = 0; c < KCH; ++c)
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[c], b[c], acc, 0, 0, 0);
    }
    part[wid][4 * q + 0][row] = acc.x;
    part[wid][4 * q + 1][row] = acc.y;
    part[wid][4 * q + 2][row] = acc.z;
    part[wid][4 * q + 3][row] = acc.w;
    __syncthreads();
    for (int t = tid; t < 256; t += WAVES * 64) {
        const int m = t / 16, n = t % 16;
        uint32_t s = 0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) s += (uint32_t)part[w][m][n];
        epi.store(m, n0 + n, (int32_t)s);
    }
}

// The same GEMV with whole-line weight loads (K % 4096 == 0): an MFMA weight
// fragment spans 16 rows x 64 B, so loading it directly makes every load
// instruction touch half of 16 cache lines, and each line is requested twice.
// Here a wave loads 4 rows x 256 B per instruction (whole 128-byte lines,
// non-temporal: the weights are streamed once) and regroups them into MFMA
// fragments through a per-wave 4 KiB LDS buffer (16 rows x 256 B, the 16-byte
// chunk c of row r stored at c ^ r: conflict-free writes and fragment reads).
// A microbenchmark of the two load patterns alone over 45 MB: 9.1 us against
// 7.7 us per launch. The activations (L2-resident, shared by every
// workgroup) are issued first, so the in-order wait for each weight group
// also covers them. Every load is unconditional (rows past M read row 0 and
// are zeroed afterwards): a load behind a branch makes the compiler wait for
// all of them before the first group.
//  * M > SMALLM: fragment-layout activation loads (16 per wave, no duplicate
//    data when M = 16).
//  * M <= SMALLM: fragment-layout loads would return mostly duplicate rows
//    (for M = 1, 1 KiB per instruction for 64 useful bytes) through the same
//    load-return path the weights need; instead each activation row of the
//    wave's K range is loaded once (1 KiB contiguous), staged in LDS and read
//    back as fragments (rows < M broadcast, the rest zero). Measured without
//    any activation loads, M = 1 over N = 11008 ran 1.2 us faster.
template <int WAVES, int SMALLM>
__global__ __launch_bounds__(WAVES * 64) void gemv_wl_kernel(
    const int8_t *__restrict__ A, const int8_t *__restrict__ W, int64_t M, int64_t N, int64_t K,
    Epilogue epi) {
    __shared__ __attribute__((aligned(16))) int8_t stage[WAVES][2][4096];
    __shared__ __attribute__((aligned(16))) int8_t astage[SMALLM > 0 ? WAVES : 1][SMALLM > 0 ? SMALLM : 1][1024];
    __shared__ int32_t part[WAVES][16][16];
    const int tid = threadIdx.x, wid = tid / 64, lane = tid % 64;
    const int row = lane & 15, q = lane >> 4;  // fragment layout
    const int lr = lane >> 4, lc = lane & 15;  // load layout: row 4r + lr, chunk lc
    const int64_t n0 = (int64_t)blockIdx.x * 16;
    const int64_t kq = K / WAVES, k0 = wid * kq;  // this wave's K range (multiple of 1024)
    const bool arow = row < M;
    const int8_t *arp = A + (arow ? row : 0) * K + k0 + q * 16;
    const v4i zero = {0, 0, 0, 0};
    // this thread's output of the epilogue (one per thread), operands first
    static_assert(WAVES * 64 == 256, "one output per thread");
    const int em = tid / 16, en = tid % 16;
    const EpiOps eo = epi.load_ops(em, n0 + en);
    const int8_t *wrp[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) wrp[r] = W + std::min<int64_t>(n0 + 4 * r + lr, N - 1) * K + k0 + lc * 16;

    v4i acc = {0, 0, 0, 0};
    for (int64_t kc = 0; kc < kq; kc += 1024) {
        v4i a[16], w[16], ar[SMALLM > 0 ? SMALLM : 1];
        if constexpr (SMALLM > 0) {
            // rows 0..SMALLM-1 of the K range, 16 bytes per lane (rows >= M
            // re-read row 0; their fragments are zeroed below)
#pragma unroll
            for (int r = 0; r < SMALLM; ++r)
                ar[r] = *reinterpret_cast<const v4i *>(A + (r < M ? r : 0) * K + k0 + kc + lane * 16);
        } else {
#pragma unroll
            for (int kb = 0; kb < 16; ++kb) a[kb] = *reinterpret_cast<const v4i *>(arp + kc + kb * 64);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                w[4 * g + r] =
                    __builtin_nontemporal_load(reinterpret_cast<const v4i *>(wrp[r] + kc + g * 256));
        const int ra = arow && row < SMALLM ? row : 0;
        if constexpr (SMALLM > 0) {
            // (the fragments are read per group below, keeping registers free)
#pragma unroll
            for (int r = 0; r < SMALLM; ++r)
                *reinterpret_cast<v4i *>(&astage[wid][r][lane * 16]) = ar[r];
        } else {
#pragma unroll
            for (int kb = 0; kb < 16; ++kb) a[kb] = arow ? a[kb] : zero;
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            int8_t *st = stage[wid][g & 1];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int rw = 4 * r + lr;
                *reinterpret_cast<v4i *>(st + rw * 256 + ((lc ^ rw) << 4)) = w[4 * g + r];
            }
            // one wave's LDS operations complete in order: no barrier needed
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const v4i b = *reinterpret_cast<const v4i *>(st + row * 256 + (((4 * kb + q) ^ row) << 4));
                v4i af = a[4 * g + kb];
                if constexpr (SMALLM > 0) {
                    const v4i x =
                        *reinterpret_cast<const v4i *>(&astage[wid][ra][(4 * g + kb) * 64 + q * 16]);
                    af = arow ? x : zero;
                }
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, b, acc, 0, 0, 0);
            }
        }
    }
    part[wid][4 * q + 0][row] = acc.x;
    part[wid][4 * q + 1][row] = acc.y;
    part[wid][4 * q + 2][row] = acc.z;
    part[wid][4 * q + 3][row] = acc.w;
    __syncthreads();
    uint32_t sum = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) sum += (uint32_t)part[w][em][en];
    epi.store_ops(em, n0 + en, (int32_t)sum, eo);
}

// Single-row decode GEMV (M = 1, K % 4096 == 0): one weight row per wave and
// two waves per workgroup, so the grid is N/2 small workgroups that the
// dispatcher deals out to CUs as they free up -- the launch shape of a plain
// streaming read -- instead of 16-row tiles dealt out whole. Per 4 KiB of the
// row a lane loads 4 x 16 bytes (each instruction 1 KiB contiguous over the
// wave, non-temporal) and the same 64 bytes of x (4 KiB shared by every wave,
// L1/L2 hits), forms the int8 dot products with v_dot4_i32_i8 (no clamp),
// and the wave's 64 partial sums are added by lane exchanges; lane 0 runs the
// epilogue. K <= 65536 bounds every partial and total sum by 2^30, so no
// int32 sum can wrap. Measured by graph replay against the per-tile and
// balanced-row kernels, weights rotated past the MALL: N = 11008 8.47 vs
// 9.18 us (same-bytes read floor 8.03), N = 4096 4.59 vs 4.77 (4.13),
// K = 8192, N = 4096 6.90 vs 7.80 (6.42); at M = 2 (x loaded per wave
// twice) 9.62 vs 9.21, so only M = 1 takes it.
constexpr int kRowWaves = 2;
constexpr int64_t kRowMaxK = 65536;
__global__ __launch_bounds__(kRowWaves * 64) void gemv_row_kernel(
    const int8_t *__restrict__ A, const int8_t *__restrict__ W, int64_t N, int64_t K,
    Epilogue epi) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int64_t n = (int64_t)blockIdx.x * kRowWaves + wid;
    // a row past N (the last workgroup of an odd N) re-reads row N-1 and
    // stores nothing
    const int8_t *wr = W + std::min<int64_t>(n, N - 1) * K + lane * 16;
    const int8_t *xr = A + lane * 16;
    // the epilogue operands first: loaded after the sum they would add a
    // dependent round trip to every wave's tail
    const EpiOps eo = epi.load_ops(0, n);
    int32_t acc = 0;
    for (int64_t kc = 0; kc < K; kc += 4096) {
        v4i x[4], w[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = *reinterpret_cast<const v4i *>(xr + kc + u * 1024);
#pragma unroll
        for (int u = 0; u < 4; ++u)
            w[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(wr + kc + u * 1024));
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            acc = __builtin_amdgcn_sdot4(w[u].x, x[u].x, acc, false);
            acc = __builtin_amdgcn_sdot4(w[u].y, x[u].y, acc, false);
            acc = __builtin_amdgcn_sdot4(w[u].z, x[u].z, acc, false);
            acc = __builtin_amdgcn_sdot4(w[u].w, x[u].w, acc, false);
        }
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) acc += __shfl_xor(acc, s, 64);
    if (lane == 0) epi.store_ops(0, n, acc, eo);
}

// Decode GEMV over balanced row ranges: workgroup b of G (8 waves, at most
// one per CU) owns weight rows [b*N/G, (b+1)*N/G), processed as up to TPW
// 16-row tiles. First the activations of each wave's K range (K/8 bytes of
// each row < M, in whole cache lines; loaded once for all tiles, where the
// per-tile kernels below load them once per tile, as many bytes as the
// weights at M = 16) and the epilogue operands; then the weights as a stream
// of 1 KiB load units (4 rows x 256 bytes of the wave's K range, tile by
// tile), with P units in flight per wave: a unit is issued as the one P
// earlier has been written to LDS. Weights and activations are read through
// buffer descriptors that end at the range's last row and at row M - 1: the
// rows that pad a tile to 16 read zeros and fetch nothing. Balanced ranges
// keep every CU's byte count within one row of the others (16-row tiles dealt
// out whole leave up to 12% of the CUs' time idle, e.g. 688 tiles over 256
// CUs). Each wave takes K/8 of a tile: the units (non-temporal) are regrouped
// into MFMA fragments through the wave's LDS slice, 256 bytes of each row at
// a time (16-byte chunk c of row r at c ^ r), 16x16x64 MFMAs against the
// activation fragments (regrouped once through the same slice and held in
// registers for all tiles), then the 8 partial tiles are summed through LDS
// (exact: wrapping int32) and the epilogue runs once per output. K = 2048 * H
// bytes (H = 1, 2).
//
// The window: plain reads of the same bytes in this launch shape (one
// workgroup per CU streaming its contiguous share; librnn_probe.so's range
// read) are fastest with 8 waves and 4 to 8 loads of 1 KiB in flight per
// wave: 45 MB in 8.38 us at 32 KiB per CU, 8.58 at 192 KiB; 16.8 MB in 4.21
// and 7.56 us (small streaming workgroups: 7.90 and 4.19). Measured against
// the previous kernel, which issued every weight load up front (192 KiB per
// CU at M = 16, N = 11008) with a barrier between tiles' loads, K = 4096
// (us, graph replay, weights rotated past the MALL): N = 11008 M = 16
// 10.54 -> 9.32 (P = 8; 9.55 at P = 4), M = 8 10.17 -> 9.07 (the per-tile
// kernel before), M = 4 9.51 -> 8.98; N = 4096 M = 16 5.16 -> 5.05 (P = 4),
// M = 8 4.87 -> 4.70; N = 16383 M = 16 14.12 -> 12.28; K = 2048, N = 11008
// M = 16 6.04 -> 5.73 (P = 4; 6.47 at P = 8), M = 8 7.98 -> 5.63.
constexpr int kGlWaves = 8;

__device__ __forceinline__ void lds_only_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int TPW, int H, int P>
__global__ __launch_bounds__(kGlWaves * 64) void gemv_rows_kernel(
    const int8_t *__restrict__ A, const int8_t *__restrict__ W, int64_t M, int64_t N,
    Epilogue epi) {
    constexpr int KW = 256 * H;        // K bytes per wave and tile
    constexpr int K = kGlWaves * KW;   // 2048 or 4096
    constexpr int KB = KW / 64;        // MFMA k-steps per wave and tile
    constexpr int LPR = KW / 16;       // lanes per activation row in a whole-line load
    constexpr int RPI = 64 / LPR;      // activation rows per load instruction
    constexpr int UPT = 4 * H;         // weight load units per wave and tile
    constexpr int U = TPW * UPT;
    static_assert(RPI * KB == 16, "KB whole-line loads cover the 16 activation rows");
    // per wave: the 16 activation rows of its K range (regrouped once), then
    // 256 bytes of each of the 16 weight rows at a time
    __shared__ __attribute__((aligned(16))) int8_t stage[kGlWaves][16 * KW];
    __shared__ int32_t part[kGlWaves][16][16];
    const int tid = threadIdx.x, wid = tid / 64, lane = tid % 64;
    const int row = lane & 15, q = lane >> 4;
    // The K slice of wave w. The older wave of each SIMD (waves 0-3) issues
    // first, so its slices should not be one contiguous half of every row:
    // with one workgroup per CU, slices are interleaved (0, 2, 4, 6 for waves
    // 0-3); with several tiles per workgroup, rotated by the workgroup, so
    // that the CUs' concurrent requests spread over the whole rows. (Measured
    // with every load issued up front, K = 4096, M = 16: N = 4096 6.5 us with
    // slices in wave order, 5.7 interleaved; N = 11008 12.5 in wave order,
    // 11.0 rotated.)
    const int k0 = (TPW == 1 ? 2 * (wid & 3) + (wid >> 2) : (wid + blockIdx.x) & 7) * KW;
    // (32-bit: the launch keeps N <= 64 rows per CU)
    const uint32_t r0 = blockIdx.x * (uint32_t)N / gridDim.x;
    const int nrows = (int)((blockIdx.x + 1) * (uint32_t)N / gridDim.x - r0);

    // every weight byte of the row range; offsets past nrows rows read 0
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t *>(W + (int64_t)r0 * K), 0, nrows * K, 0x00020000);
    // the activations, rows < M only: offsets past row M - 1 read 0
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t *>(A), 0, (int)(M * K), 0x00020000);
    // 1. this wave's K range of the activations in whole lines, RPI rows (KW
    //    bytes each) per instruction, regrouped into MFMA fragments through
    //    LDS below while the weights are in flight. Fragment-layout loads (16
    //    rows x 64 bytes per instruction) touch twice the cache lines.
    v4i al[KB];
#pragma unroll
    for (int j = 0; j < KB; ++j)
        al[j] = __builtin_bit_cast(
            v4i, __builtin_amdgcn_raw_buffer_load_b128(
                     ar, (RPI * j + lane / LPR) * K + k0 + 16 * (lane % LPR), 0, 0));
    // 2. epilogue operands of the outputs this thread finishes (one per tile)
    const int em = (tid / 16) & 15, en = tid % 16;
    EpiOps eo[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) eo[i] = epi.load_ops(em, r0 + std::min(16 * i + en, nrows - 1));
    // 3. the first P weight units. Unit u: tile u / UPT, 256-byte half
    //    (u % UPT) / 4 of the wave's K range, rows 4 (u % 4) + q of the tile.
    v4i wv[U];
    auto issue = [&](auto uc) {
        constexpr int u = decltype(uc)::value;
        if constexpr (u < U) {
            constexpr int i = u / UPT, h = (u % UPT) / 4, g = u % 4;
            wv[u] = __builtin_bit_cast(
                v4i, __builtin_amdgcn_raw_buffer_load_b128(
                         wr, (16 * i + 4 * g + q) * K + k0 + 256 * h + 16 * row, 0, 2 /* nt */));
        }
    };
    static_for<P>([&](auto uc) { issue(uc); });
    // (sched_barrier: the compiler would otherwise hoist the later units'
    // loads up here)
    __builtin_amdgcn_sched_barrier(0);

    // the activation fragments (lane (row, q) of step kb: row `row`, bytes
    // 64 kb + 16 q of the K range), through this wave's LDS slice with the
    // 16-byte chunk c of row r at c ^ r; rows past M arrived as zeros
    int8_t *st = stage[wid];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
        const int r = RPI * j + lane / LPR;
        *reinterpret_cast<v4i *>(st + r * KW + 16 * ((lane % LPR) ^ r)) = al[j];
    }
    v4i a[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
        a[kb] = *reinterpret_cast<const v4i *>(st + row * KW + 16 * ((4 * kb + q) ^ row));
    static_for<TPW>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        // (no early exit for a tile past the range: it multiplies zeros and
        // stores nothing)
        v4i acc = {0, 0, 0, 0};
        static_for<H>([&](auto hc) {
            constexpr int h = decltype(hc)::value;
            // regroup: lane (q, row) of unit (i, h, g) holds row 4g + q,
            // chunk 16h + row of this wave's K range; stored at (chunk - 16h)
            // ^ row. One wave's LDS operations complete in order, so no
            // barrier is needed between the writes, the reads and the next
            // half's writes.
            static_for<4>([&](auto gc) {
                constexpr int g = decltype(gc)::value;
                constexpr int u = i * UPT + h * 4 + g;
                const int rw = 4 * g + q;
                *reinterpret_cast<v4i *>(st + rw * 256 + 16 * (row ^ rw)) = wv[u];
                __builtin_amdgcn_sched_barrier(0);
                issue(std::integral_constant<int, u + P>{});  // unit u landed: the next one
                __builtin_amdgcn_sched_barrier(0);
            });
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const int ch = 4 * kb + q;
                const v4i b = *reinterpret_cast<const v4i *>(st + row * 256 + 16 * (ch ^ row));
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[4 * h + kb], b, acc, 0, 0, 0);
            }
        });
        part[wid][4 * q + 0][row] = acc.x;
        part[wid][4 * q + 1][row] = acc.y;
        part[wid][4 * q + 2][row] = acc.z;
        part[wid][4 * q + 3][row] = acc.w;
        lds_only_barrier();
        if (tid < 256 && 16 * i + en < nrows) {
            uint32_t sum = 0;
#pragma unroll
            for (int v = 0; v < kGlWaves; ++v) sum += (uint32_t)part[v][em][en];
            epi.store_ops(em, r0 + 16 * i + en, (int32_t)sum, eo[i]);
        }
        lds_only_barrier();  // part is rewritten by the next tile
    });
}

// the load window: 8 units (8 KiB per wave) for three or more 4096-byte
// tiles, else 4
template <int TPW, int H>
constexpr int kRowsWindow = H == 2 && TPW >= 3 ? 8 : 4;

template <int H>
static bool launch_gemv_rows_h(const int8_t *A, const int8_t *W, int64_t M, int64_t N, int grid,
                               int tpw, const Epilogue &epi, hipStream_t st) {
#define RNN_ROWS(T) \
    gemv_rows_kernel<T, H, kRowsWindow<T, H>><<<grid, kGlWaves * 64, 0, st>>>(A, W, M, N, epi)
    switch (tpw) {
    case 1: RNN_ROWS(1); return true;
    case 2: RNN_ROWS(2); return true;
    case 3: RNN_ROWS(3); return true;
    case 4: RNN_ROWS(4); return true;
    default: return false;
    }
#undef RNN_ROWS
}

// The balanced-row GEMV for M <= 16, K in {2048, 4096} and at most 64 rows
// per CU; false when the shape is outside that.
static bool launch_gemv_rows(const int8_t *A, const int8_t *W, int64_t M, int64_t N, int64_t K,
                             const Epilogue &epi, hipStream_t st) {
    if (M < 1 || M > 16 || (K != 2048 && K != 4096)) return false;
    const int64_t grid = std::min<int64_t>(device_cu_count(), ceil_div(N, 16));
    const int64_t tpw = ceil_div(ceil_div(N, grid), 16);  // tiles of the largest range
    if (tpw > 4 || N * grid >= (int64_t(1) << 32)) return false;
    return K == 4096 ? launch_gemv_rows_h<2>(A, W, M, N, (int)grid, (int)tpw, epi, st)
                     : launch_gemv_rows_h<1>(A, W, M, N, (int)grid, (int)tpw, epi, st);
}

// ------------------------------------------------------------ igemm packing
// B i8 [K,N] -> B^T [N,Kp] through a 64x64 LDS tile (zero pad k >= K).
__global__ __launch_bounds__(256) void transpose_b_kernel(const int8_t *__restrict__ b, int64_t K,
                                                          int64_t N, int64_t Kp,
                                                          int8_t *__restrict__ bt) {
    __shared__ int8_t tile[64][65];
    const int64_t k0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
    const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
    for (int r = ty; r < 64; r += 4) {
        const int64_t k = k0 + r, n = n0 + tx;
        tile[r][tx] = (k < K && n < N) ? b[k * N + n] : (int8_t)0;
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
        const int64_t n = n0 + r, k = k0 + tx;
        if (n < N && k < Kp) bt[n * Kp + k] = tile[tx][r];
    }
}

__global__ void fill_i32_kernel(int32_t *__restrict__ p, int64_t n, int32_t v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// colsum[n] = sum_k b[k,n] (wrapping int32; order-independent), as the row
// sums of the transposed B^T [N, Kp] (zero padded): one wave per row, each
// lane summing 16 contiguous bytes per step, then a wave reduction.
__global__ __launch_bounds__(256) void colsum_rows_kernel(const int8_t *__restrict__ bt, int64_t N,
                                                        int64_t Kp, int32_t *__restrict__ colsum) {
    const int lane = threadIdx.x & 63;
    const int64_t n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    const int8_t *row = bt + n * Kp;
    uint32_t s = 0;
    for (int64_t k = 16 * lane; k < Kp; k += 16 * 64) {
        const v4i v = *reinterpret_cast<const v4i *>(row + k);
        const uint32_t w[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int b = 0; b < 4; ++b) s += (uint32_t)(int32_t)(int8_t)(w[q] >> (8 * b));
    }
    for (int off = 32; off > 0; off >>= 1) s += (uint32_t)__shfl_xor((int)s, off, 64);
    if (lane == 0) colsum[n] = (int32_t)s;
}

// A u8 [M,K] -> s8 [M,Kp] (x ^ 0x80 == x - 128; pad k >= K with 0), 16 output
// bytes per thread (Kp is a multiple of 64).
__global__ void pack_a_u8_v16_kernel(const uint8_t *__restrict__ a, int64_t M, int64_t K,
                                     int64_t Kp, int8_t *__restrict__ out) {
    const int64_t chunks = M * (Kp / 16);
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < chunks;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = i / (Kp / 16), k0 = (i % (Kp / 16)) * 16;
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t v = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int64_t k = k0 + 4 * q + b;
                const uint32_t x = k < K ? (uint32_t)(a[m * K + k] ^ 0x80u) : 0u;
                v |= x << (8 * b);
            }
            w[q] = v;
        }
        *reinterpret_cast<v4i *>(out + m * Kp + k0) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
}

// ------------------------------------------------------------ dispatch
template <int BM, int BN, int WM, int WN, bool TERNARY, bool RAGGED = false, bool PERM = false>
static int launch_tiled(const int8_t *A, const void *B, int64_t M, int64_t N, int64_t K,
                        const Epilogue &epi, hipStream_t st, const char *name) {
    using C = TileGemm<BM, BN, WM, WN, TERNARY>;
    RNN_REQUIRE(ceil_div(M, BM) <= 65535, "%s: M too large", name);
    dim3 grid((unsigned)ceil_div(N, BN), (unsigned)ceil_div(M, BM));
    gemm_tiled_kernel<BM, BN, WM, WN, TERNARY, RAGGED, PERM><<<grid, C::NT, 0, st>>>(A, B, M, N, K,
                                                                                   epi);
    return check_launch(name);
}

template <int BM, int BN, int WGM, int WGN, int STAGES, bool TER = false, int KS = 1>
static int launch_dma(const int8_t *A, const int8_t *B, int64_t M, int64_t N, int64_t K,
                      const Epilogue &epi, hipStream_t st, const char *name) {
    using C = DmaCfg<BM, BN, WGM, WGN, STAGES, TER>;
    const int64_t tm = ceil_div(M, BM), tn = ceil_div(N, BN);
    RNN_REQUIRE(tm * tn <= 0x7fffffffLL, "%s: too many tiles", name);
    RNN_REQUIRE(K % (2 * kDmaBK * KS) == 0, "%s: K must be a multiple of %d here", name,
                2 * kDmaBK * KS);
    const unsigned grid = (unsigned)(tm * tn), nt = KS * C::NT;
    if (epi.y && epi.acc_out)
        gemm_dma_kernel<BM, BN, WGM, WGN, STAGES, true, true, TER, KS><<<grid, nt, 0, st>>>(
            A, B, M, N, K, (int)tm, (int)tn, epi);
    else if (epi.y)
        gemm_dma_kernel<BM, BN, WGM, WGN, STAGES, true, false, TER, KS><<<grid, nt, 0, st>>>(
            A, B, M, N, K, (int)tm, (int)tn, epi);
    else
        gemm_dma_kernel<BM, BN, WGM, WGN, STAGES, false, true, TER, KS><<<grid, nt, 0, st>>>(
            A, B, M, N, K, (int)tm, (int)tn, epi);
    return check_launch(name);
}

// The LDS-DMA kernel's preconditions: K a positive multiple of 128, 16-byte
// aligned operands, N % 4 == 0 and 16-byte aligned epilogue vectors.
static bool dma_ok(const int8_t *A, const int8_t *B, int64_t N, int64_t K, const Epilogue &epi) {
    auto al = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    return K > 0 && K % (2 * kDmaBK) == 0 && N % 4 == 0 && al(A) && al(B) && al(epi.y) &&
           al(epi.acc_out) && al(epi.sw) && al(epi.bias) && al(epi.colsum);
}

// Block-tile choice for the LDS-DMA kernel: for M > 128, 256x224 tiles with
// 8 waves (2 per SIMD, 64x112 int32 accumulators each, so one wave's barrier
// and DMA waits overlap the other's MFMAs; 2048x14336 is 512 tiles = two full
// rounds on 256 CUs, one block per CU for the 128 KiB LDS ring), else 128x128
// tiles with 4 waves of 64x64.
// The 128-byte-row kernels address their DMA sources with 32-bit offsets.
static bool l128_fits(int64_t M, int64_t N, int64_t K, bool ter) {
    const uint64_t lim = 1ull << 32;
    return (uint64_t)M * (uint64_t)K < lim && (uint64_t)N * (uint64_t)(ter ? K / 4 : K) < lim;
}
template <class C>
static int launch_l128(const int8_t *A, const int8_t *B, int64_t M, int64_t N, int64_t K,
                       const Epilogue &epi, hipStream_t st, const char *name) {
    const int64_t tm = ceil_div(M, C::BM), tn = ceil_div(N, C::BN);
    RNN_REQUIRE(tm * tn <= 0x7fffffffLL, "%s: too many tiles", name);
    RNN_REQUIRE(K % (kL * C::KS) == 0, "%s: K must be a multiple of %d here", name, kL * C::KS);
    RNN_REQUIRE(l128_fits(M, N, K, C::TER), "%s: operands of 4 GiB or more", name);
    const unsigned grid = (unsigned)(tm * tn), nt = C::KS * C::NT;
    // write-through output stores while the outputs fit a buffer range (the
    // ternary GEMM at 512 x 4096 x 4096: 11.45 -> 10.75 us, one process)
    const bool wt = (uint64_t)M * (uint64_t)N * 4u < (1ull << 31);
#define RNN_L128(Y, ACC)                                                                          \
    (wt ? gemm_l128_kernel<C, Y, ACC, true><<<grid, nt, 0, st>>>(A, B, M, N, K, (int)tm, (int)tn, epi) \
        : gemm_l128_kernel<C, Y, ACC, false><<<grid, nt, 0, st>>>(A, B, M, N, K, (int)tm, (int)tn, epi))
    if (epi.y && epi.acc_out)
        RNN_L128(true, true);
    else if (epi.y)
        RNN_L128(true, false);
    else
        RNN_L128(false, true);
#undef RNN_L128
    return check_launch(name);
}
template <class C>
static int launch_pp(const int8_t *A, const int8_t *B, int64_t M, int64_t N, int64_t K,
                     const Epilogue &epi, hipStream_t st, const char *name) {
    const int64_t tm = ceil_div(M, C::BM), tn = ceil_div(N, C::BN);
    RNN_REQUIRE(tm * tn <= 0x7fffffffLL, "%s: too many tiles", name);
    RNN_REQUIRE(K % kL == 0, "%s: K must be a multiple of %d here", name, kL);
    RNN_REQUIRE(l128_fits(M, N, K, false), "%s: operands of 4 GiB or more", name);
    const unsigned grid = (unsigned)(tm * tn);
    // write-through output stores while the outputs fit a buffer range
    const bool wt = (uint64_t)M * (uint64_t)N * 4u < (1ull << 31);
#define RNN_PP(Y, ACC)                                                                          \
    (wt ? gemm_pp_kernel<C, Y, ACC, true><<<grid, C::NT, 0, st>>>(A, B, M, N, K, (int)tm, (int)tn, epi) \
        : gemm_pp_kernel<C, Y, ACC, false><<<grid, C::NT, 0, st>>>(A, B, M, N, K, (int)tm, (int)tn, epi))
    if (epi.y && epi.acc_out)
        RNN_PP(true, true);
    else if (epi.y)
        RNN_PP(true, false);
    else
        RNN_PP(false, true);
#undef RNN_PP
    return check_launch(name);
}
static int launch_dma_auto(const int8_t *A, const int8_t *B, int64_t M, int64_t N, int64_t K,
                           const Epilogue &epi, hipStream_t st, const char *name) {
    if (M <= 128) return launch_dma<128, 128, 2, 2, 4>(A, B, M, N, K, epi, st, name);
    if (l128_fits(M, N, K, false)) {
        return launch_pp<PrefillCfg>(A, B, M, N, K, epi, st, name);
    }
    return launch_dma<256, 224, 4, 2, 4>(A, B, M, N, K, epi, st, name);
}

// Decode GEMV dispatch: one-shot workgroups of 4 waves per 16 weight rows,
// each wave keeping 16 16-byte loads in flight per lane (the whole 4096-wide
// row block of 64 KiB is requested at once). A persistent variant that walks
// row blocks with one block of prefetch measured slower (per-item memory
// latency exposed, uneven rounds), so the hardware dispatcher does the
// balancing.
static int launch_gemv(const int8_t *A, const int8_t *W, int64_t M, int64_t N, int64_t K,
                       const Epilogue &epi, hipStream_t st, const char *name) {
    // Whole-line weight loads when K % 4096 == 0. Activation rows are staged
    // in LDS (one contiguous 1 KiB load per row and wave) for M <= 8, and for
    // M <= 16 while the grid takes at most one workgroup per CU: at 16 rows
    // the 96 KiB of LDS per workgroup would otherwise cap residency. Measured
    // against fragment-layout activation loads, K = 4096: M = 8 5.19 vs
    // 6.04 us (N 4096), 10.17 vs 11.31 (N 11008); M = 16 6.21 vs 6.75
    // (N 4096), 14.96 vs 13.57 (N 11008, 688 workgroups: not taken).
    //
    // M = 1 over at least 512 rows: the single-row kernel above. The
    // balanced-row kernel (activations loaded once per workgroup, a bounded
    // load window) takes M >= 2, and M = 1 while the rows fit one tile per
    // CU; the per-tile kernels below take what it does not (K other than
    // 2048 and 4096, more than 64 rows per CU). With every weight load issued
    // up front it lost to the per-tile kernels at N = 11008, M <= 8.
    if (M == 1 && K % 4096 == 0 && K <= kRowMaxK && N >= 512 && ceil_div(N, kRowWaves) <= 0x7fffffff) {
        gemv_row_kernel<<<(unsigned)ceil_div(N, kRowWaves), kRowWaves * 64, 0, st>>>(A, W, N, K, epi);
        return check_launch(name);
    }
    const unsigned wgs = (unsigned)ceil_div(N, 16);
    if ((M > 1 || (int64_t)wgs <= device_cu_count()) && launch_gemv_rows(A, W, M, N, K, epi, st))
        return check_launch(name);
    if (K % 4096 == 0 && M <= 4)
        gemv_wl_kernel<4, 4><<<wgs, 256, 0, st>>>(A, W, M, N, K, epi);
    else if (K % 4096 == 0 && M <= 8)
        gemv_wl_kernel<4, 8><<<wgs, 256, 0, st>>>(A, W, M, N, K, epi);
    else if (K % 4096 == 0 && M <= 16 && (int64_t)wgs <= device_cu_count())
        gemv_wl_kernel<4, 16><<<wgs, 256, 0, st>>>(A, W, M, N, K, epi);
    else if (K % 4096 == 0)
        gemv_wl_kernel<4, 0><<<wgs, 256, 0, st>>>(A, W, M, N, K, epi);
    else
        gemv_kernel<4, 16><<<(unsigned)ceil_div(N, 16), 256, 0, st>>>(A, W, M, N, K, epi);
    return check_launch(name);
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace rnn

using namespace rnn;

extern "C" int rnn_w8a8_linear(const int8_t *aq, const float *sa, const int8_t *wq,
                               const float *sw, const float *bias, int64_t m, int64_t k,
                               int64_t n, unsigned flags, float *y, int32_t *acc_out,
                               void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_w8a8_linear";
    RNN_REQUIRE(m >= 0 && k >= 0 && n >= 0, "%s: negative size", name);
    RNN_REQUIRE((flags & ~(RNN_FLAG_RELU | RNN_ALGO_MASK)) == 0, "%s: unknown flags 0x%x", name, flags);
    if (m == 0 || n == 0) return RNN_OK;
    RNN_REQUIRE(y || acc_out, "%s: y and acc_out both null", name);
    RNN_REQUIRE(!y || (sa && sw), "%s: y requires sa and sw", name);
    RNN_REQUIRE(k == 0 || (aq && wq), "%s: null operand", name);
    Epilogue epi{sa, sw, bias, y, acc_out, nullptr, m, n, (flags & RNN_FLAG_RELU) ? 1 : 0};
    const unsigned algo = flags & RNN_ALGO_MASK;
    RNN_REQUIRE(algo == RNN_ALGO_AUTO || algo == RNN_ALGO_TILED || algo == RNN_ALGO_GEMV ||
                    algo == RNN_ALGO_TILED_DMA,
                "%s: unknown algo 0x%x", name, algo);
    if (algo == RNN_ALGO_GEMV)
        RNN_REQUIRE(m <= 16, "%s: RNN_ALGO_GEMV needs m <= 16", name);
    if (k % 16 != 0 || !aligned16(aq) || !aligned16(wq)) {
        // any k and alignment: the byte-assembling tiled kernel (AUTO / TILED)
        if (algo == RNN_ALGO_GEMV || algo == RNN_ALGO_TILED_DMA)
            return set_error(RNN_ERR_UNSUPPORTED,
                             "%s: the forced GEMV / LDS-DMA kernels need k %% 16 == 0 and 16-byte "
                             "aligned operands (k=%lld)",
                             name, (long long)k);
        return launch_tiled<128, 128, 64, 64, false, true>(aq, wq, m, n, k, epi, as_stream(stream),
                                                           name);
    }
    const bool dma = dma_ok(aq, wq, n, k, epi);
    if (algo == RNN_ALGO_TILED_DMA && !dma)
        return set_error(RNN_ERR_UNSUPPORTED,
                         "%s: RNN_ALGO_TILED_DMA needs k %% 128 == 0, n %% 4 == 0 and 16-byte "
                         "aligned buffers (k=%lld, n=%lld)",
                         name, (long long)k, (long long)n);
    hipStream_t st = as_stream(stream);
    if (algo == RNN_ALGO_GEMV || (algo == RNN_ALGO_AUTO && m <= 16))
        return launch_gemv(aq, wq, m, n, k, epi, st, name);
    if (algo == RNN_ALGO_TILED_DMA || (algo == RNN_ALGO_AUTO && dma))
        return launch_dma_auto(aq, wq, m, n, k, epi, st, name);
    return launch_tiled<128, 128, 64, 64, false>(aq, wq, m, n, k, epi, st, name);
}

extern "C" int rnn_ternary_gemm(const int8_t *aq, const float *sa, const uint32_t *packed,
                                const float *sw, const float *bias, int64_t m, int64_t k,
                                int64_t n, unsigned flags, float *y, int32_t *acc_out,
                                void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_ternary_gemm";
    RNN_REQUIRE(m >= 0 && k >= 0 && n >= 0, "%s: negative size", name);
    RNN_REQUIRE((flags & ~(RNN_FLAG_RELU | RNN_FLAG_TERNARY_MFMA_LAYOUT | RNN_ALGO_MASK)) == 0,
                "%s: unknown flags 0x%x", name, flags);
    const unsigned algo = flags & RNN_ALGO_MASK;
    const bool mfma_layout = (flags & RNN_FLAG_TERNARY_MFMA_LAYOUT) != 0;
    RNN_REQUIRE(algo == RNN_ALGO_AUTO || algo == RNN_ALGO_TILED || algo == RNN_ALGO_TILED_DMA,
                "%s: algo 0x%x not available for the ternary GEMM", name, algo);
    if (m == 0 || n == 0) return RNN_OK;
    RNN_REQUIRE(y || acc_out, "%s: y and acc_out both null", name);
    RNN_REQUIRE(!y || (sa && sw), "%s: y requires sa and sw", name);
    RNN_REQUIRE(k == 0 || (aq && packed), "%s: null operand", name);
    RNN_REQUIRE(((uintptr_t)packed & 3) == 0, "%s: packed must be 4-byte aligned (u32 words)",
                name);
    RNN_REQUIRE(!mfma_layout || k % 16 == 0,
                "%s: the MFMA code layout needs k %% 16 == 0 (k=%lld)", name, (long long)k);
    Epilogue epi{sa, sw, bias, y, acc_out, nullptr, m, n, (flags & RNN_FLAG_RELU) ? 1 : 0};
    hipStream_t st = as_stream(stream);
    if (k % 16 != 0 || !aligned16(aq)) {
        // rows not word aligned, or unaligned activations: the tiled kernel that
        // gathers codes from arbitrary bit offsets (AUTO / TILED)
        if (algo == RNN_ALGO_TILED_DMA)
            return set_error(RNN_ERR_UNSUPPORTED,
                             "%s: RNN_ALGO_TILED_DMA needs k %% 128 == 0 and 16-byte aligned "
                             "buffers (k=%lld)",
                             name, (long long)k);
        if (mfma_layout)  // k % 16 == 0 here: only the activations are unaligned
            return launch_tiled<128, 128, 64, 64, true, true, true>(aq, packed, m, n, k, epi, st,
                                                                    name);
        return launch_tiled<128, 128, 64, 64, true, true>(aq, packed, m, n, k, epi, st, name);
    }
    const int8_t *pb = reinterpret_cast<const int8_t *>(packed);
    // LDS-DMA path: packed rows are K/4 bytes, 16-byte aligned when k % 64 == 0
    const bool dma = dma_ok(aq, pb, n, k, epi);
    if (algo == RNN_ALGO_TILED_DMA && !dma)
        return set_error(RNN_ERR_UNSUPPORTED,
                         "%s: RNN_ALGO_TILED_DMA needs k %% 128 == 0, n %% 4 == 0 and 16-byte "
                         "aligned buffers (k=%lld, n=%lld)",
                         name, (long long)k, (long long)n);
    // 64x128 tiles of two K groups of 4 waves (64x32 each): a 512x4096 output
    // is 256 tiles, one per CU, and each weight code word is decoded once per
    // CU. Codes in the reference layout decode through the replicated LDS
    // table; codes in the MFMA layout through byte permutes.
    const bool l128 = k % (kL * L128Ter::KS) == 0 && l128_fits(m, n, k, true);
    if (algo == RNN_ALGO_TILED_DMA || (algo == RNN_ALGO_AUTO && dma)) {
        if (l128 && mfma_layout) return launch_l128<L128TerPerm>(aq, pb, m, n, k, epi, st, name);
        if (l128) return launch_l128<L128Ter>(aq, pb, m, n, k, epi, st, name);
        if (!mfma_layout) return launch_dma<128, 64, 2, 2, 4, true>(aq, pb, m, n, k, epi, st, name);
        if (algo == RNN_ALGO_TILED_DMA)
            return set_error(RNN_ERR_UNSUPPORTED,
                             "%s: RNN_ALGO_TILED_DMA on the MFMA code layout needs k %% 256 == 0 "
                             "(k=%lld)",
                             name, (long long)k);
    }
    if (mfma_layout)
        return launch_tiled<128, 128, 64, 64, true, false, true>(aq, packed, m, n, k, epi, st, name);
    return launch_tiled<128, 128, 64, 64, true>(aq, packed, m, n, k, epi, st, name);
}

// ------------------------------------------------------- ternary MFMA layout
// One thread per 32-bit word: the 16 two-bit codes are moved to the MFMA
// layout (ternary_word_to_mfma_layout). Rows stay word-aligned (K % 16 == 0),
// so the words keep their positions and a row is still K/16 words.
__global__ void ternary_prepack_kernel(const uint32_t *__restrict__ in, int64_t words,
                                       uint32_t *__restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < words;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = ternary_word_to_mfma_layout(in[i]);
}

extern "C" int rnn_ternary_prepack(const uint32_t *packed, int64_t rows, int64_t cols,
                                   uint32_t *out, void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_ternary_prepack";
    RNN_REQUIRE(rows >= 0 && cols >= 0, "%s: negative size", name);
    RNN_REQUIRE(cols % 16 == 0, "%s: cols must be a multiple of 16 (row-aligned words), got %lld",
                name, (long long)cols);
    const int64_t words = rows * cols / 16;
    if (words == 0) return RNN_OK;
    RNN_REQUIRE(packed && out, "%s: null pointer", name);
    const unsigned g = (unsigned)std::min<int64_t>(ceil_div(words, 256), 8 * device_cu_count());
    ternary_prepack_kernel<<<g, 256, 0, as_stream(stream)>>>(packed, words, out);
    return check_launch(name);
}

// ------------------------------------------------ igemm, small problems
// igemm in one launch for problems whose pack / transpose / column-sum / GEMM
// sequence would spend most of its time in its four launches (512^3: 16.9
// us, 3.3 of them in the GEMM's MFMAs and loads). A workgroup of 4 waves
// owns a 32 x 32 tile of c, a wave a 16 x 16 quarter. Per K chunk of 256 it
// stages the tile's rows of a as signed bytes (x ^ 0x80, i.e. a - 128) and
// the chunk's rows of b written transposed ([n][k]) in LDS, zero past M, N
// and K, so that both operands' fragments are 16 consecutive k per lane
// (one 16-byte LDS read). The column sums of b come from a second MFMA per
// step whose A operand is all ones; the store adds 128 x that sum (the
// identity sum (a_s8 + 128) b = sum a_s8 b + 128 colsum(b), wrapping int32).
constexpr int kIgBM = 32, kIgBN = 32, kIgKC = 256, kIgPad = 16;
constexpr double kIgSmallOps = 268435456.0;  // m n k at or below: one launch

template <bool VEC>
__global__ __launch_bounds__(256) void igemm_small_kernel(const uint8_t *__restrict__ a,
                                                          const int8_t *__restrict__ b,
                                                          int32_t *__restrict__ c, int64_t M,
                                                          int64_t K, int64_t N, int tiles_n) {
    __shared__ __attribute__((aligned(16))) int8_t as[kIgBM][kIgKC + kIgPad];
    __shared__ __attribute__((aligned(16))) int8_t bs[kIgBN][kIgKC + kIgPad];  // b transposed
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid & 1, wn = wid >> 1, fi = lane & 15, fq = lane >> 4;
    const int64_t m0 = (int64_t)(blockIdx.x / tiles_n) * kIgBM;
    const int64_t n0 = (int64_t)(blockIdx.x % tiles_n) * kIgBN;
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    v4i acc = {0, 0, 0, 0}, accs = {0, 0, 0, 0};  // a_s8 . b and the column sums of b
    for (int64_t k0 = 0; k0 < K; k0 += kIgKC) {
        {  // a: row tid / 8 of the tile, 32 bytes at (tid % 8) * 32 of the chunk
            const int r = tid >> 3, c0 = (tid & 7) * 32;
            const int64_t row = m0 + r;
            uint32_t w[8];
            if constexpr (VEC) {  // (K % 16 == 0: a 16-byte piece is wholly inside or past K)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int64_t kk = k0 + c0 + 16 * h;
                    uint4 v = {0u, 0u, 0u, 0u};
                    if (row < M && kk < K) {
                        v = *reinterpret_cast<const uint4 *>(a + row * K + kk);
                        v.x ^= 0x80808080u, v.y ^= 0x80808080u, v.z ^= 0x80808080u, v.w ^= 0x80808080u;
                    }
                    w[4 * h] = v.x, w[4 * h + 1] = v.y, w[4 * h + 2] = v.z, w[4 * h + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    uint32_t x = 0u;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int64_t kk = k0 + c0 + 4 * d + e;
                        if (row < M && kk < K) x |= (uint32_t)(a[row * K + kk] ^ 0x80u) << (8 * e);
                    }
                    w[d] = x;
                }
            }
            uint4 *dst = reinterpret_cast<uint4 *>(&as[r][c0]);
            dst[0] = uint4{w[0], w[1], w[2], w[3]};
            dst[1] = uint4{w[4], w[5], w[6], w[7]};
        }
        {  // b: k row tid of the chunk, columns n0 .. n0+31, written transposed
            const int64_t kk = k0 + tid;
            int8_t v[kIgBN];
            if constexpr (VEC) {  // (N % 16 == 0: a 16-byte half is wholly inside or past N)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    uint4 u = {0u, 0u, 0u, 0u};
                    if (kk < K && n0 + 16 * h < N)
                        u = *reinterpret_cast<const uint4 *>(b + kk * N + n0 + 16 * h);
                    const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int j = 0; j < 16; ++j) v[16 * h + j] = (int8_t)(uw[j / 4] >> (8 * (j % 4)));
                }
            } else {
#pragma unroll
                for (int j = 0; j < kIgBN; ++j)
                    v[j] = kk < K && n0 + j < N ? b[kk * N + n0 + j] : (int8_t)0;
            }
#pragma unroll
            for (int j = 0; j < kIgBN; ++j) bs[j][tid] = v[j];
        }
        __syncthreads();
#pragma unroll
        for (int kb = 0; kb < kIgKC / 64; ++kb) {
            const v4i af = *reinterpret_cast<const v4i *>(&as[16 * wm + fi][64 * kb + 16 * fq]);
            const v4i bf = *reinterpret_cast<const v4i *>(&bs[16 * wn + fi][64 * kb + 16 * fq]);
            // D[m][n]: A = rows of a, B = columns of b
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf, acc, 0, 0, 0);
            accs = __builtin_amdgcn_mfma_i32_16x16x64_i8(ones, bf, accs, 0, 0, 0);
        }
        __syncthreads();
    }
    // lane: column n0 + 16 wn + fi, rows m0 + 16 wm + 4 fq .. + 3
    const int64_t col = n0 + 16 * wn + fi;
    if (col >= N) return;
    const int32_t av[4] = {acc.x, acc.y, acc.z, acc.w}, sv[4] = {accs.x, accs.y, accs.z, accs.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + 16 * wm + 4 * fq + r;
        if (row < M) c[row * N + col] = (int32_t)((uint32_t)av[r] + 128u * (uint32_t)sv[r]);
    }
}

static bool igemm_small(int64_t m, int64_t k, int64_t n) {
    return (double)m * (double)n * (double)k <= kIgSmallOps;
}

static int launch_igemm_small(const uint8_t *a, const int8_t *b, int32_t *c, int64_t m, int64_t k,
                              int64_t n, hipStream_t st, const char *name) {
    const int64_t tm = ceil_div(m, kIgBM), tn = ceil_div(n, kIgBN);
    RNN_REQUIRE(tm * tn <= 0x7fffffffLL, "%s: too many tiles", name);
    const bool vec = k % 16 == 0 && n % 16 == 0 && aligned16(a) && aligned16(b);
    if (vec)
        igemm_small_kernel<true><<<(unsigned)(tm * tn), 256, 0, st>>>(a, b, c, m, k, n, (int)tn);
    else
        igemm_small_kernel<false><<<(unsigned)(tm * tn), 256, 0, st>>>(a, b, c, m, k, n, (int)tn);
    return check_launch(name);
}

static int64_t igemm_kp(int64_t k) { return (k + 63) / 64 * 64; }

extern "C" size_t rnn_igemm_workspace_size(int64_t m, int64_t k, int64_t n) {
    if (m <= 0 || n <= 0 || k <= 0) return 0;
    const int64_t kp = igemm_kp(k);
    auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    return (size_t)(up(m * kp) + up(n * kp) + up(4 * n));
}

// The pack / transpose / colsum / GEMM sequence of igemm on a workspace of
// rnn_igemm_workspace_size(m, k, n) bytes (16-byte aligned). Every workspace
// byte the GEMM reads is written by this call first (the packs write their
// zero padding too), so the workspace needs no clearing.
static int igemm_on_workspace(const uint8_t *a, const int8_t *b, int32_t *c, int64_t m, int64_t k,
                              int64_t n, void *workspace, hipStream_t st, const char *name) {
    const int64_t kp = igemm_kp(k);
    auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
    int8_t *ap = static_cast<int8_t *>(workspace);
    int8_t *bt = ap + up(m * kp);
    int32_t *cs = reinterpret_cast<int32_t *>(bt + up(n * kp));
    const int cus = device_cu_count();
    RNN_REQUIRE(ceil_div(kp, 64) <= 65535, "%s: k too large", name);
    pack_a_u8_v16_kernel<<<(unsigned)std::min<int64_t>(ceil_div(m * kp / 16, 256), 8 * cus), 256, 0,
                           st>>>(a, m, k, kp, ap);
    RNN_TRY(check_launch(name));
    dim3 g((unsigned)ceil_div(n, 64), (unsigned)ceil_div(kp, 64));
    transpose_b_kernel<<<g, 256, 0, st>>>(b, k, n, kp, bt);
    RNN_TRY(check_launch(name));
    colsum_rows_kernel<<<(unsigned)ceil_div(n, 4), 256, 0, st>>>(bt, n, kp, cs);
    RNN_TRY(check_launch(name));
    Epilogue epi{nullptr, nullptr, nullptr, nullptr, c, cs, m, n, 0};
    if (m <= 16) return launch_gemv(ap, bt, m, n, kp, epi, st, name);
    // 64x64 tiles while 128x128 tiles would leave most CUs idle
    if (ceil_div(m, 128) * ceil_div(n, 128) < cus)
        return launch_tiled<64, 64, 32, 32, false>(ap, bt, m, n, kp, epi, st, name);
    return launch_tiled<128, 128, 64, 64, false>(ap, bt, m, n, kp, epi, st, name);
}

// C = 0 for an empty reduction (a fill kernel, safe under graph capture).
static int igemm_empty(int32_t *c, int64_t m, int64_t n, hipStream_t st, const char *name) {
    fill_i32_kernel<<<(unsigned)std::min<int64_t>(ceil_div(m * n, 256), 8 * device_cu_count()), 256,
                      0, st>>>(c, m * n, 0);
    return check_launch(name);
}

extern "C" int rnn_igemm(const uint8_t *a, const int8_t *b, int32_t *c, int64_t m, int64_t k,
                         int64_t n, void *workspace, size_t workspace_bytes, void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_igemm";
    RNN_REQUIRE(m >= 0 && k >= 0 && n >= 0, "%s: negative size", name);
    if (m == 0 || n == 0) return RNN_OK;
    RNN_REQUIRE(c != nullptr, "%s: null c", name);
    hipStream_t st = as_stream(stream);
    if (k == 0) return igemm_empty(c, m, n, st, name);
    RNN_REQUIRE(a && b, "%s: null operand", name);
    const size_t need = rnn_igemm_workspace_size(m, k, n);
    RNN_REQUIRE(!workspace || workspace_bytes >= need, "%s: workspace %zu < %zu bytes", name,
                workspace_bytes, need);
    if (igemm_small(m, k, n)) return launch_igemm_small(a, b, c, m, k, n, st, name);
    if (workspace != nullptr) {
        RNN_REQUIRE(workspace_bytes >= need, "%s: workspace %zu < %zu bytes", name,
                    workspace_bytes, need);
        RNN_REQUIRE(aligned16(workspace), "%s: workspace must be 16-byte aligned", name);
        return igemm_on_workspace(a, b, c, m, k, n, workspace, st, name);
    }
    RNN_TRY(check_hip(hipMallocAsync(&workspace, need, st), name));
    int rc = igemm_on_workspace(a, b, c, m, k, n, workspace, st, name);
    int rf = check_hip(hipFreeAsync(workspace, st), name);
    return rc != RNN_OK ? rc : rf;
}

// ------------------------------------------------------ igemm, no allocation
// The workspace of rnn_igemm_noalloc: a file-scope device array, one copy per
// GPU, held until the process ends. Host code never uses its name as an
// address (on the host it is only a stand-in for the symbol): the device
// address comes from hipGetSymbolAddress, once per device, with that device
// current, and is kept in g_scratch_dev.
static __device__ __align__(256) int8_t scratch[RNN_IGEMM_NOALLOC_MAX_BYTES];

static std::mutex g_scratch_mu;
static void *g_scratch_dev[64];

static int scratch_address(void **out, const char *name) {
    int dev = -1;
    RNN_TRY(check_hip(hipGetDevice(&dev), name));
    RNN_REQUIRE(dev >= 0 && dev < 64, "%s: device ordinal %d out of range", name, dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_dev[dev] == nullptr) {
        void *p = nullptr;
        RNN_TRY(check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), name));
        RNN_REQUIRE(p != nullptr && aligned16(p), "%s: scratch symbol has no device address", name);
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return RNN_OK;
}

extern "C" int rnn_igemm_noalloc(const uint8_t *a, const int8_t *b, int32_t *c, int64_t m,
                                 int64_t k, int64_t n, void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_igemm_noalloc";
    RNN_REQUIRE(m >= 0 && k >= 0 && n >= 0, "%s: negative size", name);
    if (m == 0 || n == 0) return RNN_OK;
    RNN_REQUIRE(c != nullptr, "%s: null c", name);
    hipStream_t st = as_stream(stream);
    if (k == 0) return igemm_empty(c, m, n, st, name);
    RNN_REQUIRE(a && b, "%s: null operand", name);
    // one-launch problems use no workspace, so the array's size does not limit them
    if (igemm_small(m, k, n)) return launch_igemm_small(a, b, c, m, k, n, st, name);
    const size_t need = rnn_igemm_workspace_size(m, k, n);
    if (need > (size_t)RNN_IGEMM_NOALLOC_MAX_BYTES)
        return set_error(RNN_ERR_UNSUPPORTED,
                         "%s: m=%lld k=%lld n=%lld needs %zu bytes of workspace, more than the "
                         "%zu-byte device array (use rnn_igemm)",
                         name, (long long)m, (long long)k, (long long)n, need,
                         (size_t)RNN_IGEMM_NOALLOC_MAX_BYTES);
    void *ws = nullptr;
    RNN_TRY(scratch_address(&ws, name));
    return igemm_on_workspace(a, b, c, m, k, n, ws, st, name);
}
