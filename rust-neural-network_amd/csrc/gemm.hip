// gemm.hip -- int8 GEMM/GEMV on gfx950 MFMA (v_mfma_i32_16x16x64_i8).
//
//   acc[m,n] = sum_k A[m,k] * B[n,k]     A [M,K] int8, B [N,K] int8 (both
//                                        K-contiguous: the Int8Weights layout)
// Entry points: rnn_w8a8_linear (W8A8 with fused dequant epilogue), rnn_igemm
// (the reference's u8 x i8 [K,N] contract via a pack step + zero-point
// correction) and rnn_ternary_gemm (B = 2-bit codes decoded in the tile loader).
#include <algorithm>

#include "common.hpp"
#include "numerics.hpp"

namespace rnn {

// ------------------------------------------------------------------ epilogue
// Applied per output element. Float path (y != null):
//   v = ((float)acc * sa[m]) * sw[n]; v = v + bias[n]; v = max(v, 0)
// (the order of src/int8.rs:159-162 and src/tensor.rs:2025-2032).
// Raw path (acc_out != null): acc_out = acc (+ 128*colsum[n] for igemm).
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

// ------------------------------------------------------------ tiled GEMM
// Block tile BM x BN, K step 64 (one MFMA K), (BM/WM) x (BN/WN) waves, each
// wave a WM x WN tile of 16x16 MFMA blocks. Operand tiles live in LDS as
// [rows][64 bytes] with the 16-byte chunk index XOR-swizzled by
// ((r>>1) ^ (r>>3)) & 3, which keeps the ds_read_b128 fragment loads (16 rows
// x one chunk per quarter-wave) and the row-contiguous tile stores free of
// bank conflicts. Global tiles are prefetched into registers one K step
// ahead (double-buffered LDS).
constexpr int kBK = 64;

__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

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

template <int BM, int BN, int WM, int WN, bool TERNARY>
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
            ra[i] = gk < K ? *reinterpret_cast<const v4i *>(A + gm * K + gk) : v4i{0, 0, 0, 0};
        }
        if constexpr (!TERNARY) {
#pragma unroll
            for (int i = 0; i < C::B_CHUNKS; ++i) {
                const int c = tid + i * C::NT;
                const int r = c / 4, ch = c % 4;
                const int64_t gn = std::min<int64_t>(bn0 + r, N - 1);
                const int64_t gk = k0 + ch * 16;
                rb[i] = gk < K ? *reinterpret_cast<const v4i *>(B8 + gn * K + gk) : v4i{0, 0, 0, 0};
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
                            ternary_word_to_i8x16(w[ch]);
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

// ------------------------------------------------------------ igemm packing
// A u8 [M,K] -> s8 [M,Kp] (x ^ 0x80 == x - 128; pad k >= K with 0).
__global__ void pack_a_u8_kernel(const uint8_t *__restrict__ a, int64_t M, int64_t K, int64_t Kp,
                                 int8_t *__restrict__ out) {
    const int64_t total = M * Kp;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = i / Kp, k = i % Kp;
        out[i] = k < K ? (int8_t)(a[m * K + k] ^ 0x80u) : (int8_t)0;
    }
}

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

// colsum[n] = sum_k b[k,n] (wrapping int32; order-independent).
__global__ void colsum_kernel(const int8_t *__restrict__ b, int64_t K, int64_t N,
                              int32_t *__restrict__ colsum) {
    const int64_t n = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (n >= N) return;
    uint32_t s = 0;
    for (int64_t k = 0; k < K; ++k) s += (uint32_t)(int32_t)b[k * N + n];
    colsum[n] = (int32_t)s;
}

// ------------------------------------------------------------ dispatch
template <int BM, int BN, int WM, int WN, bool TERNARY>
static int launch_tiled(const int8_t *A, const void *B, int64_t M, int64_t N, int64_t K,
                        const Epilogue &epi, hipStream_t st, const char *name) {
    using C = TileGemm<BM, BN, WM, WN, TERNARY>;
    RNN_REQUIRE(ceil_div(M, BM) <= 65535, "%s: M too large", name);
    dim3 grid((unsigned)ceil_div(N, BN), (unsigned)ceil_div(M, BM));
    gemm_tiled_kernel<BM, BN, WM, WN, TERNARY><<<grid, C::NT, 0, st>>>(A, B, M, N, K, epi);
    return check_launch(name);
}

static int launch_gemv(const int8_t *A, const int8_t *W, int64_t M, int64_t N, int64_t K,
                       const Epilogue &epi, hipStream_t st, const char *name) {
    gemv_kernel<4, 4><<<(unsigned)ceil_div(N, 16), 256, 0, st>>>(A, W, M, N, K, epi);
    return check_launch(name);
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace rnn

using namespace rnn;

extern "C" int rnn_w8a8_linear(const int8_t *aq, const float *sa, const int8_t *wq,
                               const float *sw, const float *bias, int64_t m, int64_t k,
                               int64_t n, unsigned flags, float *y, int32_t *acc_out,
                               void *stream) {
    const char *name = "rnn_w8a8_linear";
    RNN_REQUIRE(m >= 0 && k >= 0 && n >= 0, "%s: negative size", name);
    RNN_REQUIRE((flags & ~(RNN_FLAG_RELU | RNN_ALGO_MASK)) == 0, "%s: unknown flags 0x%x", name, flags);
    if (m == 0 || n == 0) return RNN_OK;
    RNN_REQUIRE(y || acc_out, "%s: y and acc_out both null", name);
    RNN_REQUIRE(!y || (sa && sw), "%s: y requires sa and sw", name);
    RNN_REQUIRE(k == 0 || (aq && wq), "%s: null operand", name);
    if (k % 16 != 0 || !aligned16(aq) || !aligned16(wq))
        return set_error(RNN_ERR_UNSUPPORTED,
                         "%s: k must be a multiple of 16 and operands 16-byte aligned (k=%lld)",
                         name, (long long)k);
    Epilogue epi{sa, sw, bias, y, acc_out, nullptr, m, n, (flags & RNN_FLAG_RELU) ? 1 : 0};
    const unsigned algo = flags & RNN_ALGO_MASK;
    const bool gemv = algo == RNN_ALGO_GEMV || (algo == RNN_ALGO_AUTO && m <= 16);
    if (algo == RNN_ALGO_GEMV)
        RNN_REQUIRE(m <= 16, "%s: RNN_ALGO_GEMV needs m <= 16", name);
    hipStream_t st = as_stream(stream);
    if (gemv) return launch_gemv(aq, wq, m, n, k, epi, st, name);
    return launch_tiled<128, 128, 64, 64, false>(aq, wq, m, n, k, epi, st, name);
}

extern "C" int rnn_ternary_gemm(const int8_t *aq, const float *sa, const uint32_t *packed,
                                const float *sw, const float *bias, int64_t m, int64_t k,
                                int64_t n, unsigned flags, float *y, int32_t *acc_out,
                                void *stream) {
    const char *name = "rnn_ternary_gemm";
    RNN_REQUIRE(m >= 0 && k >= 0 && n >= 0, "%s: negative size", name);
    RNN_REQUIRE((flags & ~RNN_FLAG_RELU) == 0, "%s: unknown flags 0x%x", name, flags);
    if (m == 0 || n == 0) return RNN_OK;
    RNN_REQUIRE(y || acc_out, "%s: y and acc_out both null", name);
    RNN_REQUIRE(!y || (sa && sw), "%s: y requires sa and sw", name);
    RNN_REQUIRE(k == 0 || (aq && packed), "%s: null operand", name);
    if (k % 16 != 0 || !aligned16(aq) || ((uintptr_t)packed & 3) != 0)
        return set_error(RNN_ERR_UNSUPPORTED,
                         "%s: k must be a multiple of 16 and aq 16-byte aligned (k=%lld)", name,
                         (long long)k);
    Epilogue epi{sa, sw, bias, y, acc_out, nullptr, m, n, (flags & RNN_FLAG_RELU) ? 1 : 0};
    return launch_tiled<128, 128, 64, 64, true>(aq, packed, m, n, k, epi, as_stream(stream), name);
}

static int64_t igemm_kp(int64_t k) { return (k + 63) / 64 * 64; }

extern "C" size_t rnn_igemm_workspace_size(int64_t m, int64_t k, int64_t n) {
    if (m <= 0 || n <= 0 || k <= 0) return 0;
    const int64_t kp = igemm_kp(k);
    auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    return (size_t)(up(m * kp) + up(n * kp) + up(4 * n));
}

extern "C" int rnn_igemm(const uint8_t *a, const int8_t *b, int32_t *c, int64_t m, int64_t k,
                         int64_t n, void *workspace, size_t workspace_bytes, void *stream) {
    const char *name = "rnn_igemm";
    RNN_REQUIRE(m >= 0 && k >= 0 && n >= 0, "%s: negative size", name);
    if (m == 0 || n == 0) return RNN_OK;
    RNN_REQUIRE(c != nullptr, "%s: null c", name);
    hipStream_t st = as_stream(stream);
    if (k == 0) {  // empty reduction: C = 0 (a fill kernel, safe under graph capture)
        fill_i32_kernel<<<(unsigned)std::min<int64_t>(ceil_div(m * n, 256), 8 * device_cu_count()),
                          256, 0, st>>>(c, m * n, 0);
        return check_launch(name);
    }
    RNN_REQUIRE(a && b, "%s: null operand", name);
    const size_t need = rnn_igemm_workspace_size(m, k, n);
    bool owned = false;
    if (workspace == nullptr) {
        RNN_TRY(check_hip(hipMallocAsync(&workspace, need, st), name));
        owned = true;
    } else {
        RNN_REQUIRE(workspace_bytes >= need, "%s: workspace %zu < %zu bytes", name,
                    workspace_bytes, need);
        RNN_REQUIRE(aligned16(workspace), "%s: workspace must be 16-byte aligned", name);
    }
    const int64_t kp = igemm_kp(k);
    auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
    int8_t *ap = static_cast<int8_t *>(workspace);
    int8_t *bt = ap + up(m * kp);
    int32_t *cs = reinterpret_cast<int32_t *>(bt + up(n * kp));
    const int cus = device_cu_count();
    int rc = RNN_OK;
    pack_a_u8_kernel<<<(unsigned)std::min<int64_t>(ceil_div(m * kp, 256), 8 * cus), 256, 0, st>>>(
        a, m, k, kp, ap);
    rc = check_launch(name);
    if (rc == RNN_OK && ceil_div(kp, 64) > 65535)
        rc = set_error(RNN_ERR_UNSUPPORTED, "%s: k too large", name);
    if (rc == RNN_OK) {
        dim3 g((unsigned)ceil_div(n, 64), (unsigned)ceil_div(kp, 64));
        transpose_b_kernel<<<g, 256, 0, st>>>(b, k, n, kp, bt);
        rc = check_launch(name);
    }
    if (rc == RNN_OK) {
        colsum_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(b, k, n, cs);
        rc = check_launch(name);
    }
    if (rc == RNN_OK) {
        Epilogue epi{nullptr, nullptr, nullptr, nullptr, c, cs, m, n, 0};
        if (m <= 16)
            rc = launch_gemv(ap, bt, m, n, kp, epi, st, name);
        else
            rc = launch_tiled<128, 128, 64, 64, false>(ap, bt, m, n, kp, epi, st, name);
    }
    if (owned) {
        int rf = check_hip(hipFreeAsync(workspace, st), name);
        if (rc == RNN_OK) rc = rf;
    }
    return rc;
}
