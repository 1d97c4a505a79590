// sgemm.hip -- f32 GEMM for the BlasBackend plugin point of rust-nn
// (src/blas.rs:712-734, contract at :89-190): C = alpha*op(A)*op(B) + beta*C,
// row-major storage with leading dimensions, op = identity or transpose.
//
// Fast path (K % 32 == 0): sgemm_mfma2_kernel, below. Otherwise
// sgemm_mfma_kernel: v_mfma_f32_16x16x4f32 on 128x128 block tiles of 4 waves
// (64x64 each), K staged 32 floats at a time through double-buffered LDS:
//  * K-contiguous operands (A as stored, B transposed) are kept as 128-byte
//    LDS rows (32 floats) whose 16-byte chunks are XOR-swizzled by
//    (row >> 1) & 7. A lane reads one 16-byte chunk = 4 consecutive k and
//    feeds them to 4 successive MFMAs: MFMA s of a 16-k super-step uses, in
//    lane group q = lane/16, the k index 16*ss + 4*q + s. Both operands use the
//    same k mapping, so the sum is the same as in k order up to rounding.
//  * K-major operands (A transposed, B as stored) are kept as [k][row] tiles
//    with a 132-float row pitch (the four lane groups' rows 4 apart land 16
//    banks apart) and read 4 bytes per lane per MFMA.
// The MFMA's A operand is the op(B) fragment (16 columns n), its B operand
// the op(A) fragment (16 rows m), so a lane ends up with 4 consecutive n of
// one m and writes them as one float4.
// Other strides / alignments take a one-thread-per-output kernel.
#include "common.hpp"

namespace rnn {

namespace {

constexpr int kSgBM = 128, kSgBN = 128, kSgBK = 32;
constexpr int kSgPitch = 132;                            // K-major tile row pitch (floats)
constexpr int kSgRowTile = kSgBM * kSgBK;                 // 4096 floats (16 KiB)
constexpr int kSgKTile = kSgBK * kSgPitch;                // 4224 floats (16.5 KiB)

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int sg_swz(int r) { return (r >> 1) & 7; }

// One operand's tile of a stage: ROWS x 32 k (K-contiguous storage, KMAJ =
// false) or 32 k x ROWS (K-major storage, KMAJ = true). Each of the 256
// threads moves 4 float4 per stage.
template <bool KMAJ>
struct SgOperand {
    static constexpr int TILE = KMAJ ? kSgKTile : kSgRowTile;
    const float *p;
    int64_t ld, rows, K;  // rows: M for A, N for B
    int64_t r0;           // first row (m or n) of this block
    f4 reg[4];

    __device__ __forceinline__ void load(int64_t k0, int tid) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = tid + 256 * i;
            int64_t r, k;
            if (KMAJ) {          // k row f/32, 4 rows starting at 4*(f%32)
                k = k0 + (f >> 5);
                r = r0 + 4 * (f & 31);
            } else {             // row f/8, k chunk f%8
                r = r0 + (f >> 3);
                k = k0 + 4 * (f & 7);
            }
            // the host guarantees that the contiguous dimension is a multiple
            // of 4, so a float4 is either wholly inside or wholly outside
            const bool ok = r < rows && k < K;
            const float *src = KMAJ ? p + k * ld + r : p + r * ld + k;
            reg[i] = ok ? *reinterpret_cast<const f4 *>(src) : f4{0.f, 0.f, 0.f, 0.f};
        }
    }
    __device__ __forceinline__ void store(float *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = tid + 256 * i;
            float *dst;
            if (KMAJ)
                dst = lds + (f >> 5) * kSgPitch + 4 * (f & 31);
            else {
                const int r = f >> 3;
                dst = lds + r * kSgBK + 4 * ((f & 7) ^ sg_swz(r));
            }
            *reinterpret_cast<f4 *>(dst) = reg[i];
        }
    }
    // the 4 k values of super-step ss for fragment row `row` (tile-relative)
    // in lane group q: k = 16*ss + 4*q + s, s = 0..3
    __device__ __forceinline__ static f4 frag(const float *lds, int row, int q, int ss) {
        if (KMAJ) {
            const float *b = lds + (16 * ss + 4 * q) * kSgPitch + row;
            return f4{b[0], b[kSgPitch], b[2 * kSgPitch], b[3 * kSgPitch]};
        } else {
            return *reinterpret_cast<const f4 *>(lds + row * kSgBK + 4 * ((4 * ss + q) ^ sg_swz(row)));
        }
    }
};

template <bool TA, bool TB>
__global__ __launch_bounds__(256) void sgemm_mfma_kernel(const float *__restrict__ A, int64_t lda,
                                                         const float *__restrict__ B, int64_t ldb,
                                                         float *__restrict__ C, int64_t ldc,
                                                         int64_t M, int64_t N, int64_t Kall,
                                                         float alpha, float beta, int tiles_m,
                                                         int tiles_mn, int64_t kc, int64_t cstride) {
    using OA = SgOperand<TA>;    // op(A) rows m: K-major when A is transposed
    using OB = SgOperand<!TB>;   // op(B) rows n: K-major when B is as stored ([k][n])
    __shared__ __attribute__((aligned(16))) float smem[2 * (OA::TILE + OB::TILE)];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid & 1, wn = wid >> 1;
    const int fr = lane & 15, q = lane >> 4;
    // the K range and partial output of a split K, as in sgemm_mfma2_kernel
    const int tile = (int)(blockIdx.x % (unsigned)tiles_mn), split = (int)(blockIdx.x / (unsigned)tiles_mn);
    const int tm = tile % tiles_m, tn = tile / tiles_m;
    const int64_t m0 = (int64_t)tm * kSgBM, n0 = (int64_t)tn * kSgBN;
    const int64_t kb = (int64_t)split * kc;
    const int64_t K = std::min<int64_t>(kc, Kall - kb);
    A += TA ? kb * lda : kb;
    B += TB ? kb : kb * ldb;
    C += split * cstride;

    OA a{A, lda, M, K, m0, {}};
    OB b{B, ldb, N, K, n0, {}};
    f4 acc[4][4];  // [n tile][m tile]
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    const int nst = (int)((K + kSgBK - 1) / kSgBK);
    a.load(0, tid);
    b.load(0, tid);
    a.store(smem, tid);
    b.store(smem + OA::TILE, tid);
    __syncthreads();
    for (int s = 0; s < nst; ++s) {
        float *cur = smem + (s & 1) * (OA::TILE + OB::TILE);
        float *nxt = smem + ((s + 1) & 1) * (OA::TILE + OB::TILE);
        if (s + 1 < nst) {  // next stage's loads in flight during this stage's MFMAs
            a.load((int64_t)(s + 1) * kSgBK, tid);
            b.load((int64_t)(s + 1) * kSgBK, tid);
        }
#pragma unroll
        for (int ss = 0; ss < kSgBK / 16; ++ss) {
            f4 fa[4], fb[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) fa[j] = OA::frag(cur, wm * 64 + 16 * j + fr, q, ss);
#pragma unroll
            for (int i = 0; i < 4; ++i) fb[i] = OB::frag(cur + OA::TILE, wn * 64 + 16 * i + fr, q, ss);
#pragma unroll
            for (int k4 = 0; k4 < 4; ++k4)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fb[i][k4], fa[j][k4], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < nst) {
            a.store(nxt, tid);
            b.store(nxt + OA::TILE, tid);
        }
        __syncthreads();
    }

    // lane: m = tile row + fr, n = tile column + 4*q + e (e = 0..3)
    const bool vec_c = (ldc & 3) == 0 && (((uintptr_t)C) & 15) == 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t m = m0 + wm * 64 + 16 * j + fr;
            const int64_t n = n0 + wn * 64 + 16 * i + 4 * q;
            if (m >= M || n >= N) continue;
            float *cp = C + m * ldc + n;
            f4 v = acc[i][j];
            if (vec_c && n + 3 < N) {
                f4 o = {alpha * v.x, alpha * v.y, alpha * v.z, alpha * v.w};
                if (beta != 0.0f) {
                    const f4 c = *reinterpret_cast<const f4 *>(cp);
                    o = f4{o.x + beta * c.x, o.y + beta * c.y, o.z + beta * c.z, o.w + beta * c.w};
                }
                *reinterpret_cast<f4 *>(cp) = o;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (n + e >= N) break;
                    const float o = alpha * v[e];
                    cp[e] = beta != 0.0f ? o + beta * cp[e] : o;
                }
            }
        }
}

// K % 32 == 0: the same tiles and MFMAs with both operands in one LDS layout,
// [kq][row][4] (kq = the 4-k quad within the 32-k stage), every fragment one
// ds_read_b128. Physical row = row ^ kq ^ ((row >> 4) & 3): 16 lanes reading
// a fragment (one kq, rows base..base+15), or storing a transposed K-major
// quad (one kq, rows 4t + j for 16 consecutive t), touch 16 different 16-byte
// bank groups.
// K-contiguous operands are loaded a row's 128 bytes per 8 lanes and written
// as they come; K-major ones are loaded 512 bytes of a k-row per 32 lanes,
// 4 k-rows per thread, and transposed in registers (4 quads of one row).
// Loads go through buffer descriptors whose range ends at the operand's last
// element, so no branch guards them: rows past M or N read other rows' data
// or zeros, and only reach outputs that are not stored. Each super-step's
// fragments are read while the previous super-step's MFMAs run.
__device__ __forceinline__ int sg2_row(int row, int kq) { return row ^ kq ^ ((row >> 4) & 3); }

template <bool KMAJ>
struct SgOp2 {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t off[4];  // per-thread byte offsets within the stage (from the stage base)
    f4 reg[4];
    // row-major loads (K-contiguous): f = tid + 256 i -> row f / 8, kq f % 8;
    // K-major: kq = tid / 32, row quad tid % 32, k row 4 kq + i
    __device__ __forceinline__ void init(int64_t ld, int tid) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (KMAJ) {
                off[i] = (uint32_t)(((4 * (tid >> 5) + i) * ld + 4 * (tid & 31)) * 4);
            } else {
                const int f = tid + 256 * i;
                off[i] = (uint32_t)(((f >> 3) * ld + 4 * (f & 7)) * 4);
            }
        }
    }
    // the stage's buffer: K-contiguous from the block's first row (the k0
    // advance is the scalar offset), K-major from k row k0
    __device__ __forceinline__ void load(uint32_t soff) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            reg[i] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off[i], soff, 0));
    }
    __device__ __forceinline__ void store(float *lds, int tid) const {
        if (KMAJ) {
            const int kq = tid >> 5, r = 4 * (tid & 31);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f4 v = {reg[0][j], reg[1][j], reg[2][j], reg[3][j]};
                *reinterpret_cast<f4 *>(lds + (kq * kSgBM + sg2_row(r + j, kq)) * 4) = v;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int f = tid + 256 * i, row = f >> 3, kq = f & 7;
                *reinterpret_cast<f4 *>(lds + (kq * kSgBM + sg2_row(row, kq)) * 4) = reg[i];
            }
        }
    }
    __device__ __forceinline__ static f4 frag(const float *lds, int row, int q, int ss) {
        const int kq = 4 * ss + q;
        return *reinterpret_cast<const f4 *>(lds + (kq * kSgBM + sg2_row(row, kq)) * 4);
    }
};

constexpr int kSg2Tile = kSgBM * kSgBK;  // 4096 floats per operand and stage

// Split K (tiles_mn tiles of C, each with gridDim.x / tiles_mn workgroups):
// workgroup blockIdx.x takes tile blockIdx.x % tiles_mn over the K range
// [s kc, min((s + 1) kc, K)) with s = blockIdx.x / tiles_mn, and writes its
// tile to C + s cstride. One range (kc = K, cstride = 0) is the plain GEMM.
template <bool TA, bool TB>
__global__ __launch_bounds__(256) void sgemm_mfma2_kernel(const float *__restrict__ A, int64_t lda,
                                                          const float *__restrict__ B, int64_t ldb,
                                                          float *__restrict__ C, int64_t ldc,
                                                          int64_t M, int64_t N, int64_t Kall,
                                                          float alpha, float beta, int tiles_m,
                                                          int tiles_mn, int64_t kc, int64_t cstride) {
    constexpr bool AK = TA, BK = !TB;  // K-major storage of op(A) / op(B)
    __shared__ __attribute__((aligned(16))) float smem[2 * 2 * kSg2Tile];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid & 1, wn = wid >> 1;
    const int fr = lane & 15, q = lane >> 4;
    const int tile = (int)(blockIdx.x % (unsigned)tiles_mn), split = (int)(blockIdx.x / (unsigned)tiles_mn);
    const int tm = tile % tiles_m, tn = tile / tiles_m;
    const int64_t m0 = (int64_t)tm * kSgBM, n0 = (int64_t)tn * kSgBN;
    const int64_t kb = (int64_t)split * kc;
    const int64_t K = std::min<int64_t>(kc, Kall - kb);
    A += AK ? kb * lda : kb;
    B += BK ? kb * ldb : kb;
    C += split * cstride;

    SgOp2<AK> a;
    SgOp2<BK> b;
    a.init(lda, tid);
    b.init(ldb, tid);
    // K-contiguous: base = row r0, range to the operand's last element (at
    // most 128 rows); K-major: base = (k0, r0) per stage, range to the last
    // element, at most the stage's 32 k rows
    auto rsrc_rows = [&](const float *p, int64_t ld, int64_t rows, int64_t r0) {
        const int64_t last = std::min<int64_t>(rows - 1 - r0, kSgBM - 1) * ld + K;
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p + r0 * ld), 0, (int)(last * 4),
                                                 0x00020000);
    };
    auto rsrc_kmaj = [&](const float *p, int64_t ld, int64_t rows, int64_t r0, int64_t k0) {
        const int64_t last = std::min<int64_t>((K - 1 - k0) * ld + rows - r0, (int64_t)kSgBK * ld);
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p + k0 * ld + r0), 0,
                                                 (int)(last * 4), 0x00020000);
    };
    auto load_stage = [&](int64_t k0) {
        if (AK) {
            a.rsrc = rsrc_kmaj(A, lda, M, m0, k0);
            a.load(0);
        } else {
            a.load((uint32_t)(k0 * 4));
        }
        if (BK) {
            b.rsrc = rsrc_kmaj(B, ldb, N, n0, k0);
            b.load(0);
        } else {
            b.load((uint32_t)(k0 * 4));
        }
    };
    if (!AK) a.rsrc = rsrc_rows(A, lda, M, m0);
    if (!BK) b.rsrc = rsrc_rows(B, ldb, N, n0);

    f4 acc[4][4];  // [n tile][m tile]
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    const int nst = (int)(K / kSgBK);
    load_stage(0);
    a.store(smem, tid);
    b.store(smem + kSg2Tile, tid);
    __syncthreads();
    f4 fa[2][4], fb[2][4];
    auto read_frags = [&](const float *buf, int ss, f4 (&xa)[4], f4 (&xb)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) xa[j] = SgOp2<AK>::frag(buf, wm * 64 + 16 * j + fr, q, ss);
#pragma unroll
        for (int i = 0; i < 4; ++i) xb[i] = SgOp2<BK>::frag(buf + kSg2Tile, wn * 64 + 16 * i + fr, q, ss);
    };
    auto mfmas = [&](const f4 (&xa)[4], const f4 (&xb)[4]) {
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xb[i][k4], xa[j][k4], acc[i][j], 0, 0, 0);
    };
    read_frags(smem, 0, fa[0], fb[0]);
    for (int s = 0; s < nst; ++s) {
        const float *cur = smem + (s & 1) * 2 * kSg2Tile;
        float *nxt = smem + ((s + 1) & 1) * 2 * kSg2Tile;
        if (s + 1 < nst) load_stage((int64_t)(s + 1) * kSgBK);  // in flight during the MFMAs
        read_frags(cur, 1, fa[1], fb[1]);                          // super-step 1's fragments
        __builtin_amdgcn_sched_barrier(0);
        mfmas(fa[0], fb[0]);
        __builtin_amdgcn_sched_barrier(0);
        // the next stage into the other buffer (last read before the previous
        // barrier); after this barrier its first super-step's fragments are
        // read while this stage's second super-step runs
        if (s + 1 < nst) {
            a.store(nxt, tid);
            b.store(nxt + kSg2Tile, tid);
        }
        __syncthreads();
        if (s + 1 < nst) read_frags(nxt, 0, fa[0], fb[0]);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(fa[1], fb[1]);
        __builtin_amdgcn_sched_barrier(0);
    }

    // lane: m = tile row + fr, n = tile column + 4*q + e (e = 0..3)
    const bool vec_c = (ldc & 3) == 0 && (((uintptr_t)C) & 15) == 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t m = m0 + wm * 64 + 16 * j + fr;
            const int64_t n = n0 + wn * 64 + 16 * i + 4 * q;
            if (m >= M || n >= N) continue;
            float *cp = C + m * ldc + n;
            f4 v = acc[i][j];
            if (vec_c && n + 3 < N) {
                f4 o = {alpha * v.x, alpha * v.y, alpha * v.z, alpha * v.w};
                if (beta != 0.0f) {
                    const f4 c = *reinterpret_cast<const f4 *>(cp);
                    o = f4{o.x + beta * c.x, o.y + beta * c.y, o.z + beta * c.z, o.w + beta * c.w};
                }
                *reinterpret_cast<f4 *>(cp) = o;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (n + e >= N) break;
                    const float o = alpha * v[e];
                    cp[e] = beta != 0.0f ? o + beta * cp[e] : o;
                }
            }
        }
}

// Decode shapes of Linear::forward (C = alpha A B^T + beta C, B stored
// [n, k], m <= 16): bound by reading B once. A workgroup owns TPW 16-row
// tiles of B (n); its NW waves split K in steps of KS (4 KS bytes of a row),
// D steps in flight per wave. A step's B bytes arrive in whole-line loads
// (lane l: row l / (KS/4) + (64/(KS/4)) i, 16 bytes at 16 (l % (KS/4));
// non-temporal) and are regrouped through the wave's LDS slice so that lane
// (r = lane % 16, q = lane / 16) holds the 16-byte pieces at k + 16h + 4q of
// row n0 + r; the same pieces of A row r come straight from memory. Each
// piece feeds 4 v_mfma_f32_16x16x4f32: lane group q supplies k + 16h + 4q + s
// to MFMA s for both operands, so D[m][n] sums every k once. D rows past M
// (A rows clamped to M - 1) and columns past N (B rows clamped to N - 1) are
// not stored. The last step of a K that is not a multiple of KS zeroes the
// 16-byte pieces past K in both operands. The NW waves' partial tiles are
// added in wave order through LDS. (Measured, 16 x 11008 x 4096, B rotated
// past the MALL: 4 waves, KS = 64, D = 2, one tile per workgroup 38.1 us;
// two tiles 39.8; KS = 32 with 4 steps in flight, two tiles 42.3; 8 waves
// 40.4; D = 3 41.1; torch.matmul 36.8. Back-to-back calls on one B: the
// KS = 32 two-tile kernel with B loaded straight in the MFMA layout 62,
// with whole lines 40.7.)
template <int TPW, int KS, int NW>
__global__ __launch_bounds__(64 * NW) void sgemm_skinny_nt_kernel(const float *__restrict__ A, int64_t lda,
                                                              const float *__restrict__ B, int64_t ldb,
                                                              float *__restrict__ C, int64_t ldc,
                                                              int M, int64_t N, int64_t K, float alpha,
                                                              float beta) {
    constexpr int D = 2;          // steps in flight per wave
    constexpr int CH = KS / 4;    // 16-byte chunks of a row per step
    constexpr int RPI = 64 / CH;  // rows per whole-line load
    constexpr int L = 16 / RPI;   // whole-line loads per tile and step
    constexpr int H = KS / 16;    // MFMA-layout 16-byte pieces per lane and step
    __shared__ float part[NW][TPW][16][17];
    __shared__ f4 stage[NW][TPW][16][CH];
    // (wid in a scalar register: the step offsets below are the buffer loads'
    // scalar offsets)
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * 16 * TPW;
    const int64_t nsteps = (K + KS - 1) / KS, full = K / KS;
    const int64_t s0 = nsteps * wid / NW, s1 = nsteps * (wid + 1) / NW;
    const int64_t sf = s1 < full ? s1 : full;  // unguarded steps [s0, sf)
    // B: one buffer descriptor over the tiles' rows (the host keeps the
    // range under 2 GiB), rows past N clamped to N - 1
    const int64_t last_row = std::min<int64_t>(n0 + 16 * TPW, N) - 1;
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(B + n0 * ldb), 0, (int)(((last_row - n0) * ldb + K) * 4), 0x00020000);
    // MFMA layout (the K tail): row r, bytes 16q; whole lines (the steps):
    // row lane / CH + RPI i, bytes 16 (lane % CH), regrouped through LDS
    uint32_t boff[TPW], lineoff[TPW][L];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        boff[t] = (uint32_t)((std::min<int64_t>(n0 + 16 * t + r, last_row) - n0) * ldb * 4 + 16 * q);
#pragma unroll
        for (int i = 0; i < L; ++i)
            lineoff[t][i] = (uint32_t)((std::min<int64_t>(n0 + 16 * t + lane / CH + RPI * i, last_row) - n0) *
                                           ldb * 4 + 16 * (lane % CH));
    }
    const float *ap = A + (int64_t)(r < M ? r : M - 1) * lda + 4 * q;
    // this wave's regroup slice: 16 rows x CH 16-byte chunks per tile, chunk
    // c of row j at c ^ (j % CH)
    f4 (*stg)[16][CH] = stage[wid];

    f4 acc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    f4 xa[D][H], wb[D][TPW][L];
    auto load = [&](int d, int64_t step) {
        const int64_t k = KS * step;
#pragma unroll
        for (int h = 0; h < H; ++h) xa[d][h] = *reinterpret_cast<const f4 *>(ap + k + 16 * h);
#pragma unroll
        for (int i = 0; i < L; ++i)
#pragma unroll
            for (int t = 0; t < TPW; ++t)
                wb[d][t][i] = __builtin_bit_cast(
                    f4, __builtin_amdgcn_raw_buffer_load_b128(br, lineoff[t][i], (uint32_t)(k * 4), 2));
    };
    auto mfmas = [&](const f4 (&x)[H], const f4 (&w)[TPW][H]) {
#pragma unroll
        for (int h = 0; h < H; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int t = 0; t < TPW; ++t)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[h][e], w[t][h][e], acc[t], 0, 0, 0);
    };
    // a step's whole-line loads into the MFMA layout: lane (r, q) takes
    // chunks q and 4 + q of row r. One wave's LDS operations complete in
    // order, so the slice is rewritten by the next step without a barrier.
    auto consume = [&](int d) {
        f4 w[TPW][H];
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
#pragma unroll
            for (int i = 0; i < L; ++i) {
                const int j = lane / CH + RPI * i;
                stg[t][j][(lane % CH) ^ (j % CH)] = wb[d][t][i];
            }
#pragma unroll
            for (int h = 0; h < H; ++h) w[t][h] = stg[t][r][(4 * h + q) ^ (r % CH)];
        }
        mfmas(xa[d], w);
    };
    // D steps in flight: the steady loop refills every buffer unconditionally
    // (so the compiler's wait counts see D - 1 steps of loads still in flight
    // at each use); the first D loads are issued whole, a step past the last
    // one repeated, and the last up to 2D - 1 steps are drained after the loop
    if (sf > s0) {
#pragma unroll
        for (int d = 0; d < D; ++d) load(d, std::min<int64_t>(s0 + d, sf - 1));
        int64_t s = s0;
        for (; s + 2 * D <= sf; s += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                consume(d);
                load(d, s + d + D);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (s + d < sf) consume(d);
            if (s + d + D < sf) load(d, s + d + D);
        }
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (s + D + d < sf) consume(d);
    }
    if (s1 > full && s1 - 1 >= s0) {  // the K tail: 16-byte pieces past K are zero
        const int64_t k = KS * full;
        f4 x[H], w[TPW][H];
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const bool ok = k + 16 * h + 4 * q < K;
            x[h] = ok ? *reinterpret_cast<const f4 *>(ap + k + 16 * h) : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < TPW; ++t)
                w[t][h] = ok ? __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(
                                                          br, boff[t], (uint32_t)((k + 16 * h) * 4), 2))
                             : f4{0.f, 0.f, 0.f, 0.f};
        }
        mfmas(x, w);
    }
    // lane holds D[m = 4q + v][n = r] of each tile
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) part[wid][t][4 * q + v][r] = acc[t][v];
    __syncthreads();
    const int m = tid >> 4, nn = tid & 15;
    if (tid < 256 && m < M) {
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            const int64_t n = n0 + 16 * t + nn;
            if (n < N) {
                float sum = part[0][t][m][nn];
#pragma unroll
                for (int v = 1; v < NW; ++v) sum += part[v][t][m][nn];
                float *cp = C + (int64_t)m * ldc + n;
                const float o = alpha * sum;
                *cp = beta != 0.0f ? o + beta * *cp : o;
            }
        }
    }
}

// Decode shapes of Tensor::matmul (C = alpha A B + beta C with B stored
// [k, n], m <= 16): bound by reading B once. A workgroup owns 32 columns of
// B (two 16-column tiles); its NW waves split K in steps of 16. A step's B
// bytes arrive as whole 128-byte row segments (lane l: k row l / 8 + 8 i,
// columns 4 (l % 8) .. + 3; non-temporal) and are written transposed into
// the wave's LDS slice ([column][k], 20-float pitch), so that lane
// (r = lane % 16, q = lane / 16) reads the 4 k values 4q .. 4q + 3 of column
// r of each tile in one 16-byte read; A row r's same 4 k values come straight
// from memory. MFMA s takes k = 4q + s from both operands, so D[m][n] sums
// every k once. D rows past M (A rows clamped to M - 1) and columns past N
// (zeros from the buffer range) are not stored; the last step of a K that is
// not a multiple of 16 zeroes the k rows past K. The NW waves' partial tiles
// are added in wave order through LDS.
template <int NW>
__global__ __launch_bounds__(64 * NW) void sgemm_skinny_nn_kernel(const float *__restrict__ A, int64_t lda,
                                                                  const float *__restrict__ B, int64_t ldb,
                                                                  float *__restrict__ C, int64_t ldc,
                                                                  int M, int64_t N, int64_t K, float alpha,
                                                                  float beta) {
    constexpr int D = 4;   // steps in flight per wave
    constexpr int KS = 16; // k per step
    constexpr int LP = 20; // LDS floats per column of a step
    __shared__ float part[NW][2][16][17];
    __shared__ __attribute__((aligned(16))) float stage[NW][32 * LP];
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * 32;
    const int64_t nsteps = (K + KS - 1) / KS, full = K / KS;
    const int64_t s0 = nsteps * wid / NW, s1 = nsteps * (wid + 1) / NW;
    const int64_t sf = s1 < full ? s1 : full;
    // B from column n0: the range ends at the last element of B, so columns
    // past N in the last k row read zeros (other rows' columns past N only
    // reach outputs that are not stored); the host keeps the range under 2 GiB
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(B + n0), 0, (int)(((K - 1) * ldb + (N - n0)) * 4), 0x00020000);
    uint32_t boff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) boff[i] = (uint32_t)((((lane >> 3) + 8 * i) * ldb + 4 * (lane & 7)) * 4);
    const float *ap = A + (int64_t)(r < M ? r : M - 1) * lda + 4 * q;
    float *stg = stage[wid];

    f4 acc[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
    f4 xa[D], wb[D][2];
    auto load = [&](int d, int64_t step) {
        const int64_t k = KS * step;
        xa[d] = *reinterpret_cast<const f4 *>(ap + k);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            wb[d][i] = __builtin_bit_cast(
                f4, __builtin_amdgcn_raw_buffer_load_b128(br, boff[i], (uint32_t)(k * ldb * 4), 2));
    };
    // a step's B rows transposed into the slice, then each tile's 4 k values
    // of column r for lane group q; one wave's LDS operations complete in
    // order, so the slice is rewritten by the next step without a barrier
    auto consume = [&](const f4 &x, const f4 (&w)[2]) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int kr = (lane >> 3) + 8 * i, c = 4 * (lane & 7);
#pragma unroll
            for (int e = 0; e < 4; ++e) stg[(c + e) * LP + kr] = w[i][e];
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const f4 b = *reinterpret_cast<const f4 *>(stg + (16 * t + r) * LP + 4 * q);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[e], b[e], acc[t], 0, 0, 0);
        }
    };
    if (sf > s0) {
#pragma unroll
        for (int d = 0; d < D; ++d) load(d, std::min<int64_t>(s0 + d, sf - 1));
        int64_t s = s0;
        for (; s + 2 * D <= sf; s += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                consume(xa[d], wb[d]);
                load(d, s + d + D);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (s + d < sf) consume(xa[d], wb[d]);
            if (s + d + D < sf) load(d, s + d + D);
        }
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (s + D + d < sf) consume(xa[d], wb[d]);
    }
    if (s1 > full && s1 - 1 >= s0) {  // the K tail: k rows past K are zero
        const int64_t k = KS * full;
        const f4 z = {0.f, 0.f, 0.f, 0.f};
        const f4 x = k + 4 * q < K ? *reinterpret_cast<const f4 *>(ap + k) : z;
        f4 w[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            w[i] = k + (lane >> 3) + 8 * i < K
                       ? __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    br, boff[i], (uint32_t)(k * ldb * 4), 2))
                       : z;
        consume(x, w);
    }
    // lane holds D[m = 4q + v][n = r] of each tile
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) part[wid][t][4 * q + v][r] = acc[t][v];
    __syncthreads();
    // thread (t, m, nn) of 2 x 16 x 16 outputs: 4 waves take both tiles in
    // turn, 8 waves one each
    const int m = (tid >> 4) & 15, nn = tid & 15;
    for (int t = tid >> 8; t < 2; t += NW / 4) {
        const int64_t n = n0 + 16 * t + nn;
        if (m < M && n < N) {
            float sum = part[0][t][m][nn];
#pragma unroll
            for (int v = 1; v < NW; ++v) sum += part[v][t][m][nn];
            float *cp = C + (int64_t)m * ldc + n;
            const float o = alpha * sum;
            *cp = beta != 0.0f ? o + beta * *cp : o;
        }
    }
}

// B [K, N] (row stride ldb) -> Bt [N, K] (contiguous), 64 x 64 tiles through
// LDS: thread t loads float4 (k row t / 16 + 16 i, columns 4 (t % 16) ..),
// writes float4 (n row t / 16 + 16 i, k 4 (t % 16) ..). K and N are
// multiples of 4, so a float4 is wholly inside or outside.
__global__ __launch_bounds__(256) void sgemm_transpose_kernel(const float *__restrict__ B, int64_t ldb,
                                                              float *__restrict__ Bt, int64_t K,
                                                              int64_t N, int tiles_n) {
    __shared__ float t[64][65];
    const int tid = threadIdx.x;
    const int64_t n0 = (int64_t)(blockIdx.x % (unsigned)tiles_n) * 64, k0 = (int64_t)(blockIdx.x / (unsigned)tiles_n) * 64;
    const int c = 4 * (tid & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int kr = (tid >> 4) + 16 * i;
        f4 v = {0.f, 0.f, 0.f, 0.f};
        if (k0 + kr < K && n0 + c < N) v = *reinterpret_cast<const f4 *>(B + (k0 + kr) * ldb + n0 + c);
#pragma unroll
        for (int e = 0; e < 4; ++e) t[kr][c + e] = v[e];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int nr = (tid >> 4) + 16 * i;
        if (n0 + nr < N && k0 + c < K) {
            const f4 v = {t[c][nr], t[c + 1][nr], t[c + 2][nr], t[c + 3][nr]};
            *reinterpret_cast<f4 *>(Bt + (n0 + nr) * K + k0 + c) = v;
        }
    }
}

// Split K: C = alpha * (P_0 + P_1 + ... + P_{S-1}) + beta * C, the partial
// products P_s ([M, N], N contiguous, P_s at P + s * pstride) added in order.
constexpr int64_t kSplitMinK = 64;

__global__ __launch_bounds__(256) void sgemm_split_sum_kernel(const float *__restrict__ P, int S,
                                                              int64_t pstride, float *__restrict__ C,
                                                              int64_t ldc, int64_t M, int64_t N,
                                                              float alpha, float beta) {
    for (int64_t m = blockIdx.y; m < M; m += gridDim.y)
        for (int64_t n = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; n < N;
             n += (int64_t)gridDim.x * blockDim.x) {
            const float *p = P + m * N + n;
            float v = p[0];
            for (int s = 1; s < S; ++s) v += p[s * pstride];
            float *cp = C + m * ldc + n;
            const float o = alpha * v;
            *cp = beta != 0.0f ? o + beta * *cp : o;
        }
}

// Any strides: one thread per output, k in order with fused multiply-adds.
__global__ void sgemm_simple_kernel(int transa, int transb, const float *__restrict__ A, int64_t lda,
                                    const float *__restrict__ B, int64_t ldb, float *__restrict__ C,
                                    int64_t ldc, int64_t M, int64_t N, int64_t K, float alpha,
                                    float beta) {
    const int64_t total = M * N;
    for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = idx / N, n = idx % N;
        float s = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            const float av = transa ? A[k * lda + m] : A[m * lda + k];
            const float bv = transb ? B[n * ldb + k] : B[k * ldb + n];
            s = fmaf(av, bv, s);
        }
        float *cp = C + m * ldc + n;
        *cp = beta != 0.0f ? alpha * s + beta * *cp : alpha * s;
    }
}

// C = beta*C (beta == 0: zeros, C is not read), for k == 0 or alpha == 0
// (src/blas.rs:137-141, scale_c :191-207).
__global__ void sgemm_scale_kernel(float *__restrict__ C, int64_t ldc, int64_t M, int64_t N,
                                   float beta) {
    const int64_t total = M * N;
    for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        float *cp = C + (idx / N) * ldc + idx % N;
        *cp = beta == 0.0f ? 0.0f : beta * *cp;
    }
}

bool aligned16f(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

}  // namespace rnn

using namespace rnn;

extern "C" int rnn_sgemm(int transa, int transb, int64_t m, int64_t n, int64_t k, float alpha,
                         const float *a, int64_t lda, const float *b, int64_t ldb, float beta,
                         float *c, int64_t ldc, void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_sgemm";
    RNN_REQUIRE(m >= 0 && n >= 0 && k >= 0, "%s: negative size", name);
    RNN_REQUIRE((transa == 0 || transa == 1) && (transb == 0 || transb == 1),
                "%s: transa/transb must be 0 (as stored) or 1 (transposed)", name);
    if (m == 0 || n == 0) return RNN_OK;
    RNN_REQUIRE(c != nullptr, "%s: null C", name);
    // leading dimensions: the row strides of the stored matrices (src/blas.rs:93-101)
    RNN_REQUIRE(ldc >= n, "%s: ldc (%lld) < n (%lld)", name, (long long)ldc, (long long)n);
    hipStream_t st = as_stream(stream);
    const int cus = device_cu_count();
    if (k == 0 || alpha == 0.0f) {
        const int64_t blocks = std::min<int64_t>(ceil_div(m * n, 256), 8 * cus);
        sgemm_scale_kernel<<<(unsigned)blocks, 256, 0, st>>>(c, ldc, m, n, beta);
        return check_launch(name);
    }
    RNN_REQUIRE(a != nullptr && b != nullptr, "%s: null operand", name);
    RNN_REQUIRE(lda >= (transa ? m : k), "%s: lda (%lld) < %s (%lld)", name, (long long)lda,
                transa ? "m" : "k", (long long)(transa ? m : k));
    RNN_REQUIRE(ldb >= (transb ? k : n), "%s: ldb (%lld) < %s (%lld)", name, (long long)ldb,
                transb ? "k" : "n", (long long)(transb ? k : n));
    // The MFMA path moves float4 along each operand's contiguous dimension.
    const bool fast = (lda & 3) == 0 && (ldb & 3) == 0 && aligned16f(a) && aligned16f(b) &&
                      (transa ? m % 4 == 0 : k % 4 == 0) && (transb ? k % 4 == 0 : n % 4 == 0);
    // m <= 16 with B stored [n, k] and at least 256 rows of B: the skinny
    // kernel, one 16-row tile of B per workgroup, 8 waves while there are
    // fewer than two tiles per CU (else 4); the B range of a workgroup stays
    // under 2 GiB
    // m <= 16 with B as stored ([k, n]) and at least 256 columns: the skinny
    // NN kernel, 32 columns per workgroup over 4 waves (measured, B rotated
    // past the MALL: 16 x 11008 x 4096 52.5 us against 54.0 with 8 waves and
    // 54.2 / 57.6 with 2 / 8 steps in flight; 16 x 4096 x 11008 60.9 against
    // 63.3 with 8 waves); B's whole range stays under 2 GiB
    if (fast && !transa && !transb && m <= 16 && n >= 256 && k >= 16 &&
        ((k - 1) * ldb + n) * 4 < (int64_t(1) << 31) && (16 * ldb) * 4 < (int64_t(1) << 31)) {
        sgemm_skinny_nn_kernel<4><<<(unsigned)ceil_div(n, 32), 256, 0, st>>>(a, lda, b, ldb, c, ldc, (int)m, n, k,
                                                                        alpha, beta);
        return check_launch(name);
    }
    if (fast && !transa && transb && m <= 16 && n >= 256 && k >= 32 &&
        (16 * ldb + k) * 4 < (int64_t(1) << 31)) {
        const int64_t tiles = ceil_div(n, 16);
        if (tiles >= 2 * cus)
            sgemm_skinny_nt_kernel<1, 64, 4><<<(unsigned)tiles, 256, 0, st>>>(a, lda, b, ldb, c, ldc, (int)m, n, k, alpha, beta);
        else
            sgemm_skinny_nt_kernel<1, 64, 8><<<(unsigned)tiles, 512, 0, st>>>(a, lda, b, ldb, c, ldc, (int)m, n, k, alpha, beta);
        return check_launch(name);
    }
    if (!fast) {
        const int64_t blocks = std::min<int64_t>(ceil_div(m * n, 256), 8 * cus);
        sgemm_simple_kernel<<<(unsigned)blocks, 256, 0, st>>>(transa, transb, a, lda, b, ldb, c, ldc,
                                                              m, n, k, alpha, beta);
        return check_launch(name);
    }
    const int64_t tm = ceil_div(m, kSgBM), tn = ceil_div(n, kSgBN);
    RNN_REQUIRE(tm * tn <= 0x7fffffffLL && tm < 0x7fffffffLL, "%s: too many tiles", name);
    const unsigned grid = (unsigned)(tm * tn);
    // C = A B with B as stored and at least 2048 rows of A: B is transposed
    // into stream-ordered scratch and the product runs on the both-K-
    // contiguous kernel (the K-major B tile's loads cost the NN kernel about
    // 7%, the transpose reads and writes K N floats once; measured at 4096^3:
    // 1071 us NN against 993 NT + the transpose)
    if (!transa && !transb && m >= 2048 && grid >= (unsigned)cus && k % kSgBK == 0 &&
        k < (int64_t(1) << 22) && lda < (int64_t(1) << 22) && n * k < (int64_t(1) << 31)) {
        float *bt = nullptr;
        RNN_TRY(check_hip(hipMallocAsync(reinterpret_cast<void **>(&bt), sizeof(float) * n * k, st), name));
        const int64_t ttn = ceil_div(n, 64), ttk = ceil_div(k, 64);
        sgemm_transpose_kernel<<<(unsigned)(ttn * ttk), 256, 0, st>>>(b, ldb, bt, k, n, (int)ttn);
        int rc = check_launch(name);
        if (rc == RNN_OK) {
            sgemm_mfma2_kernel<false, true><<<grid, 256, 0, st>>>(a, lda, bt, k, c, ldc, m, n, k, alpha, beta,
                                                                 (int)tm, (int)grid, k, 0);
            rc = check_launch(name);
        }
        const int rf = check_hip(hipFreeAsync(bt, st), name);
        return rc != RNN_OK ? rc : rf;
    }
    // Fewer tiles than CUs: K is split into S ranges of whole 32-k stages
    // (the last one takes the rest; at least kSplitMinK each, S <= 16), each
    // range's tiles go to stream-ordered scratch, and sgemm_split_sum_kernel
    // adds the S partial tiles in order into C. S minimises the busiest CU's
    // k count, ceil(tiles S / CUs) (kc + 64), plus the partial sums' traffic
    // counted as S m n / 65536 k (measured, 128-row tiles at M = 16 and 256,
    // N = 11008, K = 4096: the times follow that count; the 64 is a workgroup's
    // prologue and epilogue).
    int S = 1;
    int64_t kc = k;
    if (grid < (unsigned)cus && k >= 2 * kSplitMinK) {
        int64_t best = k + 64;
        for (int s = 2; s <= 16 && s * kSplitMinK <= k; ++s) {
            const int64_t kcs = ceil_div(ceil_div(k, s), kSgBK) * kSgBK;
            const int64_t ss = ceil_div(k, kcs);
            const int64_t cost = ceil_div((int64_t)grid * ss, cus) * (kcs + 64) + ss * m * n / 65536;
            if (cost < best) best = cost, S = (int)ss, kc = kcs;
        }
    }
    float *out = c, *ws = nullptr;
    int64_t ldo = ldc;
    float al = alpha, be = beta;
    if (S > 1) {
        RNN_TRY(check_hip(hipMallocAsync(reinterpret_cast<void **>(&ws), sizeof(float) * S * m * n, st), name));
        out = ws, ldo = n, al = 1.0f, be = 0.0f;
    }
    const unsigned g2 = grid * (unsigned)S;
    const int64_t cs = S > 1 ? m * n : 0;
    // K % 32 == 0, and row strides and K below 4M floats (the buffer ranges of
    // a block or a stage stay under 2 GiB): the single-layout kernel; else
    // the guarded one (any K)
#define RNN_SG(KERNEL, TA, TB) \
    KERNEL<TA, TB><<<g2, 256, 0, st>>>(a, lda, b, ldb, out, ldo, m, n, k, al, be, (int)tm, (int)grid, kc, cs)
    if (k % kSgBK == 0 && k < (int64_t(1) << 22) && lda < (int64_t(1) << 22) &&
        ldb < (int64_t(1) << 22)) {
        if (!transa && !transb) RNN_SG(sgemm_mfma2_kernel, false, false);
        else if (!transa && transb) RNN_SG(sgemm_mfma2_kernel, false, true);
        else if (transa && !transb) RNN_SG(sgemm_mfma2_kernel, true, false);
        else RNN_SG(sgemm_mfma2_kernel, true, true);
    } else {
        if (!transa && !transb) RNN_SG(sgemm_mfma_kernel, false, false);
        else if (!transa && transb) RNN_SG(sgemm_mfma_kernel, false, true);
        else if (transa && !transb) RNN_SG(sgemm_mfma_kernel, true, false);
        else RNN_SG(sgemm_mfma_kernel, true, true);
    }
#undef RNN_SG
    if (S == 1) return check_launch(name);
    const int rc = check_launch(name);
    if (rc == RNN_OK) {
        const dim3 sg((unsigned)ceil_div(n, 256), (unsigned)std::min<int64_t>(m, 65535));
        sgemm_split_sum_kernel<<<sg, 256, 0, st>>>(ws, S, m * n, c, ldc, m, n, alpha, beta);
    }
    const int rs = rc == RNN_OK ? check_launch(name) : rc;
    const int rf = check_hip(hipFreeAsync(ws, st), name);
    return rs != RNN_OK ? rs : rf;
}
