// read_floor.hip -- measurement helpers for bench.py, not part of the C ABI of
// include/rnn_hip.h, built into librnn_probe.so: a streaming read of a device
// buffer at the best rate a plain kernel reaches (16-byte non-temporal loads,
// 4 in flight per lane, grid sized to keep every CU busy), so the decode GEMV
// and QuantizedLinear GEMV can be set beside a same-bytes, read-only floor
// timed the same way; the same read with one workgroup per CU at a chosen
// depth of loads in flight; the per-CU rate of L2-resident loads into VGPRs
// and into LDS; and a shader-clock probe.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kBlock = 256;

// Block b reads the PER * 4 KiB slab [b * PER * 4096, (b+1) * PER * 4096): each
// load instruction of the block covers 4 KiB contiguous (16 bytes per lane),
// and a lane issues all PER of its loads before using any, so a block keeps
// PER * 4 KiB in flight -- the access pattern of a one-shot weight stream.
// The XOR of every 16-byte chunk is formed per block; the sink is written only
// when it equals `magic`, which keeps the loads alive without a store per block.
template <int PER>
__global__ __launch_bounds__(kBlock) void read_floor_kernel(const u32x4 *__restrict__ p, int64_t n16,
                                                           uint32_t magic, uint32_t *sink) {
    const int64_t base = (int64_t)blockIdx.x * PER * kBlock + threadIdx.x;
    u32x4 v[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int64_t i = base + u * kBlock;
        v[u] = __builtin_nontemporal_load(p + (i < n16 ? i : n16 - 1));
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < PER; ++u)
        if (base + u * kBlock < n16) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
    __shared__ uint32_t red[kBlock / 64];
    if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t b = 0;
        for (int w = 0; w < kBlock / 64; ++w) b ^= red[w];
        if (b == magic) atomicXor(sink, b);
    }
}

template <int PER>
void launch(const void *p, int64_t n16, uint32_t magic, uint32_t *sink, hipStream_t st) {
    const int64_t g = (n16 + PER * kBlock - 1) / (PER * kBlock);
    read_floor_kernel<PER><<<(unsigned)g, kBlock, 0, st>>>(reinterpret_cast<const u32x4 *>(p), n16,
                                                          magic, sink);
}

}  // namespace

// Reads `bytes` (a multiple of 16, 16-byte aligned) from p with `per_lane`
// (4, 8, 16 or 32) 16-byte loads in flight per lane. Each block XORs its
// chunks; a block whose XOR equals `magic` XORs it into *sink. Returns 0, or 1
// for bad arguments / a failed launch.
extern "C" int rnn_probe_read(const void *p, int64_t bytes, uint32_t magic, uint32_t *sink,
                              int per_lane, void *stream) {
    if (bytes < 0 || bytes % 16 != 0 || ((uintptr_t)p & 15) != 0 || sink == nullptr) return 1;
    if (bytes == 0) return 0;
    const int64_t n16 = bytes / 16;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    switch (per_lane) {
    case 4: launch<4>(p, n16, magic, sink, st); break;
    case 8: launch<8>(p, n16, magic, sink, st); break;
    case 16: launch<16>(p, n16, magic, sink, st); break;
    case 32: launch<32>(p, n16, magic, sink, st); break;
    default: return 1;
    }
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// ---------------------------------------------------------------- range read
// One workgroup of WAVES waves per CU-sized share: workgroup g reads the
// contiguous 1 KiB chunks [g*C/G, (g+1)*C/G) of the buffer (C chunks, G
// workgroups), wave w taking chunks w, w + WAVES, ... of its share, PER loads
// (16 bytes per lane, non-temporal) issued before any is used: each workgroup
// keeps WAVES * PER KiB in flight. The access pattern of a GEMV whose
// workgroups each stream one row range, at a chosen depth of loads in flight.
// Every load stays inside the share (the last loop step re-reads the share's
// first chunk where its own would pass the end, and discards it).
template <int WAVES, int PER>
__global__ __launch_bounds__(WAVES * 64) void range_read_kernel(const u32x4 *__restrict__ p,
                                                                 int64_t nchunks, uint32_t magic,
                                                                 uint32_t *sink) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t g = blockIdx.x, G = gridDim.x;
    const int64_t c0 = nchunks * g / G, c1 = nchunks * (g + 1) / G;
    uint32_t acc = 0;
    for (int64_t j0 = 0; c0 + w + (int64_t)WAVES * j0 < c1; j0 += PER) {
        u32x4 v[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int64_t c = c0 + w + (int64_t)WAVES * (j0 + u);
            v[u] = __builtin_nontemporal_load(p + (c < c1 ? c : c0) * 64 + lane);
        }
#pragma unroll
        for (int u = 0; u < PER; ++u)
            if (c0 + w + (int64_t)WAVES * (j0 + u) < c1) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
    if (lane == 0 && acc == magic) atomicXor(sink, acc);
}

// Reads `bytes` (a multiple of 1024, 16-byte aligned, at least `groups` KiB)
// from p with `groups` workgroups of `waves` (4 or 8) waves, each keeping
// `per_lane` (2, 4, 8 or 24) loads per lane in flight. Returns 0, or 1 for bad
// arguments / a failed launch.
extern "C" int rnn_probe_range_read(const void *p, int64_t bytes, int groups, int waves,
                                    int per_lane, uint32_t magic, uint32_t *sink, void *stream) {
    if (bytes <= 0 || bytes % 1024 != 0 || ((uintptr_t)p & 15) != 0 || sink == nullptr ||
        groups <= 0 || bytes / 1024 < groups)
        return 1;
    const u32x4 *q = reinterpret_cast<const u32x4 *>(p);
    const int64_t nc = bytes / 1024;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define RNN_RR(W, P) range_read_kernel<W, P><<<(unsigned)groups, (W) * 64, 0, st>>>(q, nc, magic, sink)
    if (waves == 4 && per_lane == 2) RNN_RR(4, 2);
    else if (waves == 4 && per_lane == 4) RNN_RR(4, 4);
    else if (waves == 4 && per_lane == 8) RNN_RR(4, 8);
    else if (waves == 4 && per_lane == 24) RNN_RR(4, 24);
    else if (waves == 8 && per_lane == 2) RNN_RR(8, 2);
    else if (waves == 8 && per_lane == 4) RNN_RR(8, 4);
    else if (waves == 8 && per_lane == 8) RNN_RR(8, 8);
    else if (waves == 8 && per_lane == 24) RNN_RR(8, 24);
    else return 1;
#undef RNN_RR
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// ---------------------------------------------------------- L2 load rate
// The rate at which a CU takes in L2-resident data, with the loads writing
// VGPRs (buffer_load_dwordx4) or LDS (buffer_load_dwordx4 ... lds, the GEMM
// kernels' DMA): blocks of 8 waves, wave (b, w) walking its own 64 KiB window
// (window (8 b + w) mod the buffer's windows) in `rounds` rounds of PER 1 KiB
// loads (16 bytes per lane), each round waited for before the next is
// issued. Load j of a wave reads chunk j mod 64 of its window, so 64 loads
// read every chunk once. VGPR loads: the XOR of everything a wave loaded;
// LDS loads: the XOR of what its last round left in LDS. The sink is written
// only when that XOR equals `magic`.
template <bool TO_LDS, int PER>
__global__ __launch_bounds__(512) void l2_rate_kernel(const int8_t *__restrict__ p, uint32_t bytes,
                                                      int rounds, uint32_t magic, uint32_t *sink) {
    __shared__ __attribute__((aligned(1024))) int8_t lds[TO_LDS ? 8 * PER * 1024 : 16];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t base = ((blockIdx.x * 8u + (uint32_t)w) % (bytes >> 16)) << 16;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(p), 0, (int)bytes, 0x00020000);
    uint32_t acc = 0;
    for (int r = 0; r < rounds; ++r) {
        u32x4 v[PER];
#pragma unroll
        for (int d = 0; d < PER; ++d) {
            const uint32_t off = base + (uint32_t)(((r * PER + d) & 63) << 10) + 16u * lane;
            if constexpr (TO_LDS)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rs, (__attribute__((address_space(3))) void *)(lds + (w * PER + d) * 1024), 16,
                    off, 0, 0, 0);
            else
                v[d] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if constexpr (!TO_LDS) {
#pragma unroll
            for (int d = 0; d < PER; ++d) acc ^= v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
        }
    }
    if constexpr (TO_LDS) {
#pragma unroll
        for (int d = 0; d < PER; ++d) {
            const u32x4 t = *reinterpret_cast<const u32x4 *>(lds + (w * PER + d) * 1024 + 16 * lane);
            acc ^= t.x ^ t.y ^ t.z ^ t.w;
        }
    }
    for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
    if (lane == 0 && acc == magic) atomicXor(sink, acc);
}

// `groups` blocks of 8 waves over a buffer of `bytes` (a multiple of 64 KiB,
// at most 1 GiB, 16-byte aligned), `rounds` rounds of `per_lane` (4 or 8)
// loads per wave, into VGPRs (to_lds 0) or LDS (1). Returns 0, or 1 for bad
// arguments / a failed launch.
extern "C" int rnn_probe_l2_rate(const void *p, int64_t bytes, int groups, int to_lds, int per_lane,
                                 int rounds, uint32_t magic, uint32_t *sink, void *stream) {
    if (bytes < 65536 || bytes % 65536 != 0 || bytes > (int64_t)1 << 30 || ((uintptr_t)p & 15) != 0 ||
        sink == nullptr || groups <= 0 || rounds <= 0 || (to_lds != 0 && to_lds != 1))
        return 1;
    const int8_t *q = static_cast<const int8_t *>(p);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define RNN_L2(L, P) l2_rate_kernel<L, P><<<(unsigned)groups, 512, 0, st>>>(q, (uint32_t)bytes, rounds, magic, sink)
    if (to_lds && per_lane == 4) RNN_L2(true, 4);
    else if (to_lds && per_lane == 8) RNN_L2(true, 8);
    else if (!to_lds && per_lane == 4) RNN_L2(false, 4);
    else if (!to_lds && per_lane == 8) RNN_L2(false, 8);
    else return 1;
#undef RNN_L2
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// ---------------------------------------------------------------- clock probe
// A fixed amount of int8 MFMA work on constant operands, one wave per SIMD on
// every CU, with the shader-clock counter (s_memtime) and the 100 MHz
// real-time counter (s_memrealtime) read at the start and end of each block:
// out[4*b .. 4*b+3] = {clk0, clk1, rt0, rt1}. The ratio of the two deltas is
// the shader clock while the block ran, an independent check of clock figures
// derived from rocprofv3 counters (SQ_BUSY_CYCLES) over the same launch.
typedef int i32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void mfma_clock_kernel(int iters, uint64_t *out, int *sink) {
    const uint64_t clk0 = __builtin_amdgcn_s_memtime();
    const uint64_t rt0 = __builtin_amdgcn_s_memrealtime();
    i32x4 a = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    i32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = i32x4{0, 0, 0, 0};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, a, acc[j], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += acc[j].x;
    __syncthreads();
    const uint64_t clk1 = __builtin_amdgcn_s_memtime();
    const uint64_t rt1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        out[4 * blockIdx.x + 0] = clk0;
        out[4 * blockIdx.x + 1] = clk1;
        out[4 * blockIdx.x + 2] = rt0;
        out[4 * blockIdx.x + 3] = rt1;
    }
    if (s == 0x7fffffff) sink[0] = s;
}

// `blocks` workgroups of 4 waves run `iters` x 8 MFMAs each; out holds
// 4 * blocks u64. Returns 0, or 1 for bad arguments / a failed launch.
extern "C" int rnn_probe_mfma_clock(int blocks, int iters, uint64_t *out, int *sink, void *stream) {
    if (blocks <= 0 || iters <= 0 || out == nullptr || sink == nullptr) return 1;
    mfma_clock_kernel<<<(unsigned)blocks, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(iters, out,
                                                                                          sink);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}
