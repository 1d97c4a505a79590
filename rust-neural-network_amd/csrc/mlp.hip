// mlp.hip -- a chain of W8A8 layers (Int8Model::forward, the 784-256-128-10
// MLP of the benchmark configurations) in one launch.
//
// Per layer: the running activation's rows are quantized per row
// (scale = max|x|/127, q = round(x/scale) clamped; the rule of
// rnn_quant_rows_i8), multiplied by the layer's int8 weight [n, k] on
// v_mfma_i32_16x16x64_i8 into exact int32, dequantized in the reference's
// order ((acc * sa[m]) * sw[n] + bias[n], src/int8.rs:159-162) and, between
// layers, passed through max(., 0) (src/tensor.rs:2025-2032). The result is
// bit-identical to chaining rnn_quant_rows_i8 and rnn_w8a8_linear per layer.
//
// A workgroup owns up to 16 rows for the whole chain (fewer when the batch
// would not fill the CUs otherwise): the activation stays in LDS
// (f32 for the quantization pass, int8 codes for the MFMAs), so a layer's
// output never goes to HBM and the chain costs one launch instead of two per
// layer. Each of the 8 waves takes 16-column tiles of a layer; a tile's
// weight fragments (16 bytes per lane per 64-k block) come straight from
// global memory (each weight byte is read by one wave of each workgroup), and
// the wave's next tile is requested before the current one's MFMAs.
#include "common.hpp"
#include "numerics.hpp"

namespace rnn {

constexpr int kMlpMaxLayers = 4;
constexpr int kMlpMaxDim = 1024;   // widest layer input or output
constexpr int kMlpRows = 16;       // rows per workgroup (one MFMA row block)
constexpr int kMlpWaves = 8;
constexpr int kMlpMaxKb = kMlpMaxDim / 64;  // 64-k blocks of the widest input

struct MlpLayer {
    const int8_t *wq;   // [n, k] int8, 16-byte aligned, k % 16 == 0
    const float *sw;    // [n]
    const float *bias;  // [n] or null
    int n, k;
};

struct MlpArgs {
    MlpLayer layer[kMlpMaxLayers];
    int nlayers;
    int relu;  // ReLU between layers (not after the last)
};

constexpr int kMlpPrefetchKb = 4;  // next-layer blocks requested ahead (k <= 256)

// Workgroup barrier for LDS traffic only. __syncthreads() also orders global
// memory, which makes every wave wait for all of its outstanding loads; here
// the weight loads requested ahead must stay in flight across the barriers.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// A 16-column tile of a layer as one lane holds it.
template <int NKB>
struct MlpTile {
    v4i b[NKB];      // weight fragments, 64-k block kb
    float sw, bias;  // the dequant operands of the lane's column
};

// The weight fragments of 16-column tile t of a layer for this lane (row =
// lane & 15, q = lane >> 4): 16 bytes of column 16 t + row at k = 64 kb + 16 q.
// Every load is issued (columns past N re-read the last column), so that the
// compiler can count the loads in flight and wait for exactly the ones a use
// needs (a load skipped on some path makes it wait for all of them). They go
// through a buffer descriptor over the layer's weights: one offset register
// per tile, and bytes past the weights read as 0. Bytes past K (the next
// column's, or 0) meet zero activation codes, since the codes are zero-padded
// to whole 64-k blocks, and blocks past K take no MFMA; outputs past N are
// dropped.
template <int NKB>
__device__ __forceinline__ void mlp_load_tile(const MlpLayer &L, int t, int lane, MlpTile<NKB> &tl) {
    const int row = lane & 15, q = lane >> 4;
    const int n = min(16 * t + row, L.n - 1);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t *>(L.wq), 0, L.n * L.k, 0x00020000);  // 32-bit data format
    const uint32_t off = (uint32_t)(n * L.k + 16 * q);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
        tl.b[kb] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 64 * kb, 0, 0));
    // the column's scale and bias ride with its weights (a null bias reads the
    // scale again; the epilogue adds a bias only when there is one, and no
    // select touches these values before that use, which would wait for them)
    tl.sw = L.sw[n];
    tl.bias = (L.bias ? L.bias : L.sw)[n];
}

// Per-row quantization by one wave, a lane taking 4 consecutive elements per
// step (K % 16 == 0: a quad is wholly inside or past K). max |x| over the row
// (order-independent; fmaxf drops NaN as f32::max does):
__device__ __forceinline__ float mlp_row_max(const float *xr, int K, int lane) {
    float mx = 0.0f;
    for (int c0 = 4 * lane; c0 < K; c0 += 256) {
        const float4 v = *reinterpret_cast<const float4 *>(xr + c0);
        mx = fmaxf(mx, fabsf(v.x));
        mx = fmaxf(mx, fabsf(v.y));
        mx = fmaxf(mx, fabsf(v.z));
        mx = fmaxf(mx, fabsf(v.w));
    }
    return wave_max(mx);
}

// the codes, zero past K up to `end` (whole 64-k blocks): one 16-byte LDS
// read, 4 codes packed into one 4-byte write. q = round(x / s) through the
// reciprocal with the exact division only next to a half-integer
// (round_quotient), the same integer as the IEEE quotient rounded.
__device__ __forceinline__ void mlp_row_codes(const float *xr, int8_t *qr, int K, int end, int lane,
                                              float s, float inv) {
    for (int c0 = 4 * lane; c0 < end; c0 += 256) {
        uint32_t packed = 0u;
        if (c0 < K) {
            const float4 v = *reinterpret_cast<const float4 *>(xr + c0);
            const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float qv = clamp_rs(round_quotient(e[u], s, inv), -128.0f, 127.0f);
                packed |= (uint32_t)(uint8_t)to_i8_rs(qv) << (8 * u);
            }
        }
        *reinterpret_cast<uint32_t *>(qr + c0) = packed;
    }
}

// rows: rows of x per workgroup (1 .. 16). The MFMAs always take a 16-row
// block; rows past `rows` hold zero codes and their outputs are dropped.
// Fewer rows per workgroup spread a small batch over more CUs: each
// workgroup still streams every weight, but its share of x shrinks and a row
// is quantized by 8 / rows waves. XV: 16-byte loads of x per thread (the
// fewest that cover rows x k0 floats).
template <int XV>
__global__ __launch_bounds__(kMlpWaves * 64) void w8a8_mlp_kernel(const float *__restrict__ x,
                                                                  int64_t M, int rows, MlpArgs args,
                                                                  float *__restrict__ y) {
    __shared__ __attribute__((aligned(16))) float xf[kMlpRows][kMlpMaxDim];  // running activation
    __shared__ __attribute__((aligned(16))) int8_t xq[kMlpRows][kMlpMaxDim + 64];  // its codes
    __shared__ float sa[kMlpRows];                                        // row scales
    const int tid = threadIdx.x, wid = tid / 64, lane = tid % 64;
    const int row = lane & 15, q = lane >> 4;
    const int64_t r0 = (int64_t)blockIdx.x * rows;
    const int mr = (int)std::min<int64_t>(rows, M - r0);  // valid rows
    // the block's rows past `rows`: zero codes and scales, never written again
    for (int t = tid; t < (kMlpRows - rows) * ((kMlpMaxDim + 64) / 16); t += kMlpWaves * 64)
        reinterpret_cast<uint4 *>(&xq[rows][0])[t] = uint4{0u, 0u, 0u, 0u};
    if (tid >= rows && tid < kMlpRows) sa[tid] = 0.0f;

    // Every wave requests its input rows, then (after a barrier that waits
    // for no load, so that every wave's row requests are queued ahead of the
    // weight requests) its first tile of layer 0; a wave's next tile is
    // requested before the current one's MFMAs, and each layer requests the
    // next layer's first tile (when its k <= 256) before its quantization
    // pass, so weight latency overlaps the x load, the quantization passes and
    // the epilogues. Each CU takes in loads at about 136 GB/s, so a load
    // requested early holds up the waves that request more behind it: only
    // the first tile goes out with x. Loads complete in issue order, so each
    // wait is placed behind the loads it needs and in front of the ones that
    // may stay in flight.
    MlpTile<kMlpMaxKb> cur, ahead;
    MlpTile<kMlpPrefetchKb> nxt;
    bool have_cur = wid < (args.layer[0].n + 15) / 16;
    auto request_first_tile = [&]() {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        // issued whether or not the wave has this tile (see mlp_load_tile)
        mlp_load_tile<kMlpMaxKb>(args.layer[0], wid, lane, cur);
    };

    // the input rows (rows past M read as zeros; their outputs are dropped):
    // every load of the thread is issued before the first LDS write, from a
    // clamped (always valid) address, and masked afterwards
    const int k0 = args.layer[0].k;
    if (k0 % 4 == 0 && ((uintptr_t)x & 15) == 0) {
        const int k4 = k0 / 4, total = rows * k4;
        const float4 *x4 = reinterpret_cast<const float4 *>(x + r0 * k0);
        const int last4 = mr * k4 - 1;  // the last valid float4 of the block's rows
        float4 v[XV];
#pragma unroll
        for (int i = 0; i < XV; ++i) v[i] = x4[min(tid + i * kMlpWaves * 64, last4)];
        request_first_tile();
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int t = tid + i * kMlpWaves * 64;
            if (t < total) {
                const int r = t / k4, c = 4 * (t % k4);
                const bool ok = r < mr;
                xf[r][c] = ok ? v[i].x : 0.0f, xf[r][c + 1] = ok ? v[i].y : 0.0f;
                xf[r][c + 2] = ok ? v[i].z : 0.0f, xf[r][c + 3] = ok ? v[i].w : 0.0f;
            }
        }
    } else {
        for (int t = tid; t < rows * k0; t += kMlpWaves * 64) {
            const int r = t / k0, c = t % k0;
            xf[r][c] = r < mr ? x[(r0 + r) * k0 + c] : 0.0f;
        }
        request_first_tile();
    }
    lds_barrier();

    // a row is quantized by G waves: wave w takes rows w / G + rr * (8 / G);
    // each of them finds the row's scale (the same value, no exchange) and
    // writes the codes of every G-th 256-element chunk from chunk w % G
    const int G = rows >= kMlpWaves ? 1 : kMlpWaves / rows;
    const int rstep = kMlpWaves / G, r_w = wid / G, p_w = wid % G;
    for (int l = 0; l < args.nlayers; ++l) {
        const MlpLayer L = args.layer[l];
        const int K = L.k, N = L.n, kb_n = (K + 63) / 64;
        const bool last = l + 1 == args.nlayers;
        const bool relu = !last && args.relu;
        const int ntiles = (N + 15) / 16;
        // next layer's first tile, requested now
        bool have_nxt = false;
        if (!last) {
            const MlpLayer Ln = args.layer[l + 1];
            have_nxt = Ln.k <= 64 * kMlpPrefetchKb && wid < (Ln.n + 15) / 16;
            if (have_nxt) mlp_load_tile<kMlpPrefetchKb>(Ln, wid, lane, nxt);
        }
        // quantize: scale = max|x| / 127, then the codes, zero-padded to
        // whole 64-k blocks (combining partial maxima of a row split over
        // waves through LDS was slower than every wave finding the maximum)
#pragma unroll  // (a wave's rows: their latency chains overlap)
        for (int rr = 0; rr < kMlpRows / kMlpWaves; ++rr) {
            const int r = r_w + rr * rstep;
            if (r >= rows) break;
            const float mx = mlp_row_max(&xf[r][0], K, lane);
            const float s = mx > 0.0f ? mx / 127.0f : 1.0f;
            const float inv = __builtin_amdgcn_rcpf(s);
            if (lane == 0 && p_w == 0) sa[r] = s;
            for (int c = p_w; 256 * c < 64 * kb_n; c += G)
                mlp_row_codes(&xf[r][256 * c], &xq[r][256 * c], K - 256 * c,
                              min(256, 64 * kb_n - 256 * c), lane, s, inv);
        }
        lds_barrier();
        if (!have_cur && wid < ntiles) mlp_load_tile<kMlpMaxKb>(L, wid, lane, cur);
        for (int t = wid; t < ntiles; t += kMlpWaves) {
            const int col = 16 * t + row;
            const float w = cur.sw, bb = cur.bias;
            const bool more = t + kMlpWaves < ntiles;
            if (more) mlp_load_tile<kMlpMaxKb>(L, t + kMlpWaves, lane, ahead);
            v4i acc = {0, 0, 0, 0};
#pragma unroll
            for (int kb = 0; kb < kMlpMaxKb; ++kb) {
                if (kb < kb_n) {
                    const v4i a = *reinterpret_cast<const v4i *>(&xq[row][64 * kb + 16 * q]);
                    // D[m][n]: A = activation rows, B = weight columns
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, cur.b[kb], acc, 0, 0, 0);
                }
            }
            // lane holds column 16 t + row, rows 4 q .. 4 q + 3; the
            // reference's order: ((acc * sa[m]) * sw[n]) + bias[n], then ReLU
            if (col < N) {
                const int32_t av[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = 4 * q + e;
                    float v = (float)av[e] * sa[m] * w;
                    if (L.bias) v = v + bb;
                    if (relu) v = fmaxf(v, 0.0f);
                    if (last) {
                        if (m < mr) y[(r0 + m) * N + col] = v;
                    } else {
                        xf[m][col] = v;
                    }
                }
            }
            if (more) cur = ahead;
        }
        lds_barrier();
        have_cur = have_nxt;
        if (have_nxt) {
#pragma unroll
            for (int kb = 0; kb < kMlpPrefetchKb; ++kb) cur.b[kb] = nxt.b[kb];
#pragma unroll
            for (int kb = kMlpPrefetchKb; kb < kMlpMaxKb; ++kb) cur.b[kb] = v4i{0, 0, 0, 0};
            cur.sw = nxt.sw, cur.bias = nxt.bias;
        }
    }
}

}  // namespace rnn

using namespace rnn;

extern "C" int rnn_w8a8_mlp(const float *x, int64_t m, int nlayers, const int64_t *dims,
                            const int8_t *const *wq, const float *const *sw,
                            const float *const *bias, int relu, float *y, void *stream) {
    RNN_ENTRY();
    const char *name = "rnn_w8a8_mlp";
    RNN_REQUIRE(m >= 0, "%s: negative m", name);
    RNN_REQUIRE(nlayers >= 1 && dims && wq && sw, "%s: need at least one layer", name);
    RNN_REQUIRE(relu == 0 || relu == 1, "%s: relu must be 0 or 1", name);
    if (nlayers > kMlpMaxLayers)
        return set_error(RNN_ERR_UNSUPPORTED, "%s: at most %d layers in one launch (got %d)", name,
                         kMlpMaxLayers, nlayers);
    MlpArgs args{};
    args.nlayers = nlayers;
    args.relu = relu;
    for (int l = 0; l < nlayers; ++l) {
        const int64_t k = dims[l], n = dims[l + 1];
        RNN_REQUIRE(k > 0 && n > 0, "%s: layer %d has a zero or negative size", name, l);
        RNN_REQUIRE(wq[l] && sw[l], "%s: layer %d: null weight or scales", name, l);
        if (k > kMlpMaxDim || n > kMlpMaxDim || k % 16 != 0 || ((uintptr_t)wq[l] & 15) != 0)
            return set_error(RNN_ERR_UNSUPPORTED,
                             "%s: layer %d (%lld -> %lld): the one-launch chain needs widths <= "
                             "%d, in-features %% 16 == 0 and 16-byte aligned weights",
                             name, l, (long long)k, (long long)n, kMlpMaxDim);
        args.layer[l] = MlpLayer{wq[l], sw[l], bias ? bias[l] : nullptr, (int)n, (int)k};
    }
    if (m == 0) return RNN_OK;
    RNN_REQUIRE(x && y, "%s: null x or y", name);
    // rows per workgroup: the fewest (a power of two) that keep the
    // workgroups within one per CU. Every workgroup streams all the weights
    // through its CU, so a second workgroup on a CU costs more than the MFMA
    // rows a small batch leaves at zero (measured on 784-256-128-10: batch 1024
    // at 2 rows per workgroup ran near twice as long as at 4).
    int rows = 1;
    while (rows < kMlpRows && ceil_div(m, rows) > device_cu_count()) rows *= 2;
    const int64_t blocks = ceil_div(m, rows);
    RNN_REQUIRE(blocks <= 0x7fffffffLL, "%s: m too large", name);
    // 16-byte loads of x per thread: rows x k0 floats over 512 threads
    const int64_t xv = ceil_div((int64_t)rows * dims[0], 4 * kMlpWaves * 64);
    const hipStream_t st = as_stream(stream);
    if (xv <= 1)
        w8a8_mlp_kernel<1><<<(unsigned)blocks, kMlpWaves * 64, 0, st>>>(x, m, rows, args, y);
    else if (xv <= 2)
        w8a8_mlp_kernel<2><<<(unsigned)blocks, kMlpWaves * 64, 0, st>>>(x, m, rows, args, y);
    else if (xv <= 4)
        w8a8_mlp_kernel<4><<<(unsigned)blocks, kMlpWaves * 64, 0, st>>>(x, m, rows, args, y);
    else
        w8a8_mlp_kernel<8><<<(unsigned)blocks, kMlpWaves * 64, 0, st>>>(x, m, rows, args, y);
    return check_launch(name);
}
