/*
 * rnn_hip.h -- C ABI of the MI355X (gfx950) quantized-inference path of
 * rust-nn (gugu8intel-i9/Rust-Neural-Network): W8A8 int8 GEMM/GEMV, 2-bit
 * ternary matmul and RotorQuant KV quantize/dequantize.
 *
 * Conventions
 *  - Every tensor pointer is a DEVICE pointer (HBM) on the current HIP device.
 *    Matrices are row-major and dense; sizes are element counts.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream). Calls
 *    are asynchronous on that stream; results are visible after it syncs.
 *  - Return value: RNN_OK (0) or an RNN_ERR_* code; rnn_last_error() gives the
 *    calling thread's message for its most recent call (empty after a call
 *    that succeeded). The reference panics on the same conditions
 *    (e.g. src/int8.rs:72, src/quant.rs:136,215-220); a Rust binding maps a
 *    non-zero status to panic!.
 *  - Thread safety: no global mutable state apart from the per-thread error
 *    string; concurrent calls on different streams are independent.
 *  - Numerics follow the reference exactly: IEEE division, round half away
 *    from zero (f32::round), no FMA contraction, wrapping int32 accumulation,
 *    epilogue ((float)acc * s1) * s2 + bias in that order.
 * Each declaration names the reference interface it replaces (file:line).
 */
#ifndef RNN_HIP_H
#define RNN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RNN_HIP_ABI_VERSION 1

enum rnn_status {
    RNN_OK = 0,
    RNN_ERR_INVALID_ARG = 1, /* null pointer, bad size, bad flag            */
    RNN_ERR_HIP = 2,         /* a HIP runtime call or kernel launch failed   */
    RNN_ERR_UNSUPPORTED = 3, /* shape/alignment this entry point cannot take */
    RNN_ERR_OUT_OF_MEMORY = 4
};

/* flags for the GEMM entry points */
#define RNN_FLAG_RELU 0x1u          /* y = max(y, 0) after bias (src/tensor.rs:2025-2032) */
#define RNN_ALGO_AUTO 0x00u         /* GEMV for m <= 16, else LDS-DMA tiles (k % 128 == 0, n % 4 == 0) or register-staged tiles */
#define RNN_ALGO_TILED 0x10u        /* force the register-staged 128x128 MFMA GEMM */
#define RNN_ALGO_GEMV 0x20u         /* force the skinny GEMV (m <= 16; rnn_qt_linear_forward: per 16-row slice for any m) */
#define RNN_ALGO_TILED_DMA 0x30u    /* force the LDS-DMA pipelined big-tile GEMM (k % 128 == 0, n % 4 == 0) */
#define RNN_ALGO_GEMV_MFMA 0x40u    /* rnn_qt_linear_forward: force the f32-MFMA GEMV (per 16-row slice) */
#define RNN_ALGO_GEMV_BF16 0x50u    /* rnn_qt_linear_forward: force the bf16-MFMA GEMV (per 16-row slice) */
#define RNN_ALGO_MASK 0xF0u
#define RNN_FLAG_TERNARY_MFMA_LAYOUT 0x100u /* rnn_ternary_gemm: codes are in the layout of rnn_ternary_prepack */

int rnn_abi_version(void);
const char *rnn_last_error(void);

/* ------------------------------------------------------------ int8 (a1-a6) */

/* Per-row symmetric int8: scale[r] = max_j|x[r,j]|/127 (1.0 for an all-zero
 * row), q = (x/scale).round().clamp(-128,127).
 * Replaces Int8Weights::quantize (src/int8.rs:24-52) when x is a weight
 * [out,in], and is the per-row dynamic activation rule of
 * QuantizedTensor::quantize_int8 with group_size=cols (src/quantize.rs:296-322). */
int rnn_quant_rows_i8(const float *x, int64_t rows, int64_t cols, int8_t *q,
                      float *scale, void *stream);

/* w[r,j] = q[r,j] as f32 * scale[r].  Int8Weights::dequantize (src/int8.rs:55-65) */
int rnn_int8_dequantize(const int8_t *q, const float *scale, int64_t rows,
                        int64_t cols, float *w, void *stream);

/* Int8Weights::matmul_f32 (src/int8.rs:70-88): y[m,o] =
 * (sum_k i8((x*(1/s[o])).round().clamp) * wq[o,k]) as f32 * s[o] * s[o]. */
int rnn_int8_matmul_f32(const int8_t *wq, const float *ws, int64_t out_f,
                        int64_t in_f, const float *x, int64_t m, float *y,
                        void *stream);

/* Int8Linear::forward (src/int8.rs:134-172), reference semantics: the
 * activation is quantized with the weight's channel scale inside the output
 * loop; y = acc as f32 * s[o] * s[o] (+ bias[o]). bias may be NULL. */
int rnn_int8_linear_forward(const float *x, int64_t batch, int64_t in_f,
                            const int8_t *wq, const float *ws, int64_t out_f,
                            const float *bias, float *y, void *stream);

/* Device workspace rnn_igemm needs (bytes); 0 for m, n or k == 0. */
size_t rnn_igemm_workspace_size(int64_t m, int64_t k, int64_t n);

/* igemm (src/int8.rs:285-314) / igemm_scalar (:222-234): c[m,n] = sum_k
 * a_u8[m,k] * b_i8[k,n] in wrapping int32; a is UNSIGNED [m,k], b SIGNED
 * [k,n] (N-contiguous). Computed on signed int8 MFMA with the exact identity
 * sum (a_s8+128)*b = sum a_s8*b + 128*colsum(b). `workspace` must hold
 * rnn_igemm_workspace_size() bytes, or be NULL to let the call allocate and
 * free stream-ordered memory; problems with m*n*k <= 2^28 run in one launch
 * that stages both operands in LDS and use no workspace. */
int rnn_igemm(const uint8_t *a, const int8_t *b, int32_t *c, int64_t m,
              int64_t k, int64_t n, void *workspace, size_t workspace_bytes,
              void *stream);

/* No counterpart in the reference: rnn_igemm for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same contract and results as rnn_igemm; the workspace is
 * a file-scope device array of RNN_IGEMM_NOALLOC_MAX_BYTES that each GPU the
 * library runs on holds until the process ends. Problems with
 * m*n*k <= 2^28 run in one launch and use no workspace, at any size; larger
 * ones whose rnn_igemm_workspace_size() exceeds the array return
 * RNN_ERR_UNSUPPORTED. Nothing
 * is allocated and nothing needs clearing between calls. Calls on one GPU
 * share that GPU's array: calls ordered on one stream are safe, calls that
 * overlap on one GPU (other streams, other threads) race. */
#define RNN_IGEMM_NOALLOC_MAX_BYTES (64u << 20)
int rnn_igemm_noalloc(const uint8_t *a, const int8_t *b, int32_t *c, int64_t m,
                      int64_t k, int64_t n, void *stream);

/* W8A8 linear (the igemm contract's "caller applies scales"
 * step of src/int8.rs:283-284 fused into the GEMM store, in the multiply
 * order of src/int8.rs:159-162):
 *   acc[m,n] = sum_k aq[m,k]*wq[n,k]   (wrapping int32)
 *   y[m,n]   = ((float)acc * sa[m]) * sw[n] (+ bias[n]) (relu if flagged)
 * aq [m,k] int8 row quantized (rnn_quant_rows_i8), wq [n,k] int8 (the
 * Int8Weights layout, src/int8.rs:14-17). Any k and any operand alignment
 * (the igemm contract, src/int8.rs:288-296): k % 16 != 0 or unaligned operands
 * take a tiled kernel that assembles its chunks from byte loads (the forced
 * GEMV and LDS-DMA algos need k % 16 == 0 and 16-byte alignment).
 * bias, y and acc_out may each be NULL (not both y and acc_out). */
int rnn_w8a8_linear(const int8_t *aq, const float *sa, const int8_t *wq,
                    const float *sw, const float *bias, int64_t m, int64_t k,
                    int64_t n, unsigned flags, float *y, int32_t *acc_out,
                    void *stream);

/* Int8Model::forward in one launch: a chain of nlayers W8A8 layers over x
 * [m, dims[0]] (the 784-256-128-10 MLP of the benchmark configurations).
 * Layer l: the running activation's rows are quantized per row
 * (rnn_quant_rows_i8's rule), multiplied by wq[l] [dims[l+1], dims[l]] int8
 * (the Int8Weights layout) into int32, dequantized as
 * ((acc * sa[m]) * sw[l][n]) + bias[l][n] (src/int8.rs:159-162), and, between
 * layers when relu = 1, passed through max(., 0) (src/tensor.rs:2025-2032).
 * y [m, dims[nlayers]]. Bit-identical to chaining rnn_quant_rows_i8 and
 * rnn_w8a8_linear; the activation stays in LDS between layers. dims, wq, sw
 * and bias are HOST arrays (bias may be NULL, or hold NULL entries) of device
 * pointers. RNN_ERR_UNSUPPORTED for chains the single launch does not take:
 * more than 4 layers, a width over 1024, dims[l] % 16 != 0 or a weight that
 * is not 16-byte aligned (chain the per-layer calls instead). */
int rnn_w8a8_mlp(const float *x, int64_t m, int nlayers, const int64_t *dims,
                 const int8_t *const *wq, const float *const *sw,
                 const float *const *bias, int relu, float *y, void *stream);

/* ---------------------------------------------------------- ternary (a7-a9) */

/* pack_ternary (src/ternary.rs:46-60): 16 codes per u32, LSB first,
 * 0 -> 00, >0 -> 01, <0 -> 10; packed holds ceil(count/16) words. */
int rnn_ternary_pack(const int8_t *t, int64_t count, uint32_t *packed,
                     void *stream);
/* unpack_ternary (src/ternary.rs:63-75); code 11 decodes to 0. */
int rnn_ternary_unpack(const uint32_t *packed, int64_t count, int8_t *t,
                       void *stream);

#define RNN_TERNARY_ROWS 0    /* TernaryTensor::quantize rule (src/ternary.rs:97-137) */
#define RNN_TERNARY_ABSMEAN 1 /* per-tensor absmean gamma (BitNet b1.58), broadcast */

/* Quantize w [rows,cols] to packed ternary (flat row-major codes, as
 * TernaryTensor::packed) and scales [rows]. ROWS: delta = 0.7*mean|w|,
 * scale = max(mean|w|,1e-8) per row, sums sequential in k (bit-exact).
 * ABSMEAN: gamma = max(mean|w|,1e-8) over the tensor (row sums in f32 added
 * in double), t = round(w/gamma).clamp(-1,1), scales[r] = gamma. */
int rnn_ternary_quantize(const float *w, int64_t rows, int64_t cols, int mode,
                         uint32_t *packed, float *scales, void *stream);

/* TernaryTensor::dequantize (src/ternary.rs:140-161). */
int rnn_ternary_dequantize(const uint32_t *packed, int64_t numel,
                           const float *scales, int64_t n_scales, int64_t cols,
                           float *w, void *stream);

/* TernaryLinear::forward (src/ternary.rs:239-279), reference semantics: f32
 * shift-and-add in k order, then acc * scale[o] (+ bias[o]); bit-exact. */
int rnn_ternary_linear_forward(const float *x, int64_t batch, int64_t in_f,
                               const uint32_t *packed, const float *scales,
                               int64_t out_f, const float *bias, float *y,
                               void *stream);

/* Ternary GEMM on int8 MFMA (BASELINE ternary config): t[n,k] unpacked from
 * the 2-bit codes inside the kernel, acc = sum_k aq[m,k]*t[n,k], epilogue as
 * rnn_w8a8_linear with sw[n].
 * flags: RNN_FLAG_RELU, RNN_FLAG_TERNARY_MFMA_LAYOUT when `packed` comes
 * from rnn_ternary_prepack (k % 16 == 0), and an algo (AUTO: the LDS-DMA
 * kernel when k % 128 == 0, n % 4 == 0 and buffers are 16-byte aligned, else
 * TILED; TILED or TILED_DMA force one). Any k is accepted in the reference
 * layout: rows that start mid-word (k % 16 != 0) or unaligned activations take
 * a tiled kernel that gathers codes from arbitrary bit offsets. */
int rnn_ternary_gemm(const int8_t *aq, const float *sa, const uint32_t *packed,
                     const float *sw, const float *bias, int64_t m, int64_t k,
                     int64_t n, unsigned flags, float *y, int32_t *acc_out,
                     void *stream);

/* The packed codes of a ternary weight [rows, cols] (TernaryTensor::packed,
 * cols % 16 == 0 so that rows are whole words) rearranged for the GEMM: within
 * each 32-bit word, the code of column k0 + 4r + b moves from bits 2(4r+b) to
 * bits 8b + 2r. Same size (rows*cols/16 words), still 2 bits per weight;
 * rnn_ternary_gemm with RNN_FLAG_TERNARY_MFMA_LAYOUT reads this layout and
 * decodes it with byte permutes instead of a lookup table. A one-time weight
 * preparation (like the reference's per-call pack_b_vnni, src/int8.rs:195-218,
 * but done once); no counterpart in the reference. out may not alias packed. */
int rnn_ternary_prepack(const uint32_t *packed, int64_t rows, int64_t cols,
                        uint32_t *out, void *stream);

/* ------------------------------------------------------- RotorQuant (a10-a12) */

/* Rotor::rotation_matrix (src/quant.rs:101-113) for n rotors {s,p12,p13,p23};
 * rot9 receives n row-major 3x3 matrices. As in the reference, the sandwich
 * applies R and then its reverse both on the left (:84-89 over apply,
 * :70-81), so the matrix is |R|^2 * I (rounded as the reference rounds it):
 * the identity, up to f32 rounding, for unit rotors. */
int rnn_rotor_rotation_matrices(const float *rotors, int64_t n, float *rot9,
                                void *stream);

/* RotorQuant::quantize / Module::forward (src/quant.rs:212-252, quantize_vec
 * :170-208) over x [rows, dim]: zero-pad to padded_dim = ceil(dim/3)*3, per
 * 3-group rotate (by the rotation matrix above, so |R|^2 * I: for unit rotors
 * this is per-group absmax quantization, as the reference computes it), scale = max|rv|/qmax, q = (rv/scale).round().clamp(+-qmax),
 * rv = q*scale, inverse-rotate, trim. rotors: ceil(dim/3) x {s,p12,p13,p23}
 * (RotorQuant::rotors, src/quant.rs:127). bits in [2,8] (qmax = 2^(bits-1)-1).
 * y [rows,dim] receives the reconstruction (may be NULL when codes is set);
 * codes [rows,padded_dim] int8 and scales [rows,padded_dim/3] are optional.
 * A group with max|rv| < 1e-12 is left untouched (:189-191): codes 0, scale 0.
 * Any dim (the reference takes any): up to 2688 the rotation matrices sit in
 * LDS, beyond that each group's matrix is rebuilt from its rotor in
 * registers (same expressions, same bits). */
int rnn_rotorquant_quantize(const float *x, int64_t rows, int64_t dim, int bits,
                            const float *rotors, float *y, int8_t *codes,
                            float *scales, void *stream);

/* Reconstruction from codes + scales with the same expressions as :195-202
 * (skipped groups reconstruct to 0). */
int rnn_rotorquant_dequantize(const int8_t *codes, const float *scales,
                              int64_t rows, int64_t dim, const float *rotors,
                              float *y, void *stream);

/* --------------------------------------------- f32 GEMM (BlasBackend) */

/* C = alpha*op(A)*op(B) + beta*C, row-major with leading dimensions (row
 * strides, in elements):
 *   op(A) [m,k]: transa = 0 -> A stored [m,k], lda >= k;
 *                transa = 1 -> A stored [k,m], lda >= m;
 *   op(B) [k,n]: transb = 0 -> B stored [k,n], ldb >= n;
 *                transb = 1 -> B stored [n,k], ldb >= k;
 *   C [m,n], ldc >= n, read (unless beta == 0) and written in place.
 * beta == 0 overwrites C without reading it (NaNs in C do not propagate);
 * k == 0 or alpha == 0 gives C = beta*C; m == 0 or n == 0 is a no-op.
 * Replaces BlasBackend::sgemm and blas::sgemm (src/blas.rs:712-734, contract
 * :89-190, scale_c :191-207). Exception to the header's numeric rule: products
 * are accumulated with fused multiply-adds (MFMA) in an order of the kernel's
 * choosing, so results agree with the reference within the usual GEMM
 * rounding bound (|err| <= ~k * 2^-24 * (|alpha| |A||B| + |beta C|)), not bit
 * for bit -- as the reference's own blocked and small-matrix paths do with
 * each other. m <= 16 with n >= 256 (decode shapes, either B layout) runs a
 * kernel that reads B once and sums K in a fixed order; C = A B with B as
 * stored and m >= 2048 first transposes B into stream-ordered scratch and
 * runs the kernel for B stored [n, k]; other shapes with
 * fewer 128 x 128 tiles of C than CUs split K into up to 16 ranges whose
 * partial products (in stream-ordered scratch) are added in a fixed order:
 * the same inputs give the same bits on every call. */
int rnn_sgemm(int transa, int transb, int64_t m, int64_t n, int64_t k,
              float alpha, const float *a, int64_t lda, const float *b,
              int64_t ldb, float beta, float *c, int64_t ldc, void *stream);

/* Tensor::relu (src/tensor.rs:2025-2032): y[i] = x[i].max(0.0), NaN -> 0 as
 * f32::max returns the non-NaN operand; y may equal x. */
int rnn_relu(const float *x, int64_t n, float *y, void *stream);

/* The fused bias add + activation of Tensor::linear_layer
 * (src/tensor.rs:771-786), in place on y [rows, cols]: y = y + bias[col]
 * (skipped when bias is NULL), then with relu = 1 y = (y > 0 ? y : 0). */
int rnn_bias_act(float *y, const float *bias, int64_t rows, int64_t cols,
                 int relu, void *stream);

/* Tensor::linear_layer (src/tensor.rs:747-800) -- the call Linear::forward
 * makes (src/nn.rs:36-82): y [batch, out_f] = act(x [batch, in_f] . W^T + b)
 * with W stored [out_f, in_f] (nn::Linear::weight), as rnn_sgemm (transb = 1,
 * beta = 0) followed by rnn_bias_act. bias may be NULL (Linear without bias);
 * relu 0 = FusedAct::Identity, 1 = FusedAct::Relu. Within the rnn_sgemm
 * rounding bound of the reference. */
int rnn_linear_layer(const float *x, int64_t batch, int64_t in_f,
                     const float *w, int64_t out_f, const float *bias, int relu,
                     float *y, void *stream);

/* ------------------------------------- QuantizedTensor formats (next row) */

/* QuantFormat (src/quantize.rs:37-56), in the reference's declaration order.
 * Storage is QuantizedTensor::{data, scales, group_size} byte for byte:
 * FP16/BF16 2 bytes per element (little-endian), no scales; INT8/GGUF_Q8 one
 * int8 code per element; INT4/NF4/NVFP4/GGUF_Q4(K) 4-bit codes, each group
 * packed on its own, low nibble first; one f32 scale per group (GGUF: per
 * block of min(group, 32)). */
#define RNN_QF_FP16 0
#define RNN_QF_BF16 1
#define RNN_QF_INT8 2
#define RNN_QF_INT4 3
#define RNN_QF_NF4 4
#define RNN_QF_NVFP4 5
#define RNN_QF_GGUF_Q4 6
#define RNN_QF_GGUF_Q4K 7 /* stored as Q4_0, as the reference does (:241-243) */
#define RNN_QF_GGUF_Q8 8

/* Host-side sizes of QuantizedTensor::quantize(n elements, group_size)
 * (src/quantize.rs:231-250): data bytes, scales.len() and the stored
 * group_size field (0 means the whole tensor; GGUF caps it at 32). No GPU
 * work. */
int rnn_qt_layout(int format, int64_t n, int64_t group_size, int64_t *data_bytes,
                  int64_t *n_scales, int64_t *stored_group);

/* QuantizedTensor::quantize (src/quantize.rs:231-250, per-format :296-625)
 * of x [n] (a tensor's flat row-major data): data and scales sized by
 * rnn_qt_layout. Codes and scales are bit-exact (IEEE division, half-away
 * rounding, first-minimum NF4/E2M1 search, truncating f32->f16 and the
 * wrapping bf16 rounding of :639-703). */
int rnn_qt_quantize(int format, const float *x, int64_t n, int64_t group_size,
                    uint8_t *data, float *scales, void *stream);

/* QuantizedTensor::dequantize (src/quantize.rs:252-269, :324-632) into out
 * [n]; `group` is the stored group_size field. 4-bit formats other than GGUF
 * read byte i/2 of the whole tensor and scales[min(i/group, n_scales-1)], as
 * the reference does. Bit-exact. */
int rnn_qt_dequantize(int format, const uint8_t *data, int64_t data_bytes,
                      const float *scales, int64_t n_scales, int64_t group,
                      int64_t n, float *out, void *stream);

/* QuantizedLinear::forward (src/quantize.rs:744-754): y [m, out_f] =
 * x [m, in_f] . W^T (+ bias[out_f]) with W = the dequantized [out_f, in_f]
 * weight. AUTO: for m <= 16, in_f % 32 == 0, a group that is a multiple of
 * 32 (4-bit formats) or 16 (INT8, GGUF Q8_0) and divides or is divided by
 * in_f, and 16-byte aligned x and data, a fused GEMV that decodes the codes
 * in registers (NF4 and NVFP4 through a 16-entry table; weights read once):
 * for m >= 5 with in_f a multiple of 512 (4-bit), 256 (8-bit) or 128
 * (16-bit) a GEMV on MFMA that takes all m rows at once: for INT4, GGUF Q4,
 * INT8, GGUF Q8_0 and BF16 weights whose groups are multiples of 128 (4-bit),
 * 64 (8-bit) elements dividing in_f (or whole rows), or are 32 elements
 * (GGUF Q4_0 / Q8_0 blocks), with in_f a multiple of 1024 (4-bit), 512
 * (8-bit) or 256 (bf16), the bf16 MFMA GEMV (x split exactly into three bf16
 * parts in registers, codes exact in bf16, each group's sum scaled once, K
 * split over up to 8 workgroups whose partial sums are added in a fixed order
 * in stream-ordered scratch; RNN_ALGO_GEMV_BF16 forces it; AUTO also takes it
 * for 4- and 8-bit codes at m = 3, 4 when every CU gets at least two 16-row
 * tiles of W), else
 * the f32 MFMA GEMV (RNN_ALGO_GEMV_MFMA forces it); else the VALU GEMV
 * (m <= 4, or per 4 rows). For m > 16 the same GEMVs run on 16-row slices
 * of x and y in turn (each slice reads W again) while that is the faster
 * route: up to m = 512 when the slices take the bf16 MFMA GEMV with 4-bit
 * codes, 192 with 8-bit codes or bf16 weights, 96 for the f32 MFMA GEMV, 32
 * for the VALU GEMV; otherwise
 * dequantize into stream-ordered scratch and run rnn_sgemm. RNN_ALGO_GEMV,
 * _GEMV_MFMA and _GEMV_BF16 force their GEMV (per 16-row slice for any m;
 * error if it does not fit), RNN_ALGO_TILED the dequantize route. f32 sums in
 * the kernel's own order: within the rnn_sgemm rounding bound of the
 * reference, not bit for bit. */
int rnn_qt_linear_forward(int format, const float *x, int64_t m, int64_t in_f,
                          const uint8_t *data, int64_t data_bytes,
                          const float *scales, int64_t n_scales, int64_t group,
                          int64_t out_f, const float *bias, float *y,
                          unsigned flags, void *stream);

/* rnn_qt_linear_forward with caller-provided scratch for the bf16 MFMA
 * GEMV's split-K partial sums and counters: `workspace` (16-byte aligned) of
 * at least rnn_qt_linear_workspace_size(in_f, out_f) bytes, ZEROED before its
 * first use (every call leaves it reusable), or NULL to let the call
 * allocate stream-ordered scratch as rnn_qt_linear_forward does. A layer
 * that holds one workspace keeps allocation out of its forward (and out of
 * captured graphs). The workspace is written by the call's kernels: calls
 * that share one must be ordered on one stream. Same reference semantics
 * (src/quantize.rs:744-754). */
size_t rnn_qt_linear_workspace_size(int64_t in_f, int64_t out_f);
int rnn_qt_linear_forward_ws(int format, const float *x, int64_t m, int64_t in_f,
                             const uint8_t *data, int64_t data_bytes,
                             const float *scales, int64_t n_scales, int64_t group,
                             int64_t out_f, const float *bias, float *y,
                             void *workspace, size_t workspace_bytes,
                             unsigned flags, void *stream);

/* ------------------------------- RotorQuant KV cache + attention (next row) */

/* Page sizes for `bh` sequences of `seq` positions at head dim `dim` (ng =
 * ceil(dim/3) groups, positions rounded up to tiles of 64): u16 code elements
 * bh*ceil(seq/64)*64 * 8*ceil(ng/8), f32 scale elements bh*ceil(seq/64)*64 *
 * 4*ceil(ng/4); enough for either kind. Host only. */
int rnn_rotorquant_kv_page_elems(int64_t bh, int64_t seq, int64_t dim,
                                 int64_t *code_elems, int64_t *scale_elems);

#define RNN_RQ_PAGE_K 0
#define RNN_RQ_PAGE_V 1

/* Lays the codes and scales of rnn_rotorquant_quantize (rows = bh*seq vectors
 * of one K or V cache, codes int8 [rows, 3*ceil(dim/3)], scales f32 [rows,
 * ceil(dim/3)]) out as a KV-cache page of tiles of 64 positions: a u16 per
 * position and group holding its three 4-bit two's-complement codes
 * (c0 | c1<<4 | c2<<8) and an f32 scale. kind RNN_RQ_PAGE_K orders a tile for
 * readers with a lane per position: scales of groups 4a..4a+3 of position j at
 * ((tile*ceil(ng/4) + a)*64 + j)*4, codes of groups 8b..8b+7 at
 * ((tile*ceil(ng/8) + b)*64 + j)*8 (groups past ng are padding).
 * RNN_RQ_PAGE_V orders it for readers with a lane per group: the scale of
 * position j, group g at ((tile*16 + j/4)*ng + g)*4 + j%4, its code at
 * ((tile*8 + j/8)*ng + g)*8 + j%8. Positions past seq are zero. bits 2..4. No
 * counterpart in the reference, which keeps only the reconstruction
 * (src/quant.rs:116-121 describes RotorQuant as a KV-cache quantizer). */
int rnn_rotorquant_kv_pack(const int8_t *codes, const float *scales, int64_t bh,
                           int64_t seq, int64_t dim, int bits, int kind,
                           uint16_t *page_codes, float *page_scales, void *stream);

/* Tensor::flash_attention (src/tensor.rs:618-672) of queries q [bh, nq, dim]
 * over the K and V caches held as pages (rnn_rotorquant_kv_pack), equal to
 * the reference's attention over the RotorQuant reconstructions
 * (rnn_rotorquant_dequantize) of K and V, without forming them: scores are
 * s_g ((R_g q_g) . c_g) summed over groups and V is accumulated in the
 * rotated domain. k_* is a RNN_RQ_PAGE_K page, v_* a RNN_RQ_PAGE_V page.
 * out [bh, nq, dim]; any dim whose rotated query (16 bytes per group) fits
 * the workgroup's LDS beside 13 KB of accumulators (dim <= ~27,000 on
 * gfx950); scale multiplies q.k as in the reference.
 * f32 sums in the kernel's own order: within a floating-point bound of the
 * reference, not bit for bit. Pages 16-byte aligned. When the queries alone
 * do not fill the device, each query's sequence is split over several
 * workgroups whose softmax states the last of them merges; their scratch is
 * stream-ordered device memory here, or the caller's workspace with
 * rnn_rotorquant_kv_attention_ws. */
int rnn_rotorquant_kv_attention(const float *q, int64_t bh, int64_t nq,
                                const uint16_t *k_codes, const float *k_scales,
                                const uint16_t *v_codes, const float *v_scales,
                                const float *k_rotors, const float *v_rotors,
                                int64_t seq, int64_t dim, float scale, float *out,
                                void *stream);

/* Bytes of workspace rnn_rotorquant_kv_attention_ws needs for this shape on
 * the current device (0: the call does not split, no workspace needed).
 * No counterpart in the reference: the sequence split is this library's. */
size_t rnn_rotorquant_kv_attention_workspace_size(int64_t bh, int64_t nq, int64_t seq,
                                                  int64_t dim);

/* rnn_rotorquant_kv_attention (src/tensor.rs:618-672) with the split states
 * in a caller's workspace of workspace_bytes (at least
 * rnn_rotorquant_kv_attention_workspace_size). The workspace holds counts:
 * zero it once before its first use; every call leaves them at zero, so it
 * is reused as is. Calls sharing a workspace must be ordered on one stream.
 * workspace NULL: as rnn_rotorquant_kv_attention. */
int rnn_rotorquant_kv_attention_ws(const float *q, int64_t bh, int64_t nq,
                                   const uint16_t *k_codes, const float *k_scales,
                                   const uint16_t *v_codes, const float *v_scales,
                                   const float *k_rotors, const float *v_rotors,
                                   int64_t seq, int64_t dim, float scale, float *out,
                                   void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif
