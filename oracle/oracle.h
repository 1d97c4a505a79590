/*
 * oracle.h -- CPU restatement of rust-nn's quantized-inference path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * kernels and the timed CPU baseline in bench.py. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library (librnn_hip.so) never links or calls it.
 *
 * Each function restates one reference function expression by expression
 * (file:line into gugu8intel-i9/Rust-Neural-Network). The reference is Rust and
 * cannot be compiled in this image (no cargo/rustc), so there is no oracle/_ref
 * build; every function here is pinned instead by the reference's own
 * known-answer tests, by brute force, closed forms and invariants. The pin of
 * each function, chosen so that a dropped term, a wrong sign or index or a
 * transposed operand fails it (CPU tests under tests/):
 *   orc_lcg_bytes             reference recurrence, first outputs
 *                             (test_lcg_generator_matches_reference_recurrence)
 *   orc_igemm_scalar/_igemm   KAT [-4,7] (src/int8.rs:416-422), the 7 LCG
 *                             shapes by int64 brute force, bench inputs at
 *                             512^3, int32 wrap (test_igemm_*)
 *   orc_quant_rows_i8         closed form: max-abs/127, half-away ties, NaN,
 *                             saturation, src/int8.rs:322-327 error bound
 *   orc_int8_dequantize       round trip bound (test_int8_roundtrip_low_error)
 *   orc_int8_matmul_f32       reciprocal vs division distinguished
 *                             (test_int8_matmul_f32_uses_reciprocal)
 *   orc_int8_linear_forward   exact on integer ratios; the reference test's
 *                             max_diff < 5 against f32 (src/int8.rs:346-369)
 *   orc_w8a8_linear, orc_relu numpy int64/f32 brute force in the same order
 *   orc_pack/unpack_ternary   reference KATs (src/ternary.rs:427-446), code 11
 *   orc_ternary_quantize_*    value counts (src/ternary.rs:402-424), sequential
 *                             sum, absmean closed form
 *   orc_ternary_dequantize,
 *   orc_ternary_gemm_i8       brute force over unpacked codes
 *   orc_ternary_linear_f32    exact on integer inputs (any order agrees)
 *   orc_rotor_*               a generic Cl(3,0) geometric product (sandwich =
 *                             two left products), norm preservation and
 *                             |R|^4 scaling of non-unit rotors
 *   orc_rotorquant_*          the reference test's data and bound
 *                             (src/quant.rs:291-310), |err| <= scale/2 per
 *                             rotated component, identity rotors = plain group
 *                             quantization, the zero-group skip (:189-191)
 *   orc_sgemm                 the reference's 6 sgemm tests and KATs, float64
 *                             rounding bound with numpy transposes
 *   orc_f16/bf16 conversions  exhaustive half widening, truncation
 *                             characterisation, torch RNE for bf16
 *   orc_qt_*                  the reference's quantize tests, an independent
 *                             numpy vectorisation, odd-group and Q4_0 KATs
 *   orc_flash_attention       float64 softmax attention bound, one-hot and
 *                             uniform cases, empty cache
 * Rotors are an input everywhere (RotorQuant::rotors is a pub field): the
 * reference's seeded Rotor::random draws from the rand crate's StdRng, which
 * is not in this image, so no function here restates that generator.
 *
 * Floating point: compiled with -ffp-contract=off and no fast-math, so every
 * `a*b + c` rounds twice exactly like Rust (which never contracts), divisions
 * are IEEE, roundf() is half-away-from-zero like f32::round, fmaxf() returns the
 * non-NaN operand like f32::max, and int32 accumulation wraps (release Rust).
 */
#ifndef RNN_ORACLE_H
#define RNN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic generators used by the reference's own tests ---- */

/* src/int8.rs:382-394 (lcg_bytes): s = s*1664525 + 1013904223, byte = s>>16;
 * unsigned draws are masked with 0x7f. */
void orc_lcg_bytes(uint32_t *seed, int8_t *out, size_t n, int is_signed);

/* ---- int8 GEMM (igemm contract: A u8 [m,k], B i8 [k,n] N-contiguous) ---- */

/* src/int8.rs:222-234 */
void orc_igemm_scalar(const uint8_t *a, const int8_t *b, int32_t *c,
                      size_t m, size_t k, size_t n);

/* src/int8.rs:285-314: AVX-512 VNNI path (B repacked per call, 4-row blocks
 * spread over `nthreads` workers); scalar fallback without VNNI.
 * Returns 1 when the VNNI path ran, 0 for the scalar fallback. */
int orc_igemm(const uint8_t *a, const int8_t *b, int32_t *c,
              size_t m, size_t k, size_t n, int nthreads);

/* ---- symmetric int8 quantization (per row of a row-major matrix) ---- */

/* src/int8.rs:33-45 (Int8Weights::quantize, per output channel) and
 * src/quantize.rs:296-311 (quantize_int8 with group_size = cols): the per-row
 * dynamic activation rule is the same expression applied to rows of X. */
void orc_quant_rows_i8(const float *x, size_t rows, size_t cols,
                       int8_t *q, float *scale);

/* src/int8.rs:55-65 */
void orc_int8_dequantize(const int8_t *q, const float *scale, size_t rows,
                         size_t cols, float *w);

/* src/int8.rs:70-88 (Int8Weights::matmul_f32; activation scaled by 1/scale) */
void orc_int8_matmul_f32(const int8_t *wq, const float *ws, size_t out_f,
                         size_t in_f, const float *x, size_t m, float *y);

/* src/int8.rs:134-172 (Int8Linear::forward, reference semantics: activation
 * re-quantized with the weight's channel scale inside the output loop). */
void orc_int8_linear_forward(const float *x, size_t batch, size_t in_f,
                             const int8_t *wq, const float *ws, size_t out_f,
                             const float *bias /* nullable */, float *y);

/* W8A8 composition: acc = sum_k a[m,k]*w[n,k] (wrapping
 * int32), y = ((float)acc * sa[m]) * sw[n] (+ bias[n]) (then max(y, 0) if relu).
 * acc_out (nullable) receives the raw int32 accumulators. The epilogue keeps the
 * reference's multiply-then-add order of src/int8.rs:159-162. */
void orc_w8a8_linear(const int8_t *aq, const float *sa, const int8_t *wq,
                     const float *sw, const float *bias, size_t m, size_t k,
                     size_t n, int relu, float *y, int32_t *acc_out);

/* src/tensor.rs:2025-2032 (x.max(0.0)) */
void orc_relu(float *x, size_t n);

/* ---- ternary ---- */

/* src/ternary.rs:46-60; packed has ceil(n/16) words. */
void orc_pack_ternary(const int8_t *v, size_t n, uint32_t *packed);
/* src/ternary.rs:63-75 */
void orc_unpack_ternary(const uint32_t *packed, size_t count, int8_t *out);

/* src/ternary.rs:97-137 (reference rule: per row delta = 0.7*mean|w|,
 * scale = max(mean|w|, 1e-8)). t receives the ternary values. */
void orc_ternary_quantize_rows(const float *w, size_t rows, size_t cols,
                               int8_t *t, float *scales);

/* Config rule (BitNet-b1.58 absmean, not in the reference): per-row sequential
 * f32 sums of |w| (the reference's own sum, src/ternary.rs:114), added in row
 * order in double; gamma = max((float)(total/numel), 1e-8);
 * t = clamp(round(w/gamma), -1, 1). Returns gamma. */
float orc_ternary_quantize_absmean(const float *w, size_t rows, size_t cols,
                                   int8_t *t);

/* src/ternary.rs:140-161 */
void orc_ternary_dequantize(const uint32_t *packed, size_t numel,
                            const float *scales, size_t n_scales, size_t cols,
                            float *w);

/* src/ternary.rs:239-279 (reference f32 shift-and-add, k order sequential). */
void orc_ternary_linear_f32(const float *x, size_t batch, size_t in_f,
                            const uint32_t *packed, const float *scales,
                            size_t out_f, const float *bias, float *y);

/* Config ternary GEMM: acc = sum_k a[m,k]*t[n,k] with t unpacked from the
 * 2-bit codes, epilogue as orc_w8a8_linear with sw[n] (= gamma broadcast). */
void orc_ternary_gemm_i8(const int8_t *aq, const float *sa,
                         const uint32_t *packed, const float *sw,
                         const float *bias, size_t m, size_t k, size_t n,
                         int relu, float *y, int32_t *acc_out);

/* ---- Cl(3,0) rotors and RotorQuant ---- */

/* src/quant.rs:84-89 and :92-96 on a multivector [1,e1,e2,e3,e12,e13,e23,e123]
 * with rotor r = {s, p12, p13, p23}. */
void orc_rotor_sandwich(const float r[4], const float x[8], float out[8]);
void orc_rotor_inv_sandwich(const float r[4], const float x[8], float out[8]);
/* src/quant.rs:101-113; row-major 3x3. */
void orc_rotor_rotation_matrix(const float r[4], float rot[9]);

/* src/quant.rs:212-239 with quantize_vec :170-208. x is [rows, dim]; rotors
 * holds ceil(dim/3) rotors of {s,p12,p13,p23}. y receives the reconstruction.
 * codes (nullable) receives [rows, padded_dim] int8 codes q, scales (nullable)
 * [rows, n_groups] per-group scales; a group skipped by the max_abs < 1e-12
 * rule (:189-191) gets codes 0 and scale 0 while y keeps its input values. */
void orc_rotorquant_quantize(const float *x, size_t rows, size_t dim, int bits,
                             const float *rotors, float *y, int8_t *codes,
                             float *scales);

/* Reconstruction from codes + scales: rv = q*scale, out = rot^T rv, the same
 * expressions as :195-202. Skipped groups (scale 0) reconstruct to 0. */
void orc_rotorquant_dequantize(const int8_t *codes, const float *scales,
                               size_t rows, size_t dim, const float *rotors,
                               float *y);

/* ---- f32 GEMM (BlasBackend contract) ---- */

/* src/blas.rs:104-190 (sgemm contract, scale_c :191-207) with the small-matrix
 * order of gemm_small (:214-264): per row i, C row *= beta (zeroed for beta
 * == 0), then for p in k order, skipping op(A)[i][p] == 0,
 * C[i][j] += (alpha*op(A)[i][p]) * op(B)[p][j], each product and sum rounded
 * separately. k == 0 or alpha == 0 gives C = beta*C. The reference's blocked
 * path (m*n*k >= 4096) sums in another order, so its results differ from this
 * one by rounding only. transa/transb: 0 = as stored, 1 = transposed. */
void orc_sgemm(int transa, int transb, size_t m, size_t n, size_t k, float alpha,
               const float *a, size_t lda, const float *b, size_t ldb, float beta,
               float *c, size_t ldc);

/* ---- QuantizedTensor formats (src/quantize.rs) ---- */

/* QuantFormat (src/quantize.rs:37-56), in the reference's declaration order. */
enum {
    ORC_QF_FP16 = 0, ORC_QF_BF16 = 1, ORC_QF_INT8 = 2, ORC_QF_INT4 = 3,
    ORC_QF_NF4 = 4, ORC_QF_NVFP4 = 5, ORC_QF_GGUF_Q4 = 6, ORC_QF_GGUF_Q4K = 7,
    ORC_QF_GGUF_Q8 = 8
};

/* Half/bfloat conversions of src/quantize.rs:639-708 (f32_to_f16 truncates;
 * f32_to_bf16 adds with wrap-around as release Rust does). */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t b);
/* The same over arrays (bit patterns, signalling NaNs included, kept as is). */
void orc_f32_to_f16_array(const float *x, size_t n, uint16_t *h);
void orc_f16_to_f32_array(const uint16_t *h, size_t n, float *x);
void orc_f32_to_bf16_array(const float *x, size_t n, uint16_t *h);
void orc_bf16_to_f32_array(const uint16_t *h, size_t n, float *x);

/* Bytes of QuantizedTensor::data for n elements; *n_scales and
 * *stored_group receive scales.len() and the group_size field
 * (src/quantize.rs:231-250, :515, :558). */
size_t orc_qt_layout(int fmt, size_t n, size_t group_size, size_t *n_scales,
                     size_t *stored_group);

/* QuantizedTensor::quantize (src/quantize.rs:231-250 and :296-625). */
void orc_qt_quantize(int fmt, const float *x, size_t n, size_t group_size,
                     uint8_t *data, float *scales);

/* QuantizedTensor::dequantize (src/quantize.rs:252-269 and :324-632); group is
 * the stored group_size field. */
void orc_qt_dequantize(int fmt, const uint8_t *data, const float *scales,
                       size_t n_scales, size_t group, size_t n, float *out);

/* QuantizedLinear::forward (src/quantize.rs:744-754): dequantize, x.W^T with
 * orc_sgemm's order, then + bias (may be NULL). */
void orc_qt_linear_forward(int fmt, const float *x, size_t m, size_t in_f,
                           const uint8_t *data, const float *scales, size_t n_scales,
                           size_t group, size_t out_f, const float *bias, float *y);

/* ---- attention (src/tensor.rs:618-672) ---- */

/* Tensor::flash_attention: out[b,i] = softmax_j(scale * q[b,i].k[b,j]) . v[b,j]
 * by the reference's sequential online softmax (expf, no contraction). q is
 * [batch, nq, dim], k and v [batch, skv, dim]; nq == skv is the reference's
 * own signature, nq = 1 a decode step over a cache of skv keys. */
void orc_flash_attention(const float *q, const float *k, const float *v, size_t batch,
                         size_t nq, size_t skv, size_t dim, float scale, float *out);

#ifdef __cplusplus
}
#endif
#endif
