/*
 * oracle.c -- CPU restatement of rust-nn's quantized-inference path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and timed CPU baseline); see
 * oracle.h for the contract, the floating-point rules and what pins each
 * function. Built by oracle/Makefile with -ffp-contract=off.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* Rust `f32 as i8` after clamp: NaN -> 0, values already in range. */
static inline int8_t f32_to_i8_sat(float v) {
    if (v != v) return 0;
    if (v <= -128.0f) return -128;
    if (v >= 127.0f) return 127;
    return (int8_t)v;
}

/* Rust f32::clamp(lo, hi): NaN passes through. */
static inline float clampf_rs(float x, float lo, float hi) {
    if (x < lo) return lo;
    if (x > hi) return hi;
    return x;
}

/* ------------------------------------------------------------------ */
/* src/int8.rs:382-394                                                  */
/* ------------------------------------------------------------------ */
void orc_lcg_bytes(uint32_t *seed, int8_t *out, size_t n, int is_signed) {
    uint32_t s = *seed;
    for (size_t i = 0; i < n; ++i) {
        s = s * 1664525u + 1013904223u;
        uint8_t b = (uint8_t)(s >> 16);
        out[i] = is_signed ? (int8_t)b : (int8_t)(b & 0x7f);
    }
    *seed = s;
}

/* ------------------------------------------------------------------ */
/* src/int8.rs:222-234  igemm_scalar (wrapping int32)                   */
/* ------------------------------------------------------------------ */
void orc_igemm_scalar(const uint8_t *a, const int8_t *b, int32_t *c,
                      size_t m, size_t k, size_t n) {
    for (size_t i = 0; i < m; ++i) {
        for (size_t j = 0; j < n; ++j) {
            uint32_t s = 0;
            for (size_t p = 0; p < k; ++p)
                s += (uint32_t)((int32_t)a[i * k + p] * (int32_t)b[p * n + j]);
            c[i * n + j] = (int32_t)s;
        }
    }
}

/* ------------------------------------------------------------------ */
/* src/int8.rs:195-314  igemm: VNNI repack of B + 4-row blocks          */
/* ------------------------------------------------------------------ */
#if defined(__x86_64__)
/* B [k,n] -> tiles of (4 k x 16 n): tile (kq, nb) is 64 bytes, lane l holds
 * b[4kq+0..3, 16nb+l] little-endian (the vpdpbusd operand order), zero padded
 * to kp x np. Same layout as src/int8.rs:191-218. */
static uint8_t *vnni_pack_b(const int8_t *b, size_t k, size_t n, size_t kp,
                            size_t np) {
    size_t nblk = np / 16;
    uint8_t *out = (uint8_t *)calloc((kp / 4) * nblk * 64, 1);
    for (size_t kq = 0; kq < kp / 4; ++kq)
        for (size_t nb = 0; nb < nblk; ++nb) {
            uint8_t *tile = out + (kq * nblk + nb) * 64;
            for (size_t l = 0; l < 16; ++l) {
                size_t col = nb * 16 + l;
                for (size_t j = 0; j < 4; ++j) {
                    size_t row = kq * 4 + j;
                    tile[l * 4 + j] =
                        (row < k && col < n) ? (uint8_t)b[row * n + col] : 0;
                }
            }
        }
    return out;
}

/* One block of up to 4 rows starting at row0: acc[r][16] per 16-column
 * block, accumulated with vpdpbusd over the packed K. */
__attribute__((target("avx512f,avx512bw,avx512vnni")))
static void vnni_rows4(const uint8_t *apad, const uint8_t *bpack, int32_t *crow,
                       size_t row0, size_t nrows, size_t kp, size_t np) {
    size_t nblk = np / 16;
    for (size_t nb = 0; nb < nblk; ++nb) {
        __m512i acc0 = _mm512_setzero_si512(), acc1 = acc0, acc2 = acc0,
                acc3 = acc0;
        const uint8_t *bt = bpack + nb * 64;
        const uint8_t *a0 = apad + (row0 + 0) * kp;
        const uint8_t *a1 = apad + (row0 + 1) * kp;
        const uint8_t *a2 = apad + (row0 + 2) * kp;
        const uint8_t *a3 = apad + (row0 + 3) * kp;
        for (size_t kq = 0; kq < kp / 4; ++kq) {
            __m512i bv = _mm512_loadu_si512((const void *)(bt + kq * nblk * 64));
            int32_t w0, w1, w2, w3;
            memcpy(&w0, a0 + 4 * kq, 4);
            memcpy(&w1, a1 + 4 * kq, 4);
            memcpy(&w2, a2 + 4 * kq, 4);
            memcpy(&w3, a3 + 4 * kq, 4);
            acc0 = _mm512_dpbusd_epi32(acc0, _mm512_set1_epi32(w0), bv);
            acc1 = _mm512_dpbusd_epi32(acc1, _mm512_set1_epi32(w1), bv);
            acc2 = _mm512_dpbusd_epi32(acc2, _mm512_set1_epi32(w2), bv);
            acc3 = _mm512_dpbusd_epi32(acc3, _mm512_set1_epi32(w3), bv);
        }
        __m512i accs[4] = {acc0, acc1, acc2, acc3};
        for (size_t r = 0; r < nrows; ++r)
            _mm512_storeu_si512((void *)(crow + r * np + nb * 16), accs[r]);
    }
}

struct vnni_job {
    const uint8_t *apad, *bpack;
    int32_t *ctmp;
    size_t m, kp, np, nblocks;
    atomic_size_t next;
};

static void *vnni_worker(void *arg) {
    struct vnni_job *j = (struct vnni_job *)arg;
    for (;;) {
        size_t blk = atomic_fetch_add(&j->next, 1);
        if (blk >= j->nblocks) break;
        size_t row0 = blk * 4;
        size_t nrows = j->m - row0 < 4 ? j->m - row0 : 4;
        vnni_rows4(j->apad, j->bpack, j->ctmp + row0 * j->np, row0, nrows,
                   j->kp, j->np);
    }
    return NULL;
}
#endif

int orc_igemm(const uint8_t *a, const int8_t *b, int32_t *c, size_t m,
              size_t k, size_t n, int nthreads) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512vnni") && m > 0 && n > 0) {
        size_t kp = (k + 3) & ~(size_t)3, np = (n + 15) & ~(size_t)15,
               mp = (m + 3) & ~(size_t)3;
        uint8_t *apad = (uint8_t *)calloc((mp * kp) > 0 ? (mp * kp) : 1, 1);
        for (size_t i = 0; i < m; ++i) memcpy(apad + i * kp, a + i * k, k);
        uint8_t *bpack = vnni_pack_b(b, k, n, kp ? kp : 4, np);
        int32_t *ctmp = (int32_t *)malloc(m * np * sizeof(int32_t));
        struct vnni_job job = {apad, bpack, ctmp, m, kp, np, (m + 3) / 4, 0};
        if (kp == 0) {
            memset(ctmp, 0, m * np * sizeof(int32_t));
        } else {
            int nt = nthreads < 1 ? 1 : nthreads;
            if ((size_t)nt > job.nblocks) nt = (int)job.nblocks;
            pthread_t th[256];
            if (nt > 256) nt = 256;
            for (int t = 1; t < nt; ++t)
                pthread_create(&th[t], NULL, vnni_worker, &job);
            vnni_worker(&job);
            for (int t = 1; t < nt; ++t) pthread_join(th[t], NULL);
        }
        for (size_t i = 0; i < m; ++i)
            memcpy(c + i * n, ctmp + i * np, n * sizeof(int32_t));
        free(apad);
        free(bpack);
        free(ctmp);
        return 1;
    }
#endif
    (void)nthreads;
    orc_igemm_scalar(a, b, c, m, k, n);
    return 0;
}

/* ------------------------------------------------------------------ */
/* src/int8.rs:33-45, src/quantize.rs:296-311  per-row symmetric int8   */
/* ------------------------------------------------------------------ */
void orc_quant_rows_i8(const float *x, size_t rows, size_t cols, int8_t *q,
                       float *scale) {
    for (size_t r = 0; r < rows; ++r) {
        const float *row = x + r * cols;
        float max_abs = 0.0f;
        for (size_t j = 0; j < cols; ++j) max_abs = fmaxf(max_abs, fabsf(row[j]));
        float s = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
        scale[r] = s;
        for (size_t j = 0; j < cols; ++j)
            q[r * cols + j] = f32_to_i8_sat(clampf_rs(roundf(row[j] / s), -128.0f, 127.0f));
    }
}

/* src/int8.rs:55-65 */
void orc_int8_dequantize(const int8_t *q, const float *scale, size_t rows,
                         size_t cols, float *w) {
    for (size_t i = 0; i < rows; ++i)
        for (size_t j = 0; j < cols; ++j)
            w[i * cols + j] = (float)q[i * cols + j] * scale[i];
}

/* src/int8.rs:70-88 */
void orc_int8_matmul_f32(const int8_t *wq, const float *ws, size_t out_f,
                         size_t in_f, const float *x, size_t m, float *y) {
    for (size_t row = 0; row < m; ++row)
        for (size_t col = 0; col < out_f; ++col) {
            uint32_t acc = 0;
            for (size_t p = 0; p < in_f; ++p) {
                float inv = 1.0f / ws[col];
                int8_t av = f32_to_i8_sat(
                    clampf_rs(roundf(x[row * in_f + p] * inv), -128.0f, 127.0f));
                acc += (uint32_t)((int32_t)av * (int32_t)wq[col * in_f + p]);
            }
            y[row * out_f + col] = (float)(int32_t)acc * ws[col] * ws[col];
        }
}

/* src/int8.rs:134-172 */
void orc_int8_linear_forward(const float *x, size_t batch, size_t in_f,
                             const int8_t *wq, const float *ws, size_t out_f,
                             const float *bias, float *y) {
    for (size_t b = 0; b < batch; ++b)
        for (size_t o = 0; o < out_f; ++o) {
            uint32_t acc = 0;
            float s = ws[o];
            for (size_t p = 0; p < in_f; ++p) {
                int8_t aq = f32_to_i8_sat(
                    clampf_rs(roundf(x[b * in_f + p] / s), -128.0f, 127.0f));
                acc += (uint32_t)((int32_t)aq * (int32_t)wq[o * in_f + p]);
            }
            float v = (float)(int32_t)acc * s * s;
            if (bias) v = v + bias[o];
            y[b * out_f + o] = v;
        }
}

/* W8A8 composition; epilogue order of src/int8.rs:159-162. */
void orc_w8a8_linear(const int8_t *aq, const float *sa, const int8_t *wq,
                     const float *sw, const float *bias, size_t m, size_t k,
                     size_t n, int relu, float *y, int32_t *acc_out) {
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) {
            uint32_t acc = 0;
            const int8_t *ar = aq + i * k, *wr = wq + j * k;
            for (size_t p = 0; p < k; ++p)
                acc += (uint32_t)((int32_t)ar[p] * (int32_t)wr[p]);
            if (acc_out) acc_out[i * n + j] = (int32_t)acc;
            float v = (float)(int32_t)acc * sa[i] * sw[j];
            if (bias) v = v + bias[j];
            if (relu) v = fmaxf(v, 0.0f);
            y[i * n + j] = v;
        }
}

/* src/tensor.rs:2025-2032 */
void orc_relu(float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = fmaxf(x[i], 0.0f);
}

/* ------------------------------------------------------------------ */
/* src/ternary.rs:46-75  2-bit packing, 16 codes per u32, LSB first     */
/* ------------------------------------------------------------------ */
void orc_pack_ternary(const int8_t *v, size_t n, uint32_t *packed) {
    memset(packed, 0, ((n + 15) / 16) * sizeof(uint32_t));
    for (size_t i = 0; i < n; ++i) {
        uint32_t code = v[i] == 0 ? 0u : (v[i] > 0 ? 1u : 2u);
        packed[i / 16] |= code << ((i % 16) * 2);
    }
}

void orc_unpack_ternary(const uint32_t *packed, size_t count, int8_t *out) {
    for (size_t i = 0; i < count; ++i) {
        uint32_t code = (packed[i / 16] >> ((i % 16) * 2)) & 3u;
        out[i] = code == 1 ? 1 : (code == 2 ? -1 : 0);
    }
}

/* src/ternary.rs:97-137 */
void orc_ternary_quantize_rows(const float *w, size_t rows, size_t cols,
                               int8_t *t, float *scales) {
    for (size_t r = 0; r < rows; ++r) {
        const float *row = w + r * cols;
        float sum = 0.0f;
        for (size_t j = 0; j < cols; ++j) sum = sum + fabsf(row[j]);
        float mean_abs = sum / (float)(cols > 0 ? cols : 1);
        float threshold = 0.7f * mean_abs;
        scales[r] = fmaxf(mean_abs, 1e-8f);
        for (size_t j = 0; j < cols; ++j) {
            float v = row[j];
            t[r * cols + j] = fabsf(v) < threshold ? 0 : (v > 0.0f ? 1 : -1);
        }
    }
}

float orc_ternary_quantize_absmean(const float *w, size_t rows, size_t cols,
                                   int8_t *t) {
    double total = 0.0;
    for (size_t r = 0; r < rows; ++r) {
        float sum = 0.0f;
        for (size_t j = 0; j < cols; ++j) sum = sum + fabsf(w[r * cols + j]);
        total = total + (double)sum;
    }
    size_t numel = rows * cols;
    float gamma = (float)(total / (double)(numel > 0 ? numel : 1));
    gamma = fmaxf(gamma, 1e-8f);
    for (size_t i = 0; i < numel; ++i)
        t[i] = f32_to_i8_sat(clampf_rs(roundf(w[i] / gamma), -1.0f, 1.0f));
    return gamma;
}

/* src/ternary.rs:140-161 */
void orc_ternary_dequantize(const uint32_t *packed, size_t numel,
                            const float *scales, size_t n_scales, size_t cols,
                            float *w) {
    for (size_t i = 0; i < numel; ++i) {
        uint32_t code = (packed[i / 16] >> ((i % 16) * 2)) & 3u;
        int tv = code == 1 ? 1 : (code == 2 ? -1 : 0);
        size_t r = i / cols;
        if (r > n_scales - 1) r = n_scales - 1;
        w[i] = (float)tv * scales[r];
    }
}

/* src/ternary.rs:239-279 */
void orc_ternary_linear_f32(const float *x, size_t batch, size_t in_f,
                            const uint32_t *packed, const float *scales,
                            size_t out_f, const float *bias, float *y) {
    for (size_t b = 0; b < batch; ++b)
        for (size_t o = 0; o < out_f; ++o) {
            float acc = 0.0f;
            for (size_t i = 0; i < in_f; ++i) {
                size_t idx = o * in_f + i;
                uint32_t code = (packed[idx / 16] >> ((idx % 16) * 2)) & 3u;
                float xv = x[b * in_f + i];
                if (code == 1) acc = acc + xv;
                else if (code == 2) acc = acc - xv;
            }
            float v = acc * scales[o];
            if (bias) v = v + bias[o];
            y[b * out_f + o] = v;
        }
}

void orc_ternary_gemm_i8(const int8_t *aq, const float *sa,
                         const uint32_t *packed, const float *sw,
                         const float *bias, size_t m, size_t k, size_t n,
                         int relu, float *y, int32_t *acc_out) {
    int8_t *wt = (int8_t *)malloc((n * k) > 0 ? (n * k) : 1);
    orc_unpack_ternary(packed, n * k, wt);
    orc_w8a8_linear(aq, sa, wt, sw, bias, m, k, n, relu, y, acc_out);
    free(wt);
}

/* ------------------------------------------------------------------ */
/* src/quant.rs:70-113  Cl(3,0) rotor sandwich                          */
/* ------------------------------------------------------------------ */
/* Sparse geometric product rotor*x for rotor (s,p12,p13,p23); multivector
 * layout [1,e1,e2,e3,e12,e13,e23,e123] (src/quant.rs:23-24, :70-81). */
static void rotor_apply(const float x[8], float s, float p12, float p13,
                        float p23, float o[8]) {
    o[0] = s * x[0] - p12 * x[4] - p13 * x[5] - p23 * x[6];
    o[1] = s * x[1] + p12 * x[2] + p13 * x[3] + p23 * x[7];
    o[2] = s * x[2] - p12 * x[1] + p23 * x[3] - p13 * x[7];
    o[3] = s * x[3] - p13 * x[1] - p23 * x[2] + p12 * x[7];
    o[4] = s * x[4] + p12 * x[0];
    o[5] = s * x[5] + p13 * x[0];
    o[6] = s * x[6] + p23 * x[0];
    o[7] = s * x[7] - p23 * x[1] + p13 * x[2] - p12 * x[3];
}

void orc_rotor_sandwich(const float r[4], const float x[8], float out[8]) {
    float t[8];
    rotor_apply(x, r[0], r[1], r[2], r[3], t);
    rotor_apply(t, r[0], -r[1], -r[2], -r[3], out);
}

void orc_rotor_inv_sandwich(const float r[4], const float x[8], float out[8]) {
    float t[8];
    rotor_apply(x, r[0], -r[1], -r[2], -r[3], t);
    rotor_apply(t, r[0], r[1], r[2], r[3], out);
}

void orc_rotor_rotation_matrix(const float r[4], float rot[9]) {
    float e[3][8], img[3][8];
    memset(e, 0, sizeof e);
    e[0][1] = 1.0f;
    e[1][2] = 1.0f;
    e[2][3] = 1.0f;
    for (int j = 0; j < 3; ++j) orc_rotor_sandwich(r, e[j], img[j]);
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) rot[i * 3 + j] = img[j][1 + i];
}

/* ------------------------------------------------------------------ */
/* src/quant.rs:164-239  RotorQuant                                     */
/* ------------------------------------------------------------------ */
void orc_rotorquant_quantize(const float *x, size_t rows, size_t dim, int bits,
                             const float *rotors, float *y, int8_t *codes,
                             float *scales) {
    size_t padded = (dim + 2) / 3 * 3, ng = padded / 3;
    float qmax = (float)((1u << (bits - 1)) - 1u);
    float *rot = (float *)malloc((ng ? ng : 1) * 9 * sizeof(float));
    for (size_t g = 0; g < ng; ++g) orc_rotor_rotation_matrix(rotors + 4 * g, rot + 9 * g);
    float *row = (float *)malloc((padded ? padded : 1) * sizeof(float));
    for (size_t r = 0; r < rows; ++r) {
        for (size_t t = 0; t < padded; ++t) row[t] = t < dim ? x[r * dim + t] : 0.0f;
        for (size_t g = 0; g < ng; ++g) {
            const float *R = rot + 9 * g;
            float v0 = row[3 * g], v1 = row[3 * g + 1], v2 = row[3 * g + 2];
            float rv[3] = {R[0] * v0 + R[1] * v1 + R[2] * v2,
                           R[3] * v0 + R[4] * v1 + R[5] * v2,
                           R[6] * v0 + R[7] * v1 + R[8] * v2};
            float max_abs = 0.0f;
            for (int i = 0; i < 3; ++i) max_abs = fmaxf(max_abs, fabsf(rv[i]));
            if (max_abs < 1e-12f) {
                if (codes) codes[r * padded + 3 * g] = codes[r * padded + 3 * g + 1] =
                               codes[r * padded + 3 * g + 2] = 0;
                if (scales) scales[r * ng + g] = 0.0f;
                continue;
            }
            float scale = max_abs / qmax;
            for (int i = 0; i < 3; ++i) {
                float q = clampf_rs(roundf(rv[i] / scale), -qmax, qmax);
                if (codes) codes[r * padded + 3 * g + i] = f32_to_i8_sat(q);
                rv[i] = q * scale;
            }
            if (scales) scales[r * ng + g] = scale;
            row[3 * g] = R[0] * rv[0] + R[3] * rv[1] + R[6] * rv[2];
            row[3 * g + 1] = R[1] * rv[0] + R[4] * rv[1] + R[7] * rv[2];
            row[3 * g + 2] = R[2] * rv[0] + R[5] * rv[1] + R[8] * rv[2];
        }
        for (size_t t = 0; t < dim; ++t) y[r * dim + t] = row[t];
    }
    free(row);
    free(rot);
}

void orc_rotorquant_dequantize(const int8_t *codes, const float *scales,
                               size_t rows, size_t dim, const float *rotors,
                               float *y) {
    size_t padded = (dim + 2) / 3 * 3, ng = padded / 3;
    float *rot = (float *)malloc((ng ? ng : 1) * 9 * sizeof(float));
    for (size_t g = 0; g < ng; ++g) orc_rotor_rotation_matrix(rotors + 4 * g, rot + 9 * g);
    float *row = (float *)malloc((padded ? padded : 1) * sizeof(float));
    for (size_t r = 0; r < rows; ++r) {
        for (size_t g = 0; g < ng; ++g) {
            const float *R = rot + 9 * g;
            float s = scales[r * ng + g];
            const int8_t *q = codes + r * padded + 3 * g;
            float rv[3] = {(float)q[0] * s, (float)q[1] * s, (float)q[2] * s};
            row[3 * g] = R[0] * rv[0] + R[3] * rv[1] + R[6] * rv[2];
            row[3 * g + 1] = R[1] * rv[0] + R[4] * rv[1] + R[7] * rv[2];
            row[3 * g + 2] = R[2] * rv[0] + R[5] * rv[1] + R[8] * rv[2];
        }
        for (size_t t = 0; t < dim; ++t) y[r * dim + t] = row[t];
    }
    free(row);
    free(rot);
}

/* ------------------------------------------------------------------ */
/* src/blas.rs:104-264 (sgemm contract, gemm_small order)              */
/* ------------------------------------------------------------------ */
void orc_sgemm(int transa, int transb, size_t m, size_t n, size_t k, float alpha,
               const float *a, size_t lda, const float *b, size_t ldb, float beta,
               float *c, size_t ldc) {
    if (m == 0 || n == 0) return;
    for (size_t i = 0; i < m; ++i) {
        float *crow = c + i * ldc;
        if (beta == 0.0f) {
            for (size_t j = 0; j < n; ++j) crow[j] = 0.0f;
        } else if (beta != 1.0f) {
            for (size_t j = 0; j < n; ++j) crow[j] *= beta;
        }
        if (k == 0 || alpha == 0.0f) continue;
        for (size_t p = 0; p < k; ++p) {
            const float av = transa ? a[p * lda + i] : a[i * lda + p];
            if (av == 0.0f) continue;
            const float aav = alpha * av;
            for (size_t j = 0; j < n; ++j) {
                const float bv = transb ? b[j * ldb + p] : b[p * ldb + j];
                crow[j] += aav * bv;
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* src/quantize.rs: QuantizedTensor (multi-format weight quantization)  */
/* ------------------------------------------------------------------ */

/* src/quantize.rs:96-114 */
static const float NF4_LUT[16] = {
    -1.0f, -0.6961928f, -0.52507305f, -0.3949175f, -0.28444138f, -0.18477343f,
    -0.091050036f, 0.0f, 0.0795803f, 0.1609302f, 0.2461123f, 0.33791524f,
    0.44070983f, 0.562617f, 0.72295684f, 1.0f};
/* src/quantize.rs:138-144 (index 8 is -0.0) */
static const float NVFP4_LUT[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,
                                    4.0f,  6.0f,  -0.0f, -0.5f, -1.0f, -1.5f,
                                    -2.0f, -3.0f, -4.0f, -6.0f};

/* src/quantize.rs:117-129: first index of the strictly smallest |v - x|. */
static uint8_t nf4_index(float x) {
    uint8_t best = 0;
    float best_d = INFINITY;
    for (int i = 0; i < 16; ++i) {
        float d = fabsf(NF4_LUT[i] - x);
        if (d < best_d) { best_d = d; best = (uint8_t)i; }
    }
    return best;
}

/* src/quantize.rs:146-161 */
static uint8_t nvfp4_index(float x) {
    static const float mags[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    float ax = fabsf(x);
    uint8_t sign = x < 0.0f ? 8 : 0;
    uint8_t best = 0;
    float best_d = INFINITY;
    for (int i = 0; i < 8; ++i) {
        float d = fabsf(mags[i] - ax);
        if (d < best_d) { best_d = d; best = (uint8_t)i; }
    }
    return sign | best;
}

/* src/quantize.rs:639-666 (truncating; release-mode integer semantics) */
uint16_t orc_f32_to_f16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 0xFF) return sign | 0x7C00u | (mant != 0 ? 0x200u : 0u);
    int32_t new_exp = exp - 127 + 15;
    if (new_exp >= 31) return sign | 0x7C00u;
    if (new_exp <= 0) {
        if (14 - new_exp >= 24) return sign;
        uint32_t m = mant | 0x800000u;
        uint32_t shift = (uint32_t)(14 - new_exp);
        return sign | (uint16_t)(m >> shift);
    }
    return sign | (uint16_t)((uint32_t)new_exp << 10) | (uint16_t)(mant >> 13);
}

/* src/quantize.rs:668-695. The subnormal loop decrements an unsigned
 * exponent below zero for mantissas under 0x200; release Rust wraps, and the
 * `as i32` then gives the intended negative value, so this follows the
 * release arithmetic (debug builds would panic on that overflow). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t mant = (uint32_t)h & 0x3FFu;
    uint32_t val;
    if (exp == 0) {
        if (mant == 0) {
            val = sign;
        } else {
            uint32_t e = 1, m = mant;
            while ((m & 0x400u) == 0) { m <<= 1; e -= 1; }
            m &= 0x3FFu;
            val = sign | ((uint32_t)(127 - 15 + (int32_t)e) << 23) | (m << 13);
        }
    } else if (exp == 31) {
        val = sign | 0x7F800000u | (mant << 13);
    } else {
        val = sign | ((exp + 112) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &val, 4);
    return f;
}

/* src/quantize.rs:697-703: bits + ((bits>>16)&1) + 0x7FFF, wrapping (release). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint32_t r = bits + ((bits >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)(r >> 16);
}

/* src/quantize.rs:705-708 */
float orc_bf16_to_f32(uint16_t b) {
    uint32_t v = (uint32_t)b << 16;
    float f;
    memcpy(&f, &v, 4);
    return f;
}

/* Array forms (the results stay bit patterns in memory; a float returned by
 * value through a foreign-function layer may have its signalling NaNs
 * quieted on the way). */
void orc_f32_to_f16_array(const float *x, size_t n, uint16_t *h) {
    for (size_t i = 0; i < n; ++i) h[i] = orc_f32_to_f16(x[i]);
}
void orc_f16_to_f32_array(const uint16_t *h, size_t n, float *x) {
    for (size_t i = 0; i < n; ++i) x[i] = orc_f16_to_f32(h[i]);
}
void orc_f32_to_bf16_array(const float *x, size_t n, uint16_t *h) {
    for (size_t i = 0; i < n; ++i) h[i] = orc_f32_to_bf16(x[i]);
}
void orc_bf16_to_f32_array(const uint16_t *h, size_t n, float *x) {
    for (size_t i = 0; i < n; ++i) x[i] = orc_bf16_to_f32(h[i]);
}

static int qf_is4(int fmt) {
    return fmt == ORC_QF_INT4 || fmt == ORC_QF_NF4 || fmt == ORC_QF_NVFP4 ||
           fmt == ORC_QF_GGUF_Q4 || fmt == ORC_QF_GGUF_Q4K;
}

/* Storage of QuantizedTensor::quantize (src/quantize.rs:231-250): the group
 * (or GGUF block, min(group,32), :515/:558) every format uses, with
 * group_size 0 meaning the whole tensor (:235). */
size_t orc_qt_layout(int fmt, size_t n, size_t group_size, size_t *n_scales,
                     size_t *stored_group) {
    if (fmt == ORC_QF_FP16 || fmt == ORC_QF_BF16) {
        *n_scales = 0;
        *stored_group = 0;
        return 2 * n;
    }
    size_t g = group_size == 0 ? n : group_size;
    if (fmt == ORC_QF_GGUF_Q4 || fmt == ORC_QF_GGUF_Q4K || fmt == ORC_QF_GGUF_Q8)
        g = g < 32 ? g : 32;
    *stored_group = g;
    if (g == 0) { *n_scales = 0; return 0; }
    size_t ng = (n + g - 1) / g;
    *n_scales = ng;
    if (!qf_is4(fmt)) return n;
    if (ng == 0) return 0;
    size_t last = n - (ng - 1) * g;
    return (ng - 1) * ((g + 1) / 2) + (last + 1) / 2;
}

/* src/quantize.rs:296-322 (INT8), :334-375 (INT4), :398-438 (NF4),
 * :456-496 (NVFP4), :514-536 with :171-190 (GGUF Q4_0), :556-583 (GGUF Q8_0),
 * :589-602 (FP16), :612-625 (BF16). 4-bit formats pack each group on its own
 * (low nibble first, a zero high nibble after an odd count). */
void orc_qt_quantize(int fmt, const float *x, size_t n, size_t group_size,
                     uint8_t *data, float *scales) {
    if (fmt == ORC_QF_FP16 || fmt == ORC_QF_BF16) {
        for (size_t i = 0; i < n; ++i) {
            uint16_t h = fmt == ORC_QF_FP16 ? orc_f32_to_f16(x[i]) : orc_f32_to_bf16(x[i]);
            data[2 * i] = (uint8_t)(h & 0xFF);
            data[2 * i + 1] = (uint8_t)(h >> 8);
        }
        return;
    }
    size_t ns, g;
    orc_qt_layout(fmt, n, group_size, &ns, &g);
    size_t off = 0;
    for (size_t gi = 0; gi < ns; ++gi) {
        size_t start = gi * g, end = start + g < n ? start + g : n;
        float max_abs = 0.0f;
        for (size_t i = start; i < end; ++i) max_abs = fmaxf(max_abs, fabsf(x[i]));
        float s;
        switch (fmt) {
        case ORC_QF_INT8: case ORC_QF_GGUF_Q8:
            s = max_abs > 0.0f ? max_abs / 127.0f : 1.0f; break;
        case ORC_QF_INT4: s = max_abs > 0.0f ? max_abs / 7.0f : 1.0f; break;
        case ORC_QF_NF4: s = max_abs > 0.0f ? max_abs : 1.0f; break;
        case ORC_QF_NVFP4: s = max_abs > 0.0f ? max_abs / 6.0f : 1.0f; break;
        default: /* GGUF Q4_0, :174-176 */
            s = max_abs / -8.0f;
            if (s == 0.0f) s = 1.0f;
            break;
        }
        scales[gi] = s;
        if (!qf_is4(fmt)) {
            for (size_t i = start; i < end; ++i)
                data[i] = (uint8_t)f32_to_i8_sat(clampf_rs(roundf(x[i] / s), -128.0f, 127.0f));
            continue;
        }
        for (size_t i = start; i < end; i += 2) {
            uint8_t c[2] = {0, 0};
            for (size_t t = 0; t < 2 && i + t < end; ++t) {
                float v = x[i + t] / s;
                switch (fmt) {
                case ORC_QF_NF4: c[t] = nf4_index(v); break;
                case ORC_QF_NVFP4: c[t] = nvfp4_index(v); break;
                default: /* INT4 and Q4_0: round, clamp to [-8,7], low 4 bits */
                    c[t] = (uint8_t)f32_to_i8_sat(clampf_rs(roundf(v), -8.0f, 7.0f)) & 0xF;
                    break;
                }
            }
            data[off++] = (uint8_t)(c[0] | (c[1] << 4));
        }
    }
}

static float nib_signed(uint8_t nib) { return (float)((nib & 0x8) ? (int)nib - 16 : (int)nib); }

/* src/quantize.rs:252-269 and the per-format dequantizers :324-332 (INT8,
 * GGUF Q8_0 :585-587), :377-396 (INT4), :440-454 (NF4), :498-512 (NVFP4),
 * :538-554 with :192-211 (GGUF Q4_0), :604-610 (FP16), :627-632 (BF16).
 * INT4/NF4/NVFP4 index bytes as data[i/2] over the whole tensor and scales as
 * scales[min(i/group, n_scales-1)] (:326, :380, :442, :500), exactly as the
 * reference does; GGUF Q4_0 walks its blocks with a running byte offset. */
void orc_qt_dequantize(int fmt, const uint8_t *data, const float *scales,
                       size_t n_scales, size_t group, size_t n, float *out) {
    if (fmt == ORC_QF_FP16 || fmt == ORC_QF_BF16) {
        for (size_t i = 0; i < n; ++i) {
            uint16_t h = (uint16_t)(data[2 * i] | (data[2 * i + 1] << 8));
            out[i] = fmt == ORC_QF_FP16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
        }
        return;
    }
    if (fmt == ORC_QF_GGUF_Q4 || fmt == ORC_QF_GGUF_Q4K) {
        size_t off = 0;
        for (size_t b = 0; b * group < n; ++b) {
            size_t start = b * group, end = start + group < n ? start + group : n;
            float s = scales[b];
            for (size_t i = 0; i < end - start; ++i) {
                uint8_t byte = data[off + i / 2];
                uint8_t nib = (i % 2 == 0) ? (byte & 0xF) : ((byte >> 4) & 0xF);
                out[start + i] = nib_signed(nib) * s;
            }
            off += (end - start + 1) / 2;
        }
        return;
    }
    if (n_scales == 0 || group == 0) return; /* the reference panics here */
    for (size_t i = 0; i < n; ++i) {
        size_t gi = i / group;
        float s = scales[gi < n_scales - 1 ? gi : n_scales - 1];
        if (fmt == ORC_QF_INT8 || fmt == ORC_QF_GGUF_Q8) {
            out[i] = (float)(int8_t)data[i] * s;
            continue;
        }
        uint8_t byte = data[i / 2];
        uint8_t nib = (i % 2 == 0) ? (byte & 0xF) : ((byte >> 4) & 0xF);
        if (fmt == ORC_QF_INT4) out[i] = nib_signed(nib) * s;
        else if (fmt == ORC_QF_NF4) out[i] = NF4_LUT[nib] * s;
        else out[i] = NVFP4_LUT[nib] * s;
    }
}

/* QuantizedLinear::forward (src/quantize.rs:744-754): W = dequantize()
 * [out_f, in_f], y = x.matmul(W^T) (blas sgemm, restated by orc_sgemm), then
 * y + bias broadcast over rows. */
void orc_qt_linear_forward(int fmt, const float *x, size_t m, size_t in_f,
                           const uint8_t *data, const float *scales, size_t n_scales,
                           size_t group, size_t out_f, const float *bias, float *y) {
    size_t nw = out_f * in_f;
    float *w = (float *)malloc(sizeof(float) * (nw > 0 ? nw : 1));
    orc_qt_dequantize(fmt, data, scales, n_scales, group, out_f * in_f, w);
    orc_sgemm(0, 1, m, out_f, in_f, 1.0f, x, in_f, w, in_f, 0.0f, y, out_f);
    free(w);
    if (bias)
        for (size_t i = 0; i < m; ++i)
            for (size_t j = 0; j < out_f; ++j) y[i * out_f + j] = y[i * out_f + j] + bias[j];
}

/* ------------------------------------------------------------------ */
/* src/tensor.rs:618-672 Tensor::flash_attention                        */
/* ------------------------------------------------------------------ */
/* Online softmax per query row, sequential over keys, every product and sum
 * rounded on its own (no contraction), exp through libm expf as f32::exp.
 * The reference takes q, k, v of one shape [batch, seq, dim]; nq and skv are
 * kept apart here so that a decode query (nq = 1) over a cache of skv keys
 * follows the same expressions; nq == skv is the reference function. */
void orc_flash_attention(const float *q, const float *k, const float *v, size_t batch,
                         size_t nq, size_t skv, size_t dim, float scale, float *out) {
    float *acc = (float *)malloc((dim ? dim : 1) * sizeof(float));
    for (size_t b = 0; b < batch; ++b) {
        for (size_t i = 0; i < nq; ++i) {
            const float *qr = q + (b * nq + i) * dim;
            float row_max = -INFINITY, row_sum = 0.0f;
            for (size_t t = 0; t < dim; ++t) acc[t] = 0.0f;
            for (size_t j = 0; j < skv; ++j) {
                const float *kr = k + (b * skv + j) * dim, *vr = v + (b * skv + j) * dim;
                float s = 0.0f;
                for (size_t t = 0; t < dim; ++t) s += qr[t] * kr[t];
                s *= scale;
                float m_new = fmaxf(row_max, s);
                float exp_old = expf(row_max - m_new);
                float p = expf(s - m_new);
                row_sum = exp_old * row_sum + p;
                for (size_t t = 0; t < dim; ++t) acc[t] = exp_old * acc[t] + p * vr[t];
                row_max = m_new;
            }
            float inv = row_sum > 0.0f ? 1.0f / row_sum : 0.0f;
            float *o = out + (b * nq + i) * dim;
            for (size_t t = 0; t < dim; ++t) o[t] = acc[t] * inv;
        }
    }
    free(acc);
}
