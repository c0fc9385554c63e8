/*
 * rdl_oracle.c -- CPU restatement of rustml's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (see rdl_oracle.h): the checker for the HIP
 * product path and the timed CPU baseline, never part of the product.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include "rdl_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* Block geometry: rustml/quant/main/src/api/types.rs:1-17 and
 * rustml/gguf/main/src/api/types.rs:62,69-76 (Q4_K = 256 elements / 144 B). */
enum {
    QK = 32,
    Q8_0_BYTES = 34,
    Q4_0_BYTES = 18,
    Q4_1_BYTES = 20,
    QK_K = 256,
    Q4_K_BYTES = 144,
    Q6_K_BYTES = 210,
};

/* ------------------------------------------------------------------------ */
/* binary16 <-> binary32                                                     */
/* ------------------------------------------------------------------------ */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        /* zero or subnormal: value = man * 2^-24, exact in binary32 */
        float v = ldexpf((float)man, -24);
        return sign ? -v : v;
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) {
        if (man) return (uint16_t)(sign | 0x7E00u | (man >> 13)); /* quiet NaN */
        return (uint16_t)(sign | 0x7C00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e; /* 14..24 */
        uint32_t hm = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    uint32_t h = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) h++; /* carry may reach inf */
    return (uint16_t)h;
}

static inline uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline float rd_f16(const uint8_t* p) { return orc_f16_to_f32(rd_u16(p)); }

/* ------------------------------------------------------------------------ */
/* block dots                                                                */
/* ------------------------------------------------------------------------ */

float orc_dot_q8_block_scalar(const float* x, const int8_t* q, float scale) {
    float sum = 0.0f;
    for (int i = 0; i < 32; i++) sum += x[i] * (float)q[i];
    return sum * scale;
}

float orc_dot_q4_block_scalar(const float* x, const uint8_t* packed, float scale) {
    float sum = 0.0f;
    for (int j = 0; j < 16; j++) {
        int lo = (packed[j] & 0x0F) - 8;
        int hi = ((packed[j] >> 4) & 0x0F) - 8;
        sum += x[j] * (float)lo;
        sum += x[j + 16] * (float)hi;
    }
    return sum * scale;
}

int32_t orc_dot_q4q8_block(const uint8_t* packed, const int8_t* q8) {
    int32_t sum = 0;
    for (int j = 0; j < 16; j++) {
        int32_t lo = (packed[j] & 0x0F) - 8;
        int32_t hi = ((packed[j] >> 4) & 0x0F) - 8;
        sum += lo * (int32_t)q8[j];
        sum += hi * (int32_t)q8[j + 16];
    }
    return sum;
}

void orc_dot_q4_1_q8_block(const uint8_t* packed, const int8_t* q8, int32_t* dot, int32_t* q8_sum) {
    int32_t d = 0, s = 0;
    for (int j = 0; j < 16; j++) {
        int32_t lo = packed[j] & 0x0F;
        int32_t hi = (packed[j] >> 4) & 0x0F;
        d += lo * (int32_t)q8[j];
        d += hi * (int32_t)q8[j + 16];
        s += (int32_t)q8[j];
        s += (int32_t)q8[j + 16];
    }
    *dot = d;
    *q8_sum = s;
}

/* The AVX2 reduction tree of simd.rs:69-107 / 110-151 applied to 32 products
 * p[0..32) (p[8c+i] = lane i of chunk c):
 *   t_i = (p_i + p_{8+i}) + (p_{16+i} + p_{24+i})      i = 0..7
 *   u_i = t_i + t_{i+4}                                i = 0..3  (hi128 + lo128)
 *   r   = (u_0 + u_1) + (u_2 + u_3)                    (movehdup add, movehl add_ss)
 */
static inline float avx2_tree(const float* p) {
    float t[8], u[4];
    for (int i = 0; i < 8; i++) t[i] = (p[i] + p[8 + i]) + (p[16 + i] + p[24 + i]);
    for (int i = 0; i < 4; i++) u[i] = t[i] + t[i + 4];
    return (u[0] + u[1]) + (u[2] + u[3]);
}

static float dot_q8_block_lanes(const float* x, const int8_t* q, float scale) {
    float p[32];
    for (int i = 0; i < 32; i++) p[i] = x[i] * (float)q[i];
    return avx2_tree(p) * scale;
}

static float dot_q4_block_lanes(const float* x, const uint8_t* packed, float scale) {
    float w[32], p[32];
    for (int j = 0; j < 16; j++) {
        w[j] = (float)((packed[j] & 0x0F) - 8);
        w[j + 16] = (float)(((packed[j] >> 4) & 0x0F) - 8);
    }
    for (int i = 0; i < 32; i++) p[i] = x[i] * w[i];
    return avx2_tree(p) * scale;
}

#if defined(__x86_64__)
__attribute__((target("avx2"))) static inline float hsum_tree_avx2(__m256 a0, __m256 a1, __m256 a2,
                                                                   __m256 a3) {
    __m256 s = _mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3));
    __m128 hi = _mm256_extractf128_ps(s, 1);
    __m128 lo = _mm256_castps256_ps128(s);
    __m128 s128 = _mm_add_ps(lo, hi);
    __m128 sh = _mm_movehdup_ps(s128);
    __m128 sums = _mm_add_ps(s128, sh);
    __m128 sh2 = _mm_movehl_ps(sums, sums);
    return _mm_cvtss_f32(_mm_add_ss(sums, sh2));
}

__attribute__((target("avx2"))) static float dot_q8_block_avx2(const float* x, const int8_t* q,
                                                               float scale) {
    __m256 acc[4];
    for (int c = 0; c < 4; c++) {
        float qf[8];
        for (int j = 0; j < 8; j++) qf[j] = (float)q[8 * c + j];
        acc[c] = _mm256_mul_ps(_mm256_loadu_ps(x + 8 * c), _mm256_loadu_ps(qf));
    }
    return hsum_tree_avx2(acc[0], acc[1], acc[2], acc[3]) * scale;
}

__attribute__((target("avx2"))) static float dot_q4_block_avx2(const float* x,
                                                               const uint8_t* packed,
                                                               float scale) {
    float w[32];
    for (int j = 0; j < 16; j++) {
        w[j] = (float)((packed[j] & 0x0F) - 8);
        w[j + 16] = (float)(((packed[j] >> 4) & 0x0F) - 8);
    }
    __m256 acc[4];
    for (int c = 0; c < 4; c++)
        acc[c] = _mm256_mul_ps(_mm256_loadu_ps(x + 8 * c), _mm256_loadu_ps(w + 8 * c));
    return hsum_tree_avx2(acc[0], acc[1], acc[2], acc[3]) * scale;
}

static int have_avx2(void) {
    static int cached = -1;
    if (cached < 0) cached = __builtin_cpu_supports("avx2") ? 1 : 0;
    return cached;
}
#else
static int have_avx2(void) { return 0; }
static float dot_q8_block_avx2(const float* x, const int8_t* q, float s) {
    return dot_q8_block_lanes(x, q, s);
}
static float dot_q4_block_avx2(const float* x, const uint8_t* p, float s) {
    return dot_q4_block_lanes(x, p, s);
}
#endif

/* Both branches give identical bits (same op sequence, no contraction); the
 * intrinsic branch is only faster.  tests/test_oracle_dots.py checks that. */
float orc_dot_q8_block(const float* x, const int8_t* q, float scale) {
    return have_avx2() ? dot_q8_block_avx2(x, q, scale) : dot_q8_block_lanes(x, q, scale);
}

float orc_dot_q4_block(const float* x, const uint8_t* packed, float scale) {
    return have_avx2() ? dot_q4_block_avx2(x, packed, scale) : dot_q4_block_lanes(x, packed, scale);
}

/* Exposed for the oracle's own self-check (lane restatement vs intrinsics). */
float orc_dot_q8_block_lanes(const float* x, const int8_t* q, float scale) {
    return dot_q8_block_lanes(x, q, scale);
}
float orc_dot_q4_block_lanes(const float* x, const uint8_t* packed, float scale) {
    return dot_q4_block_lanes(x, packed, scale);
}

/* ------------------------------------------------------------------------ */
/* quantize_row_q8_0 (quantize.rs:164-193)                                   */
/* ------------------------------------------------------------------------ */

/* f32::max: returns the other operand when one is NaN. */
static inline float rust_fmax(float a, float b) { return fmaxf(a, b); }

/* `v.round().clamp(-128.0, 127.0) as i8`: round half away from zero, clamp,
 * saturating cast with NaN -> 0 (Rust float->int `as` semantics). */
static inline int8_t round_clamp_i8(float v) {
    float r = roundf(v);
    if (isnan(r)) return 0;
    if (r < -128.0f) r = -128.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)(int)r;
}

void orc_quantize_row_q8_0(const float* input, size_t n, uint8_t* output, float* scales) {
    size_t nb = n / QK;
    for (size_t b = 0; b < nb; b++) {
        const float* blk = input + b * QK;
        uint8_t* dst = output + b * Q8_0_BYTES;
        float amax = 0.0f;
        for (int i = 0; i < QK; i++) amax = rust_fmax(amax, fabsf(blk[i]));
        float scale = (amax == 0.0f) ? 0.0f : amax / 127.0f;
        uint16_t sh = orc_f32_to_f16(scale);
        float scale_rt = orc_f16_to_f32(sh);
        float inv = (scale_rt == 0.0f) ? 0.0f : 1.0f / scale_rt;
        dst[0] = (uint8_t)(sh & 0xFF);
        dst[1] = (uint8_t)(sh >> 8);
        for (int i = 0; i < QK; i++) dst[2 + i] = (uint8_t)round_clamp_i8(blk[i] * inv);
        scales[b] = scale_rt;
    }
}

/* ------------------------------------------------------------------------ */
/* matmuls                                                                   */
/* ------------------------------------------------------------------------ */

typedef enum { K_Q8, K_Q4, K_Q4_NATIVE, K_Q4_1, K_Q4_1_NATIVE, K_Q4K, K_Q6K } kind_t;

typedef struct {
    kind_t kind;
    const float* x;
    const uint8_t* w;
    size_t m, k, n;
    float* y;
    size_t row_begin, row_end; /* input rows (tokens) */
    size_t col_begin, col_end; /* output columns */
} job_t;

static size_t block_bytes_of(kind_t kd) {
    switch (kd) {
        case K_Q8: return Q8_0_BYTES;
        case K_Q4:
        case K_Q4_NATIVE: return Q4_0_BYTES;
        case K_Q4_1:
        case K_Q4_1_NATIVE: return Q4_1_BYTES;
        case K_Q4K: return Q4_K_BYTES;
        case K_Q6K: return Q6_K_BYTES;
    }
    return 0;
}

static void run_row(const job_t* j, size_t r, uint8_t* q8buf, float* q8s, float* wrow) {
    const size_t k = j->k;
    const float* xr = j->x + r * k;
    float* yr = j->y + r * j->n;
    if (j->kind == K_Q4K || j->kind == K_Q6K) {
        const size_t nsb = k / QK_K;
        const size_t row_bytes = nsb * block_bytes_of(j->kind);
        for (size_t c = j->col_begin; c < j->col_end; c++) {
            if (j->kind == K_Q4K)
                orc_dequantize_q4k(j->w + c * row_bytes, row_bytes, k, wrow);
            else
                orc_dequantize_q6k(j->w + c * row_bytes, row_bytes, k, wrow);
            float dot = 0.0f;
            for (size_t l = 0; l < k; l++) dot += xr[l] * wrow[l];
            yr[c] = dot;
        }
        return;
    }
    const size_t nb = k / QK;
    const size_t bb = block_bytes_of(j->kind);
    const size_t row_bytes = nb * bb;
    if (j->kind == K_Q4_NATIVE || j->kind == K_Q4_1_NATIVE) orc_quantize_row_q8_0(xr, k, q8buf, q8s);
    for (size_t c = j->col_begin; c < j->col_end; c++) {
        const uint8_t* wr = j->w + c * row_bytes;
        float dot = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t* blk = wr + b * bb;
            switch (j->kind) {
                case K_Q8:
                    dot += orc_dot_q8_block(xr + b * QK, (const int8_t*)(blk + 2), rd_f16(blk));
                    break;
                case K_Q4:
                    dot += orc_dot_q4_block(xr + b * QK, blk + 2, rd_f16(blk));
                    break;
                case K_Q4_NATIVE: {
                    float ws = rd_f16(blk);
                    int32_t id = orc_dot_q4q8_block(blk + 2, (const int8_t*)(q8buf + b * Q8_0_BYTES + 2));
                    dot += (float)id * q8s[b] * ws;
                    break;
                }
                case K_Q4_1: {
                    float d = rd_f16(blk), mv = rd_f16(blk + 2);
                    const uint8_t* p = blk + 4;
                    const float* xb = xr + b * QK;
                    float bd = 0.0f, is = 0.0f;
                    for (int t = 0; t < 16; t++) {
                        float lo = (float)(p[t] & 0x0F), hi = (float)((p[t] >> 4) & 0x0F);
                        bd += xb[t] * lo;
                        bd += xb[t + 16] * hi;
                        is += xb[t];
                        is += xb[t + 16];
                    }
                    dot += d * bd + mv * is;
                    break;
                }
                case K_Q4_1_NATIVE: {
                    float d = rd_f16(blk), mv = rd_f16(blk + 2);
                    int32_t ud, qs;
                    orc_dot_q4_1_q8_block(blk + 4, (const int8_t*)(q8buf + b * Q8_0_BYTES + 2), &ud, &qs);
                    dot += q8s[b] * (d * (float)ud + mv * (float)qs);
                    break;
                }
                default: break;
            }
        }
        yr[c] = dot;
    }
}

static void* job_thread(void* arg) {
    job_t* j = (job_t*)arg;
    size_t nb = j->k / QK + 1;
    uint8_t* q8buf = (uint8_t*)malloc(nb * Q8_0_BYTES);
    float* q8s = (float*)malloc(nb * sizeof(float));
    float* wrow = (j->kind == K_Q4K || j->kind == K_Q6K) ? (float*)malloc(j->k * sizeof(float)) : NULL;
    for (size_t r = j->row_begin; r < j->row_end; r++) run_row(j, r, q8buf, q8s, wrow);
    free(q8buf);
    free(q8s);
    free(wrow);
    return NULL;
}

/* Split [0, total) into `parts` contiguous ranges; run each on its own thread. */
static void run_split(job_t proto, int by_rows, int threads) {
    size_t total = by_rows ? proto.m : proto.n;
    if (threads < 1) threads = 1;
    if ((size_t)threads > total) threads = (int)(total ? total : 1);
    if (threads == 1) {
        job_thread(&proto);
        return;
    }
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * threads);
    job_t* jobs = (job_t*)malloc(sizeof(job_t) * threads);
    for (int t = 0; t < threads; t++) {
        jobs[t] = proto;
        size_t b = total * (size_t)t / threads, e = total * (size_t)(t + 1) / threads;
        if (by_rows) {
            jobs[t].row_begin = b;
            jobs[t].row_end = e;
        } else {
            jobs[t].col_begin = b;
            jobs[t].col_end = e;
        }
        pthread_create(&th[t], NULL, job_thread, &jobs[t]);
    }
    for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

static int matmul_common(kind_t kd, const float* x, const uint8_t* w, size_t w_len, size_t m,
                         size_t k, size_t n, float* y, int threads, int by_rows) {
    size_t unit = (kd == K_Q4K || kd == K_Q6K) ? QK_K : QK;
    if (k % unit != 0) return ORC_ERR_BLOCK_ALIGNMENT;
    if (w_len < n * (k / unit) * block_bytes_of(kd)) return ORC_ERR_SHAPE_MISMATCH;
    job_t j = {kd, x, w, m, k, n, y, 0, m, 0, n};
    run_split(j, by_rows, threads);
    return ORC_OK;
}

int orc_matmul_f32_q8(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k, size_t n,
                      float* y, int threads) {
    return matmul_common(K_Q8, x, w, w_len, m, k, n, y, threads, 1);
}
int orc_matmul_f32_q4(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k, size_t n,
                      float* y, int threads) {
    return matmul_common(K_Q4, x, w, w_len, m, k, n, y, threads, 1);
}
int orc_matmul_f32_q4_native(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                             size_t n, float* y, int threads) {
    return matmul_common(K_Q4_NATIVE, x, w, w_len, m, k, n, y, threads, 1);
}
int orc_matmul_f32_q4_1(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                        size_t n, float* y, int threads) {
    return matmul_common(K_Q4_1, x, w, w_len, m, k, n, y, threads, 1);
}
int orc_matmul_f32_q4_1_native(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                               size_t n, float* y, int threads) {
    return matmul_common(K_Q4_1_NATIVE, x, w, w_len, m, k, n, y, threads, 1);
}
int orc_matmul_f32_q4_cols(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                           size_t n, float* y, int threads) {
    return matmul_common(K_Q4, x, w, w_len, m, k, n, y, threads, 0);
}
int orc_matmul_f32_q4k(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k, size_t n,
                       float* y, int threads) {
    return matmul_common(K_Q4K, x, w, w_len, m, k, n, y, threads, 0);
}

int orc_matmul_f32_q6k(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k, size_t n,
                       float* y, int threads) {
    return matmul_common(K_Q6K, x, w, w_len, m, k, n, y, threads, 0);
}

int orc_q4_0_q8_0_block_dots(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                             size_t n, int32_t* part) {
    if (k % QK != 0) return ORC_ERR_BLOCK_ALIGNMENT;
    size_t nb = k / QK;
    if (w_len < n * nb * Q4_0_BYTES) return ORC_ERR_SHAPE_MISMATCH;
    uint8_t* q8 = (uint8_t*)malloc(nb * Q8_0_BYTES);
    float* s = (float*)malloc(nb * sizeof(float));
    for (size_t r = 0; r < m; r++) {
        orc_quantize_row_q8_0(x + r * k, k, q8, s);
        for (size_t c = 0; c < n; c++)
            for (size_t b = 0; b < nb; b++)
                part[(r * n + c) * nb + b] = orc_dot_q4q8_block(
                    w + (c * nb + b) * Q4_0_BYTES + 2, (const int8_t*)(q8 + b * Q8_0_BYTES + 2));
    }
    free(q8);
    free(s);
    return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* dequantizers                                                              */
/* ------------------------------------------------------------------------ */

int orc_to_f32_q4_0(const uint8_t* w, size_t w_len, size_t n_elements, float* out) {
    if (n_elements % QK) return ORC_ERR_BLOCK_ALIGNMENT;
    size_t nb = n_elements / QK;
    if (w_len < nb * Q4_0_BYTES) return ORC_ERR_SHAPE_MISMATCH;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = w + b * Q4_0_BYTES;
        float s = rd_f16(blk);
        for (int j = 0; j < 16; j++) {
            uint8_t byte = blk[2 + j];
            out[b * QK + j] = s * (float)((int)(byte & 0x0F) - 8);
            out[b * QK + j + 16] = s * (float)((int)((byte >> 4) & 0x0F) - 8);
        }
    }
    return ORC_OK;
}

int orc_to_f32_q4_1(const uint8_t* w, size_t w_len, size_t n_elements, float* out) {
    if (n_elements % QK) return ORC_ERR_BLOCK_ALIGNMENT;
    size_t nb = n_elements / QK;
    if (w_len < nb * Q4_1_BYTES) return ORC_ERR_SHAPE_MISMATCH;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = w + b * Q4_1_BYTES;
        float d = rd_f16(blk), mv = rd_f16(blk + 2);
        for (int j = 0; j < 16; j++) {
            uint8_t byte = blk[4 + j];
            out[b * QK + j] = d * (float)(byte & 0x0F) + mv;
            out[b * QK + j + 16] = d * (float)((byte >> 4) & 0x0F) + mv;
        }
    }
    return ORC_OK;
}

int orc_to_f32_q8_0(const uint8_t* w, size_t w_len, size_t n_elements, float* out) {
    if (n_elements % QK) return ORC_ERR_BLOCK_ALIGNMENT;
    size_t nb = n_elements / QK;
    if (w_len < nb * Q8_0_BYTES) return ORC_ERR_SHAPE_MISMATCH;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = w + b * Q8_0_BYTES;
        float s = rd_f16(blk);
        for (int j = 0; j < 32; j++) out[b * QK + j] = s * (float)(int8_t)blk[2 + j];
    }
    return ORC_OK;
}

int orc_dequantize_q4k(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    if (n_elements % QK_K) return ORC_ERR_BLOCK_ALIGNMENT;
    size_t nb = n_elements / QK_K;
    if (data_len < nb * Q4_K_BYTES) return ORC_ERR_SHAPE_MISMATCH;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = data + b * Q4_K_BYTES;
        float d = rd_f16(blk), dmin = rd_f16(blk + 2);
        const uint8_t* s = blk + 4;
        const uint8_t* qs = blk + 16;
        uint8_t sc[8], mn[8];
        for (int i = 0; i < 4; i++) {
            sc[i] = s[i] & 63;
            mn[i] = s[i + 4] & 63;
            sc[i + 4] = (uint8_t)(((s[i] >> 6) & 3) | ((s[i + 8] & 0xF) << 2));
            mn[i + 4] = (uint8_t)(((s[i + 4] >> 6) & 3) | ((s[i + 8] >> 4) << 2));
        }
        float* o = out + b * QK_K;
        for (int c = 0; c < 4; c++) {
            const uint8_t* q = qs + 32 * c;
            float d1 = d * (float)sc[2 * c], m1 = dmin * (float)mn[2 * c];
            float d2 = d * (float)sc[2 * c + 1], m2 = dmin * (float)mn[2 * c + 1];
            for (int l = 0; l < 32; l++) o[64 * c + l] = d1 * (float)(q[l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) o[64 * c + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
        }
    }
    return ORC_OK;
}

/* parser.rs:510-547: two halves of 128 elements; element half*128 + 32*t + l
 * takes its low four bits from ql (byte half*64 + l for t = 0, 2 and
 * half*64 + 32 + l for t = 1, 3; low nibble for t < 2, high for t >= 2), its
 * high two bits from bits 2t, 2t+1 of qh[half*32 + l], and the signed scale
 * scales[half*8 + l/16 + 2t]; value (d * scale) * (q - 32). */
int orc_dequantize_q6k(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    if (n_elements % QK_K) return ORC_ERR_BLOCK_ALIGNMENT;
    size_t nb = n_elements / QK_K;
    if (data_len < nb * Q6_K_BYTES) return ORC_ERR_SHAPE_MISMATCH;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = data + b * Q6_K_BYTES;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        const float d = rd_f16(blk + 208);
        float* o = out + b * QK_K;
        for (int half = 0; half < 2; half++) {
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const uint8_t lo = ql[half * 64 + l], hi = ql[half * 64 + 32 + l], h = qh[half * 32 + l];
                const int q1 = (int)((lo & 0xF) | (((h >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((hi & 0xF) | (((h >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((lo >> 4) | (((h >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((hi >> 4) | (((h >> 6) & 3) << 4)) - 32;
                o[half * 128 + l] = d * (float)sc[half * 8 + is] * (float)q1;
                o[half * 128 + l + 32] = d * (float)sc[half * 8 + is + 2] * (float)q2;
                o[half * 128 + l + 64] = d * (float)sc[half * 8 + is + 4] * (float)q3;
                o[half * 128 + l + 96] = d * (float)sc[half * 8 + is + 6] * (float)q4;
            }
        }
    }
    return ORC_OK;
}

/* ---- the other load-time dequantizers (parser.rs:371-760) ----------------
 * Each writes n_elements / block_size whole blocks (the reference's block
 * count); elements past them keep the zero the reference's output Vec holds. */

static float rd_f32le(const uint8_t* p) {
    float f;
    memcpy(&f, p, 4);  /* the host is little-endian, as the file */
    return f;
}
static uint32_t rd_u32le(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* parser.rs:386-408: [f16 d][f16 m][16 B]; d * nibble + m */
int orc_dequantize_q4_1_legacy(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    size_t nb = n_elements / 32;
    if (data_len < nb * 20) return ORC_ERR_SHAPE_MISMATCH;
    memset(out, 0, n_elements * sizeof(float));
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = data + b * 20;
        float d = rd_f16(blk), m = rd_f16(blk + 2);
        for (int j = 0; j < 16; j++) {
            out[b * 32 + j] = d * (float)(blk[4 + j] & 0xF) + m;
            out[b * 32 + j + 16] = d * (float)(blk[4 + j] >> 4) + m;
        }
    }
    return ORC_OK;
}

/* parser.rs:411-437: [f16 d][u32 qh][16 B]; d * ((nibble | bit << 4) - 16) */
int orc_dequantize_q5_0(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    size_t nb = n_elements / 32;
    if (data_len < nb * 22) return ORC_ERR_SHAPE_MISMATCH;
    memset(out, 0, n_elements * sizeof(float));
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = data + b * 22;
        float d = rd_f16(blk);
        uint32_t qh = rd_u32le(blk + 2);
        for (int j = 0; j < 16; j++) {
            int lo = (blk[6 + j] & 0xF) | (int)(((qh >> j) & 1) << 4);
            int hi = (blk[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1) << 4);
            out[b * 32 + j] = d * ((float)lo - 16.0f);
            out[b * 32 + j + 16] = d * ((float)hi - 16.0f);
        }
    }
    return ORC_OK;
}

/* parser.rs:440-467: [f16 d][f16 m][u32 qh][16 B]; d * (nibble | bit << 4) + m */
int orc_dequantize_q5_1(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    size_t nb = n_elements / 32;
    if (data_len < nb * 24) return ORC_ERR_SHAPE_MISMATCH;
    memset(out, 0, n_elements * sizeof(float));
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = data + b * 24;
        float d = rd_f16(blk), m = rd_f16(blk + 2);
        uint32_t qh = rd_u32le(blk + 4);
        for (int j = 0; j < 16; j++) {
            uint32_t lo = (uint32_t)(blk[8 + j] & 0xF) | (((qh >> j) & 1) << 4);
            uint32_t hi = (uint32_t)(blk[8 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4);
            out[b * 32 + j] = d * (float)lo + m;
            out[b * 32 + j + 16] = d * (float)hi + m;
        }
    }
    return ORC_OK;
}

/* parser.rs:470-489: [f32 d][f32 s][32 x i8]; d * q (s unused) */
int orc_dequantize_q8_1(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    size_t nb = n_elements / 32;
    if (data_len < nb * 40) return ORC_ERR_SHAPE_MISMATCH;
    memset(out, 0, n_elements * sizeof(float));
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = data + b * 40;
        float d = rd_f32le(blk);
        for (int j = 0; j < 32; j++) out[b * 32 + j] = d * (float)(int8_t)blk[8 + j];
    }
    return ORC_OK;
}

/* parser.rs:595-646: [f16 d][f16 dmin][12 B scales][32 B qh][128 B qs]; the
 * Q4_K scale/min unpack; element 64c + l (+32): d*sc * (nibble + 16 * bit) - dmin*mn,
 * the bit of qh[l] at 2c (lo nibbles) or 2c + 1 (hi nibbles). */
int orc_dequantize_q5k(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    size_t nb = n_elements / QK_K;
    if (data_len < nb * 176) return ORC_ERR_SHAPE_MISMATCH;
    memset(out, 0, n_elements * sizeof(float));
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = data + b * 176;
        float d = rd_f16(blk), dmin = rd_f16(blk + 2);
        const uint8_t* s = blk + 4;
        const uint8_t* qh = blk + 16;
        const uint8_t* qs = blk + 48;
        uint8_t sc[8], mn[8];
        for (int i = 0; i < 4; i++) {
            sc[i] = s[i] & 63;
            mn[i] = s[i + 4] & 63;
            sc[i + 4] = (uint8_t)(((s[i] >> 6) & 3) | ((s[i + 8] & 0xF) << 2));
            mn[i + 4] = (uint8_t)(((s[i + 4] >> 6) & 3) | ((s[i + 8] >> 4) << 2));
        }
        float* o = out + b * QK_K;
        uint8_t u1 = 1, u2 = 2;
        for (int c = 0; c < 4; c++) {
            float d1 = d * (float)sc[2 * c], m1 = dmin * (float)mn[2 * c];
            float d2 = d * (float)sc[2 * c + 1], m2 = dmin * (float)mn[2 * c + 1];
            for (int l = 0; l < 32; l++) {
                int hb = (qh[l] & u1) ? 16 : 0;
                o[64 * c + l] = d1 * (float)((qs[32 * c + l] & 0xF) + hb) - m1;
            }
            for (int l = 0; l < 32; l++) {
                int hb = (qh[l] & u2) ? 16 : 0;
                o[64 * c + 32 + l] = d2 * (float)((qs[32 * c + l] >> 4) + hb) - m2;
            }
            u1 = (uint8_t)(u1 << 2);
            u2 = (uint8_t)(u2 << 2);
        }
    }
    return ORC_OK;
}

/* parser.rs:649-667: [f32 d][256 x i8][32 B bsums]; d * q */
int orc_dequantize_q8k(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    size_t nb = n_elements / QK_K;
    if (data_len < nb * 292) return ORC_ERR_SHAPE_MISMATCH;
    memset(out, 0, n_elements * sizeof(float));
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = data + b * 292;
        float d = rd_f32le(blk);
        for (int j = 0; j < 256; j++) out[b * QK_K + j] = d * (float)(int8_t)blk[4 + j];
    }
    return ORC_OK;
}

/* parser.rs:669-735: [32 B hmask][64 B qs][12 B scales][f16 d].  The sixteen
 * 6-bit scales: low nibbles from bytes 0..7 (scale i < 8: low nibble of byte
 * i; 8 <= i < 16: high nibble of byte i - 8), high bit pairs from bytes 8..11
 * (scale i: bits 2(i / 4) .. +1 of byte 8 + i % 4), each minus 32.  Element
 * order: two halves of 128, four shift steps of 32 (16 + 16 with scales is,
 * is + 1), value d*(scale - 32) * (2-bit q + (hmask bit set ? 0 : -4)). */
int orc_dequantize_q3k(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    size_t nb = n_elements / QK_K;
    if (data_len < nb * 110) return ORC_ERR_SHAPE_MISMATCH;
    memset(out, 0, n_elements * sizeof(float));
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = data + b * 110;
        const uint8_t* hm = blk;
        const uint8_t* qs = blk + 32;
        const uint8_t* sr = blk + 96;
        const float d_all = rd_f16(blk + 108);
        /* the aux-word unpack of :682-698 */
        const uint32_t km1 = 0x03030303u, km2 = 0x0f0f0f0fu;
        uint32_t a0 = rd_u32le(sr), a1 = rd_u32le(sr + 4), tmp = rd_u32le(sr + 8);
        uint32_t aux[4];
        aux[2] = ((a0 >> 4) & km2) | (((tmp >> 4) & km1) << 4);
        aux[3] = ((a1 >> 4) & km2) | (((tmp >> 6) & km1) << 4);
        aux[0] = (a0 & km2) | (((tmp >> 0) & km1) << 4);
        aux[1] = (a1 & km2) | (((tmp >> 2) & km1) << 4);
        int8_t scb[16];
        for (int i = 0; i < 16; i++) scb[i] = (int8_t)((aux[i / 4] >> (8 * (i % 4))) & 0xFF);
        float* o = out + b * QK_K;
        int y = 0, is = 0;
        uint8_t m = 1;
        for (int half = 0; half < 2; half++) {
            const uint8_t* q = qs + 32 * half;
            int shift = 0;
            for (int j = 0; j < 4; j++) {
                float dl = d_all * ((float)scb[is] - 32.0f);
                for (int l = 0; l < 16; l++) {
                    int q2 = (q[l] >> shift) & 3;
                    int hb = (hm[l] & m) ? 0 : -4;
                    o[y++] = dl * (float)(q2 + hb);
                }
                dl = d_all * ((float)scb[is + 1] - 32.0f);
                for (int l = 0; l < 16; l++) {
                    int q2 = (q[l + 16] >> shift) & 3;
                    int hb = (hm[l + 16] & m) ? 0 : -4;
                    o[y++] = dl * (float)(q2 + hb);
                }
                is += 2;
                shift += 2;
                m = (uint8_t)(m << 1);
            }
        }
    }
    return ORC_OK;
}

/* parser.rs:737-776: [16 B scales][64 B qs][f16 d][f16 dmin]; scale byte:
 * low nibble scale, high nibble min; value d*sc * q2 - dmin*mn, same element
 * order as Q3_K. */
int orc_dequantize_q2k(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    size_t nb = n_elements / QK_K;
    if (data_len < nb * 84) return ORC_ERR_SHAPE_MISMATCH;
    memset(out, 0, n_elements * sizeof(float));
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = data + b * 84;
        const uint8_t* sc = blk;
        const uint8_t* qs = blk + 16;
        const float d = rd_f16(blk + 80), dmin = rd_f16(blk + 82);
        float* o = out + b * QK_K;
        int y = 0, is = 0;
        for (int half = 0; half < 2; half++) {
            const uint8_t* q = qs + 32 * half;
            int shift = 0;
            for (int j = 0; j < 4; j++) {
                uint8_t s = sc[is++];
                float dl = d * (float)(s & 0xF), ml = dmin * (float)(s >> 4);
                for (int l = 0; l < 16; l++) o[y++] = dl * (float)((q[l] >> shift) & 3) - ml;
                s = sc[is++];
                dl = d * (float)(s & 0xF);
                ml = dmin * (float)(s >> 4);
                for (int l = 0; l < 16; l++) o[y++] = dl * (float)((q[l + 16] >> shift) & 3) - ml;
                shift += 2;
            }
        }
    }
    return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* F32 GEMV used as the timed part of the reference Q4_K path                */
/* ------------------------------------------------------------------------ */

typedef struct {
    const float* x;
    const float* w;
    size_t m, k, n;
    float* y;
    size_t c0, c1;
} f32job_t;

#if defined(__x86_64__)
__attribute__((target("avx2,fma"))) static float dot_f32_avx2(const float* a, const float* b,
                                                              size_t k) {
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    __m256 acc2 = _mm256_setzero_ps(), acc3 = _mm256_setzero_ps();
    size_t l = 0;
    for (; l + 32 <= k; l += 32) {
        acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + l), _mm256_loadu_ps(b + l), acc0);
        acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + l + 8), _mm256_loadu_ps(b + l + 8), acc1);
        acc2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + l + 16), _mm256_loadu_ps(b + l + 16), acc2);
        acc3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + l + 24), _mm256_loadu_ps(b + l + 24), acc3);
    }
    float r = hsum_tree_avx2(acc0, acc1, acc2, acc3);
    for (; l < k; l++) r += a[l] * b[l];
    return r;
}
#endif

static void* f32_thread(void* arg) {
    f32job_t* j = (f32job_t*)arg;
    for (size_t r = 0; r < j->m; r++)
        for (size_t c = j->c0; c < j->c1; c++) {
            const float* a = j->x + r * j->k;
            const float* b = j->w + c * j->k;
            float d;
#if defined(__x86_64__)
            if (have_avx2()) {
                d = dot_f32_avx2(a, b, j->k);
            } else
#endif
            {
                d = 0.0f;
                for (size_t l = 0; l < j->k; l++) d += a[l] * b[l];
            }
            j->y[r * j->n + c] = d;
        }
    return NULL;
}

int orc_matmul_f32_f32(const float* x, const float* w, size_t m, size_t k, size_t n, float* y,
                       int threads) {
    if (threads < 1) threads = 1;
    if ((size_t)threads > n) threads = (int)(n ? n : 1);
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * threads);
    f32job_t* jobs = (f32job_t*)malloc(sizeof(f32job_t) * threads);
    for (int t = 0; t < threads; t++) {
        f32job_t j = {x, w, m, k, n, y, n * (size_t)t / threads, n * (size_t)(t + 1) / threads};
        jobs[t] = j;
        pthread_create(&th[t], NULL, f32_thread, &jobs[t]);
    }
    for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
    return ORC_OK;
}

/* ---- decoder pieces ---- */

void orc_rope_tables(int head_dim, int max_seq, float theta, float* cos_out, float* sin_out) {
    /* rope.rs:97-105 */
    const int half = head_dim / 2;
    for (int pos = 0; pos < max_seq; pos++)
        for (int i = 0; i < half; i++) {
            const float freq = 1.0f / powf(theta, 2.0f * (float)i / (float)head_dim);
            const float angle = (float)pos * freq;
            cos_out[(size_t)pos * half + i] = cosf(angle);
            sin_out[(size_t)pos * half + i] = sinf(angle);
        }
}

void orc_rms_norm_row(const float* row, const float* gamma, size_t dim, float eps, float* out) {
    if (dim < 8) { /* scalar fallback, ops.rs:735-744 */
        float sum_sq = 0.0f;
        for (size_t i = 0; i < dim; i++) sum_sq += row[i] * row[i];
        const float rms = sqrtf(sum_sq / (float)dim + eps);
        for (size_t j = 0; j < dim; j++) out[j] = row[j] / rms * gamma[j];
        return;
    }
    float acc0[8] = {0}, acc1[8] = {0};
    size_t i = 0;
    for (; i + 16 <= dim; i += 16) /* ops.rs:23-29 */
        for (int l = 0; l < 8; l++) {
            const float v0 = row[i + l], v1 = row[i + 8 + l];
            acc0[l] = acc0[l] + v0 * v0;
            acc1[l] = acc1[l] + v1 * v1;
        }
    for (; i + 8 <= dim; i += 8) /* ops.rs:30-34 */
        for (int l = 0; l < 8; l++) acc0[l] = acc0[l] + row[i + l] * row[i + l];
    float sv[8];
    for (int l = 0; l < 8; l++) sv[l] = acc0[l] + acc1[l];
    /* ops.rs:35-43: lo + hi, movehdup, movehl, add_ss */
    float s128[4];
    for (int l = 0; l < 4; l++) s128[l] = sv[l] + sv[4 + l];
    const float sums0 = s128[0] + s128[1], sums2 = s128[2] + s128[3];
    float sum_sq = sums0 + sums2;
    for (; i < dim; i++) sum_sq += row[i] * row[i]; /* ops.rs:44-48 */
    const float rms = sqrtf(sum_sq / (float)dim + eps); /* ops.rs:51-53 */
    const float inv_rms = 1.0f / rms;
    for (size_t j = 0; j < dim; j++) out[j] = (row[j] * inv_rms) * gamma[j];
}
