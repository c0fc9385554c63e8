/*
 * rdl_oracle.h -- CPU restatement of rustml's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * product path is compared against.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product library
 * (librdlquant.so) never links, loads or calls it, and there is no CPU
 * fallback from the product to this code.
 *
 * Every function restates one reference function; the citation next to each
 * declaration names the file:line it follows (paths relative to the
 * rust-deeplearning repository root).  Arithmetic is IEEE binary32 with no
 * FMA contraction (the build uses -ffp-contract=off), as the Rust reference
 * never contracts a mul+add.
 *
 * Pinning (how each function is checked against something other than
 * itself) is listed in tests/test_oracle_*.py; functions without an
 * independent check are marked "parity unpinned" below.
 */
#ifndef RDL_ORACLE_H
#define RDL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: the same numbering as include/rdl_quant.h. */
#define ORC_OK 0
#define ORC_ERR_SHAPE_MISMATCH 2
#define ORC_ERR_BLOCK_ALIGNMENT 3

/* ---- binary16 (half 2.7.1: f16::from_f32 is RNE with subnormals,
 *      f16::to_f32 is exact) -------------------------------------------- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* ---- block dots (rustml/quant/main/src/core/simd.rs) ----------------- */
/* dot_q8_block_scalar, simd.rs:12-18 */
float orc_dot_q8_block_scalar(const float* x, const int8_t* q, float scale);
/* dot_q4_block_scalar, simd.rs:21-31 */
float orc_dot_q4_block_scalar(const float* x, const uint8_t* packed, float scale);
/* dot_q4q8_block (every variant is exact integer arithmetic), simd.rs:34-43, 154-193 */
int32_t orc_dot_q4q8_block(const uint8_t* packed, const int8_t* q8);
/* dot_q4_1_q8_block, simd.rs:50-62, 196-238 */
void orc_dot_q4_1_q8_block(const uint8_t* packed, const int8_t* q8, int32_t* dot, int32_t* q8_sum);
/* dot_q8_block as dispatched on x86_64 with AVX2 (dot_q8_block_avx2, simd.rs:69-107):
 * four 8-lane products, (acc0+acc1)+(acc2+acc3), 128-bit hi+lo fold,
 * movehdup add, movehl add_ss, then * scale.  Restated lane by lane. */
float orc_dot_q8_block(const float* x, const int8_t* q, float scale);
/* dot_q4_block as dispatched on x86_64 with AVX2 (dot_q4_block_avx2, simd.rs:110-151). */
float orc_dot_q4_block(const float* x, const uint8_t* packed, float scale);

/* ---- activation quantizer (quantize.rs:164-193) ---------------------- */
void orc_quantize_row_q8_0(const float* input, size_t n, uint8_t* output, float* scales);

/* ---- matmuls (quantize.rs); y[M,N] = x[M,K] . W[N,K]^T ---------------
 * `threads` mirrors rayon's decomposition: one task per input row
 * (par_chunks_mut(out_features), quantize.rs:220-223); the pool size is
 * min(threads, m).  Returns ORC_ERR_BLOCK_ALIGNMENT when K % 32 != 0,
 * ORC_ERR_SHAPE_MISMATCH when a buffer is too short (the reference would
 * panic on the out-of-range slice instead). */
int orc_matmul_f32_q8(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                      size_t n, float* y, int threads);                       /* :201-260 */
int orc_matmul_f32_q4(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                      size_t n, float* y, int threads);                       /* :265-320 */
int orc_matmul_f32_q4_native(const float* x, const uint8_t* w, size_t w_len, size_t m,
                             size_t k, size_t n, float* y, int threads);      /* :326-394 */
int orc_matmul_f32_q4_1(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                        size_t n, float* y, int threads);                     /* :429-495 */
int orc_matmul_f32_q4_1_native(const float* x, const uint8_t* w, size_t w_len, size_t m,
                               size_t k, size_t n, float* y, int threads);    /* :501-572 */

/* Same skeleton as the Q4_0 matmuls but split over output columns on all
 * `threads`: NOT the reference decomposition (the reference runs an M=1
 * GEMV on one core); reported as a labelled extra CPU figure only. */
int orc_matmul_f32_q4_cols(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                           size_t n, float* y, int threads);

/* int32 block partials of the native path: part[r][c][b] = dot_q4q8_block(W[c,b], q8(x_r)[b])
 * (quantize.rs:383), shape [M, N, K/32]. */
int orc_q4_0_q8_0_block_dots(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                             size_t n, int32_t* part);

/* ---- dequantizers ------------------------------------------------------ */
/* Tensor::to_f32, Q4_0 branch: rustml/core/main/src/core/tensor/tensor.rs:535-570 */
int orc_to_f32_q4_0(const uint8_t* w, size_t w_len, size_t n_elements, float* out);
/* Tensor::to_f32, Q4_1 branch: tensor.rs:571-607 */
int orc_to_f32_q4_1(const uint8_t* w, size_t w_len, size_t n_elements, float* out);
/* Tensor::to_f32, Q8_0 branch: tensor.rs:608-639 */
int orc_to_f32_q8_0(const uint8_t* w, size_t w_len, size_t n_elements, float* out);
/* dequantize_q4k: rustml/gguf/main/src/core/parser.rs:549-593 (6-bit scale/min
 * unpack exactly as :562-569, which places the two high bits of sub-blocks 4..7
 * differently from ggml's get_scale_min_k4) */
int orc_dequantize_q4k(const uint8_t* data, size_t data_len, size_t n_elements, float* out);

/* Q4_K "GEMV" as the reference runs it: W dequantized at load (parser.rs:321-325),
 * then the F32 Linear path x . W^T (linear.rs:167-170 -> faer).  faer's summation
 * order is internal to faer 0.20.2 / gemm 0.18.2: this restatement sums each dot
 * sequentially in f32 -- parity unpinned beyond the f64 tolerance check. */
int orc_matmul_f32_q4k(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                       size_t n, float* y, int threads);
/* dequantize_q6k: rustml/gguf/main/src/core/parser.rs:510-547 (ql low nibbles,
 * qh high bit pairs, int8 scales per 16 elements, f16 d at byte 208). */
int orc_dequantize_q6k(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
/* The remaining load-time dequantizers of load_tensors (parser.rs:371-760):
 * Q4_1 (:386-408), Q5_0 (:411-437), Q5_1 (:440-467), Q8_1 (:470-489), Q5_K
 * (:595-646), Q8_K (:649-667), Q3_K (:669-735), Q2_K (:737-776).  Whole
 * blocks of n_elements only; the rest of out is zero, as in the reference. */
int orc_dequantize_q4_1_legacy(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
int orc_dequantize_q5_0(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
int orc_dequantize_q5_1(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
int orc_dequantize_q8_1(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
int orc_dequantize_q5k(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
int orc_dequantize_q8k(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
int orc_dequantize_q3k(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
int orc_dequantize_q2k(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
/* Q6_K "GEMV" as the reference runs it: dequantized at load (parser.rs:321-325),
 * then the F32 Linear; each dot summed sequentially in f32 (parity unpinned
 * beyond the f64 tolerance check, as for Q4_K). */
int orc_matmul_f32_q6k(const float* x, const uint8_t* w, size_t w_len, size_t m, size_t k,
                       size_t n, float* y, int threads);
/* The timed part of the reference Q4_K path: an F32 GEMV over an already
 * dequantized [N,K] matrix, split over output rows on `threads`. */
int orc_matmul_f32_f32(const float* x, const float* w, size_t m, size_t k, size_t n, float* y,
                       int threads);

/* ---- decoder pieces (config 5) ---- */

/* RoPEFreqs::new (rustml/nn/main/src/core/rope.rs:93-108): cos/sin tables
 * [max_seq][head_dim/2] in f32: freq = 1 / powf(theta, 2i/hd), angle =
 * pos * freq, with the C library's powf / cosf / sinf (the calls Rust's f32
 * powf / cos / sin make). */
void orc_rope_tables(int head_dim, int max_seq, float theta, float* cos_out, float* sin_out);

/* Tensor::rms_norm for one row (rustml/core/main/src/core/tensor/ops.rs:688-751)
 * on its AVX2 path (rms_norm_row_avx2, ops.rs:14-69, taken for dim >= 8):
 * two 8-lane sum-of-squares accumulators over 16-element steps, the 8-lane
 * tail, the hi/lo + movehdup + movehl horizontal sum, the scalar remainder;
 * out = (x * (1 / sqrt(sum / dim + eps))) * g. */
void orc_rms_norm_row(const float* row, const float* gamma, size_t dim, float eps, float* out);

#ifdef __cplusplus
}
#endif
#endif
