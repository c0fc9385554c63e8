/*
 * rdl_quant.h -- C ABI of librdlquant.so, the MI355X (gfx950) implementation
 * of rustml's GGUF block-quantized matmul path (Q8_0, Q4_0, Q4_1, Q4_K, Q6_K).
 *
 * Reference interface replaced (paths relative to the rust-deeplearning
 * repository root):
 *   rustml_quant facade        rustml/quant/main/src/saf/mod.rs:1-4
 *   matmul_f32_q8              rustml/quant/main/src/core/quantize.rs:201-260
 *   matmul_f32_q4              rustml/quant/main/src/core/quantize.rs:265-320
 *   matmul_f32_q4_native       rustml/quant/main/src/core/quantize.rs:326-394
 *   matmul_f32_q4_1            rustml/quant/main/src/core/quantize.rs:429-495
 *   matmul_f32_q4_1_native     rustml/quant/main/src/core/quantize.rs:501-572
 *   quantize_row_q8_0          rustml/quant/main/src/core/quantize.rs:164-193
 *   QuantError                 rustml/quant/main/src/api/error.rs:1-18
 *   Linear::forward dispatch   rustml/nn/main/src/core/linear.rs:119-177
 *
 * Conventions
 *   - Every entry point returns an rdl_status; nothing throws or aborts across
 *     the ABI.  rdl_last_error() gives the detail text of the calling thread's
 *     last failure (the String inside QuantError::BlockAlignment etc.).
 *   - Rust slices become (pointer, length) pairs.  The reference does not check
 *     slice lengths (an out-of-range slice panics); this ABI checks them and
 *     returns RDL_ERR_SHAPE_MISMATCH instead.
 *   - K % 32 != 0 (K % 256 for Q4_K / Q6_K) returns RDL_ERR_BLOCK_ALIGNMENT, checked
 *     before any length check, as in quantize.rs:208-213 / 272-277 / 333-338.
 *   - Host-pointer entry points (rdl_matmul_*, rdl_quantize_row_q8_0) are
 *     synchronous, like the reference's Vec-returning functions: inputs are
 *     copied to the device, the result is copied back before return.
 *   - Device entry points (suffix _dev) take device pointers and a hipStream_t
 *     passed as void*; they are stream-ordered and return after the launch.
 *   - Weight bytes are the GGUF block layout, row-major [N, K/block] blocks, and
 *     stay in that layout in HBM (no repacking).
 *   - Thread safety: distinct threads may call concurrently on distinct
 *     streams.  Weight handles are immutable after creation.
 */
#ifndef RDL_QUANT_H
#define RDL_QUANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
typedef int32_t rdl_status;
enum {
    RDL_OK = 0,
    RDL_ERR_DTYPE_MISMATCH = 1,  /* QuantError::DTypeMismatch  (error.rs:6-7)  */
    RDL_ERR_SHAPE_MISMATCH = 2,  /* QuantError::ShapeMismatch  (error.rs:9-10) */
    RDL_ERR_BLOCK_ALIGNMENT = 3, /* QuantError::BlockAlignment (error.rs:12-13) */
    RDL_ERR_INVALID_DATA = 4,    /* QuantError::InvalidData    (error.rs:15-16) */
    RDL_ERR_NULL_POINTER = 5,    /* a required pointer was NULL (a Rust slice never is) */
    RDL_ERR_HIP = 6,             /* a HIP runtime call failed */
    RDL_ERR_NO_DEVICE = 7,       /* no gfx950 device is visible */
    RDL_ERR_UNSUPPORTED = 8      /* shape beyond a documented kernel limit */
};

/* ---- weight dtypes: GGML type ids (rustml/gguf/main/src/api/types.rs:5-20) */
enum {
    RDL_DTYPE_Q4_0 = 2,
    RDL_DTYPE_Q4_1 = 3,
    RDL_DTYPE_Q8_0 = 8,
    RDL_DTYPE_Q4_K = 12, /* additive extension: rustml_core::DType has no Q4_K */
    RDL_DTYPE_Q6_K = 14  /* additive extension: rustml_core::DType has no Q6_K */
};

/* ---- arithmetic modes (Linear::use_native_q4, linear.rs:23-24, 96-98) ---- */
enum {
    RDL_MODE_FLOAT = 0, /* f32 activations: matmul_f32_q4 / _q8 / _q4_1 semantics */
    RDL_MODE_NATIVE = 1 /* activations quantized to Q8_0, int32 block dots:
                           matmul_f32_q4_native / _q4_1_native semantics */
};

/* Text of a status code; never NULL. */
const char* rdl_status_string(rdl_status status);
/* Detail message of the calling thread's last non-OK status ("" if none). */
const char* rdl_last_error(void);
/* The extents of the calling thread's last status when it was
 * RDL_ERR_SHAPE_MISMATCH, as QuantError::ShapeMismatch { expected, actual }
 * carries them (error.rs:9-10): up to RDL_SHAPE_MAX_DIMS values each
 * (lengths in elements or bytes, or tensor dims, as rdl_last_error's text
 * names them), the counts in *n_expected / *n_actual, unused entries 0.
 * RDL_ERR_INVALID_DATA when the last status was anything else; neither case
 * changes the thread's last status. */
#define RDL_SHAPE_MAX_DIMS 4
rdl_status rdl_last_shape_mismatch(size_t* expected, size_t* n_expected, size_t* actual, size_t* n_actual);
/* Library version string. */
const char* rdl_version(void);
/* Number of visible gfx950 devices (0 when there is no GPU; never an error). */
int32_t rdl_device_count(void);

/* Testing switch (no reference counterpart).  The Q4_0 GEMMs for 5-64 rows
 * split K over workgroups whose partials the last one of each strip adds.
 * RDL_COMBINE_AUTO (the default): where the device deals each launch's
 * workgroups round-robin over its XCDs (probed once per device), a strip's
 * slices share one XCD and its L2, and the partials stay there.
 * RDL_COMBINE_COHERENT: every launch takes the agent-coherent combine
 * (write-through partials, device-scope counter).  Both give the same bits.
 * Process-wide; set it while no call is in flight. */
enum { RDL_COMBINE_AUTO = 0, RDL_COMBINE_COHERENT = 1 };
rdl_status rdl_set_gemm_combine(int32_t mode);
/* The switch's mode, and *local = 1 when the current device's next split
 * GEMM launch takes the XCD-local combine (the placement probe, which the
 * first such launch runs, has passed). */
rdl_status rdl_get_gemm_combine(int32_t* mode, int32_t* local);

/* Instrumentation (no reference counterpart): the next GEMV/GEMM kernel the
 * calling thread launches records its start and end into these hipEvent_t
 * (created with timing enabled) at the kernel boundaries, through
 * hipExtLaunchKernel -- the same interval a kernel trace reports. */
rdl_status rdl_time_next_launch(void* start_event, void* stop_event);

/* ---- host-pointer drop-ins for rustml_quant ------------------------------
 * input_data: f32 [m, in_features]; weight_bytes: blocks of [out_features,
 * in_features]; output: f32 [m, out_features] (output_len >= m*out_features). */

/* replaces matmul_f32_q8, quantize.rs:201-260 */
rdl_status rdl_matmul_f32_q8(const float* input_data, size_t input_len,
                             const uint8_t* weight_bytes, size_t weight_len, size_t m,
                             size_t in_features, size_t out_features, float* output,
                             size_t output_len);
/* replaces matmul_f32_q4, quantize.rs:265-320 */
rdl_status rdl_matmul_f32_q4(const float* input_data, size_t input_len,
                             const uint8_t* weight_bytes, size_t weight_len, size_t m,
                             size_t in_features, size_t out_features, float* output,
                             size_t output_len);
/* replaces matmul_f32_q4_native, quantize.rs:326-394 */
rdl_status rdl_matmul_f32_q4_native(const float* input_data, size_t input_len,
                                    const uint8_t* weight_bytes, size_t weight_len, size_t m,
                                    size_t in_features, size_t out_features, float* output,
                                    size_t output_len);
/* replaces matmul_f32_q4_1, quantize.rs:429-495 */
rdl_status rdl_matmul_f32_q4_1(const float* input_data, size_t input_len,
                               const uint8_t* weight_bytes, size_t weight_len, size_t m,
                               size_t in_features, size_t out_features, float* output,
                               size_t output_len);
/* replaces matmul_f32_q4_1_native, quantize.rs:501-572 */
rdl_status rdl_matmul_f32_q4_1_native(const float* input_data, size_t input_len,
                                      const uint8_t* weight_bytes, size_t weight_len, size_t m,
                                      size_t in_features, size_t out_features, float* output,
                                      size_t output_len);
/* Additive extension (no reference counterpart): Q4_K weights kept resident.
 * The reference dequantizes Q4_K at load (rustml/gguf/main/src/core/parser.rs:321-325,
 * dequantize_q4k :549-593) and runs the F32 Linear path (linear.rs:167-170); this
 * computes the same product straight from the 144-byte super-blocks: GEMVs
 * for m < 16 rows, the matrix-core tile GEMM from 16 rows (in_features <=
 * 16384; longer rows take the GEMV). */
rdl_status rdl_matmul_f32_q4_k(const float* input_data, size_t input_len,
                               const uint8_t* weight_bytes, size_t weight_len, size_t m,
                               size_t in_features, size_t out_features, float* output,
                               size_t output_len);
/* Additive extension (no reference counterpart): Q6_K weights kept resident.
 * The reference dequantizes Q6_K at load (parser.rs:321-325, dequantize_q6k
 * :510-547) and runs the F32 Linear path; this computes the same product
 * straight from the 210-byte super-blocks (GEMVs below 16 rows, the
 * matrix-core tile GEMM from 16 rows as for Q4_K).  in_features % 256 == 0. */
rdl_status rdl_matmul_f32_q6_k(const float* input_data, size_t input_len,
                               const uint8_t* weight_bytes, size_t weight_len, size_t m,
                               size_t in_features, size_t out_features, float* output,
                               size_t output_len);

/* replaces quantize_row_q8_0, quantize.rs:164-193.  Byte-exact: output holds
 * input_len/32 blocks of [f16 scale][32 x i8], scales the f16-rounded scales. */
rdl_status rdl_quantize_row_q8_0(const float* input, size_t input_len, uint8_t* output,
                                 size_t output_len, float* scales, size_t scales_len);

/* Debug view of matmul_f32_q4_native's integer stage (quantize.rs:383):
 * partials[(r*out_features + c)*(in_features/32) + b] = dot_q4q8_block(W[c,b], q8(x_r)[b]),
 * the exact int32 value the reference accumulates before scaling. */
rdl_status rdl_q4_0_q8_0_block_dots(const float* input_data, size_t input_len,
                                    const uint8_t* weight_bytes, size_t weight_len, size_t m,
                                    size_t in_features, size_t out_features, int32_t* partials,
                                    size_t partials_len);

/* ---- device-resident weights ---------------------------------------------
 * A weight handle owns (or wraps) the GGUF-layout bytes of one [N, K] matrix
 * in HBM; the reference equivalent is Linear::weight (linear.rs:14) whose
 * bytes come from Tensor::as_raw_bytes (rustml/core/main/src/core/tensor/tensor.rs:413-422). */
typedef struct rdl_weight rdl_weight;

/* Copy host bytes into a new device allocation. */
rdl_status rdl_weight_upload(const uint8_t* bytes, size_t len, int32_t dtype,
                             size_t out_features, size_t in_features, rdl_weight** out);
/* Wrap caller-owned device bytes (no copy; the caller keeps them alive). */
rdl_status rdl_weight_wrap_device(const void* dev_bytes, size_t len, int32_t dtype,
                                  size_t out_features, size_t in_features, rdl_weight** out);
/* Free a handle (and its allocation when it owns one).  NULL is a no-op. */
rdl_status rdl_weight_free(rdl_weight* w);

/* Linear::forward for a device-resident weight (linear.rs:119-177 minus the bias,
 * which Llama does not use): y_dev[m, N] = x_dev[m, K] . W^T.  mode is
 * RDL_MODE_FLOAT or RDL_MODE_NATIVE (NATIVE applies to Q4_0 and Q4_1 only, as in
 * the reference).  Batch-1..small m runs the decode GEMV; larger m the MFMA GEMM.
 * Scratch (the prefill GEMM's activation split or K-slice partials, activation
 * records of the other paths) comes from work memory the library keeps per
 * (device, stream), shared by all handles used on that stream: allocated by
 * the stream's first call that needs it and grown (hipFree of the old memory
 * waits for the device) by a call that needs more, never otherwise; held
 * until the process ends.  Under HIP graph capture of the stream the call
 * instead records stream-ordered allocation and free nodes (and a kernel that
 * zeroes the GEMM's counters), so every replay owns its scratch. */
rdl_status rdl_linear_forward_dev(const rdl_weight* w, const float* x_dev, size_t m,
                                  float* y_dev, int32_t mode, void* stream);

/* rdl_linear_forward_dev plus Linear::forward's optional F32 bias
 * (linear.rs:172-176, output.add(bias)): y_dev[i][j] = product + bias_dev[j],
 * one f32 add an output, as a second launch on the stream after the product.
 * bias_dev: out_features floats on the device, or NULL (then exactly
 * rdl_linear_forward_dev).  m x out_features must stay below 2^32
 * (RDL_ERR_UNSUPPORTED). */
rdl_status rdl_linear_forward_bias_dev(const rdl_weight* w, const float* x_dev, size_t m,
                                       const float* bias_dev, float* y_dev, int32_t mode, void* stream);

/* Frees the work memory the device entry points keep for `stream` on the
 * current device (rdl_linear_forward_dev and the other device calls above),
 * after waiting for the stream.  No counterpart in the reference: for
 * callers that create and destroy streams (a stream per request), whose
 * streams' work memory would otherwise stay until the process ends; call it
 * before destroying such a stream.  A later call on the stream allocates
 * again.  The caller must not make device calls on the same stream from other
 * threads while this runs (their launches could still be reading the memory
 * freed here).  Not while the stream is being captured into a graph (the
 * wait is refused: RDL_ERR_HIP).  A stream with no work memory: RDL_OK.  Allocation
 * and release (hipMalloc / hipFree, on a stream's first call, on growth, and
 * here) wait for the device, so they must not overlap another thread's
 * graph capture in global capture mode. */
rdl_status rdl_release_stream_work(void* stream);

/* rdl_linear_forward_dev without any device allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * Where rdl_linear_forward_dev uses its work memory (the activation split or
 * K-slice partials of the prefill GEMM, activation records for m > 4 in
 * native mode or for other types), this entry point uses one static device
 * array of RDL_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; its
 * last 64 KiB hold the prefill GEMM's counters (zero at load, left at zero by
 * every launch).  Products needing more than the rest return
 * RDL_ERR_UNSUPPORTED before launching anything.  Every call on one GPU
 * shares that array: calls that overlap in time on one GPU (other streams,
 * other threads) race and must be serialized by the caller.  Results equal
 * rdl_linear_forward_dev's (same kernels). */
#define RDL_NOALLOC_SCRATCH_BYTES (16u << 20)
rdl_status rdl_linear_forward_dev_noalloc(const rdl_weight* w, const float* x_dev, size_t m,
                                          float* y_dev, int32_t mode, void* stream);

/* Measurement aid, no reference counterpart: one streaming read of `bytes`
 * (a multiple of 16, below 2^31) of device memory at buf_dev by 2 x CUs
 * workgroups, each XOR-folding its contiguous share into out_dev[workgroup]
 * (out_len >= 2 x CUs words).  The HBM read rate of a plain kernel, timed
 * like the product launches (rdl_time_next_launch). */
rdl_status rdl_stream_read_dev(const void* buf_dev, size_t bytes, uint32_t* out_dev, size_t out_len,
                               void* stream);

/* ---- device building blocks ----------------------------------------------
 * The product kernels read activations as per-32-element "records" (an exact
 * 24-bit fixed-point code in float mode, the Q8_0 code of quantize_row_q8_0 in
 * native mode).  A caller that owns its scratch memory (a decode loop, a HIP
 * graph) prepares the records itself and reuses them for every weight that
 * consumes the same activations (q/k/v, gate/up).  No reference counterpart:
 * this is the split of Linear::forward's work at the record boundary. */

/* Bytes of the record buffer for m activation rows of length k in `mode`. */
size_t rdl_activation_record_bytes(size_t m, size_t k, int32_t mode);
/* x_dev f32 [m, k] -> rec_dev (rdl_activation_record_bytes bytes, 16-byte aligned). */
rdl_status rdl_prepare_activations_dev(const float* x_dev, size_t m, size_t k, int32_t mode,
                                       void* rec_dev, void* stream);
/* y_dev[m, N] = W . x from prepared records (same mode they were prepared in). */
rdl_status rdl_linear_prepared_dev(const rdl_weight* w, const void* rec_dev, size_t m,
                                   float* y_dev, int32_t mode, void* stream);

/* Fused decode-loop Linear, Q4_0 weights, float mode (the GEMV of
 * matmul_f32_q4, quantize.rs:265-320), m <= 4 rows, in_features / 32 even:
 *   prologue RDL_PROLOGUE_NONE:    x as given;
 *   prologue RDL_PROLOGUE_RMSNORM: rms_norm(x, gamma, eps) per row first
 *     (Tensor::rms_norm, rustml/core/main/src/core/tensor/ops.rs:688-751);
 *   prologue RDL_PROLOGUE_SWIGLU:  silu(x[:, :k]) * x[:, k:2k] first, each x
 *     row holding [gate | up] (FeedForward::forward, feed_forward.rs:138-150);
 *   epilogue RDL_EPILOGUE_STORE:    y = result;
 *   epilogue RDL_EPILOGUE_RESIDUAL: y += result (Tensor::add_inplace,
 *     transformer_block.rs:333,352), y read before it is written;
 *   epilogue RDL_EPILOGUE_SWIGLU:   the weight rows 2j, 2j+1 are gate_j, up_j
 *     and y[j] = silu(result[2j]) * result[2j+1] (y rows out_features/2 long;
 *     out_features even, in_features <= 8192).
 * x_stride = floats between x rows (>= k, >= 2k for the SWIGLU prologue;
 * multiple of 4; x 16-byte aligned).  No counterpart in the reference: there
 * these are separate tensor operations; here one launch, no scratch memory. */
enum { RDL_PROLOGUE_NONE = 0, RDL_PROLOGUE_RMSNORM = 1, RDL_PROLOGUE_SWIGLU = 2 };
enum { RDL_EPILOGUE_STORE = 0, RDL_EPILOGUE_RESIDUAL = 1, RDL_EPILOGUE_SWIGLU = 2 };
rdl_status rdl_linear_fused_dev(const rdl_weight* w, const float* x_dev, size_t x_stride, size_t m,
                                float* y_dev, int32_t prologue, const float* gamma_dev, float eps,
                                int32_t epilogue, void* stream);

/* quantize_row_q8_0 on device: x_dev f32 [n] -> out_dev (n/32)*34 bytes and
 * scales_dev f32 [n/32] (scales_dev may be NULL). */
rdl_status rdl_quantize_row_q8_0_dev(const float* x_dev, size_t n, uint8_t* out_dev,
                                     float* scales_dev, void* stream);

/* Tensor::to_f32 for Q4_0 / Q4_1 / Q8_0 rows (tensor.rs:535-639),
 * dequantize_q4k for Q4_K rows (rustml/gguf/main/src/core/parser.rs:549-593)
 * and dequantize_q6k for Q6_K rows (parser.rs:510-547): dequantize the rows
 * `row_ids[0..n_rows)` (int32, device, each < N) of a weight into out_dev f32
 * [n_rows, K], bit-exact.  This is the embedding gather of the decode loop
 * (rustml/nn/main/src/core/embedding.rs:50-76) on a matrix kept quantized,
 * and the load-time F32 expansion of K-quant tensors (parser.rs:321-325) when
 * a caller wants it. */
rdl_status rdl_dequantize_rows_dev(const rdl_weight* w, const int32_t* row_ids_dev,
                                   size_t n_rows, float* out_dev, void* stream);

/* Debug/device form of rdl_q4_0_q8_0_block_dots (one activation row). */
rdl_status rdl_q4_0_q8_0_block_dots_dev(const rdl_weight* w, const float* x_dev,
                                        int32_t* partials_dev, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* RDL_QUANT_H */
