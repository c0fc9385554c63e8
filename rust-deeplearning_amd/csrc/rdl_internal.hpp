// rdl_internal.hpp -- declarations shared by the HIP translation units of
// librdlquant.so (kernels, launchers and the C ABI).  Not part of the ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <initializer_list>

#include "../../include/rdl_quant.h"

// HIP_TRY for functions returning rdl_status: a failing HIP call sets the
// thread's last-error text and returns RDL_ERR_HIP.
#define HIP_TRY(expr)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess)                                                                  \
            return ::rdl::api_fail(RDL_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

namespace rdl {

// Error reporting shared by the C ABI translation units (capi.hip).
rdl_status api_fail(rdl_status st, const char* fmt, ...);
// RDL_ERR_SHAPE_MISMATCH with the extents QuantError::ShapeMismatch carries
// (expected, actual: at most RDL_SHAPE_MAX_DIMS values each), kept for
// rdl_last_shape_mismatch; the text reads "<what>: expected [..], got [..]".
rdl_status api_shape_fail(const char* what, const size_t* expected, size_t n_expected, const size_t* actual,
                          size_t n_actual);
inline rdl_status api_shape_fail(const char* what, std::initializer_list<size_t> expected,
                                 std::initializer_list<size_t> actual) {
    return api_shape_fail(what, expected.begin(), expected.size(), actual.begin(), actual.size());
}
rdl_status api_ok();
rdl_status api_require_device();

// GGUF block geometry (rustml/quant/main/src/api/types.rs:1-17,
// rustml/gguf/main/src/api/types.rs:54-76).
constexpr int QK = 32;          // elements per Q4_0 / Q4_1 / Q8_0 block
constexpr int Q4_0_BYTES = 18;  // [f16 d][16 B nibbles]
constexpr int Q4_1_BYTES = 20;  // [f16 d][f16 m][16 B nibbles]
constexpr int Q8_0_BYTES = 34;  // [f16 d][32 x i8]
constexpr int QK_K = 256;       // elements per Q4_K / Q6_K super-block
constexpr int Q4_K_BYTES = 144; // [f16 d][f16 dmin][12 B scales][128 B nibbles]
constexpr int Q6_K_BYTES = 210; // [128 B ql][64 B qh][16 x i8 scales][f16 d]

// ---------------------------------------------------------------------------
// Prepared activations.
//
// The GEMV/GEMM kernels never read f32 activations directly: a small pass
// converts each 32-element block of x into a record the integer dot units
// (v_dot4_i32_i8) consume.
//
// FloatRec (float mode, 128 B): x_j ~= S * (a_j + b_j/256 + c_j/65536) with
// S = amax/127 and signed 8-bit digits a, b, c (a 24-bit fixed-point code per
// block; absolute error <= amax * 2^-23 per element).  A block dot against
// integer weights q_j is then S * (A + (B + C/256)/256) with A = sum q_j a_j,
// etc., computed exactly in int32.  sa/sb/sc are sum(a), sum(b), sum(c) (for
// the Q4_0 "-8" offset) and xsum is sum(x_j) in f32 (for Q4_1/Q4_K minimums).
// A block holding a NaN or Inf gets S = NaN, which makes every output it
// touches NaN.
//
// NativeRec (native mode, 48 B): the Q8_0 quantization of the block exactly as
// quantize_row_q8_0 (quantize.rs:164-193) produces it: q8 bytes, the
// f16-rounded scale as f32, and sum(q8).
// ---------------------------------------------------------------------------
struct alignas(16) FloatRec {
    int32_t a[8];
    int32_t b[8];
    int32_t c[8];
    float S;
    int32_t sa, sb, sc;
    float xsum;
    int32_t pad[3];
};
static_assert(sizeof(FloatRec) == 128, "FloatRec layout");

struct alignas(16) NativeRec {
    int32_t q[8];
    float scale;
    int32_t qsum;
    int32_t pad[2];
};
static_assert(sizeof(NativeRec) == 48, "NativeRec layout");

enum class WType : int { Q4_0 = 2, Q4_1 = 3, Q8_0 = 8, Q4_K = 12, Q6_K = 14 };

inline size_t block_elems(WType t) { return (t == WType::Q4_K || t == WType::Q6_K) ? QK_K : QK; }
inline size_t block_bytes(WType t) {
    switch (t) {
        case WType::Q4_0: return Q4_0_BYTES;
        case WType::Q4_1: return Q4_1_BYTES;
        case WType::Q8_0: return Q8_0_BYTES;
        case WType::Q4_K: return Q4_K_BYTES;
        case WType::Q6_K: return Q6_K_BYTES;
    }
    return 0;
}

// ---- host -> device staging ------------------------------------------------
// Two pinned buffers of CHUNK bytes: the host copy of one chunk into a buffer
// overlaps the DMA of the other buffer's chunk.  Used to move GGUF tensor
// bytes from a file mapping into HBM.  Not thread-safe; synchronous (returns
// once every byte has reached the device).
struct Stager {
    static constexpr size_t CHUNK = (size_t)32 << 20;
    uint8_t* buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    ~Stager();
    hipError_t init();
    // `rows` rows of row_bytes each, packed in src, to dst with row pitch
    // dpitch (dpitch == row_bytes: one packed copy of any length; otherwise
    // row_bytes <= CHUNK).
    hipError_t copy2d(const void* src, size_t row_bytes, size_t rows, void* dst, size_t dpitch, hipStream_t s);
};

// ---- kernel-boundary timing -----------------------------------------------
// When set (rdl_time_next_launch), the next product-kernel launch of this
// thread records its start/end into these events via hipExtLaunchKernel.
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local LaunchEvents g_launch_events;

template <typename F, typename... Args>
inline void launch_kernel(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                          Args... args) {
    LaunchEvents& ev = g_launch_events;
    if (ev.start || ev.stop) {
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, ev.start, ev.stop, 0, args...);
        ev = LaunchEvents{};
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
    }
}

// ---- launchers (return hipSuccess or the launch error) --------------------

// x [m, k] f32 -> FloatRec [m, k/32]
hipError_t launch_prep_float(const float* x, size_t m, size_t k, FloatRec* rec, hipStream_t s);
// x [m, k] f32 -> NativeRec [m, k/32] (rec may be NULL); optionally also the
// Q8_0 bytes [m, k/32 * 34] and the f32 scales [m, k/32] of quantize_row_q8_0.
hipError_t launch_prep_native(const float* x, size_t m, size_t k, NativeRec* rec,
                              uint8_t* q8_bytes, float* scales, hipStream_t s);
// The same quantization as contiguous int8 codes [m, k] and f32 scales [m, k/32].
hipError_t launch_prep_native_codes(const float* x, size_t m, size_t k, int8_t* codes, float* scales,
                                    hipStream_t s);

// y[m, n] = x . W^T from prepared activations, one GEMV per activation row.
hipError_t launch_gemv(WType t, bool native, const uint8_t* w, size_t n, size_t k,
                       const void* xrec, size_t m, float* y, hipStream_t s);

// Single-launch GEMV with the activation preparation fused in (x f32 [m, k],
// 16-byte aligned); valid for k <= fused_max_k(t) and weights of at most
// FUSED_MAX_WEIGHT_BYTES (its loads use 32-bit buffer offsets).
constexpr uint64_t FUSED_MAX_WEIGHT_BYTES = 0x7FFFFF00u;
size_t fused_max_k(WType t);
hipError_t launch_gemv_fused(WType t, bool native, const uint8_t* w, size_t n, size_t k,
                             const float* x, size_t m, float* y, hipStream_t s);

// Compute units of the current device (queried once; 256 on MI355X).
int device_cu_count();

// Prefill GEMM for Q4_0 weights on the matrix cores: y[m, n] = x[m, k] . W^T.
// Float mode (matmul_f32_q4): `scratch` holds gemm_scratch_bytes(m, n, k,
// false) bytes (the f16 x split; for m <= GEMM_SMALL_M the skinny kernel's
// K-slice partials, none when it runs unsplit) and `counters` points to
// gemm_counter_count(n, k) ints that are zero before the first call and that
// every call leaves at zero (memory no other code writes; NULL runs the
// skinny kernels unsplit).  Native mode (matmul_f32_q4_native): x quantized
// to Q8_0 codes, int8 MFMA block dots; gemm_scratch_bytes(m, n, k, true)
// bytes of scratch; partials != NULL writes the int32 block dots to
// partials[(i * n + j) * (k / 32) + b] instead of y.
constexpr size_t GEMM_SMALL_M = 64;
constexpr size_t GEMM_XTILE_M = 64;  // float products of at most this many rows: x tiles as MFMA A operands, 128-row strips
constexpr size_t KQ_GEMM_MIN_M = 16;  // Q4_K / Q6_K / Q8_0 / Q4_1 float products of at least this many rows: the LDS tile GEMM
size_t gemm_scratch_bytes(size_t m, size_t n, size_t k, bool native);
// ints of the GEMM's strip counters for out_features n, in_features k
size_t gemm_counter_count(size_t n, size_t k);
// Zeroes `count` GEMM counters with a kernel (no memset node under graph capture).
hipError_t launch_zero_counters(int* counters, size_t count, hipStream_t s);
// The skinny / x-tile GEMMs' K-slice combine: on = every launch takes the
// agent-coherent combine (a testing switch; off: XCD-local where the probed
// placement holds).
void set_combine_coherent(bool on);
bool combine_is_coherent();
// True when the current device's next combine runs XCD-local (placement
// probed and a rotation, switch off); does not probe.
bool combine_local_now();
hipError_t launch_gemm_q4_0(const uint8_t* w, size_t n, size_t k, const float* x, size_t m, float* y,
                            void* scratch, int* counters, hipStream_t s);
hipError_t launch_gemm_q4_0_native(const uint8_t* w, size_t n, size_t k, const float* x, size_t m, float* y,
                                   int32_t* partials, void* scratch, hipStream_t s);
// Float-mode products on the LDS tile GEMM, Q4_0 (more than GEMM_XTILE_M
// rows), Q4_K, Q6_K, Q8_0 or Q4_1 weights (any row count; k a multiple of
// the block, k <= 16384), with the decoder's neighbouring steps folded in; hipErrorInvalidValue
// (nothing launched) for shapes it does not take.  x rows go through pro 1
// RMSNorm (weights g, eps; x [m, k]) or pro 2 SwiGLU (x [m, 2k] interleaved
// gate / up) before the product (pro 0: none); accumulate: y += product (the
// residual add) instead of y = product.  scratch: gemm_tiles_scratch_bytes(m,
// k) bytes (Q4_0 needs only gemm_scratch_bytes(m, n, k, false) of them).
hipError_t launch_gemm_tiles_ex(WType t, const uint8_t* w, size_t n, size_t k, const float* x, size_t m, float* y,
                                void* scratch, int pro, const float* g, float eps, bool accumulate, hipStream_t s);
size_t gemm_tiles_scratch_bytes(size_t m, size_t k);
// The float-mode product y = x W^T of Q4_K, Q6_K, Q8_0 or Q4_1 weights on
// the LDS tile GEMM (the reference's dequantize_q4k / dequantize_q6k + F32
// matmul, parser.rs:510-593; matmul_f32_q8, quantize.rs:201-260;
// matmul_f32_q4_1, quantize.rs:429-495).
hipError_t launch_gemm_typed(WType t, const uint8_t* w, size_t n, size_t k, const float* x, size_t m, float* y,
                             void* scratch, hipStream_t s);

// Decoder fusion of the Q4_0 float-mode fused GEMV (m <= 4, k / 32 even,
// x 16-byte aligned): prologue 0 none, 1 RMSNorm with weights g and eps,
// 2 SwiGLU of [gate | up] x rows (row stride xstride >= 2k); epilogue 0 y = W x,
// 1 y += W x, 2 y[j] = silu(W x)[2j] * (W x)[2j+1] (n even, y rows n/2 long).
hipError_t launch_gemv_q4_0_fused_ex(const uint8_t* w, size_t n, size_t k, const float* x, size_t xstride,
                                     size_t m, float* y, int prologue, const float* g, float eps,
                                     int epilogue, hipStream_t s);

// prologue / epilogue codes of the decoder-fusion launches
constexpr int GEMV_PRO_NONE = 0, GEMV_PRO_RMSNORM = 1;
constexpr int GEMV_EPI_STORE = 0, GEMV_EPI_RESIDUAL = 1, GEMV_EPI_SWIGLU = 2;

// Decoder fusion of the Q4_K / Q6_K fused GEMVs (m <= 4, k % 256 == 0, x and
// g 16-byte aligned, x rows xstride floats apart, y rows ystride): (prologue,
// epilogue) = (0, 0) y = W x, (1, 0) y = W rms_norm(x, g), (0, 1) y += W x,
// (1, 2) y[j] = silu(v[2j]) * v[2j+1] with v = W rms_norm(x, g) (n even).
hipError_t launch_gemv_kquant_ex(WType t, const uint8_t* w, size_t n, size_t k, const float* x, size_t xstride,
                                 size_t m, float* y, size_t ystride, int prologue, const float* g, float eps,
                                 int epilogue, hipStream_t s);

// The decoder's q/k/v projection in one launch: y = rms_norm(x, g) . [Wq; Wk; Wv]^T
// with RoPE at positions *pos + row applied to q (in y) and k, and k, v
// written into the paged cache (pages of KV_PAGE positions through kv_table,
// [n_pages][n_kv][KV_PAGE][hd] per layer, f16 or f32); m <= 4.
hipError_t launch_gemv_q4_0_rope_kv(const uint8_t* w, size_t n, size_t k, const float* x, size_t m, float* y,
                                    const float* g, float eps, const int* pos, const float* cos_t,
                                    const float* sin_t, void* kc, void* vc, int n_heads, int n_kv, int hd,
                                    const int* kv_table, bool kv_f16, hipStream_t s);

// launch_gemv_q4_0_rope_kv for one activation row (a decode step) with the
// decode attention of that row in the same launch: att_out[n_heads * hd] =
// attention over the cache positions 0 .. *pos (paged, kv_table), spans of
// ATT_SPAN keys combined through att_part ([n_heads][nspan][hd + 2]) /
// att_cnt as the attention launch does, `spans` span workgroups a head (those
// past the position exit at once); xch = the layer's exchange of n tagged
// q / k / v words (zero on an empty cache; *pos must grow from one launch on
// the same exchange to the next), err = a flag set if a wait runs out.
// With wo set, the same launch also applies the o projection: x_res[n_o] +=
// att W_o^T (W_o Q4_0, n_heads * hd columns), the attention outputs passing
// through oxch (n_heads * hd tagged words, same rules as xch) instead of
// att_out; the results equal the separate o launch's bit for bit.
// With wd set as well, the launch starts with the previous layer's down
// projection x_res[k] += h W_d^T (W_d Q4_0, k_d columns, h the SwiGLU row):
// its results reach the q/k/v workgroups (whose weight loads run meanwhile)
// and the o workgroups as tagged words through xx ([k], same rules as xch),
// and x_res is written once, by the o projection; the results equal the
// separate down launch's and this launch's without it bit for bit.
// hipErrorInvalidValue for shapes it does not take (then use
// launch_gemv_q4_0_rope_kv, the attention launch and the o launch).
hipError_t launch_qkv_attention(const uint8_t* w, size_t n, size_t k, const float* x, float* y, const float* g,
                                float eps, const int* pos, const float* cos_t, const float* sin_t, void* kc, void* vc,
                                const int* kv_table, int n_heads, int n_kv, int hd, bool kv_f16, float* att_part,
                                int nspan, int spans, int* att_cnt, float* att_out, uint64_t* xch, int* err,
                                const uint8_t* wo, size_t n_o, float* x_res, uint64_t* oxch, hipStream_t s,
                                const uint8_t* wd = nullptr, size_t k_d = 0, const float* h = nullptr,
                                uint64_t* xx = nullptr);

// launch_gemv_q4_0_rope_kv for a Q4_K or Q6_K [Wq; Wk; Wv], or for the rows of
// heads head0 .. head0 + n / hd - 1 of it (head0 = 0, or past the q heads:
// [Wq; Wk] and Wv as two launches): m <= 4 activation rows (k floats apart)
// at positions *pos + row0 + row, q rows ystride apart.
hipError_t launch_gemv_kquant_rope_kv(WType t, const uint8_t* w, size_t n, size_t k, const float* x, size_t m,
                                      size_t row0, float* y, size_t ystride, const float* g, float eps,
                                      const int* pos, const float* cos_t, const float* sin_t, void* kc, void* vc,
                                      int n_heads, int n_kv, int hd, int head0, const int* kv_table, bool kv_f16,
                                      hipStream_t s);

// int32 block partials of the Q4_0 x Q8_0 path for one activation row.
hipError_t launch_q4_0_block_dots(const uint8_t* w, size_t n, size_t k, const NativeRec* rec,
                                  int32_t* partials, hipStream_t s);

// GGMLType block geometry (elements, bytes per block); false for unknown ids.
bool ggml_geometry(int32_t ggml_type, int* block_size, int* block_bytes);
// Any GGML tensor type to f32 (load_tensors + Tensor::to_f32): the whole
// blocks of n_elements, zeros after them; dst 16-byte aligned.
hipError_t launch_dequant_gguf(int32_t ggml_type, const uint8_t* src, size_t n_elements, float* dst,
                               hipStream_t s);

// y[i][j] += bias[j] for m rows of n (m * n < 2^32).
hipError_t launch_bias_add(float* y, const float* bias, size_t m, size_t n, hipStream_t s);

// Dequantize selected rows of a Q4_0 / Q4_1 / Q8_0 matrix to f32.
hipError_t launch_dequant_rows(WType t, const uint8_t* w, size_t n, size_t k,
                               const int32_t* rows, size_t n_rows, float* out, hipStream_t s);

}  // namespace rdl
