// capi.hip -- the extern "C" boundary of librdlquant.so (include/rdl_quant.h).
//
// Argument checks follow the reference's error behaviour
// (rustml/quant/main/src/core/quantize.rs:208-213, 272-277, 333-338: K % 32 is
// checked first and reported as QuantError::BlockAlignment) and add the
// slice-length checks the reference leaves to a panic.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/rdl_quant.h"
#include "../../include/rdl_gguf.h"
#include "rdl_internal.hpp"

namespace rdl {
thread_local LaunchEvents g_launch_events;
}

using rdl::FloatRec;
using rdl::NativeRec;
using rdl::WType;

struct rdl_weight {
    void* dev;
    size_t len;
    WType type;
    size_t n, k;
    bool owned;
};

namespace rdl {

thread_local std::string g_err;

// The extents of the calling thread's last RDL_ERR_SHAPE_MISMATCH (n_* = 0:
// the last status was something else).
struct ShapeDetail {
    size_t expected[RDL_SHAPE_MAX_DIMS], actual[RDL_SHAPE_MAX_DIMS];
    size_t n_expected, n_actual;
};
thread_local ShapeDetail g_shape{};

rdl_status api_fail(rdl_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    g_shape.n_expected = g_shape.n_actual = 0;
    return st;
}

rdl_status api_shape_fail(const char* what, const size_t* expected, size_t n_expected, const size_t* actual,
                          size_t n_actual) {
    auto list = [](const size_t* v, size_t n) {
        std::string t = "[";
        for (size_t i = 0; i < n; i++) t += (i ? ", " : "") + std::to_string(v[i]);
        return t + "]";
    };
    g_err = std::string(what) + ": expected " + list(expected, n_expected) + ", got " + list(actual, n_actual);
    ShapeDetail d{};
    d.n_expected = std::min<size_t>(n_expected, RDL_SHAPE_MAX_DIMS);
    d.n_actual = std::min<size_t>(n_actual, RDL_SHAPE_MAX_DIMS);
    for (size_t i = 0; i < d.n_expected; i++) d.expected[i] = expected[i];
    for (size_t i = 0; i < d.n_actual; i++) d.actual[i] = actual[i];
    g_shape = d;
    return RDL_ERR_SHAPE_MISMATCH;
}

rdl_status api_ok() {
    g_err.clear();
    g_shape.n_expected = g_shape.n_actual = 0;
    return RDL_OK;
}

}  // namespace rdl

namespace {

using rdl::g_err;
constexpr auto fail = rdl::api_fail;
constexpr auto ok = rdl::api_ok;

const char* type_name(WType t) {
    switch (t) {
        case WType::Q4_0: return "Q4_0";
        case WType::Q4_1: return "Q4_1";
        case WType::Q8_0: return "Q8_0";
        case WType::Q4_K: return "Q4_K";
        case WType::Q6_K: return "Q6_K";
    }
    return "?";
}

bool valid_type(int32_t d) {
    return d == RDL_DTYPE_Q4_0 || d == RDL_DTYPE_Q4_1 || d == RDL_DTYPE_Q8_0 || d == RDL_DTYPE_Q4_K ||
           d == RDL_DTYPE_Q6_K;
}

// Visible gfx950 devices; 0 without a GPU.
int count_devices() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    int good = 0;
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) == hipSuccess && strncmp(p.gcnArchName, "gfx950", 6) == 0)
            good++;
    }
    return good;
}

}  // namespace

rdl_status rdl::api_require_device() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fail(RDL_ERR_NO_DEVICE, "no HIP device is visible");
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return fail(RDL_ERR_NO_DEVICE, "hipGetDevice failed");
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, cur) != hipSuccess)
        return fail(RDL_ERR_NO_DEVICE, "hipGetDeviceProperties failed");
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(RDL_ERR_NO_DEVICE, "device %d is %s, this library is built for gfx950", cur,
                    p.gcnArchName);
    return RDL_OK;
}

namespace {

constexpr auto require_device = rdl::api_require_device;

// Shape checks shared by every matmul entry point.
rdl_status check_matmul(WType t, const float* x, size_t x_len, const uint8_t* w, size_t w_len,
                        size_t m, size_t k, size_t n, const void* y, size_t y_len) {
    const size_t be = rdl::block_elems(t);
    if (k % be != 0)
        return fail(RDL_ERR_BLOCK_ALIGNMENT, "in_features %zu not divisible by %s block size %zu", k,
                    type_name(t), be);
    // With no output rows or columns the reference never slices its inputs.
    if (m == 0 || n == 0) return RDL_OK;
    const size_t need_w = n * (k / be) * rdl::block_bytes(t);
    if (w_len < need_w)
        return rdl::api_shape_fail("weight bytes", {need_w}, {w_len});
    if (x_len < m * k)
        return rdl::api_shape_fail("input length", {m * k}, {x_len});
    if (y_len < m * n)
        return rdl::api_shape_fail("output length", {m * n}, {y_len});
    if ((m * k && !x) || (need_w && !w) || (m * n && !y))
        return fail(RDL_ERR_NULL_POINTER, "NULL buffer with non-zero length");
    return RDL_OK;
}

size_t rec_bytes(bool native, size_t m, size_t k) {
    return m * (k / rdl::QK) * (native ? sizeof(NativeRec) : sizeof(FloatRec));
}

// Activation rows up to which one fused launch (prep in LDS + GEMV) is used.
constexpr size_t FUSED_MAX_M = 4;

bool use_fused(WType t, size_t m, size_t n, size_t k, const float* x_dev) {
    return m <= FUSED_MAX_M && k > 0 && k <= rdl::fused_max_k(t) && ((uintptr_t)x_dev & 15) == 0 &&
           (uint64_t)n * (k / rdl::block_elems(t)) * rdl::block_bytes(t) <= rdl::FUSED_MAX_WEIGHT_BYTES;
}

// How a product runs: one fused GEMV launch (m <= 4), the matrix-core GEMM
// (Q4_0, more rows: f16 MFMA in float mode, int8 MFMA in native mode; Q4_K,
// Q6_K, Q8_0 and float-mode Q4_1 from KQ_GEMM_MIN_M rows), or activation
// records + the records GEMV.
enum class Path { Fused, Gemm, Records };

// The GEMM addresses x and W with 32-bit offsets; the x prep of the other
// types holds a row in registers (k <= 16384).
bool gemm_fits(WType t, bool native, size_t m, size_t n, size_t k) {
    if (k == 0 || (uint64_t)m * k * 2 > rdl::FUSED_MAX_WEIGHT_BYTES) return false;
    if (t == WType::Q4_K || t == WType::Q6_K || t == WType::Q8_0 || (t == WType::Q4_1 && !native)) {
        const size_t be = rdl::block_elems(t);
        return m >= rdl::KQ_GEMM_MIN_M && k % be == 0 && k <= 16384 &&
               (uint64_t)n * (k / be) * rdl::block_bytes(t) <= rdl::FUSED_MAX_WEIGHT_BYTES;
    }
    return t == WType::Q4_0 && (uint64_t)n * (k / rdl::QK) * rdl::Q4_0_BYTES <= rdl::FUSED_MAX_WEIGHT_BYTES;
}

Path pick_path(WType t, bool native, size_t m, size_t n, size_t k, const float* x_dev) {
    if (use_fused(t, m, n, k, x_dev)) return Path::Fused;
    if (gemm_fits(t, native, m, n, k)) return Path::Gemm;
    return Path::Records;
}

size_t scratch_bytes(WType t, Path p, bool native, size_t m, size_t n, size_t k) {
    switch (p) {
        case Path::Fused: return 0;
        case Path::Gemm:
            return t == WType::Q4_0 ? rdl::gemm_scratch_bytes(m, n, k, native) : rdl::gemm_tiles_scratch_bytes(m, k);
        case Path::Records: return rec_bytes(native, m, k);
    }
    return 0;
}

// Run the product on `s`; `work` holds scratch_bytes(path) bytes of device
// memory, `counters` gemm_counter_count(n, k) ints of the GEMM (zero between calls).
rdl_status run_linear(WType t, bool native, const uint8_t* w_dev, size_t n, size_t k,
                      const float* x_dev, size_t m, float* y_dev, void* work, int* counters, hipStream_t s,
                      Path path) {
    if (m == 0 || n == 0) return RDL_OK;
    // k == 0: no blocks; the GEMV then writes zeros (empty dot, as in the reference).
    if (k == 0) {
        HIP_TRY(rdl::launch_gemv(t, native, w_dev, n, k, work, m, y_dev, s));
        return RDL_OK;
    }
    if (path == Path::Fused) {
        HIP_TRY(rdl::launch_gemv_fused(t, native, w_dev, n, k, x_dev, m, y_dev, s));
        return RDL_OK;
    }
    if (path == Path::Gemm) {
        if (t != WType::Q4_0)
            HIP_TRY(rdl::launch_gemm_typed(t, w_dev, n, k, x_dev, m, y_dev, work, s));
        else if (native)
            HIP_TRY(rdl::launch_gemm_q4_0_native(w_dev, n, k, x_dev, m, y_dev, nullptr, work, s));
        else
            HIP_TRY(rdl::launch_gemm_q4_0(w_dev, n, k, x_dev, m, y_dev, work, counters, s));
        return RDL_OK;
    }
    void* xrec = work;
    if (native)
        HIP_TRY(rdl::launch_prep_native(x_dev, m, k, (NativeRec*)xrec, nullptr, nullptr, s));
    else
        HIP_TRY(rdl::launch_prep_float(x_dev, m, k, (FloatRec*)xrec, s));
    HIP_TRY(rdl::launch_gemv(t, native, w_dev, n, k, xrec, m, y_dev, s));
    return RDL_OK;
}

// ---- static scratch of rdl_linear_forward_dev_noalloc ----------------------
// One array per device, for callers that cannot allocate.  In host code the
// name `scratch` is only a stand-in for the symbol: its device address comes
// from hipGetSymbolAddress, taken once per device (with that device current)
// and kept in scratch_dev[]; only that address is ever passed to kernels.
__device__ __align__(256) uint8_t scratch[RDL_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_dev[MAX_DEVICES] = {};

// The last NOALLOC_COUNTER_BYTES of `scratch` hold the prefill GEMM's counters
// (zero from load time and left at zero by every launch); nothing else is
// ever written there.
constexpr size_t NOALLOC_COUNTER_BYTES = 64 * 1024;
constexpr size_t NOALLOC_DATA_BYTES = (size_t)RDL_NOALLOC_SCRATCH_BYTES - NOALLOC_COUNTER_BYTES;

// The current device's address of `scratch`.
rdl_status noalloc_scratch(void** out) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES) return fail(RDL_ERR_UNSUPPORTED, "device index %d beyond %d", dev, MAX_DEVICES);
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_dev[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(RDL_ERR_HIP, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
        scratch_dev[dev] = p;
    }
    *out = scratch_dev[dev];
    return RDL_OK;
}

// RAII device buffer for the synchronous host entry points.
struct DevBuf {
    void* p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    hipError_t alloc(size_t bytes) { return hipMalloc(&p, bytes ? bytes : 4); }
};

// Work memory of the device entry points, one per (device, stream) and
// shared by every weight handle used on that stream (calls on one stream run
// in order; calls on two streams get two): scratch grown to the largest call
// so far, and the prefill GEMM's counters (zeroed when allocated, left at
// zero by every launch), grown to the largest out_features so far.  Growth
// frees the old memory with hipFree, which waits for the device; calls that
// fit allocate nothing.  Held until the process ends.
struct StreamWork {
    int dev;
    hipStream_t stream;
    void* p;
    size_t bytes;
    int* counters;
    size_t ncnt;
};
std::mutex work_mu;
std::vector<StreamWork> work_pool;

rdl_status stream_work(hipStream_t s, size_t bytes, size_t ncnt, void** p, int** counters) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(work_mu);
    StreamWork* e = nullptr;
    for (auto& x : work_pool)
        if (x.dev == dev && x.stream == s) e = &x;
    if (!e) {
        work_pool.push_back({dev, s, nullptr, 0, nullptr, 0});
        e = &work_pool.back();
    }
    if (bytes > e->bytes) {
        if (e->p) HIP_TRY(hipFree(e->p));
        e->p = nullptr;
        e->bytes = 0;
        HIP_TRY(hipMalloc(&e->p, bytes));
        e->bytes = bytes;
    }
    if (ncnt > e->ncnt) {
        if (e->counters) HIP_TRY(hipFree(e->counters));
        e->counters = nullptr;
        e->ncnt = 0;
        HIP_TRY(hipMalloc(&e->counters, ncnt * sizeof(int)));
        HIP_TRY(hipMemset(e->counters, 0, ncnt * sizeof(int)));
        e->ncnt = ncnt;
    }
    *p = e->p;
    *counters = e->counters;
    return RDL_OK;
}

// Device memory of one call on stream `s`: `bytes` of scratch and, when
// `counters` is wanted, the GEMM counters.  Outside graph capture they are
// the stream's work memory.  Under capture (where hipMalloc is not
// allowed) the call takes stream-ordered memory that the graph allocates and
// frees on every replay, with the counters zeroed by a kernel; release()
// frees it after the call's launches.
struct CallWork {
    void* p = nullptr;
    int* counters = nullptr;
    bool graph_owned = false;
    rdl_status get(const rdl_weight* w, hipStream_t s, size_t bytes, bool want_counters) {
        if (!bytes && !want_counters) return RDL_OK;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        HIP_TRY(hipStreamIsCapturing(s, &cs));
        if (cs != hipStreamCaptureStatusActive) {
            void* q = nullptr;
            int* c = nullptr;
            rdl_status st = stream_work(s, bytes, want_counters ? rdl::gemm_counter_count(w->n, w->k) : 0, &q, &c);
            p = q;
            counters = want_counters ? c : nullptr;
            return st;
        }
        const size_t data = (bytes + 255) & ~(size_t)255;
        const size_t nc = want_counters ? rdl::gemm_counter_count(w->n, w->k) : 0;
        HIP_TRY(hipMallocAsync(&p, data + nc * sizeof(int) + 4, s));
        graph_owned = true;
        if (want_counters) {
            counters = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(p) + data);
            HIP_TRY(rdl::launch_zero_counters(counters, nc, s));
        }
        return RDL_OK;
    }
    rdl_status release(hipStream_t s) {
        if (graph_owned && p) HIP_TRY(hipFreeAsync(p, s));
        p = nullptr;
        return RDL_OK;
    }
};

rdl_status host_matmul(WType t, bool native, const float* x, size_t x_len, const uint8_t* w,
                       size_t w_len, size_t m, size_t k, size_t n, float* y, size_t y_len) {
    rdl_status st = check_matmul(t, x, x_len, w, w_len, m, k, n, y, y_len);
    if (st != RDL_OK) return st;
    if (m == 0 || n == 0) return ok();
    if ((st = require_device()) != RDL_OK) return st;
    const size_t wb = n * (k / rdl::block_elems(t)) * rdl::block_bytes(t);
    DevBuf dx, dw, dy, dr;
    HIP_TRY(dx.alloc(m * k * sizeof(float)));
    HIP_TRY(dw.alloc(wb + 64));
    HIP_TRY(dy.alloc(m * n * sizeof(float)));
    HIP_TRY(hipMemcpy(dx.p, x, m * k * sizeof(float), hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(dw.p, w, wb, hipMemcpyHostToDevice));
    const Path path = pick_path(t, native, m, n, k, (const float*)dx.p);
    const size_t sb = scratch_bytes(t, path, native, m, n, k);
    if (sb) HIP_TRY(dr.alloc(sb));
    DevBuf dc;
    HIP_TRY(dc.alloc(rdl::gemm_counter_count(n, k) * sizeof(int)));
    HIP_TRY(hipMemset(dc.p, 0, rdl::gemm_counter_count(n, k) * sizeof(int)));
    st = run_linear(t, native, (const uint8_t*)dw.p, n, k, (const float*)dx.p, m, (float*)dy.p,
                    dr.p, (int*)dc.p, nullptr, path);
    if (st != RDL_OK) return st;
    HIP_TRY(hipMemcpy(y, dy.p, m * n * sizeof(float), hipMemcpyDeviceToHost));
    return ok();
}

}  // namespace

extern "C" {

const char* rdl_status_string(rdl_status s) {
    switch (s) {
        case RDL_OK: return "ok";
        case RDL_ERR_DTYPE_MISMATCH: return "dtype mismatch";
        case RDL_ERR_SHAPE_MISMATCH: return "shape mismatch";
        case RDL_ERR_BLOCK_ALIGNMENT: return "block alignment error";
        case RDL_ERR_INVALID_DATA: return "invalid data";
        case RDL_ERR_NULL_POINTER: return "null pointer";
        case RDL_ERR_HIP: return "HIP runtime error";
        case RDL_ERR_NO_DEVICE: return "no gfx950 device";
        case RDL_ERR_UNSUPPORTED: return "unsupported shape";
        case RDL_ERR_GGUF_IO: return "IO error";
        case RDL_ERR_GGUF_INVALID_FORMAT: return "Invalid GGUF format";
        case RDL_ERR_GGUF_UNSUPPORTED_TYPE: return "Unsupported GGML type";
        case RDL_ERR_GGUF_MISSING_METADATA: return "Missing metadata";
        case RDL_ERR_NOT_FOUND: return "not found";
    }
    return "unknown status";
}

const char* rdl_last_error(void) { return g_err.c_str(); }

rdl_status rdl_last_shape_mismatch(size_t* expected, size_t* n_expected, size_t* actual, size_t* n_actual) {
    if (!expected || !n_expected || !actual || !n_actual) return RDL_ERR_NULL_POINTER;
    const rdl::ShapeDetail& d = rdl::g_shape;
    if (d.n_expected == 0 && d.n_actual == 0) return RDL_ERR_INVALID_DATA;  // keeps g_err / g_shape as they are
    for (size_t i = 0; i < RDL_SHAPE_MAX_DIMS; i++) {
        expected[i] = i < d.n_expected ? d.expected[i] : 0;
        actual[i] = i < d.n_actual ? d.actual[i] : 0;
    }
    *n_expected = d.n_expected;
    *n_actual = d.n_actual;
    return RDL_OK;
}

const char* rdl_version(void) { return "rdlquant 0.1.0 (gfx950)"; }

int32_t rdl_device_count(void) { return count_devices(); }

rdl_status rdl_set_gemm_combine(int32_t mode) {
    if (mode != RDL_COMBINE_AUTO && mode != RDL_COMBINE_COHERENT)
        return fail(RDL_ERR_INVALID_DATA, "unknown combine mode %d", mode);
    rdl::set_combine_coherent(mode == RDL_COMBINE_COHERENT);
    return ok();
}

rdl_status rdl_get_gemm_combine(int32_t* mode, int32_t* local) {
    if (!mode || !local) return fail(RDL_ERR_NULL_POINTER, "NULL argument");
    *mode = rdl::combine_is_coherent() ? RDL_COMBINE_COHERENT : RDL_COMBINE_AUTO;
    *local = rdl::combine_local_now() ? 1 : 0;
    return ok();
}

rdl_status rdl_time_next_launch(void* start_event, void* stop_event) {
    rdl::g_launch_events.start = (hipEvent_t)start_event;
    rdl::g_launch_events.stop = (hipEvent_t)stop_event;
    return ok();
}

rdl_status rdl_matmul_f32_q8(const float* x, size_t x_len, const uint8_t* w, size_t w_len,
                             size_t m, size_t k, size_t n, float* y, size_t y_len) {
    return host_matmul(WType::Q8_0, false, x, x_len, w, w_len, m, k, n, y, y_len);
}
rdl_status rdl_matmul_f32_q4(const float* x, size_t x_len, const uint8_t* w, size_t w_len,
                             size_t m, size_t k, size_t n, float* y, size_t y_len) {
    return host_matmul(WType::Q4_0, false, x, x_len, w, w_len, m, k, n, y, y_len);
}
rdl_status rdl_matmul_f32_q4_native(const float* x, size_t x_len, const uint8_t* w, size_t w_len,
                                    size_t m, size_t k, size_t n, float* y, size_t y_len) {
    return host_matmul(WType::Q4_0, true, x, x_len, w, w_len, m, k, n, y, y_len);
}
rdl_status rdl_matmul_f32_q4_1(const float* x, size_t x_len, const uint8_t* w, size_t w_len,
                               size_t m, size_t k, size_t n, float* y, size_t y_len) {
    return host_matmul(WType::Q4_1, false, x, x_len, w, w_len, m, k, n, y, y_len);
}
rdl_status rdl_matmul_f32_q4_1_native(const float* x, size_t x_len, const uint8_t* w,
                                      size_t w_len, size_t m, size_t k, size_t n, float* y,
                                      size_t y_len) {
    return host_matmul(WType::Q4_1, true, x, x_len, w, w_len, m, k, n, y, y_len);
}
rdl_status rdl_matmul_f32_q4_k(const float* x, size_t x_len, const uint8_t* w, size_t w_len,
                               size_t m, size_t k, size_t n, float* y, size_t y_len) {
    return host_matmul(WType::Q4_K, false, x, x_len, w, w_len, m, k, n, y, y_len);
}

rdl_status rdl_matmul_f32_q6_k(const float* x, size_t x_len, const uint8_t* w, size_t w_len,
                               size_t m, size_t k, size_t n, float* y, size_t y_len) {
    return host_matmul(WType::Q6_K, false, x, x_len, w, w_len, m, k, n, y, y_len);
}

rdl_status rdl_quantize_row_q8_0(const float* input, size_t input_len, uint8_t* output,
                                 size_t output_len, float* scales, size_t scales_len) {
    if (input_len % rdl::QK != 0)
        return fail(RDL_ERR_BLOCK_ALIGNMENT, "Q8_0 requires element count divisible by 32, got %zu",
                    input_len);
    const size_t nb = input_len / rdl::QK;
    if (output_len < nb * rdl::Q8_0_BYTES)
        return rdl::api_shape_fail("output bytes", {nb * rdl::Q8_0_BYTES}, {output_len});
    if (scales_len < nb)
        return rdl::api_shape_fail("scales length", {nb}, {scales_len});
    if (nb == 0) return ok();
    if (!input || !output || !scales) return fail(RDL_ERR_NULL_POINTER, "NULL buffer");
    rdl_status st = require_device();
    if (st != RDL_OK) return st;
    DevBuf dx, dq, ds;
    HIP_TRY(dx.alloc(input_len * sizeof(float)));
    HIP_TRY(dq.alloc(nb * rdl::Q8_0_BYTES));
    HIP_TRY(ds.alloc(nb * sizeof(float)));
    HIP_TRY(hipMemcpy(dx.p, input, input_len * sizeof(float), hipMemcpyHostToDevice));
    HIP_TRY(rdl::launch_prep_native((const float*)dx.p, 1, input_len, nullptr, (uint8_t*)dq.p,
                                    (float*)ds.p, nullptr));
    HIP_TRY(hipMemcpy(output, dq.p, nb * rdl::Q8_0_BYTES, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(scales, ds.p, nb * sizeof(float), hipMemcpyDeviceToHost));
    return ok();
}

rdl_status rdl_q4_0_q8_0_block_dots(const float* x, size_t x_len, const uint8_t* w, size_t w_len,
                                    size_t m, size_t k, size_t n, int32_t* partials,
                                    size_t partials_len) {
    rdl_status st = check_matmul(WType::Q4_0, x, x_len, w, w_len, m, k, n, partials,
                                 partials_len);
    if (st != RDL_OK) return st;
    const size_t nb = k / rdl::QK;
    if (partials_len < m * n * nb)
        return rdl::api_shape_fail("partials length", {m * n * nb}, {partials_len});
    if (m * n * nb == 0) return ok();
    if ((st = require_device()) != RDL_OK) return st;
    DevBuf dx, dw, dp, dr;
    HIP_TRY(dx.alloc(m * k * sizeof(float)));
    HIP_TRY(dw.alloc(n * nb * rdl::Q4_0_BYTES + 64));
    HIP_TRY(dp.alloc(m * n * nb * sizeof(int32_t)));
    HIP_TRY(hipMemcpy(dx.p, x, m * k * sizeof(float), hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(dw.p, w, n * nb * rdl::Q4_0_BYTES, hipMemcpyHostToDevice));
    if (m > FUSED_MAX_M && gemm_fits(WType::Q4_0, true, m, n, k)) {
        // the rows matmul_f32_q4_native takes to the int8 GEMM: its own MFMA block dots
        HIP_TRY(dr.alloc(rdl::gemm_scratch_bytes(m, n, k, true)));
        HIP_TRY(rdl::launch_gemm_q4_0_native((const uint8_t*)dw.p, n, k, (const float*)dx.p, m, nullptr,
                                             (int32_t*)dp.p, dr.p, nullptr));
    } else {
        HIP_TRY(dr.alloc(m * nb * sizeof(NativeRec)));
        HIP_TRY(rdl::launch_prep_native((const float*)dx.p, m, k, (NativeRec*)dr.p, nullptr, nullptr,
                                        nullptr));
        for (size_t r = 0; r < m; r++)
            HIP_TRY(rdl::launch_q4_0_block_dots((const uint8_t*)dw.p, n, k,
                                                (const NativeRec*)dr.p + r * nb,
                                                (int32_t*)dp.p + r * n * nb, nullptr));
    }
    HIP_TRY(hipMemcpy(partials, dp.p, m * n * nb * sizeof(int32_t), hipMemcpyDeviceToHost));
    return ok();
}

rdl_status rdl_weight_upload(const uint8_t* bytes, size_t len, int32_t dtype,
                             size_t out_features, size_t in_features, rdl_weight** out) {
    if (!out) return fail(RDL_ERR_NULL_POINTER, "out is NULL");
    *out = nullptr;
    if (!valid_type(dtype)) return fail(RDL_ERR_DTYPE_MISMATCH, "unsupported dtype %d", dtype);
    const WType t = (WType)dtype;
    const size_t be = rdl::block_elems(t);
    if (in_features % be)
        return fail(RDL_ERR_BLOCK_ALIGNMENT, "in_features %zu not divisible by %s block size %zu",
                    in_features, type_name(t), be);
    const size_t need = out_features * (in_features / be) * rdl::block_bytes(t);
    if (len < need) return rdl::api_shape_fail("weight bytes", {need}, {len});
    if (need && !bytes) return fail(RDL_ERR_NULL_POINTER, "bytes is NULL");
    rdl_status st = require_device();
    if (st != RDL_OK) return st;
    void* d = nullptr;
    HIP_TRY(hipMalloc(&d, need + 64));
    if (need) {
        hipError_t e = hipMemcpy(d, bytes, need, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(d);
            return fail(RDL_ERR_HIP, "hipMemcpy failed: %s", hipGetErrorString(e));
        }
    }
    *out = new rdl_weight{d, need, t, out_features, in_features, true};
    return ok();
}

rdl_status rdl_weight_wrap_device(const void* dev_bytes, size_t len, int32_t dtype,
                                  size_t out_features, size_t in_features, rdl_weight** out) {
    if (!out) return fail(RDL_ERR_NULL_POINTER, "out is NULL");
    *out = nullptr;
    if (!valid_type(dtype)) return fail(RDL_ERR_DTYPE_MISMATCH, "unsupported dtype %d", dtype);
    const WType t = (WType)dtype;
    const size_t be = rdl::block_elems(t);
    if (in_features % be)
        return fail(RDL_ERR_BLOCK_ALIGNMENT, "in_features %zu not divisible by %s block size %zu",
                    in_features, type_name(t), be);
    const size_t need = out_features * (in_features / be) * rdl::block_bytes(t);
    if (len < need) return rdl::api_shape_fail("weight bytes", {need}, {len});
    if (need && !dev_bytes) return fail(RDL_ERR_NULL_POINTER, "dev_bytes is NULL");
    if (t == WType::Q4_K && ((uintptr_t)dev_bytes & 15))
        return fail(RDL_ERR_INVALID_DATA, "Q4_K device bytes must be 16-byte aligned");
    if ((uintptr_t)dev_bytes & 3)
        return fail(RDL_ERR_INVALID_DATA, "device bytes must be 4-byte aligned");
    rdl_status st = require_device();
    if (st != RDL_OK) return st;
    *out = new rdl_weight{const_cast<void*>(dev_bytes), need, t, out_features, in_features, false};
    return ok();
}

rdl_status rdl_weight_free(rdl_weight* w) {
    if (!w) return ok();
    if (w->owned && w->dev) (void)hipFree(w->dev);
    delete w;
    return ok();
}

rdl_status rdl_linear_forward_dev(const rdl_weight* w, const float* x_dev, size_t m, float* y_dev,
                                  int32_t mode, void* stream) {
    if (!w) return fail(RDL_ERR_NULL_POINTER, "weight handle is NULL");
    if (mode != RDL_MODE_FLOAT && mode != RDL_MODE_NATIVE)
        return fail(RDL_ERR_INVALID_DATA, "unknown mode %d", mode);
    if (m == 0 || w->n == 0) return ok();
    if (!x_dev || !y_dev) return fail(RDL_ERR_NULL_POINTER, "NULL activation pointer");
    // Linear::forward honours use_native_q4 only for Q4_0 / Q4_1 (linear.rs:128-153).
    const bool native = mode == RDL_MODE_NATIVE && (w->type == WType::Q4_0 || w->type == WType::Q4_1);
    hipStream_t s = (hipStream_t)stream;
    const Path path = pick_path(w->type, native, m, w->n, w->k, x_dev);
    const bool want_counters = path == Path::Gemm && w->type == WType::Q4_0 && !native && m <= rdl::GEMM_SMALL_M;
    CallWork cw;
    rdl_status st = cw.get(w, s, scratch_bytes(w->type, path, native, m, w->n, w->k), want_counters);
    if (st != RDL_OK) return st;
    st = run_linear(w->type, native, (const uint8_t*)w->dev, w->n, w->k, x_dev, m, y_dev, cw.p, cw.counters, s,
                    path);
    const rdl_status rs = cw.release(s);
    if (st != RDL_OK) return st;
    return rs == RDL_OK ? ok() : rs;
}

rdl_status rdl_linear_forward_bias_dev(const rdl_weight* w, const float* x_dev, size_t m, const float* bias_dev,
                                       float* y_dev, int32_t mode, void* stream) {
    if (bias_dev && w && m * (size_t)w->n >= ((size_t)1 << 32))
        return fail(RDL_ERR_UNSUPPORTED, "bias over %zu x %zu outputs: at most 2^32 - 1", m, w->n);
    rdl_status st = rdl_linear_forward_dev(w, x_dev, m, y_dev, mode, stream);
    if (st != RDL_OK || !bias_dev || m == 0 || w->n == 0) return st;
    HIP_TRY(rdl::launch_bias_add(y_dev, bias_dev, m, w->n, (hipStream_t)stream));
    return ok();
}

rdl_status rdl_release_stream_work(void* stream) {
    hipStream_t s = (hipStream_t)stream;
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(work_mu);
    for (auto it = work_pool.begin(); it != work_pool.end(); ++it) {
        if (it->dev != dev || it->stream != s) continue;
        // the stream's calls may still run on the device
        HIP_TRY(hipStreamSynchronize(s));
        if (it->p) HIP_TRY(hipFree(it->p));
        it->p = nullptr;
        if (it->counters) HIP_TRY(hipFree(it->counters));
        work_pool.erase(it);
        break;
    }
    return ok();
}

rdl_status rdl_linear_forward_dev_noalloc(const rdl_weight* w, const float* x_dev, size_t m, float* y_dev,
                                          int32_t mode, void* stream) {
    if (!w) return fail(RDL_ERR_NULL_POINTER, "weight handle is NULL");
    if (mode != RDL_MODE_FLOAT && mode != RDL_MODE_NATIVE)
        return fail(RDL_ERR_INVALID_DATA, "unknown mode %d", mode);
    if (m == 0 || w->n == 0) return ok();
    if (!x_dev || !y_dev) return fail(RDL_ERR_NULL_POINTER, "NULL activation pointer");
    const bool native = mode == RDL_MODE_NATIVE && (w->type == WType::Q4_0 || w->type == WType::Q4_1);
    const Path path = pick_path(w->type, native, m, w->n, w->k, x_dev);
    const size_t rb = scratch_bytes(w->type, path, native, m, w->n, w->k);
    if (rb > NOALLOC_DATA_BYTES)
        return fail(RDL_ERR_UNSUPPORTED,
                    "m=%zu rows of in_features %zu need %zu scratch bytes; the static scratch holds %zu",
                    m, w->k, rb, NOALLOC_DATA_BYTES);
    if (rdl::gemm_counter_count(w->n, w->k) * sizeof(int) > NOALLOC_COUNTER_BYTES)
        return fail(RDL_ERR_UNSUPPORTED, "out_features %zu beyond the static scratch's GEMM counters", w->n);
    void* work = nullptr;
    rdl_status st = noalloc_scratch(&work);
    if (st != RDL_OK) return st;
    int* counters = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(work) + NOALLOC_DATA_BYTES);
    st = run_linear(w->type, native, (const uint8_t*)w->dev, w->n, w->k, x_dev, m, y_dev, work, counters,
                    (hipStream_t)stream, path);
    return st == RDL_OK ? ok() : st;
}

size_t rdl_activation_record_bytes(size_t m, size_t k, int32_t mode) {
    return rec_bytes(mode == RDL_MODE_NATIVE, m, k);
}

rdl_status rdl_prepare_activations_dev(const float* x_dev, size_t m, size_t k, int32_t mode,
                                       void* rec_dev, void* stream) {
    if (mode != RDL_MODE_FLOAT && mode != RDL_MODE_NATIVE)
        return fail(RDL_ERR_INVALID_DATA, "unknown mode %d", mode);
    if (k % rdl::QK)
        return fail(RDL_ERR_BLOCK_ALIGNMENT, "activation length %zu not divisible by 32", k);
    if (m * k == 0) return ok();
    if (!x_dev || !rec_dev) return fail(RDL_ERR_NULL_POINTER, "NULL device pointer");
    if ((uintptr_t)rec_dev & 15) return fail(RDL_ERR_INVALID_DATA, "record buffer must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    if (mode == RDL_MODE_NATIVE)
        HIP_TRY(rdl::launch_prep_native(x_dev, m, k, (NativeRec*)rec_dev, nullptr, nullptr, s));
    else
        HIP_TRY(rdl::launch_prep_float(x_dev, m, k, (FloatRec*)rec_dev, s));
    return ok();
}

rdl_status rdl_linear_prepared_dev(const rdl_weight* w, const void* rec_dev, size_t m, float* y_dev,
                                   int32_t mode, void* stream) {
    if (!w) return fail(RDL_ERR_NULL_POINTER, "weight handle is NULL");
    if (mode != RDL_MODE_FLOAT && mode != RDL_MODE_NATIVE)
        return fail(RDL_ERR_INVALID_DATA, "unknown mode %d", mode);
    const bool native = mode == RDL_MODE_NATIVE;
    if (native && w->type != WType::Q4_0 && w->type != WType::Q4_1)
        return fail(RDL_ERR_DTYPE_MISMATCH, "native records apply to Q4_0 / Q4_1 weights only");
    if (m == 0 || w->n == 0) return ok();
    if (!y_dev || (w->k && !rec_dev)) return fail(RDL_ERR_NULL_POINTER, "NULL device pointer");
    HIP_TRY(rdl::launch_gemv(w->type, native, (const uint8_t*)w->dev, w->n, w->k, rec_dev, m, y_dev,
                             (hipStream_t)stream));
    return ok();
}

rdl_status rdl_linear_fused_dev(const rdl_weight* w, const float* x_dev, size_t x_stride, size_t m,
                                float* y_dev, int32_t prologue, const float* gamma_dev, float eps,
                                int32_t epilogue, void* stream) {
    if (!w) return fail(RDL_ERR_NULL_POINTER, "weight handle is NULL");
    if (w->type != WType::Q4_0) return fail(RDL_ERR_DTYPE_MISMATCH, "fused Linear takes Q4_0 weights");
    if (prologue < RDL_PROLOGUE_NONE || prologue > RDL_PROLOGUE_SWIGLU)
        return fail(RDL_ERR_INVALID_DATA, "unknown prologue %d", prologue);
    if (epilogue < RDL_EPILOGUE_STORE || epilogue > RDL_EPILOGUE_SWIGLU)
        return fail(RDL_ERR_INVALID_DATA, "unknown epilogue %d", epilogue);
    if (m == 0 || w->n == 0) return ok();
    if (!x_dev || !y_dev || (prologue == RDL_PROLOGUE_RMSNORM && !gamma_dev))
        return fail(RDL_ERR_NULL_POINTER, "NULL device pointer");
    const size_t k = w->k, nb = k / rdl::QK;
    if (m > 4 || nb == 0 || (nb & 1) || k > rdl::fused_max_k(WType::Q4_0) || (x_stride & 3) ||
        ((uintptr_t)x_dev & 15) || x_stride < (prologue == RDL_PROLOGUE_SWIGLU ? 2 * k : k) ||
        w->len > rdl::FUSED_MAX_WEIGHT_BYTES ||
        (epilogue == RDL_EPILOGUE_SWIGLU && ((w->n & 1) || nb > 256)))
        return fail(RDL_ERR_UNSUPPORTED,
                    "fused Linear: m <= 4, in_features/32 even and <= 16384, x 16-byte aligned, "
                    "x_stride a multiple of 4 covering the row (m=%zu k=%zu stride=%zu)", m, k, x_stride);
    HIP_TRY(rdl::launch_gemv_q4_0_fused_ex((const uint8_t*)w->dev, w->n, k, x_dev, x_stride, m, y_dev, prologue,
                                           gamma_dev, eps, epilogue, (hipStream_t)stream));
    return ok();
}

rdl_status rdl_quantize_row_q8_0_dev(const float* x_dev, size_t n, uint8_t* out_dev,
                                     float* scales_dev, void* stream) {
    if (n % rdl::QK)
        return fail(RDL_ERR_BLOCK_ALIGNMENT, "Q8_0 requires element count divisible by 32, got %zu", n);
    if (n == 0) return ok();
    if (!x_dev || !out_dev) return fail(RDL_ERR_NULL_POINTER, "NULL device pointer");
    HIP_TRY(rdl::launch_prep_native(x_dev, 1, n, nullptr, out_dev, scales_dev, (hipStream_t)stream));
    return ok();
}

rdl_status rdl_dequantize_rows_dev(const rdl_weight* w, const int32_t* row_ids_dev, size_t n_rows,
                                   float* out_dev, void* stream) {
    if (!w) return fail(RDL_ERR_NULL_POINTER, "weight handle is NULL");
    if (n_rows == 0) return ok();
    if (!row_ids_dev || !out_dev) return fail(RDL_ERR_NULL_POINTER, "NULL device pointer");
    HIP_TRY(rdl::launch_dequant_rows(w->type, (const uint8_t*)w->dev, w->n, w->k, row_ids_dev,
                                     n_rows, out_dev, (hipStream_t)stream));
    return ok();
}

rdl_status rdl_q4_0_q8_0_block_dots_dev(const rdl_weight* w, const float* x_dev,
                                        int32_t* partials_dev, void* stream) {
    if (!w) return fail(RDL_ERR_NULL_POINTER, "weight handle is NULL");
    if (w->type != WType::Q4_0) return fail(RDL_ERR_DTYPE_MISMATCH, "weight must be Q4_0");
    if (w->n == 0 || w->k == 0) return ok();
    if (!x_dev || !partials_dev) return fail(RDL_ERR_NULL_POINTER, "NULL device pointer");
    hipStream_t s = (hipStream_t)stream;
    CallWork cw;
    rdl_status st = cw.get(w, s, rec_bytes(true, 1, w->k), false);
    if (st != RDL_OK) return st;
    hipError_t e = rdl::launch_prep_native(x_dev, 1, w->k, (NativeRec*)cw.p, nullptr, nullptr, s);
    if (e == hipSuccess)
        e = rdl::launch_q4_0_block_dots((const uint8_t*)w->dev, w->n, w->k, (const NativeRec*)cw.p, partials_dev,
                                        s);
    const rdl_status rs = cw.release(s);
    HIP_TRY(e);
    return rs == RDL_OK ? ok() : rs;
}

}  // extern "C"
