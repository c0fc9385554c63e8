// stream_read.hip -- a plain streaming read of device memory: the HBM read
// rate the quantized GEMV launches are compared with, measured with the same
// launch machinery (one kernel, no arithmetic beyond keeping the loads live).
// No reference counterpart.
#include <hip/hip_runtime.h>

#include "../../include/rdl_quant.h"
#include "rdl_device.hpp"
#include "rdl_internal.hpp"

namespace rdl {
namespace {

constexpr int SR_THREADS = 512, SR_INFLIGHT = 8;

// Workgroup g reads the 16-byte units [g * per, (g + 1) * per) in rounds of
// SR_THREADS * SR_INFLIGHT units (SR_INFLIGHT loads in flight per thread),
// XORs them and writes one word (so that no load can be dropped).
__global__ __launch_bounds__(SR_THREADS) void stream_read_kernel(const uint8_t* __restrict__ p, uint32_t bytes,
                                                                 uint32_t per, uint32_t* __restrict__ out) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p, bytes);
    const uint32_t u0 = blockIdx.x * per, u1 = min(u0 + per, bytes / 16u);
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (uint32_t base = u0 + threadIdx.x; base < u1; base += SR_THREADS * SR_INFLIGHT) {
        u32x4 v[SR_INFLIGHT];
#pragma unroll
        for (int i = 0; i < SR_INFLIGHT; i++) {
            const uint32_t u = base + (uint32_t)i * SR_THREADS;
            v[i] = buf_load_b128(rs, u < u1 ? u * 16u : RSRC_OOB);
        }
#pragma unroll
        for (int i = 0; i < SR_INFLIGHT; i++) acc ^= v[i];
    }
    const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    __shared__ uint32_t red[SR_THREADS / 64];
    uint32_t w = x;
    for (int o = 32; o >= 1; o >>= 1) w ^= (uint32_t)__shfl_xor((int)w, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = w;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int i = 0; i < SR_THREADS / 64; i++) t ^= red[i];
        out[blockIdx.x] = t;
    }
}

}  // namespace
}  // namespace rdl

extern "C" rdl_status rdl_stream_read_dev(const void* buf, size_t bytes, uint32_t* out_dev, size_t out_len,
                                          void* stream) {
    if (!buf || !out_dev) return rdl::api_fail(RDL_ERR_NULL_POINTER, "NULL device pointer");
    if (bytes % 16 || bytes == 0 || bytes >= ((size_t)1 << 31))
        return rdl::api_fail(RDL_ERR_INVALID_DATA, "bytes %zu: a multiple of 16 in (0, 2^31)", bytes);
    // two workgroups per CU, each a contiguous share
    const uint32_t wgs = (uint32_t)(2 * rdl::device_cu_count());
    if (out_len < wgs) return rdl::api_fail(RDL_ERR_SHAPE_MISMATCH, "out_len %zu < %u", out_len, wgs);
    const uint32_t units = (uint32_t)(bytes / 16), per = (units + wgs - 1) / wgs;
    rdl::launch_kernel(rdl::stream_read_kernel, dim3(wgs), dim3(rdl::SR_THREADS), 0, (hipStream_t)stream,
                       (const uint8_t*)buf, (uint32_t)bytes, per, out_dev);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return rdl::api_fail(RDL_ERR_HIP, "stream read launch: %s", hipGetErrorString(e));
    return rdl::api_ok();
}
