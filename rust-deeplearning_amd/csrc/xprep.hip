// xprep.hip -- activation preparation kernels.
//
//  * prep_native: quantize_row_q8_0 (rustml/quant/main/src/core/quantize.rs:164-193),
//    byte-exact.  One lane per element, 32 lanes per block:
//      amax  = max(0, |x_j|) over the block (f32::max ignores NaN, :176)
//      scale = amax == 0 ? 0 : amax / 127          (IEEE division, :177)
//      h     = f16 RNE of scale; rt = f32(h)        (:178-179)
//      inv   = rt == 0 ? 0 : 1 / rt                 (:180)
//      q_j   = clamp(round_half_away(x_j * inv), -128, 127), NaN -> 0   (:187)
//  * prep_float: the 24-bit fixed-point digit record (FloatRec) that the float-mode
//    kernels consume; see rdl_internal.hpp.
#include "rdl_device.hpp"
#include "rdl_internal.hpp"

namespace rdl {

namespace {

constexpr int PREP_THREADS = 256;  // 8 blocks of 32 elements per workgroup

__device__ __forceinline__ float group_max32(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 32));
    return v;
}
__device__ __forceinline__ int group_sum32(int v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 32);
    return v;
}
__device__ __forceinline__ float group_sumf32(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 32);
    return v;
}

__global__ __launch_bounds__(PREP_THREADS) void prep_native_kernel(
    const float* __restrict__ x, size_t total_blocks, NativeRec* __restrict__ rec,
    uint8_t* __restrict__ q8_bytes, float* __restrict__ scales, int8_t* __restrict__ codes) {
    const size_t gid = (size_t)blockIdx.x * PREP_THREADS + threadIdx.x;
    const size_t blk = gid >> 5;
    const int j = threadIdx.x & 31;
    const bool valid = blk < total_blocks;
    const float v = valid ? x[gid] : 0.0f;

    // fmaxf(0, |v|) maps NaN to 0 exactly as the fold from 0.0 with f32::max does.
    const float amax = group_max32(fmaxf(0.0f, fabsf(v)));
    const float scale = (amax == 0.0f) ? 0.0f : amax / 127.0f;
    const uint32_t h = f2h_rne(scale);
    const float rt = h2f(h);
    const float inv = (rt == 0.0f) ? 0.0f : 1.0f / rt;
    float r = roundf(v * inv);
    int q;
    if (r != r) {
        q = 0;
    } else {
        r = fminf(fmaxf(r, -128.0f), 127.0f);
        q = (int)r;
    }
    const int qsum = group_sum32(q);
    if (!valid) return;

    if (rec) {  // NULL: only the Q8_0 bytes / scales are wanted
        NativeRec* out = rec + blk;
        reinterpret_cast<int8_t*>(out->q)[j] = (int8_t)q;
        if (j == 0) {
            out->scale = rt;
            out->qsum = qsum;
            out->pad[0] = 0;
            out->pad[1] = 0;
        }
    }
    if (q8_bytes) {
        uint8_t* ob = q8_bytes + blk * Q8_0_BYTES;
        ob[2 + j] = (uint8_t)(int8_t)q;
        if (j == 0) {
            ob[0] = (uint8_t)(h & 0xFFu);
            ob[1] = (uint8_t)(h >> 8);
        }
    }
    if (scales && j == 0) scales[blk] = rt;
    if (codes) codes[gid] = (int8_t)q;
}

__global__ __launch_bounds__(PREP_THREADS) void prep_float_kernel(const float* __restrict__ x,
                                                                 size_t total_blocks,
                                                                 FloatRec* __restrict__ rec) {
    const size_t gid = (size_t)blockIdx.x * PREP_THREADS + threadIdx.x;
    const size_t blk = gid >> 5;
    const int j = threadIdx.x & 31;
    const bool valid = blk < total_blocks;
    const float v = valid ? x[gid] : 0.0f;

    // Any NaN/Inf in the block poisons the block's scale.
    const unsigned long long bad = __ballot(!isfinite(v));
    const bool block_bad = ((bad >> (threadIdx.x & 32)) & 0xFFFFFFFFull) != 0;
    const float amax = group_max32(fabsf(v));
    int t = 0;
    float S = 0.0f;
    if (block_bad) {
        S = __builtin_nanf("");
    } else if (amax > 0.0f) {
        // t = x * (127 * 65536) / amax, |t| <= 8323072 + 1 < 2^23
        t = (int)rintf((v / amax) * 8323072.0f);
        S = amax / 127.0f;
    }
    // signed base-256 digits: t = a*65536 + b*256 + c, each in [-128, 127]
    const int c = (int)(int8_t)(t & 0xFF);
    const int t1 = (t - c) >> 8;
    const int b = (int)(int8_t)(t1 & 0xFF);
    const int a = (t1 - b) >> 8;
    const int sa = group_sum32(a);
    const int sb = group_sum32(b);
    const int sc = group_sum32(c);
    const float xs = group_sumf32(block_bad ? 0.0f : v);
    if (!valid) return;

    FloatRec* out = rec + blk;
    reinterpret_cast<int8_t*>(out->a)[j] = (int8_t)a;
    reinterpret_cast<int8_t*>(out->b)[j] = (int8_t)b;
    reinterpret_cast<int8_t*>(out->c)[j] = (int8_t)c;
    if (j == 0) {
        out->S = S;
        out->sa = sa;
        out->sb = sb;
        out->sc = sc;
        out->xsum = block_bad ? __builtin_nanf("") : xs;
        out->pad[0] = out->pad[1] = out->pad[2] = 0;
    }
}

}  // namespace

hipError_t launch_prep_native(const float* x, size_t m, size_t k, NativeRec* rec,
                              uint8_t* q8_bytes, float* scales, hipStream_t s) {
    const size_t total = m * (k / QK);
    if (total == 0) return hipSuccess;
    const size_t grid = (total * QK + PREP_THREADS - 1) / PREP_THREADS;
    hipLaunchKernelGGL(prep_native_kernel, dim3((unsigned)grid), dim3(PREP_THREADS), 0, s, x,
                       total, rec, q8_bytes, scales, (int8_t*)nullptr);
    return hipGetLastError();
}

hipError_t launch_prep_native_codes(const float* x, size_t m, size_t k, int8_t* codes, float* scales,
                                    hipStream_t s) {
    const size_t total = m * (k / QK);
    if (total == 0) return hipSuccess;
    const size_t grid = (total * QK + PREP_THREADS - 1) / PREP_THREADS;
    hipLaunchKernelGGL(prep_native_kernel, dim3((unsigned)grid), dim3(PREP_THREADS), 0, s, x, total,
                       (NativeRec*)nullptr, (uint8_t*)nullptr, scales, codes);
    return hipGetLastError();
}

hipError_t launch_prep_float(const float* x, size_t m, size_t k, FloatRec* rec, hipStream_t s) {
    const size_t total = m * (k / QK);
    if (total == 0) return hipSuccess;
    const size_t grid = (total * QK + PREP_THREADS - 1) / PREP_THREADS;
    hipLaunchKernelGGL(prep_float_kernel, dim3((unsigned)grid), dim3(PREP_THREADS), 0, s, x,
                       total, rec);
    return hipGetLastError();
}

}  // namespace rdl
