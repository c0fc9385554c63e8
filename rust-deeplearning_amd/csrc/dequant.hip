// dequant.hip -- every GGML tensor type to f32 on the device: the load-time
// expansion of GGUFFile::load_tensors (rustml/gguf/main/src/core/parser.rs:
// 292-346, 371-776) and Tensor::to_f32 (rustml/core/main/src/core/tensor/
// tensor.rs:535-639), bit-exact.
//
// One thread per 32 output elements: a whole block of the 32-element types,
// one eighth of a 256-element K-quant super-block.  Reads are byte loads (the
// source may start anywhere); every product below is exact in f32 or a
// single rounding, the same operations in the same order as the reference.
#include "../../include/rdl_gguf.h"
#include "rdl_device.hpp"
#include "rdl_internal.hpp"

namespace rdl {
namespace {

__device__ __forceinline__ float ld_f16(const uint8_t* p) { return h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
__device__ __forceinline__ float ld_f32(const uint8_t* p) { return __builtin_bit_cast(float, ld_u32(p)); }

// Q4_K / Q5_K 6-bit scale and min of sub-block j (parser.rs:562-569, :611-616)
__device__ __forceinline__ void k_scale_min(const uint8_t* s, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = ((s[j - 4] >> 6) & 3) | ((s[j + 4] & 0xF) << 2);
        mn = ((s[j] >> 6) & 3) | ((s[j + 4] >> 4) << 2);
    }
}

// The 32 elements of group g (block b = g / G, part p = g % G) into o.
template <int T>
__device__ void decode32(const uint8_t* __restrict__ src, size_t g, float* __restrict__ o) {
    if constexpr (T == 1) {  // F16
        const uint8_t* p = src + g * 64;
        for (int l = 0; l < 32; l++) o[l] = ld_f16(p + 2 * l);
    } else if constexpr (T == 2) {  // Q4_0 (tensor.rs:553-563)
        const uint8_t* p = src + g * 18;
        const float d = ld_f16(p);
        for (int j = 0; j < 16; j++) {
            o[j] = d * (float)((int)(p[2 + j] & 0xF) - 8);
            o[j + 16] = d * (float)((int)(p[2 + j] >> 4) - 8);
        }
    } else if constexpr (T == 3) {  // Q4_1 (parser.rs:386-408)
        const uint8_t* p = src + g * 20;
        const float d = ld_f16(p), m = ld_f16(p + 2);
        for (int j = 0; j < 16; j++) {
            o[j] = d * (float)(p[4 + j] & 0xF) + m;
            o[j + 16] = d * (float)(p[4 + j] >> 4) + m;
        }
    } else if constexpr (T == 6) {  // Q5_0 (parser.rs:411-437)
        const uint8_t* p = src + g * 22;
        const float d = ld_f16(p);
        const uint32_t qh = ld_u32(p + 2);
        for (int j = 0; j < 16; j++) {
            const int lo = (p[6 + j] & 0xF) | (int)(((qh >> j) & 1) << 4);
            const int hi = (p[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1) << 4);
            o[j] = d * ((float)lo - 16.0f);
            o[j + 16] = d * ((float)hi - 16.0f);
        }
    } else if constexpr (T == 7) {  // Q5_1 (parser.rs:440-467)
        const uint8_t* p = src + g * 24;
        const float d = ld_f16(p), m = ld_f16(p + 2);
        const uint32_t qh = ld_u32(p + 4);
        for (int j = 0; j < 16; j++) {
            const uint32_t lo = (uint32_t)(p[8 + j] & 0xF) | (((qh >> j) & 1) << 4);
            const uint32_t hi = (uint32_t)(p[8 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4);
            o[j] = d * (float)lo + m;
            o[j + 16] = d * (float)hi + m;
        }
    } else if constexpr (T == 8) {  // Q8_0 (tensor.rs:608-639)
        const uint8_t* p = src + g * 34;
        const float d = ld_f16(p);
        for (int j = 0; j < 32; j++) o[j] = d * (float)(int8_t)p[2 + j];
    } else if constexpr (T == 9) {  // Q8_1 (parser.rs:470-489): f32 d, the sum unused
        const uint8_t* p = src + g * 40;
        const float d = ld_f32(p);
        for (int j = 0; j < 32; j++) o[j] = d * (float)(int8_t)p[8 + j];
    } else if constexpr (T == 10 || T == 11) {  // Q2_K (parser.rs:737-776), Q3_K (:669-735)
        // group 4h + j: two runs of 16 with scales 8h + 2j, 8h + 2j + 1, the
        // 2-bit field 2j of qs bytes 32h + 16 part + l
        const int part8 = (int)(g % 8), h = part8 >> 2, j = part8 & 3;
        if constexpr (T == 10) {
            const uint8_t* p = src + (g / 8) * 84;
            const float d = ld_f16(p + 80), dmin = ld_f16(p + 82);
            for (int part = 0; part < 2; part++) {
                const uint8_t s = p[8 * h + 2 * j + part];
                const float dl = d * (float)(s & 0xF), ml = dmin * (float)(s >> 4);
                const uint8_t* q = p + 16 + 32 * h + 16 * part;
                for (int l = 0; l < 16; l++) o[16 * part + l] = dl * (float)((q[l] >> (2 * j)) & 3) - ml;
            }
        } else {
            const uint8_t* p = src + (g / 8) * 110;
            const float d_all = ld_f16(p + 108);
            const uint8_t* sr = p + 96;
            for (int part = 0; part < 2; part++) {
                // 6-bit scale i: low nibble from byte i (i < 8) or the high
                // nibble of byte i - 8, high pair from bits 2 (i / 4) of byte 8 + i % 4
                const int i = 8 * h + 2 * j + part;
                const int lo4 = i < 8 ? (sr[i] & 0xF) : (sr[i - 8] >> 4);
                const int sc = lo4 | (((sr[8 + (i & 3)] >> (2 * (i >> 2))) & 3) << 4);
                const float dl = d_all * ((float)(int8_t)sc - 32.0f);
                const uint8_t* q = p + 32 + 32 * h + 16 * part;
                const uint8_t* hm = p + 16 * part;
                const uint8_t m = (uint8_t)(1u << (4 * h + j));
                for (int l = 0; l < 16; l++) {
                    const int q2 = (q[l] >> (2 * j)) & 3;
                    const int hb = (hm[l] & m) ? 0 : -4;
                    o[16 * part + l] = dl * (float)(q2 + hb);
                }
            }
        }
    } else if constexpr (T == 12 || T == 13) {  // Q4_K (parser.rs:549-593), Q5_K (:595-646)
        constexpr int BB = T == 12 ? Q4_K_BYTES : 176;
        const int sub = (int)(g % 8), c = sub >> 1;
        const uint8_t* p = src + (g / 8) * BB;
        const float d = ld_f16(p), dmin = ld_f16(p + 2);
        int sc, mn;
        k_scale_min(p + 4, sub, sc, mn);
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        const int sh = (sub & 1) * 4;
        if constexpr (T == 12) {
            const uint8_t* q = p + 16 + 32 * c;
            for (int l = 0; l < 32; l++) o[l] = d1 * (float)((q[l] >> sh) & 0xF) - m1;
        } else {
            const uint8_t* qh = p + 16;
            const uint8_t* q = p + 48 + 32 * c;
            const uint8_t u = (uint8_t)(1u << sub);  // bit 2c for low nibbles, 2c + 1 for high
            for (int l = 0; l < 32; l++) {
                const int hb = (qh[l] & u) ? 16 : 0;
                o[l] = d1 * (float)(((q[l] >> sh) & 0xF) + hb) - m1;
            }
        }
    } else if constexpr (T == 14) {  // Q6_K (parser.rs:510-547), column 4 half + t
        const int col = (int)(g % 8), half = col >> 2, t = col & 3;
        const uint8_t* p = src + (g / 8) * Q6_K_BYTES;
        const float d = ld_f16(p + 208);
        const uint8_t* ql = p + 64 * half + 32 * (t & 1);
        const uint8_t* qh = p + 128 + 32 * half;
        const int8_t* sc = reinterpret_cast<const int8_t*>(p + 192 + 8 * half + 2 * t);
        for (int l = 0; l < 32; l++) {
            const int code = ((ql[l] >> (4 * (t >> 1))) & 0xF) | (((qh[l] >> (2 * t)) & 3) << 4);
            o[l] = d * (float)sc[l >> 4] * (float)(code - 32);
        }
    } else if constexpr (T == 15) {  // Q8_K (parser.rs:649-667)
        const uint8_t* p = src + (g / 8) * 292;
        const float d = ld_f32(p);
        const uint8_t* q = p + 4 + 32 * (g % 8);
        for (int l = 0; l < 32; l++) o[l] = d * (float)(int8_t)q[l];
    }
}

template <int T>
__global__ __launch_bounds__(256) void dequant_gguf_kernel(const uint8_t* __restrict__ src, size_t groups,
                                                           float* __restrict__ dst) {
    const size_t g = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= groups) return;
    float o[32];
    decode32<T>(src, g, o);
    float4* d4 = reinterpret_cast<float4*>(dst + g * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) d4[i] = make_float4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}

// F16 elements that do not fill a group of 32, and the zero tail.
__global__ void dequant_tail_kernel(const uint8_t* __restrict__ src, size_t first, size_t f16_end, size_t n,
                                    float* __restrict__ dst) {
    const size_t i = first + (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    dst[i] = i < f16_end ? ld_f16(src + 2 * i) : 0.0f;
}

}  // namespace

// GGMLType block geometry (rustml/gguf/main/src/api/types.rs:49-77); false for
// ids that GGMLType::from_u32 rejects.
bool ggml_geometry(int32_t t, int* block_size, int* block_bytes) {
    static const int tab[16][2] = {{1, 4}, {1, 2}, {32, 18}, {32, 20}, {0, 0}, {0, 0}, {32, 22}, {32, 24},
                                   {32, 34}, {32, 40}, {256, 84}, {256, 110}, {256, 144}, {256, 176},
                                   {256, 210}, {256, 292}};
    if (t < 0 || t > 15 || tab[t][0] == 0) return false;
    *block_size = tab[t][0];
    *block_bytes = tab[t][1];
    return true;
}

hipError_t launch_dequant_gguf(int32_t t, const uint8_t* src, size_t n_elements, float* dst, hipStream_t s) {
    int bs = 0, bb = 0;
    if (!ggml_geometry(t, &bs, &bb)) return hipErrorInvalidValue;
    if (t == 0) {  // F32: the bytes themselves
        return n_elements ? hipMemcpyAsync(dst, src, n_elements * 4, hipMemcpyDeviceToDevice, s) : hipSuccess;
    }
    // whole blocks only (the reference's n_elements / block_size); F16 in groups of 32
    const size_t full = (bs > 1) ? n_elements / bs * bs : n_elements;
    const size_t groups = full / 32;
    if ((uintptr_t)dst & 15) return hipErrorInvalidValue;
    if (groups) {
        const dim3 grid((unsigned)((groups + 255) / 256)), block(256);
        switch (t) {
            case 1: hipLaunchKernelGGL(dequant_gguf_kernel<1>, grid, block, 0, s, src, groups, dst); break;
            case 2: hipLaunchKernelGGL(dequant_gguf_kernel<2>, grid, block, 0, s, src, groups, dst); break;
            case 3: hipLaunchKernelGGL(dequant_gguf_kernel<3>, grid, block, 0, s, src, groups, dst); break;
            case 6: hipLaunchKernelGGL(dequant_gguf_kernel<6>, grid, block, 0, s, src, groups, dst); break;
            case 7: hipLaunchKernelGGL(dequant_gguf_kernel<7>, grid, block, 0, s, src, groups, dst); break;
            case 8: hipLaunchKernelGGL(dequant_gguf_kernel<8>, grid, block, 0, s, src, groups, dst); break;
            case 9: hipLaunchKernelGGL(dequant_gguf_kernel<9>, grid, block, 0, s, src, groups, dst); break;
            case 10: hipLaunchKernelGGL(dequant_gguf_kernel<10>, grid, block, 0, s, src, groups, dst); break;
            case 11: hipLaunchKernelGGL(dequant_gguf_kernel<11>, grid, block, 0, s, src, groups, dst); break;
            case 12: hipLaunchKernelGGL(dequant_gguf_kernel<12>, grid, block, 0, s, src, groups, dst); break;
            case 13: hipLaunchKernelGGL(dequant_gguf_kernel<13>, grid, block, 0, s, src, groups, dst); break;
            case 14: hipLaunchKernelGGL(dequant_gguf_kernel<14>, grid, block, 0, s, src, groups, dst); break;
            case 15: hipLaunchKernelGGL(dequant_gguf_kernel<15>, grid, block, 0, s, src, groups, dst); break;
        }
    }
    const size_t done = groups * 32;
    if (done < n_elements) {
        const size_t f16_end = (t == 1) ? n_elements : done;
        hipLaunchKernelGGL(dequant_tail_kernel, dim3((unsigned)((n_elements - done + 255) / 256)), dim3(256), 0, s,
                           src, done, f16_end, n_elements, dst);
    }
    return hipGetLastError();
}

}  // namespace rdl

extern "C" {

rdl_status rdl_dequantize_gguf_dev(int32_t ggml_type, const void* src_dev, size_t src_len, size_t n_elements,
                                   float* dst_dev, void* stream) {
    int bs = 0, bb = 0;
    if (!rdl::ggml_geometry(ggml_type, &bs, &bb))
        return rdl::api_fail(RDL_ERR_GGUF_UNSUPPORTED_TYPE, "GGML type: %d", ggml_type);
    const size_t need = (bs > 1 ? n_elements / bs : n_elements) * (size_t)bb;
    if (src_len < need)
        return rdl::api_shape_fail("source bytes", {need}, {src_len});
    if (n_elements == 0) return rdl::api_ok();
    if (!dst_dev || (need && !src_dev)) return rdl::api_fail(RDL_ERR_NULL_POINTER, "NULL device pointer");
    if ((uintptr_t)dst_dev & 15) return rdl::api_fail(RDL_ERR_INVALID_DATA, "destination must be 16-byte aligned");
    rdl_status st = rdl::api_require_device();
    if (st != RDL_OK) return st;
    HIP_TRY(rdl::launch_dequant_gguf(ggml_type, static_cast<const uint8_t*>(src_dev), n_elements, dst_dev,
                                     (hipStream_t)stream));
    return rdl::api_ok();
}

}  // extern "C"
