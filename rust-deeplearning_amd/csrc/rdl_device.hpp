// rdl_device.hpp -- small device helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rdl {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Reinterpret an int32 as f32.  Takes the value (not an lvalue): clang lowers
// __builtin_bit_cast of an ext_vector_type component such as v.y as a load
// from the start of the vector, i.e. it returns v.x.  Use this helper for
// vector components.
__device__ __forceinline__ float as_f32(int32_t v) { return __builtin_bit_cast(float, v); }

// IEEE binary16 -> binary32 through the hardware converter (exact, keeps
// subnormals: kernels run with f16 denormals enabled, the HSA default).
__device__ __forceinline__ float h2f(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
    return (float)h;
}

// binary32 -> binary16, round to nearest even, subnormals kept, overflow to
// inf, NaN quieted: the conversion half 2.7.1's f16::from_f32 performs.
// Written in integer arithmetic so the result never depends on the FP mode.
__device__ __forceinline__ uint32_t f2h_rne(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFFu) return sign | (man ? (0x7E00u | (man >> 13)) : 0x7C00u);
    int e = (int)exp - 112;
    if (e >= 31) return sign | 0x7C00u;
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e;
        uint32_t hm = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return sign | hm;
    }
    uint32_t hm = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    uint32_t h = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) h++;
    return h;
}

// v_dot4_i32_i8: acc + sum of the four signed byte products of a and b.
__device__ __forceinline__ int32_t dot4(uint32_t a, int32_t b, int32_t acc) {
    return __builtin_amdgcn_sdot4((int32_t)a, b, acc, false);
}

// Pick 4 bytes out of the 8-byte pair {hi:lo}; sel bytes 0-3 address lo, 4-7 hi.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

}  // namespace rdl
