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

// ---- cross-lane reductions without an LDS round trip ----------------------
// DPP lane patterns (a DPP row is 16 lanes).
constexpr int DPP_QUAD_XOR1 = 0xB1;        // quad_perm [1,0,3,2]: lane i <- i^1
constexpr int DPP_QUAD_XOR2 = 0x4E;        // quad_perm [2,3,0,1]: lane i <- i^2
constexpr int DPP_ROW_HALF_MIRROR = 0x141; // lane i <- 7-i within each 8 lanes
constexpr int DPP_ROW_MIRROR = 0x140;      // lane i <- 15-i within each 16 lanes

// Every pattern used here reads a lane of the same row, so no lane takes the
// out-of-bounds value; bound_ctrl lets the compiler fold the move into the
// instruction that consumes it (v_add_f32_dpp, v_max_u32_dpp, ...).
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return as_f32(dpp_i32<CTRL>(__builtin_bit_cast(int32_t, v)));
}

// Sum / max over each aligned group of 4 or 8 lanes, returned in every lane
// of the group.  Each step pairs a lane with one in the other half of its
// group, and both lanes of a pair compute the same (commutative) result, so
// every lane of a group ends up with identical bits.
__device__ __forceinline__ int sum4_i32(int v) {
    v += dpp_i32<DPP_QUAD_XOR1>(v);
    return v + dpp_i32<DPP_QUAD_XOR2>(v);
}
__device__ __forceinline__ float sum4_f32(float v) {
    v += dpp_f32<DPP_QUAD_XOR1>(v);
    return v + dpp_f32<DPP_QUAD_XOR2>(v);
}
__device__ __forceinline__ float max4_f32(float v) {
    v = fmaxf(v, dpp_f32<DPP_QUAD_XOR1>(v));
    return fmaxf(v, dpp_f32<DPP_QUAD_XOR2>(v));
}
// Maximum of non-negative float bit patterns as unsigned integers: the same
// order as the floats for finite values, and an Inf or NaN in the group
// comes out on top (>= 0x7F800000), so one reduction gives both the largest
// magnitude and whether the group holds a non-finite value.
__device__ __forceinline__ uint32_t max4_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp_i32<DPP_QUAD_XOR1>((int)v));
    return max(v, (uint32_t)dpp_i32<DPP_QUAD_XOR2>((int)v));
}
__device__ __forceinline__ uint32_t max8_u32(uint32_t v) {
    v = max4_u32(v);
    return max(v, (uint32_t)dpp_i32<DPP_ROW_HALF_MIRROR>((int)v));
}
__device__ __forceinline__ uint32_t abs_bits(float x) { return __builtin_bit_cast(uint32_t, x) & 0x7FFFFFFFu; }
__device__ __forceinline__ int sum8_i32(int v) {
    v = sum4_i32(v);
    return v + dpp_i32<DPP_ROW_HALF_MIRROR>(v);
}
__device__ __forceinline__ float sum8_f32(float v) {
    v = sum4_f32(v);
    return v + dpp_f32<DPP_ROW_HALF_MIRROR>(v);
}
__device__ __forceinline__ float max8_f32(float v) {
    v = max4_f32(v);
    return fmaxf(v, dpp_f32<DPP_ROW_HALF_MIRROR>(v));
}

// gfx950 v_permlane32_swap / v_permlane16_swap folds.
// fold32(x, y): lanes 0-31 get x[l] + x[l+32], lanes 32-63 get y[l-32] + y[l].
// fold16(x, y): lanes of the even 16-lane rows get x[l] + x[l+16], lanes of
// the odd rows get y[l-16] + y[l].
__device__ __forceinline__ float fold32(float x, float y) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                    __builtin_bit_cast(uint32_t, y), false, false);
    const uint32_t lo = r[0], hi = r[1];  // by value: see as_f32
    return __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
}
__device__ __forceinline__ float fold16(float x, float y) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x),
                                                    __builtin_bit_cast(uint32_t, y), false, false);
    const uint32_t lo = r[0], hi = r[1];  // by value: see as_f32
    return __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
}

// Row sums of a wave: v[r] holds lane partials of row r (R <= 4).  Returns,
// in every lane, the 64-lane total of row (lane >> 4) for R = 3, 4, of row
// (lane >> 5) for R = 2 and of row 0 for R = 1 (rows >= R read as zero).
template <int R>
__device__ __forceinline__ float wave_reduce_rows(const float (&v)[R]) {
    static_assert(R >= 1 && R <= 4, "rows per wave");
    float s;
    if constexpr (R >= 3) {
        const float a = fold32(v[0], v[2]);
        const float b = fold32(v[1], R == 4 ? v[R == 4 ? 3 : 0] : 0.0f);
        s = fold16(a, b);
    } else if constexpr (R == 2) {
        s = fold32(v[0], v[1]);
        s = fold16(s, s);
    } else {
        s = fold32(v[0], v[0]);
        s = fold16(s, s);
    }
    s += dpp_f32<DPP_QUAD_XOR1>(s);
    s += dpp_f32<DPP_QUAD_XOR2>(s);
    s += dpp_f32<DPP_ROW_HALF_MIRROR>(s);
    return s + dpp_f32<DPP_ROW_MIRROR>(s);
}
// log2 of the lanes that share one row total after wave_reduce_rows<R>.
template <int R>
constexpr int reduce_span_log2() { return R >= 3 ? 4 : R == 2 ? 5 : 6; }

// ---- buffer loads ---------------------------------------------------------
// Raw buffer loads over [base, base + bytes): an offset at or beyond `bytes`
// returns zero without touching memory, which gives branch-free loads for
// lanes that have nothing to load (offset RSRC_OOB).  bytes < 2^31.
constexpr uint32_t RSRC_OOB = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    // 0x00020000: the gfx9-family descriptor word 3 (32-bit data format).
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}
__device__ __forceinline__ u32x4 buf_load_b128(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load_b32(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load_b16(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)off, 0, 0);
}

// ---- Q6_K units ---------------------------------------------------------------
// A unit is one 32-element column of a 256-element Q6_K super-block: column
// j = 4 * half + t holds elements 128 * half + 32 * t + l, l < 32.  Its codes
// (dequantize_q6k, rustml/gguf/main/src/core/parser.rs:510-547): low four bits
// from ql[64 * half + 32 * (t & 1) + l] (low nibble for t < 2, high for t >= 2),
// high two bits from bits 2t, 2t + 1 of qh[32 * half + l]; element value
// (d * scales[8 * half + 2t + l / 16]) * (code - 32), scales int8, d f16 at
// byte 208.  Blocks are 210 bytes, so a block starts on a 2- or 4-byte
// boundary; the 32-byte ql and qh runs are read as nine-dword windows from
// the dword below them and realigned with v_perm_b32.
struct Q6KUnit {
    uint32_t ql, qh;  // first byte of the unit's ql / qh run
    uint32_t sc;      // its two scales (l < 16, l >= 16)
    uint32_t d;       // the block's f16 scale
    int t;            // column within the half
};
__device__ __forceinline__ Q6KUnit q6k_unit(uint32_t block, int j) {
    const uint32_t half = (uint32_t)j >> 2, t = (uint32_t)j & 3;
    return {block + 64 * half + 32 * (t & 1), block + 128 + 32 * half, block + 192 + 8 * half + 2 * t,
            block + 208, (int)t};
}
// v_perm selector taking the 4 bytes that start at run & 3 (0 or 2) in {w[k+1]:w[k]}
__device__ __forceinline__ uint32_t q6k_sel(uint32_t run) { return (run & 2) ? 0x05040302u : 0x03020100u; }

// The 32 codes (0..63) of a unit as 8 dwords of bytes (dword k: elements 4k..4k+3).
__device__ __forceinline__ void q6k_codes(const uint32_t (&wl)[9], const uint32_t (&wh)[9], uint32_t sel, int t,
                                          uint32_t (&q)[8]) {
    const uint32_t nsh = 4 * (uint32_t)(t >> 1);
    // the 2-bit field at bits 2t, 2t+1 of each qh byte moves to bits 4, 5 by
    // one rotation of the dword (right by 2t - 4, i.e. left by 4 - 2t): no bit
    // that lands there crosses a byte
    const uint32_t rot = (2 * (uint32_t)t + 28) & 31;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t lo = perm(wl[k + 1], wl[k], sel), hi = perm(wh[k + 1], wh[k], sel);
        const uint32_t h2 = __builtin_amdgcn_alignbit(hi, hi, rot) & 0x30303030u;
        q[k] = ((lo >> nsh) & 0x0F0F0F0Fu) | h2;
    }
}

// Starting values of the unit's six digit sums: -32 * (sum of the a / b / c
// digits over elements 0..15 and 16..31), so that the dots below give
// sum (code - 32) * digit exactly.  X: a float-mode record view (a0, a1 =
// a digits of elements 0..15 / 16..31, likewise b, c; sa, sb, sc = sums over
// all 32).
template <class X>
__device__ __forceinline__ void q6k_offsets(const X& x, int (&off)[6]) {
    constexpr int ONE4 = 0x01010101;
    auto half_sum = [](const i32x4& v) {
        return dot4(ONE4, v.x, dot4(ONE4, v.y, dot4(ONE4, v.z, dot4(ONE4, v.w, 0))));
    };
    const int a = half_sum(x.a0), b = half_sum(x.b0), c = half_sum(x.c0);
    off[0] = -32 * a;
    off[1] = -32 * (x.sa - a);
    off[2] = -32 * b;
    off[3] = -32 * (x.sb - b);
    off[4] = -32 * c;
    off[5] = -32 * (x.sc - c);
}

// sum over the unit of scale * (code - 32) * x_digits, combined as
// A + (B + C / 256) / 256 (exact in int32 up to the final conversion);
// sc0 / sc1: the scales of elements 0..15 / 16..31.
template <class X>
__device__ __forceinline__ float q6k_dot(const uint32_t (&q)[8], const X& x, const int (&off)[6], int sc0,
                                         int sc1) {
    int A0 = off[0], A1 = off[1], B0 = off[2], B1 = off[3], C0 = off[4], C1 = off[5];
    A0 = dot4(q[0], x.a0.x, A0); A0 = dot4(q[1], x.a0.y, A0); A0 = dot4(q[2], x.a0.z, A0); A0 = dot4(q[3], x.a0.w, A0);
    A1 = dot4(q[4], x.a1.x, A1); A1 = dot4(q[5], x.a1.y, A1); A1 = dot4(q[6], x.a1.z, A1); A1 = dot4(q[7], x.a1.w, A1);
    B0 = dot4(q[0], x.b0.x, B0); B0 = dot4(q[1], x.b0.y, B0); B0 = dot4(q[2], x.b0.z, B0); B0 = dot4(q[3], x.b0.w, B0);
    B1 = dot4(q[4], x.b1.x, B1); B1 = dot4(q[5], x.b1.y, B1); B1 = dot4(q[6], x.b1.z, B1); B1 = dot4(q[7], x.b1.w, B1);
    C0 = dot4(q[0], x.c0.x, C0); C0 = dot4(q[1], x.c0.y, C0); C0 = dot4(q[2], x.c0.z, C0); C0 = dot4(q[3], x.c0.w, C0);
    C1 = dot4(q[4], x.c1.x, C1); C1 = dot4(q[5], x.c1.y, C1); C1 = dot4(q[6], x.c1.z, C1); C1 = dot4(q[7], x.c1.w, C1);
    // |A0|, |A1| <= 16 * 63 * 128 + 32 * 16 * 128 < 2^18, |scale| <= 128: no int32 overflow
    const int IA = sc0 * A0 + sc1 * A1, IB = sc0 * B0 + sc1 * B1, IC = sc0 * C0 + sc1 * C1;
    return fmaf(fmaf((float)IC, 1.0f / 256.0f, (float)IB), 1.0f / 256.0f, (float)IA);
}

// ---- paged KV cache -------------------------------------------------------
// Cached positions live in pages of KV_PAGE positions.  A layer's K (or V)
// pool is [n_pages][n_kv][KV_PAGE][hd]: physical page pg holds every KV
// head's rows of one run of KV_PAGE positions; table[pos / KV_PAGE] is the
// physical page of a position (KVCache's contiguous [n_kv][max_seq][hd] is
// the identity table).  One attention chunk (64 keys) is one page.
constexpr int KV_PAGE = 64;
__device__ __forceinline__ size_t kv_row(const int* __restrict__ table, int n_kv, int kvh, int pos, int hd) {
    return (((size_t)table[pos / KV_PAGE] * n_kv + kvh) * KV_PAGE + (pos % KV_PAGE)) * hd;
}

}  // namespace rdl
