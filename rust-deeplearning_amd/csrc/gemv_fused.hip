// gemv_fused.hip -- single-launch decode GEMV: activation preparation fused
// into the GEMV, y = W x for one activation row per blockIdx.y.
//
// Reference semantics are those of gemv.hip (matmul_f32_q8 / _q4 / _q4_native /
// _q4_1 / _q4_1_native, quantize.rs:201-572; Q4_K parser.rs:549-593; Q6_K
// parser.rs:510-547).
//
// Shape of a launch (MI355X: 256 CUs):
//   * about one workgroup of NW = 16 waves per CU; workgroup g owns rows
//     [g*rpw, (g+1)*rpw) and hands them to its waves round-robin, so wave w
//     owns at most R rows;
//   * phase 0: every wave issues the loads of all its weight blocks (R rows x
//     up to CPL columns per lane) before anything else -- the weight stream
//     does not depend on x;
//   * phase 1: while those loads are in flight the workgroup converts x into
//     per-column records in LDS (same encodings as FloatRec / NativeRec,
//     stored as eight 16-byte groups per column, group-major, so that 64 lanes
//     reading 64 consecutive columns hit 64 consecutive 16-byte slots);
//   * phase 2: each lane dots its blocks against its columns' records on
//     v_dot4_i32_i8; the R row sums are reduced across the wave.
#include <algorithm>
#include <type_traits>

#include "attention.hpp"
#include "rdl_device.hpp"
#include "rdl_internal.hpp"

namespace rdl {

namespace {

// waves per workgroup (template parameter NW of the kernels); NT = NW * 64
constexpr uint32_t NIB = 0x0F0F0F0Fu;
constexpr uint32_t ONES = 0x01010101u;

// ---- phase 1: records in LDS ---------------------------------------------------
// Group layout per column c (i32x4 slots at lds[g * nb + c]):
//   float:  g0,g1 = a digits (dwords 0-3, 4-7), g2,g3 = b, g4,g5 = c,
//           g6 = {S, sum a, sum b, sum c}, g7 = {sum x, 0, 0, 0}
//   native: g0,g1 = q8 codes, g2 = {scale, sum q8, 0, 0}
// Eight threads share a column; thread k of the eight handles elements 4k..4k+3,
// which form digit dword k.

__device__ __forceinline__ int lds_word(int g, int k4, int nb, int c) {  // dword index
    return (g * nb + c) * 4 + k4;
}


// 24-bit fixed-point digits of x_j * (127*65536 / amax):  t + 0x808080 is in
// [0, 2^24), its bytes u are the digits biased by 128, and u ^ 0x80 is the
// int8 pattern of the signed digit, so e = (t + 0x808080) ^ 0x808080 holds
// the digits c (byte 0), b (byte 1), a (byte 2).
// x loads for the prep, issued before the weight stream so they return first.
// The prep's x loads are issued first, by inline asm, so that they precede
// every weight load in the wave's in-order load queue; wait_prep_x<N>() then
// waits for them alone ("vmcnt <= N" with N = the number of weight loads the
// wave issued after them) while the weight stream stays in flight.  The
// compiler does not track these asm loads, so the explicit wait is the only
// guard: N must not exceed the number of load instructions actually issued
// between the two points (the "memory" clobbers keep every load in between).
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int NW, int PI>
__device__ __forceinline__ void load_prep_x(const float* __restrict__ x, int nb, f32x4 (&xv)[PI]) {
    constexpr int NT = NW * 64;
#pragma unroll
    for (int j = 0; j < PI; j++) {
        const int p = min((int)threadIdx.x + j * NT, nb * 8 - 1);
        const float* ptr = x + (p >> 3) * 32 + (p & 7) * 4;
        asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(xv[j]) : "v"(ptr) : "memory");
    }
}

template <int N>
__device__ __forceinline__ void wait_prep_x() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The compiler takes an asm load's result as ready right after the load and
// may move arithmetic on it above the explicit wait.  Passing each result
// through an empty volatile asm placed after the wait makes every use depend
// on a value defined after it.
template <int PI>
__device__ __forceinline__ void after_wait(f32x4 (&v)[PI]) {
#pragma unroll
    for (int j = 0; j < PI; j++) asm volatile("" : "+v"(v[j]));
}
template <int PI>
__device__ __forceinline__ void after_wait(f32x4 (&v)[PI][2]) {
#pragma unroll
    for (int j = 0; j < PI; j++) asm volatile("" : "+v"(v[j][0]), "+v"(v[j][1]));
}

// SUMS: also the digit sums (the Q4_0 -8 offset terms); the K-quant kernels
// do not read them.
template <int NW, int PI, bool SUMS = true>
__device__ void prep_float_lds(const f32x4 (&xv)[PI], int nb, int* __restrict__ lds) {
    constexpr int NT = NW * 64;
#pragma unroll
    for (int j = 0; j < PI; j++) {
        const int p = threadIdx.x + j * NT;
        if (j * NT >= nb * 8) break;  // uniform
        const int c = p >> 3, k = p & 7;
        const f32x4 v = xv[j];
        // the block's largest magnitude; an Inf or NaN shows as bits >= 0x7F800000
        const uint32_t ab = max8_u32(max(max(abs_bits(v.x), abs_bits(v.y)), max(abs_bits(v.z), abs_bits(v.w))));
        const bool anybad = ab >= 0x7F800000u;
        const float amax = __builtin_bit_cast(float, ab);
        // scale tiny blocks by 2^64 so that 8323072/amax stays finite (exact)
        // (the reciprocal's 1 ulp keeps |t| within 8323075, far inside the digits' range)
        const float pw = (amax < 0x1p-60f) ? 0x1p64f : 1.0f;
        const float inv = (amax > 0.0f && !anybad) ? 8323072.0f * __builtin_amdgcn_rcpf(amax * pw) : 0.0f;
        const float f = anybad ? 0.0f : pw * inv;
        uint32_t e0 = (uint32_t)(rintf(v.x * f) + 8421504.0f) ^ 0x808080u;
        uint32_t e1 = (uint32_t)(rintf(v.y * f) + 8421504.0f) ^ 0x808080u;
        uint32_t e2 = (uint32_t)(rintf(v.z * f) + 8421504.0f) ^ 0x808080u;
        uint32_t e3 = (uint32_t)(rintf(v.w * f) + 8421504.0f) ^ 0x808080u;
        if (anybad) e0 = e1 = e2 = e3 = 0u;  // S is NaN for this block anyway
        // gather byte k of e0..e3 into one dword per digit
        const uint32_t p01 = perm(e1, e0, 0x05010400u);   // c0 c1 b0 b1
        const uint32_t p23 = perm(e3, e2, 0x05010400u);   // c2 c3 b2 b3
        const uint32_t q01 = perm(e1, e0, 0x0c0c0602u);   // a0 a1 0 0
        const uint32_t q23 = perm(e3, e2, 0x0c0c0602u);   // a2 a3 0 0
        const uint32_t dc = perm(p23, p01, 0x05040100u);
        const uint32_t db = perm(p23, p01, 0x07060302u);
        const uint32_t da = perm(q23, q01, 0x05040100u);
        const int g = k >> 2, k4 = k & 3;
        if (p < nb * 8) {
            lds[lds_word(0 + g, k4, nb, c)] = (int)da;
            lds[lds_word(2 + g, k4, nb, c)] = (int)db;
            lds[lds_word(4 + g, k4, nb, c)] = (int)dc;
        }
        const float xs = sum8_f32((v.x + v.y) + (v.z + v.w));
        if constexpr (SUMS) {
            const int sa = sum8_i32(__builtin_amdgcn_sdot4((int)da, (int)ONES, 0, false));
            const int sb = sum8_i32(__builtin_amdgcn_sdot4((int)db, (int)ONES, 0, false));
            const int sc = sum8_i32(__builtin_amdgcn_sdot4((int)dc, (int)ONES, 0, false));
            if (k == 0 && p < nb * 8) {
                lds[lds_word(6, 1, nb, c)] = sa;
                lds[lds_word(6, 2, nb, c)] = sb;
                lds[lds_word(6, 3, nb, c)] = sc;
            }
        }
        if (k == 0 && p < nb * 8) {
            const float nan = __builtin_nanf("");
            lds[lds_word(6, 0, nb, c)] = __builtin_bit_cast(int, anybad ? nan : amax * (1.0f / 127.0f));
            lds[lds_word(7, 0, nb, c)] = __builtin_bit_cast(int, anybad ? nan : xs);
        }
    }
}

// quantize_row_q8_0 (quantize.rs:164-193), byte-exact, into LDS records.
template <int NW, int PI>
__device__ void prep_native_lds(const f32x4 (&xv)[PI], int nb, int* __restrict__ lds) {
    constexpr int NT = NW * 64;
#pragma unroll
    for (int j = 0; j < PI; j++) {
        const int p = threadIdx.x + j * NT;
        if (j * NT >= nb * 8) break;  // uniform
        const int c = p >> 3, k = p & 7;
        const f32x4 v = xv[j];
        // fmaxf(0, |x|) drops NaN as the fold from 0.0 with f32::max does
        float amax = fmaxf(fmaxf(fmaxf(0.0f, fabsf(v.x)), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        amax = max8_f32(amax);
        const float scale = (amax == 0.0f) ? 0.0f : amax / 127.0f;
        const float rt = h2f(f2h_rne(scale));
        const float inv = (rt == 0.0f) ? 0.0f : 1.0f / rt;
        const float vv[4] = {v.x, v.y, v.z, v.w};
        uint32_t d = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float r = roundf(vv[j] * inv);
            const int q = (r != r) ? 0 : (int)fminf(fmaxf(r, -128.0f), 127.0f);
            d |= ((uint32_t)q & 0xFFu) << (8 * j);
        }
        if (p < nb * 8) lds[lds_word(k >> 2, k & 3, nb, c)] = (int)d;
        const int qs = sum8_i32(__builtin_amdgcn_sdot4((int)d, (int)ONES, 0, false));
        if (k == 0 && p < nb * 8) {
            lds[lds_word(2, 0, nb, c)] = __builtin_bit_cast(int, rt);
            lds[lds_word(2, 1, nb, c)] = qs;
        }
    }
}

// ---- int4-digit records for Q4_0 / Q4_1 (float mode) --------------------------------
// x_j ~= S4 * t_j with t_j = rint(x_j * 7829364 / amax), a signed 24-bit code
// (|t| <= 0x777777 = 7829367, the largest code the digits hold; the scale
// leaves three units for the rounding of amax * (7829364 * rcp(amax)))
// held as six signed base-16 digits: t + 0x888888 is in [0, 2^24), so the
// nibbles of e = (t + 0x888888) ^ 0x888888 are the digits as int4 (nibble L
// weighs 16^L).  The digit dwords follow the Q4 nibble order (byte j of a
// block holds element j low and j+16 high), so that v_dot8_i32_i4 multiplies
// the weight nibbles in place: dword k of level L holds the digits of elements
// 4k, 4k+16, 4k+1, 4k+17, 4k+2, 4k+18, 4k+3, 4k+19.
// Group layout per column (i32x4 at lds[g * nb + c]): g0..g5 = level 0..5
// (dwords k = 0..3), g6 = {S4, sum x, 0, 0}.  Four threads share a column;
// thread k handles elements 4k..4k+3 and 4k+16..4k+19.


// Nibble levels 2b and 2b+1 of the eight codes: P holds byte b of elements
// 4k..4k+3, Q byte b of elements 4k+16..4k+19.
__device__ __forceinline__ void nib_levels(uint32_t P, uint32_t Q, uint32_t& lo, uint32_t& hi) {
    lo = (P & 0x0F0F0F0Fu) | ((Q & 0x0F0F0F0Fu) << 4);
    hi = ((P >> 4) & 0x0F0F0F0Fu) | (Q & 0xF0F0F0F0u);
}

// Prologues applied to x as the prep reads it (decoder fusion):
//   PRO_RMSNORM: x_j * (1 / sqrt(sum(x^2) / K + eps)) * g_j (ops.rs:688-751),
//                aux = g, the sum formed by the workgroup;
//   PRO_SWIGLU:  silu(x_j) * x_{K + j}, silu(v) = v * (1 / (1 + exp(-v)))
//                (feed_forward.rs:138-150, ops.rs:441-446), aux = x + K.
constexpr int PRO_NONE = 0, PRO_RMSNORM = 1, PRO_SWIGLU = 2;

// Fusion arguments of one launch (unused fields are ignored).
struct Fuse {
    const float* g;  // RMSNorm weights
    float eps;
    int xstride;     // floats between activation rows
    // EPI_ROPE_KV (rope.rs:134-200, kv_cache.rs:94-106)
    const int* pos;             // cache position of activation row 0
    const float* cos_t;         // [max_seq][hd / 2]
    const float* sin_t;
    void* kc;                   // paged pool [n_pages][n_kv][KV_PAGE][hd], f16 or f32
    void* vc;
    const int* kv_table;        // physical page of each logical page
    int n_heads, n_kv, hd, kv_f16;
    uint64_t* xch;              // PUB: the layer's exchange, one tagged value per q / k / v row
    int* err;                   // XIO_IN: set when a wait runs out (never in a correct launch)
    // XIO_IN: x read as tagged words from xin instead of X; XIO_OUT: outputs
    // published as tagged words to xout instead of Y; the tag is *pos + 1
    const uint64_t* xin;
    uint64_t* xout;
};

// How a fused GEMV body exchanges its activation within a launch: XIO_NONE
// (x read from memory, y stored), XIO_IN (x polled from another role's
// published words; the weight stream starts before x exists), XIO_OUT (y
// published as tagged words for another role of the same launch).
constexpr int XIO_NONE = 0, XIO_IN = 1, XIO_OUT = 2;

template <int NW, int PI, int PRO = PRO_NONE>
__device__ __forceinline__ void load_prep_x4(const float* __restrict__ x, const float* __restrict__ aux, int nb,
                                             f32x4 (&xv)[PI][2], f32x4 (&av)[PI][2]) {
    constexpr int NT = NW * 64;
#pragma unroll
    for (int j = 0; j < PI; j++) {
        const int p = min((int)threadIdx.x + j * NT, nb * 4 - 1);
        const int o = (p >> 2) * 32 + (p & 3) * 4;
        const float* ptr = x + o;
        asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(xv[j][0]) : "v"(ptr) : "memory");
        asm volatile("global_load_dwordx4 %0, %1, off offset:64" : "=v"(xv[j][1]) : "v"(ptr) : "memory");
        if constexpr (PRO != PRO_NONE) {
            const float* aptr = aux + o;
            asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(av[j][0]) : "v"(aptr) : "memory");
            asm volatile("global_load_dwordx4 %0, %1, off offset:64" : "=v"(av[j][1]) : "v"(aptr) : "memory");
        }
    }
}

template <int NW, int PI, int PRO = PRO_NONE>
__device__ void prep_float4_lds(const f32x4 (&xv)[PI][2], const f32x4 (&av)[PI][2], float eps, int nb,
                                int* __restrict__ lds) {
    constexpr int NT = NW * 64;
    float inv = 1.0f;
    if constexpr (PRO == PRO_RMSNORM) {
        // sum of squares over the row: this thread's elements, then the
        // workgroup (fixed reduction tree: every workgroup gets the same bits)
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < PI; j++) {
            if ((int)threadIdx.x + j * NT < nb * 4) {
                const f32x4 a = xv[j][0], b = xv[j][1];
                ss += ((a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w)) +
                      ((b.x * b.x + b.y * b.y) + (b.z * b.z + b.w * b.w));
            }
        }
        ss = sum8_f32(ss);
        ss += dpp_f32<DPP_ROW_MIRROR>(ss);
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        float* red = reinterpret_cast<float*>(lds + 7 * 4 * nb);  // group 7 is free in int4 records
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) tot += red[w];
        inv = 1.0f / sqrtf(tot / (float)(nb * 32) + eps);
    }
#pragma unroll
    for (int j = 0; j < PI; j++) {
        const int p = threadIdx.x + j * NT;
        if (j * NT >= nb * 4) break;  // uniform
        const int c = p >> 2, k = p & 3;
        const f32x4 va = xv[j][0], vb = xv[j][1];
        float v[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
        if constexpr (PRO != PRO_NONE) {
            const f32x4 ga = av[j][0], gb = av[j][1];
            const float a[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if constexpr (PRO == PRO_RMSNORM) {
                    v[i] = (v[i] * inv) * a[i];
                } else {
                    const float sig = 1.0f / (1.0f + expf(-v[i]));
                    v[i] = (v[i] * sig) * a[i];
                }
            }
        }
        // the block's largest magnitude; an Inf or NaN shows as bits >= 0x7F800000
        uint32_t ab = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) ab = max(ab, abs_bits(v[i]));
        ab = max4_u32(ab);
        const bool anybad = ab >= 0x7F800000u;
        const float amax = __builtin_bit_cast(float, ab);
        // 7829364 / amax through the reciprocal (1 ulp): |t| <= 7829366, one
        // code inside the digits' range 0x777777 = 7829367
        const float pw = (amax < 0x1p-60f) ? 0x1p64f : 1.0f;
        const float f = (amax > 0.0f && !anybad) ? pw * (7829364.0f * __builtin_amdgcn_rcpf(amax * pw)) : 0.0f;
        uint32_t e[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            e[i] = anybad ? 0u : ((uint32_t)(rintf(v[i] * f) + 8947848.0f) ^ 0x888888u);
        // byte b of e[0..3] -> P_b, of e[4..7] -> Q_b
        const uint32_t a01 = perm(e[1], e[0], 0x05010400u), a23 = perm(e[3], e[2], 0x05010400u);
        const uint32_t b01 = perm(e[5], e[4], 0x05010400u), b23 = perm(e[7], e[6], 0x05010400u);
        const uint32_t P0 = perm(a23, a01, 0x05040100u), P1 = perm(a23, a01, 0x07060302u);
        const uint32_t Q0 = perm(b23, b01, 0x05040100u), Q1 = perm(b23, b01, 0x07060302u);
        const uint32_t c01 = perm(e[1], e[0], 0x0c0c0602u), c23 = perm(e[3], e[2], 0x0c0c0602u);
        const uint32_t d01 = perm(e[5], e[4], 0x0c0c0602u), d23 = perm(e[7], e[6], 0x0c0c0602u);
        const uint32_t P2 = perm(c23, c01, 0x05040100u), Q2 = perm(d23, d01, 0x05040100u);
        uint32_t L[6];
        nib_levels(P0, Q0, L[0], L[1]);
        nib_levels(P1, Q1, L[2], L[3]);
        nib_levels(P2, Q2, L[4], L[5]);
        float xs = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) xs += v[i];
        xs = sum4_f32(xs);
        if (p < nb * 4) {
#pragma unroll
            for (int lv = 0; lv < 6; lv++) lds[lds_word(lv, k, nb, c)] = (int)L[lv];
            if (k == 0) {
                const float nan = __builtin_nanf("");
                lds[lds_word(6, 0, nb, c)] = __builtin_bit_cast(int, anybad ? nan : amax * (1.0f / 7829364.0f));
                lds[lds_word(6, 1, nb, c)] = __builtin_bit_cast(int, anybad ? nan : xs);
            }
        }
    }
}

// Only vector members: S and sum(x) stay packed in `meta` (as loaded) and are
// bit-cast where they are used.
struct RF4 {
    i32x4 lv[6];
    i32x4 meta;  // {S4, sum x, 0, 0}
    __device__ float S() const { return as_f32(meta.x); }
    __device__ float xsum() const { return as_f32(meta.y); }
};
__device__ __forceinline__ RF4 read_rf4(const i32x4* __restrict__ l4, int nb, int c) {
    RF4 r;
#pragma unroll
    for (int lv = 0; lv < 6; lv++) r.lv[lv] = l4[lv * nb + c];
    r.meta = l4[6 * nb + c];
    return r;
}

// The three-address v_dot8_i32_i4 on a zero accumulator: the first product
// of a chain (the compiler otherwise zeroes a register for the two-address
// v_dot8c form).
__device__ __forceinline__ int dot8z(uint32_t a, int b) {
    int r;
    asm("v_dot8_i32_i4 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// sum_j w_j * t_j for signed int4 weight nibbles w (four dwords), as a float.
__device__ __forceinline__ float dot_i4(const uint32_t (&w)[4], const RF4& x) {
    int D[6];
#pragma unroll
    for (int lv = 0; lv < 6; lv++) {
        int a = dot8z(w[0], x.lv[lv].x);
        a = __builtin_amdgcn_sdot8((int)w[1], x.lv[lv].y, a, false);
        a = __builtin_amdgcn_sdot8((int)w[2], x.lv[lv].z, a, false);
        D[lv] = __builtin_amdgcn_sdot8((int)w[3], x.lv[lv].w, a, false);
    }
    // |D| <= 32 * 8 * 8, so each three-level Horner sum stays far inside int32
    const int hi = (((D[5] << 4) + D[4]) << 4) + D[3];
    const int lo = (((D[2] << 4) + D[1]) << 4) + D[0];
    return fmaf((float)hi, 4096.0f, (float)lo);
}

// ---- records from LDS -------------------------------------------------------------
struct RF {
    i32x4 a0, a1, b0, b1, c0, c1;
    float S;
    int sa, sb, sc;
    float xsum;
};
__device__ __forceinline__ RF read_rf(const i32x4* __restrict__ l4, int nb, int c) {
    RF r;
    r.a0 = l4[0 * nb + c];
    r.a1 = l4[1 * nb + c];
    r.b0 = l4[2 * nb + c];
    r.b1 = l4[3 * nb + c];
    r.c0 = l4[4 * nb + c];
    r.c1 = l4[5 * nb + c];
    const i32x4 m = l4[6 * nb + c];
    r.S = as_f32(m.x);
    r.sa = m.y;
    r.sb = m.z;
    r.sc = m.w;
    r.xsum = as_f32(l4[7 * nb + c].x);
    return r;
}
struct RN {
    i32x4 q0, q1;
    float scale;
    int qsum;
};
__device__ __forceinline__ RN read_rn(const i32x4* __restrict__ l4, int nb, int c) {
    RN r;
    r.q0 = l4[0 * nb + c];
    r.q1 = l4[1 * nb + c];
    const i32x4 m = l4[2 * nb + c];
    r.scale = as_f32(m.x);
    r.qsum = m.y;
    return r;
}

__device__ __forceinline__ float dot3(const uint32_t (&w)[8], const RF& x, int ia, int ib, int ic) {
    int A = ia, B = ib, C = ic;
    A = dot4(w[0], x.a0.x, A); A = dot4(w[1], x.a0.y, A); A = dot4(w[2], x.a0.z, A); A = dot4(w[3], x.a0.w, A);
    A = dot4(w[4], x.a1.x, A); A = dot4(w[5], x.a1.y, A); A = dot4(w[6], x.a1.z, A); A = dot4(w[7], x.a1.w, A);
    B = dot4(w[0], x.b0.x, B); B = dot4(w[1], x.b0.y, B); B = dot4(w[2], x.b0.z, B); B = dot4(w[3], x.b0.w, B);
    B = dot4(w[4], x.b1.x, B); B = dot4(w[5], x.b1.y, B); B = dot4(w[6], x.b1.z, B); B = dot4(w[7], x.b1.w, B);
    C = dot4(w[0], x.c0.x, C); C = dot4(w[1], x.c0.y, C); C = dot4(w[2], x.c0.z, C); C = dot4(w[3], x.c0.w, C);
    C = dot4(w[4], x.c1.x, C); C = dot4(w[5], x.c1.y, C); C = dot4(w[6], x.c1.z, C); C = dot4(w[7], x.c1.w, C);
    const float t = fmaf((float)C, 1.0f / 256.0f, (float)B);
    return fmaf(t, 1.0f / 256.0f, (float)A);
}
// dot3(w, x, 0, 0, 0) with each digit's chain started by the three-address
// v_dot4_i32_i8 on a zero accumulator (the compiler otherwise zeroes a
// register for the two-address v_dot4c form: three moves a call)
__device__ __forceinline__ int dot4z(uint32_t a, int b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float dot3z(const uint32_t (&w)[8], const RF& x) {
    int A = dot4z(w[0], x.a0.x), B = dot4z(w[0], x.b0.x), C = dot4z(w[0], x.c0.x);
    A = dot4(w[1], x.a0.y, A); A = dot4(w[2], x.a0.z, A); A = dot4(w[3], x.a0.w, A);
    A = dot4(w[4], x.a1.x, A); A = dot4(w[5], x.a1.y, A); A = dot4(w[6], x.a1.z, A); A = dot4(w[7], x.a1.w, A);
    B = dot4(w[1], x.b0.y, B); B = dot4(w[2], x.b0.z, B); B = dot4(w[3], x.b0.w, B);
    B = dot4(w[4], x.b1.x, B); B = dot4(w[5], x.b1.y, B); B = dot4(w[6], x.b1.z, B); B = dot4(w[7], x.b1.w, B);
    C = dot4(w[1], x.c0.y, C); C = dot4(w[2], x.c0.z, C); C = dot4(w[3], x.c0.w, C);
    C = dot4(w[4], x.c1.x, C); C = dot4(w[5], x.c1.y, C); C = dot4(w[6], x.c1.z, C); C = dot4(w[7], x.c1.w, C);
    const float t = fmaf((float)C, 1.0f / 256.0f, (float)B);
    return fmaf(t, 1.0f / 256.0f, (float)A);
}
__device__ __forceinline__ int dot1(const uint32_t (&w)[8], const RN& x, int acc) {
    acc = dot4(w[0], x.q0.x, acc); acc = dot4(w[1], x.q0.y, acc);
    acc = dot4(w[2], x.q0.z, acc); acc = dot4(w[3], x.q0.w, acc);
    acc = dot4(w[4], x.q1.x, acc); acc = dot4(w[5], x.q1.y, acc);
    acc = dot4(w[6], x.q1.z, acc); acc = dot4(w[7], x.q1.w, acc);
    return acc;
}

// ---- weight windows ------------------------------------------------------------------
template <int WT> struct Geo;
template <> struct Geo<(int)WType::Q4_0> { static constexpr int BYTES = 18, WORDS = 5; };
template <> struct Geo<(int)WType::Q4_1> { static constexpr int BYTES = 20, WORDS = 5; };
template <> struct Geo<(int)WType::Q8_0> { static constexpr int BYTES = 34, WORDS = 9; };

// Window of WORDS dwords from the dword-aligned base at or below byte `off`
// (off = RSRC_OOB: no load, zeros).  Branch-free.
// GUARD: the last dword may end 2 bytes past the matrix (an aligned block at
// the very end); it is then read as the matrix's last dword shifted down 16.
template <int WORDS, bool GUARD>
__device__ __forceinline__ void load_window(__amdgpu_buffer_rsrc_t rs, uint32_t off,
                                            uint32_t wbytes, uint32_t (&w)[WORDS]) {
    const uint32_t base = off & ~3u;
    const u32x4 v0 = buf_load_b128(rs, base);
    w[0] = v0.x; w[1] = v0.y; w[2] = v0.z; w[3] = v0.w;
    if constexpr (WORDS == 9) {
        const u32x4 v1 = buf_load_b128(rs, base + 16);
        w[4] = v1.x; w[5] = v1.y; w[6] = v1.z; w[7] = v1.w;
    }
    const uint32_t toff = base + 4 * (WORDS - 1);
    if constexpr (GUARD) {
        const bool over = base < wbytes && base + 4 * WORDS > wbytes;
        w[WORDS - 1] = buf_load_b32(rs, over ? wbytes - 4 : toff) >> (over ? 16 : 0);
    } else {
        w[WORDS - 1] = buf_load_b32(rs, toff);
    }
}

// Per-block decode + dot; returns the block's contribution to y.
template <int WT, bool NATIVE>
struct BlockDot;

template <>
struct BlockDot<(int)WType::Q4_0, false> {
    __device__ static float run(const uint32_t (&w)[5], uint32_t sel, uint32_t dsh, const RF& x,
                                int ia, int ib, int ic) {
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t nbl = perm(w[k + 1], w[k], sel);
            q[k] = nbl & NIB;
            q[k + 4] = (nbl >> 4) & NIB;
        }
        const float d = h2f((w[0] >> dsh) & 0xFFFFu);
        return (x.S * d) * dot3(q, x, ia, ib, ic);
    }
};
template <>
struct BlockDot<(int)WType::Q8_0, false> {
    __device__ static float run(const uint32_t (&w)[9], uint32_t sel, uint32_t dsh, const RF& x,
                                int, int, int) {
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 8; k++) q[k] = perm(w[k + 1], w[k], sel);
        const float d = h2f((w[0] >> dsh) & 0xFFFFu);
        return (x.S * d) * dot3z(q, x);
    }
};
template <>
struct BlockDot<(int)WType::Q4_1, false> {
    __device__ static float run(const uint32_t (&w)[5], uint32_t, uint32_t, const RF& x, int, int,
                                int) {
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            q[k] = w[k + 1] & NIB;
            q[k + 4] = (w[k + 1] >> 4) & NIB;
        }
        const float d = h2f(w[0] & 0xFFFFu), m = h2f(w[0] >> 16);
        return fmaf(x.S * d, dot3z(q, x), m * x.xsum);
    }
};
template <>
struct BlockDot<(int)WType::Q4_0, true> {
    __device__ static float run(const uint32_t (&w)[5], uint32_t sel, uint32_t dsh, const RN& x) {
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t nbl = perm(w[k + 1], w[k], sel);
            q[k] = nbl & NIB;
            q[k + 4] = (nbl >> 4) & NIB;
        }
        const float d = h2f((w[0] >> dsh) & 0xFFFFu);
        // dot_q4q8_block = sum q*q8 - 8 sum q8 (exact); (int as f32) * sx * sw
        return ((float)dot1(q, x, -8 * x.qsum) * x.scale) * d;
    }
};
template <>
struct BlockDot<(int)WType::Q4_1, true> {
    __device__ static float run(const uint32_t (&w)[5], uint32_t, uint32_t, const RN& x) {
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            q[k] = w[k + 1] & NIB;
            q[k + 4] = (w[k + 1] >> 4) & NIB;
        }
        const float d = h2f(w[0] & 0xFFFFu), m = h2f(w[0] >> 16);
        // q8_scale * (d * unsigned_dot + m * q8_sum)   (quantize.rs:562)
        return x.scale * (d * (float)dot1(q, x, 0) + m * (float)x.qsum);
    }
};

// Q4_0 / Q4_1 float mode on int4 digits.
template <int WT>
__device__ __forceinline__ float block_dot_i4(const uint32_t (&w)[5], uint32_t sel, uint32_t dsh,
                                              const RF4& x) {
    uint32_t q[4];
    if (WT == (int)WType::Q4_0) {
#pragma unroll
        for (int k = 0; k < 4; k++) q[k] = perm(w[k + 1], w[k], sel) ^ 0x88888888u;  // q - 8
        const float d = h2f((w[0] >> dsh) & 0xFFFFu);
        return (x.S() * d) * dot_i4(q, x);
    } else {
#pragma unroll
        for (int k = 0; k < 4; k++) q[k] = w[k + 1] ^ 0x88888888u;  // q - 8
        const float d = h2f(w[0] & 0xFFFFu), m = h2f(w[0] >> 16);
        // sum q x = sum (q-8) x + 8 sum x
        return fmaf(x.S() * d, dot_i4(q, x), fmaf(8.0f, d, m) * x.xsum());
    }
}


// ---- the fused kernel (Q4_0 / Q4_1 / Q8_0) ----------------------------------------------
// Block g of the matrix starts at byte g*BYTES; with BYTES = 18 or 34 its
// dword alignment alternates with g.  When nb is even the parity of g is the
// parity of the column, so the realignment selectors are per column.
//
// A wave owns R rows x CPL columns = NB blocks per lane, visited row-major.
// The loads run PF blocks ahead of the compute in program order: a wave issues
// its instructions in order and the memory pipeline accepts only so many
// loads per CU, so interleaving load issue with compute is what lets the dot
// products overlap the weight stream.
// Epilogues: EPI_STORE y = W x; EPI_RESIDUAL y += W x in place (the residual
// add of transformer_block.rs:333,352); EPI_SWIGLU: W holds [gate_j; up_j]
// as rows 2j, 2j+1 and y[j] = silu(gate_j) * up_j (feed_forward.rs:138-150) --
// a wave then owns row pairs, so both halves of a pair meet in one wave.
// EPI_ROPE_KV: W holds [Wq; Wk; Wv] and a wave owns the RoPE pairs (i, i + hd/2)
// of a head: q rows are rotated in place in y, k rows rotated and v rows
// copied into the KV cache at the row's position (y's k / v rows unwritten).
constexpr int EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_ROPE_KV = 3;

// PRO: prologue on x (PRO_NONE / PRO_RMSNORM / PRO_SWIGLU, int4 records only).
// The body of one workgroup (bx, by): row group bx, activation row by.
// PUB (EPI_ROPE_KV only): every q / k / v output (after RoPE) is also written
// to the exchange fz.xch as one tagged 8-byte value (xch_put, tag = position
// + 1), which the fused decode attention of the same launch polls; the q
// rows are then not written to y (nothing else reads them).
// XIO (int4 records, one activation row): see XIO_NONE / XIO_IN / XIO_OUT;
// XIO_IN takes PRO_RMSNORM and issues every weight block before polling x,
// XIO_OUT takes EPI_RESIDUAL (the old y still read from Y).
template <int WT, bool NATIVE, int R, int CPL, bool NB_EVEN, int NW, int PRO = PRO_NONE, int EPI = EPI_STORE,
          bool PUB = false, int XIO = XIO_NONE>
__device__ __forceinline__ void gemv_fused_body(int bx, int by, i32x4* __restrict__ lds4, const uint8_t* __restrict__ W,
                                                int n, int nb, int rpw, const float* __restrict__ X,
                                                float* __restrict__ Y, const Fuse& fz) {
    static_assert(!PUB || EPI == EPI_ROPE_KV, "publication is for the q/k/v epilogue");
    static_assert(XIO != XIO_IN || PRO == PRO_RMSNORM, "x from the exchange feeds the RMSNorm prologue");
    static_assert(XIO != XIO_OUT || EPI == EPI_RESIDUAL, "published outputs are residual sums");
    constexpr int BYTES = Geo<WT>::BYTES, WORDS = Geo<WT>::WORDS;
    constexpr int LPB = (WORDS == 9) ? 3 : 2;    // load instructions per block
    constexpr int NB = R * CPL;                   // blocks per lane
    // Q4_0 / Q4_1 float mode use int4-digit records (four threads per column),
    // everything else int8 records (eight threads per column)
    constexpr bool I4 = !NATIVE && (WT == (int)WType::Q4_0 || WT == (int)WType::Q4_1);
    // PF blocks in flight ahead of the compute; only P0 <= PF of them are
    // issued before the prep.  The prep waits for its x loads, which queue in
    // the CU behind every weight load issued before them, so the longer prep
    // of the int4 records wants fewer weight loads in front of it (measured on
    // MI355X: P0 = 2, PF = 3 for int4 records, 4 / 4 otherwise).
    // (int4 records with 16 blocks a lane -- 8 rows a wave -- keep 5 in flight)
    constexpr int PF_I4 = NB >= 16 ? 5 : 3;
    // (the q/k/v launch of a decode step, 8 blocks a lane on 192 of the
    // CUs: all of them in flight, 4 before the prep; 7B decode 812 -> 820
    // tokens/s against 3 / 2, and against 8 / 8: 804)
    // (XIO_IN: every block before x exists)
    constexpr int PF = (EPI == EPI_ROPE_KV || XIO == XIO_IN) ? NB : (NB < (I4 ? PF_I4 : 4)) ? NB : (I4 ? PF_I4 : 4);
    constexpr int P0 = XIO == XIO_IN ? NB
                       : EPI == EPI_ROPE_KV ? (PF < 4 ? PF : 4) : (PF < (I4 ? 2 : 4)) ? PF : (I4 ? 2 : 4);
    constexpr int PI = I4 ? (CPL * 4 + NW - 1) / NW : (CPL * 8 + NW - 1) / NW;
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int r0 = bx * rpw;
    const int rend = min(n, r0 + rpw);
    static_assert(PRO == PRO_NONE || I4, "prologues run on the int4-record prep");
    constexpr bool PAIRS = (EPI == EPI_SWIGLU || EPI == EPI_ROPE_KV);
    static_assert(!PAIRS || R % 2 == 0, "row pairs need an even row count per wave");
    const float* x = X + (size_t)by * fz.xstride;
    float* y = Y + (size_t)by * (EPI == EPI_SWIGLU ? n / 2 : n);
    const int half = fz.hd >> 1;
    // The wave's r-th row as a linear row in [r0, r0 + rpw) (validity against
    // rend) and as a matrix row (addressing).  Pairs (r, r + 1 even/odd):
    // SwiGLU rows 2j, 2j + 1; RoPE: linear pair p is the partners (i, i + hd/2)
    // of head p / (hd/2), i = p % (hd/2).
    auto row_of = [&](int r) {  // linear
        if constexpr (PAIRS) return r0 + 2 * (wv + (r >> 1) * NW) + (r & 1);
        return r0 + wv + r * NW;
    };
    auto mat_row = [&](int lin) {
        if constexpr (EPI == EPI_ROPE_KV) {
            const int pp = lin >> 1;
            return (pp / half) * fz.hd + pp % half + (lin & 1) * half;
        }
        return lin;
    };
    const uint32_t row_bytes = (uint32_t)nb * BYTES;
    const uint32_t wbytes = (uint32_t)n * row_bytes;

    // Branch-free load issue (a slot past the workgroup's rows or the row's
    // blocks loads nothing: out-of-range buffer offset), so the compiler's
    // wait counts are exact.  With nb even the last block of the matrix has an
    // odd index and its window ends exactly at the end of the matrix; only odd
    // nb needs the guarded tail load.
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(W, wbytes);
    uint32_t win[NB][WORDS];
    auto issue = [&](int b) {
        const int r = b / CPL, i = b % CPL;
        const int row = row_of(r), col = lane + 64 * i;
        const uint32_t off = (row < rend && col < nb)
                                 ? (uint32_t)mat_row(row) * row_bytes + (uint32_t)col * BYTES
                                 : RSRC_OOB;
        load_window<WORDS, !NB_EVEN>(rs, off, wbytes, win[b]);
    };

    // The lane that stores row row_of(lane >> SH) after the reduction
    // (EPI_SWIGLU / EPI_ROPE_KV: the pair starting there) fetches what its
    // epilogue reads ahead of the stream, so no load waits at the kernel's
    // end: the residual's old y (here), the RoPE position (a scalar load) and
    // cos / sin (after the prep).
    // R = 8 (store and SwiGLU epilogues): rows reduced and stored in two
    // groups of four
    constexpr int RG = R > 4 ? 4 : R;
    constexpr int NGRP = R / RG;
    static_assert(R <= 4 || (R == 8 && (EPI == EPI_STORE || EPI == EPI_SWIGLU)), "rows per wave");
    constexpr int SH = reduce_span_log2<RG>();
    const bool st_lane = (lane & (((PAIRS ? 2 : 1) << SH) - 1)) == 0;
    const int st_row = row_of(lane >> SH);
    float y_old = 0.0f;
    if constexpr (EPI == EPI_RESIDUAL) {
        if (st_lane && st_row < rend) y_old = y[st_row];
    }
    int rope_pos = 0;
    if constexpr (EPI == EPI_ROPE_KV) rope_pos = *fz.pos + by;

    // ---- x for the prep first, then the first PF blocks ----
    __builtin_amdgcn_s_setprio(2);  // the prep ahead of other workgroups' streams
    if constexpr (XIO == XIO_IN) {
        // the weight stream first (it does not depend on x), then the
        // RMSNorm weights, then x: this thread's pieces (load_prep_x4's
        // elements) polled from the exchange until all carry the tag
        static_assert(I4, "int4 records");
#pragma unroll
        for (int b = 0; b < P0; b++) issue(b);
        f32x4 xv[PI][2], av[PI][2];
        constexpr int NT = NW * 64;
#pragma unroll
        for (int j = 0; j < PI; j++) {
            const int p = min((int)threadIdx.x + j * NT, nb * 4 - 1);
            const int o = (p >> 2) * 32 + (p & 3) * 4;
            av[j][0] = *reinterpret_cast<const f32x4*>(fz.g + o);
            av[j][1] = *reinterpret_cast<const f32x4*>(fz.g + o + 16);
        }
        const int xtag = *fz.pos + 1;
        // Each wave first watches one word (wave w: the last of the w-th
        // eighth of x), sleeping between reads, and polls its pieces only
        // once that word is there.  Where these workgroups share the CUs
        // with the down workgroups, hundreds of them polling every word at
        // once kept the down workgroups' stores from landing for the
        // whole bounded wait (MI355X, 2 workgroups a CU: 60 ms).
        {
            const uint64_t* watch = fz.xin + min((wv + 1) * nb * 4, nb * 32) - 1;
            for (int spins = 0;; spins++) {
                if (att::xch_ok(att::xch_get(watch), xtag) || spins > (1 << 16)) break;
                __builtin_amdgcn_s_sleep(2);
            }
        }
#pragma unroll
        for (int j = 0; j < PI; j++) {
            const int p = min((int)threadIdx.x + j * NT, nb * 4 - 1);
            const uint64_t* src = fz.xin + (p >> 2) * 32 + (p & 3) * 4;
            uint64_t v[8];
            for (int spins = 0;; spins++) {
                bool ok = true;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    v[i] = att::xch_get(src + (i & 3) + (i >> 2) * 16);
                    ok = ok && att::xch_ok(v[i], xtag);
                }
                if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
                if (spins > (1 << 16)) {  // only a broken launch gets here
                    if ((threadIdx.x & 63) == 0)
                        __hip_atomic_store(fz.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            xv[j][0] = f32x4{att::xch_val(v[0]), att::xch_val(v[1]), att::xch_val(v[2]), att::xch_val(v[3])};
            xv[j][1] = f32x4{att::xch_val(v[4]), att::xch_val(v[5]), att::xch_val(v[6]), att::xch_val(v[7])};
        }
        prep_float4_lds<NW, PI, PRO>(xv, av, fz.eps, nb, reinterpret_cast<int*>(lds4));
    } else if constexpr (I4) {
        f32x4 xv[PI][2], av[PI][2];
        const float* aux = (PRO == PRO_RMSNORM) ? fz.g : x + nb * 32;
        load_prep_x4<NW, PI, PRO>(x, aux, nb, xv, av);
        // every wave's x loads enter the CU's memory pipeline ahead of any
        // wave's weight loads (an execution barrier only: no wait for the loads)
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int b = 0; b < P0; b++) issue(b);
        wait_prep_x<P0 * LPB>();
        after_wait<PI>(xv);
        if constexpr (PRO != PRO_NONE) after_wait<PI>(av);
        prep_float4_lds<NW, PI, PRO>(xv, av, fz.eps, nb, reinterpret_cast<int*>(lds4));
    } else {
        f32x4 xv[PI];
        load_prep_x<NW, PI>(x, nb, xv);
#pragma unroll
        for (int b = 0; b < P0; b++) issue(b);
        wait_prep_x<P0 * LPB>();
        after_wait<PI>(xv);
        if constexpr (NATIVE)
            prep_native_lds<NW, PI>(xv, nb, reinterpret_cast<int*>(lds4));
        else
            prep_float_lds<NW, PI>(xv, nb, reinterpret_cast<int*>(lds4));
    }
    __syncthreads();
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int b = P0; b < PF; b++) issue(b);
    float rope_c = 0.0f, rope_s = 0.0f;
    if constexpr (EPI == EPI_ROPE_KV) {
        if (st_lane && st_row < rend) {
            const int r1 = mat_row(st_row), head = r1 / fz.hd, i = r1 % fz.hd;
            if (head < fz.n_heads + fz.n_kv) {
                rope_c = fz.cos_t[(size_t)rope_pos * half + i];
                rope_s = fz.sin_t[(size_t)rope_pos * half + i];
            }
        }
    }

    // column records: kept in registers when a lane has at most two columns
    constexpr bool KEEP = (CPL <= 2);
    using Rec = typename std::conditional<NATIVE, RN, typename std::conditional<I4, RF4, RF>::type>::type;
    Rec keep[KEEP ? CPL : 1];
    auto read_rec = [&](int col) -> Rec {
        if constexpr (NATIVE) return read_rn(lds4, nb, col);
        else if constexpr (I4) return read_rf4(lds4, nb, col);
        else return read_rf(lds4, nb, col);
    };
    if constexpr (KEEP) {
#pragma unroll
        for (int i = 0; i < CPL; i++) keep[i] = read_rec(min(lane + 64 * i, nb - 1));
    }

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        if (b + PF < NB) issue(b + PF);
        const int r = b / CPL, i = b % CPL;
        const int row = row_of(r);
        const int col = lane + 64 * i;
        if (row < rend && col < nb) {
            const bool odd = NB_EVEN ? (col & 1) : (((row * nb + col) & 1) != 0);
            const uint32_t sel = odd ? 0x07060504u : 0x05040302u;
            const uint32_t dsh = odd ? 16u : 0u;
            if constexpr (NATIVE) {
                const RN xr = KEEP ? keep[KEEP ? i : 0] : read_rec(col);
                acc[r] += BlockDot<WT, true>::run(win[b], sel, dsh, xr);
            } else if constexpr (I4) {
                const RF4 xr = KEEP ? keep[KEEP ? i : 0] : read_rec(col);
                acc[r] += block_dot_i4<WT>(win[b], sel, dsh, xr);
            } else {
                const RF xr = KEEP ? keep[KEEP ? i : 0] : read_rec(col);
                const int ia = (WT == (int)WType::Q4_0) ? -8 * xr.sa : 0;
                const int ib = (WT == (int)WType::Q4_0) ? -8 * xr.sb : 0;
                const int ic = (WT == (int)WType::Q4_0) ? -8 * xr.sc : 0;
                acc[r] += BlockDot<WT, false>::run(win[b], sel, dsh, xr, ia, ib, ic);
            }
        }
    }
    const bool has_rows = row_of(0) < rend;  // wave-uniform
    if (!has_rows) return;  // the wave had nothing to store

    // ---- reduce and store ----
#pragma unroll
    for (int grp = 0; grp < NGRP; grp++) {
        float accg[RG];
#pragma unroll
        for (int r = 0; r < RG; r++) accg[r] = acc[grp * RG + r];
        const float s = wave_reduce_rows<RG>(accg);
        if constexpr (EPI == EPI_SWIGLU) {
            // rows r (gate, even) and r + 1 (up) sit in adjacent lane groups
            const float up = __shfl_down(s, 1 << SH);
            if ((lane & ((2 << SH) - 1)) == 0) {
                const int g = row_of(grp * RG + (lane >> SH));
                if (g + 1 < rend) y[g >> 1] = (s * (1.0f / (1.0f + expf(-s)))) * up;
            }
        } else if constexpr (EPI == EPI_ROPE_KV) {
            const float x2 = __shfl_down(s, 1 << SH);
            if ((lane & ((2 << SH) - 1)) == 0) {
                const int l1 = row_of(grp * RG + (lane >> SH));
                if (l1 < rend) {
                    const int r1 = mat_row(l1);  // row of x1; x2's row is r1 + half
                    const int head = r1 / fz.hd, i = r1 % fz.hd;
                    const int pos = rope_pos;
                    const float x1 = s;
                    if (head < fz.n_heads + fz.n_kv) {
                        const float c = rope_c, sn = rope_s;
                        const float o1 = x1 * c - x2 * sn, o2 = x1 * sn + x2 * c;
                        if constexpr (PUB) {  // the attention of this launch reads the tagged copies
                            xch_put(fz.xch + r1, o1, pos + 1);
                            xch_put(fz.xch + r1 + half, o2, pos + 1);
                        }
                        if (head < fz.n_heads) {
                            if constexpr (!PUB) {
                                y[r1] = o1;
                                y[r1 + half] = o2;
                            }
                        } else {
                            const size_t ko = kv_row(fz.kv_table, fz.n_kv, head - fz.n_heads, pos, fz.hd) + i;
                            if (fz.kv_f16) {
                                reinterpret_cast<_Float16*>(fz.kc)[ko] = (_Float16)o1;
                                reinterpret_cast<_Float16*>(fz.kc)[ko + half] = (_Float16)o2;
                            } else {
                                reinterpret_cast<float*>(fz.kc)[ko] = o1;
                                reinterpret_cast<float*>(fz.kc)[ko + half] = o2;
                            }
                        }
                    } else {
                        if constexpr (PUB) {
                            xch_put(fz.xch + r1, x1, pos + 1);
                            xch_put(fz.xch + r1 + half, x2, pos + 1);
                        }
                        const size_t vo = kv_row(fz.kv_table, fz.n_kv, head - fz.n_heads - fz.n_kv, pos, fz.hd) + i;
                        if (fz.kv_f16) {
                            reinterpret_cast<_Float16*>(fz.vc)[vo] = (_Float16)x1;
                            reinterpret_cast<_Float16*>(fz.vc)[vo + half] = (_Float16)x2;
                        } else {
                            reinterpret_cast<float*>(fz.vc)[vo] = x1;
                            reinterpret_cast<float*>(fz.vc)[vo + half] = x2;
                        }
                    }
                }
            }
        } else if ((lane & ((1 << SH) - 1)) == 0) {
            const int row = row_of(grp * RG + (lane >> SH));
            if (row < rend) {
                if constexpr (XIO == XIO_OUT)
                    att::xch_put(fz.xout + row, s + y_old, *fz.pos + 1);
                else if constexpr (EPI == EPI_RESIDUAL)
                    y[row] = s + y_old;
                else
                    y[row] = s;
            }
        }
    }
}


template <int WT, bool NATIVE, int R, int CPL, bool NB_EVEN, int NW, int PRO = PRO_NONE, int EPI = EPI_STORE>
__global__ __launch_bounds__(NW * 64) void gemv_fused_kernel(const uint8_t* __restrict__ W, int n,
                                                        int nb, int rpw,
                                                        const float* __restrict__ X,
                                                        float* __restrict__ Y, Fuse fz) {
    extern __shared__ i32x4 lds4[];
    gemv_fused_body<WT, NATIVE, R, CPL, NB_EVEN, NW, PRO, EPI, false>(blockIdx.x, blockIdx.y, lds4, W, n, nb, rpw, X,
                                                                      Y, fz);
}

// The o projection of a fused decode step: x += att W_o^T over rows [0, n)
// of W_o (Q4_0, nb blocks a row), the attention outputs read from the
// exchange xch ([n_heads * hd] tagged words, tag t).
struct OProj {
    const uint8_t* w;
    int n, nb;
    float* x;              // residual stream [n]
    const uint64_t* xch;
    // when set: the residual stream's current values as tagged words (the
    // launch's tag) published by another role of the launch (x is then only
    // written)
    const uint64_t* xin;
};

// One o-projection workgroup of the fused decode launch: rows r0 + wv + 8 r
// (r < RO) of W_o, wave wv.  Its weight blocks do not depend on the
// attention, so all of them are loaded at the start (RO * 2 windows a lane)
// and arrive while the q/k/v workgroups and the attention run.  The
// attention outputs are then polled from the exchange (each wave first
// watches one word with a single lane, then takes its lanes' pieces once
// they all carry tag t), and go through the same records, block order and
// per-row reduction as the o launch of the unfused step (gemv_fused_kernel,
// one row a wave), so both give the same bits.  Bounded: a wait that runs
// out sets *err (never in a correct launch).
template <int RO>
__device__ __forceinline__ void o_proj_body(int j, i32x4* __restrict__ lds4, const OProj& op, int t, int* err) {
    constexpr int NW = 8, CPL = 2, NB = RO * CPL, PI = 1;
    constexpr int WORDS = Geo<(int)WType::Q4_0>::WORDS, BYTES = Geo<(int)WType::Q4_0>::BYTES;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nb = op.nb, n = op.n;
    const int r0 = j * NW * RO;
    const uint32_t row_bytes = (uint32_t)nb * BYTES, wbytes = (uint32_t)n * row_bytes;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(op.w, wbytes);
    uint32_t win[NB][WORDS];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int row = r0 + wv + (b / CPL) * NW, col = lane + 64 * (b % CPL);
        const uint32_t off = (row < n && col < nb) ? (uint32_t)row * row_bytes + (uint32_t)col * BYTES : RSRC_OOB;
        load_window<WORDS, false>(rs, off, wbytes, win[b]);
    }
    float y_old[RO];
    if (op.xin) {
        // every lane polls the wave's RO words (the same addresses)
        uint64_t v[RO];
        for (int spins = 0;; spins++) {
            bool ok = true;
#pragma unroll
            for (int r = 0; r < RO; r++) {
                const int row = min(r0 + wv + r * NW, n - 1);
                v[r] = att::xch_get(op.xin + row);
                ok = ok && att::xch_ok(v[r], t);
            }
            if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
            if (spins > (1 << 16)) {  // only a broken launch gets here
                if (lane == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int r = 0; r < RO; r++) y_old[r] = att::xch_val(v[r]);
    } else {
#pragma unroll
        for (int r = 0; r < RO; r++) {
            const int row = r0 + wv + r * NW;
            y_old[r] = row < n ? op.x[row] : 0.0f;
        }
    }
    // this thread's activation pieces (load_prep_x4's): block c, elements
    // 32 c + 4 k + {0..3} and + 16
    const int p = min((int)threadIdx.x, nb * 4 - 1);
    const int o = (p >> 2) * 32 + (p & 3) * 4;
    const uint64_t* src = op.xch + o;
    const uint64_t* watch = op.xch + min(wv * 512 + 511, nb * 32 - 1);
    for (int spins = 0;; spins++) {
        const bool ready = att::xch_ok(att::xch_get(watch), t);
        if (ready || spins > (1 << 16)) break;
        __builtin_amdgcn_s_sleep(2);
    }
    uint64_t v[8];
    for (int spins = 0;; spins++) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[i] = att::xch_get(src + (i & 3) + (i >> 2) * 16);
            ok = ok && att::xch_ok(v[i], t);
        }
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
        if (spins > (1 << 16)) {  // tens of milliseconds: only a broken launch gets here
            if (lane == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    f32x4 xv[PI][2], av[PI][2];
    xv[0][0] = f32x4{att::xch_val(v[0]), att::xch_val(v[1]), att::xch_val(v[2]), att::xch_val(v[3])};
    xv[0][1] = f32x4{att::xch_val(v[4]), att::xch_val(v[5]), att::xch_val(v[6]), att::xch_val(v[7])};
    prep_float4_lds<NW, PI, PRO_NONE>(xv, av, 0.0f, nb, reinterpret_cast<int*>(lds4));
    __syncthreads();
    RF4 keep[CPL];
#pragma unroll
    for (int i = 0; i < CPL; i++) keep[i] = read_rf4(lds4, nb, min(lane + 64 * i, nb - 1));
#pragma unroll
    for (int r = 0; r < RO; r++) {
        const int row = r0 + wv + r * NW;
        float acc[1] = {0.0f};
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int col = lane + 64 * i;
            if (row < n && col < nb) {
                const bool odd = (col & 1) != 0;
                acc[0] += block_dot_i4<(int)WType::Q4_0>(win[r * CPL + i], odd ? 0x07060504u : 0x05040302u,
                                                         odd ? 16u : 0u, keep[i]);
            }
        }
        const float s = wave_reduce_rows<1>(acc);
        if (lane == 0 && row < n) op.x[row] = s + y_old[r];
    }
}

// Rows of W_o an o-projection workgroup owns (8 waves x O_ROWS_PER_WAVE).
constexpr int O_ROWS_PER_WAVE = 4;

// One decode step's q/k/v projection (RMSNorm prologue, RoPE + KV-cache
// epilogue) with the decode attention fused into the same launch: workgroups
// [0, n_gemv) are the GEMV's, the next n_att attention workgroups (head,
// span) that load their older K/V rows at once, wait for their KV group's
// q/k/v values (tagged exchange) and then read q and the current row; with
// op.w set, the rest are o-projection workgroups (o_proj_body) that wait for
// the attention outputs.  Every wait is on workgroups with smaller ids, and
// the device dispatches a launch's workgroups in id order (workgroup i on
// XCD i % 8, each XCD in id order, measured on MI355X), so the oldest
// unfinished workgroup is always resident and its producers are done: the
// grid may exceed what the CUs hold at once (7B: 352 workgroups, one a CU).
// The waits are bounded besides: one that runs out sets *err.
// The previous layer's down projection (x += h W_down^T, Q4_0) as the first
// role of a fused decode launch (DOWN): its workgroups publish the new x as
// tagged words (Fuse::xout) instead of storing it; the q/k/v workgroups,
// whose weight blocks are all in flight meanwhile, take x from there for
// their RMSNorm, and the o workgroups take it for their residual add.
struct DownPart {
    const uint8_t* w;
    int n, nb, rpw, n_wg;  // rows (dim), blocks a row (ffn / 32), rows a workgroup, workgroups
    const float* h;        // the SwiGLU row (ffn floats)
    float* x;              // residual stream (the old values are read)
    Fuse fz;               // pos, xout
};
constexpr int DOWN_R = 2;  // down rows a wave (16 a workgroup)

template <typename KV, int HD, int R, int CPL, bool DOWN>
__global__ __launch_bounds__(512) void qkv_attention_kernel(const uint8_t* __restrict__ W, int n, int nb, int rpw,
                                                            const float* __restrict__ X, float* __restrict__ Y, Fuse fz,
                                                            AttArgs<KV> aa, int n_gemv, int n_att, OProj op,
                                                            DownPart dp) {
    extern __shared__ i32x4 lds4[];
    int b = (int)blockIdx.x;
    if constexpr (DOWN) {
        if (b < dp.n_wg) {
            gemv_fused_body<(int)WType::Q4_0, false, DOWN_R, 8, true, 8, PRO_NONE, EPI_RESIDUAL, false, XIO_OUT>(
                b, 0, lds4, dp.w, dp.n, dp.nb, dp.rpw, dp.h, dp.x, dp.fz);
            return;
        }
        b -= dp.n_wg;
    }
    if (b < n_gemv) {
        gemv_fused_body<(int)WType::Q4_0, false, R, CPL, true, 8, PRO_RMSNORM, EPI_ROPE_KV, true,
                        DOWN ? XIO_IN : XIO_NONE>(b, 0, lds4, W, n, nb, rpw, X, Y, fz);
    } else if (b < n_gemv + n_att) {
        const int a = b - n_gemv;
        attention_body<KV, HD, true>(a % aa.n_heads, 0, a / aa.n_heads, reinterpret_cast<float*>(lds4), aa);
    } else {
        o_proj_body<O_ROWS_PER_WAVE>(b - n_gemv - n_att, lds4, op, *fz.pos + 1, aa.err);
    }
}

// ---- K-quant decoder fusion -------------------------------------------------------------
// The Q4_K / Q6_K kernels below take the decoder's RMSNorm as a prologue on
// x (PRO_RMSNORM) and one of three epilogues: EPI_STORE, EPI_RESIDUAL
// (y += W x) or EPI_SWIGLU (rows 2j, 2j + 1 are gate j, up j; y_j =
// silu(gate_j) * up_j).
struct KqFuse {
    const float* g;  // RMSNorm weights (PRO_RMSNORM)
    float eps;
    int xstride;     // floats between activation rows
    int ystride;     // floats between output rows
    // EPI_ROPE_KV (rope.rs:134-200, kv_cache.rs:94-106): the launch's rows are
    // heads head0, head0 + 1, ... of [q heads | k heads | v heads]
    const int* pos;  // cache position of activation row 0 is *pos + row0
    int row0;
    const float* cos_t;  // [max_seq][hd / 2]
    const float* sin_t;
    void* kc;            // paged pool [n_pages][n_kv][KV_PAGE][hd], f16 or f32
    void* vc;
    const int* kv_table; // physical page of each logical page
    int n_heads, n_kv, hd, kv_f16, head0;
};

// Matrix row of linear row `lin` under the RoPE pairing: linear rows 2p, 2p + 1
// are the partners (i, i + hd/2) of head p / (hd/2), i = p % (hd/2).
__device__ __forceinline__ int rope_row(int lin, int hd) {
    const int half = hd >> 1, pp = lin >> 1;
    return (pp / half) * hd + pp % half + (lin & 1) * half;
}

// Partners x1 (matrix row r1) and x2 (row r1 + hd/2) of one activation row:
// q heads rotated into y, k heads rotated into the key cache, v heads copied
// into the value cache, at position *pos + row0 + blockIdx.y.
__device__ __forceinline__ void rope_kv_pair(const KqFuse& fz, int r1, float x1, float x2, float* __restrict__ y) {
    const int hd = fz.hd, half = hd >> 1;
    const int head = fz.head0 + r1 / hd, i = r1 % hd;
    const int pos = *fz.pos + fz.row0 + blockIdx.y;
    if (head < fz.n_heads + fz.n_kv) {
        const float c = fz.cos_t[(size_t)pos * half + i], sn = fz.sin_t[(size_t)pos * half + i];
        const float o1 = x1 * c - x2 * sn, o2 = x1 * sn + x2 * c;
        if (head < fz.n_heads) {
            y[r1] = o1;
            y[r1 + half] = o2;
        } else {
            const size_t ko = kv_row(fz.kv_table, fz.n_kv, head - fz.n_heads, pos, hd) + i;
            if (fz.kv_f16) {
                reinterpret_cast<_Float16*>(fz.kc)[ko] = (_Float16)o1;
                reinterpret_cast<_Float16*>(fz.kc)[ko + half] = (_Float16)o2;
            } else {
                reinterpret_cast<float*>(fz.kc)[ko] = o1;
                reinterpret_cast<float*>(fz.kc)[ko + half] = o2;
            }
        }
    } else {
        const size_t vo = kv_row(fz.kv_table, fz.n_kv, head - fz.n_heads - fz.n_kv, pos, hd) + i;
        if (fz.kv_f16) {
            reinterpret_cast<_Float16*>(fz.vc)[vo] = (_Float16)x1;
            reinterpret_cast<_Float16*>(fz.vc)[vo + half] = (_Float16)x2;
        } else {
            reinterpret_cast<float*>(fz.vc)[vo] = x1;
            reinterpret_cast<float*>(fz.vc)[vo + half] = x2;
        }
    }
}

// x pieces as load_prep_x, then (PRO_RMSNORM) the matching pieces of g: both
// ahead of the weight stream, both covered by wait_prep_x.
template <int NW, int PI, int PRO>
__device__ __forceinline__ void load_prep_xg(const float* __restrict__ x, const float* __restrict__ g, int nb,
                                             f32x4 (&xv)[PI], f32x4 (&gv)[PI]) {
    load_prep_x<NW, PI>(x, nb, xv);
    if constexpr (PRO == PRO_RMSNORM) load_prep_x<NW, PI>(g, nb, gv);
}

// x_j <- (x_j * (1 / sqrt(sum(x^2) / K + eps))) * g_j (ops.rs:688-751) on the
// pieces of load_prep_x, the sum formed by the workgroup in a fixed order.
// `red` holds NW floats of LDS that nothing else uses until the next barrier.
template <int NW, int PI>
__device__ void rmsnorm_pieces(f32x4 (&xv)[PI], const f32x4 (&gv)[PI], float eps, int nb, float* red) {
    constexpr int NT = NW * 64;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < PI; j++) {
        if ((int)threadIdx.x + j * NT < nb * 8) {  // clamped duplicates past the row count once
            const f32x4 a = xv[j];
            ss += (a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w);
        }
    }
    ss = sum8_f32(ss);
    ss += dpp_f32<DPP_ROW_MIRROR>(ss);
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) tot += red[w];
    const float inv = 1.0f / sqrtf(tot / (float)(nb * 32) + eps);
#pragma unroll
    for (int j = 0; j < PI; j++) {
        xv[j].x = (xv[j].x * inv) * gv[j].x;
        xv[j].y = (xv[j].y * inv) * gv[j].y;
        xv[j].z = (xv[j].z * inv) * gv[j].z;
        xv[j].w = (xv[j].w * inv) * gv[j].w;
    }
}

// silu(gate) * up as the fused Q4_0 epilogue forms it (feed_forward.rs:138-150)
__device__ __forceinline__ float swiglu1(float gate, float up) {
    return (gate * (1.0f / (1.0f + expf(-gate)))) * up;
}

// Final store of the split-K kernels: rb[k * RPW + i] holds slice k's sum of
// local row i of the rows from r0.
// Linear rows are matrix rows except under EPI_ROPE_KV (rope_row).
template <int KS, int RPW, int NW, int EPI>
__device__ __forceinline__ void store_slices(const float* rb, int r0, int n, float* __restrict__ y,
                                             const KqFuse& fz) {
    if constexpr (EPI == EPI_SWIGLU || EPI == EPI_ROPE_KV) {
        for (int i = threadIdx.x; i < RPW / 2; i += NW * 64) {
            float t0 = rb[2 * i], t1 = rb[2 * i + 1];
#pragma unroll
            for (int k = 1; k < KS; k++) {
                t0 += rb[k * RPW + 2 * i];
                t1 += rb[k * RPW + 2 * i + 1];
            }
            if (r0 + 2 * i + 1 < n) {
                if constexpr (EPI == EPI_SWIGLU) y[(r0 >> 1) + i] = swiglu1(t0, t1);
                else rope_kv_pair(fz, rope_row(r0 + 2 * i, fz.hd), t0, t1, y);
            }
        }
    } else {
        for (int i = threadIdx.x; i < RPW; i += NW * 64) {
            float t = rb[i];
#pragma unroll
            for (int k = 1; k < KS; k++) t += rb[k * RPW + i];
            if (r0 + i < n) {
                if constexpr (EPI == EPI_RESIDUAL) y[r0 + i] = t + y[r0 + i];
                else y[r0 + i] = t;
            }
        }
    }
}

// ---- Q4_K (float mode) ------------------------------------------------------------------
// A unit is one 32-byte chunk of a super-block's nibbles: sub-block 2c (lo
// nibbles) and 2c+1 (hi nibbles) of super-block sb (parser.rs:574-589).
// The same four 6-bit values packed as bytes {sc1, sc2, mn1, mn2}, for a lane
// whose chunk c is fixed: Q4kSel holds its byte selectors, so a row costs two
// byte permutes and a few packed-byte operations (both forms, then a select).
struct Q4kSel {
    uint32_t p, w;  // v_perm selectors: {s[b], s[b+1], s[b+4], s[b+5]}, {s[b+8], s[b+9]} twice
    uint32_t hi;    // all ones when c >= 2: the split form (parser.rs:567-568)
};
__device__ __forceinline__ Q4kSel q4k_sel(int c) {
    const uint32_t b = 2 * (c & 1);
    return Q4kSel{b | (b + 1) << 8 | (b + 4) << 16 | (b + 5) << 24, b | (b + 1) << 8 | b << 16 | (b + 1) << 24,
                  c >= 2 ? ~0u : 0u};
}
__device__ __forceinline__ uint32_t q4k_scales4(const u32x4& h, const Q4kSel& q) {
    const uint32_t p = perm(h.z, h.y, q.p);  // s[b], s[b+1] (scales), s[b+4], s[b+5] (mins)
    const uint32_t w = perm(h.w, h.w, q.w);  // s[b+8], s[b+9], s[b+8], s[b+9]
    // j < 4: the low 6 bits                                           (parser.rs:565-566)
    const uint32_t lo = p & 0x3F3F3F3Fu;
    // j >= 4: the top 2 bits of s[i] / s[i+4] and a nibble of s[i+8]  (parser.rs:567-568)
    const uint32_t top = (p >> 6) & 0x03030303u;
    const uint32_t nib = (w & 0x00000F0Fu) | ((w >> 4) & 0x0F0F0000u);
    return ((top | (nib << 2)) & q.hi) | (lo & ~q.hi);  // a bit select, no branch
}

// Loads of Q4_K rows in flight ahead of the arithmetic (both Q4_K kernels).
constexpr int Q4K_AHEAD = 2;
// gemv_q4k_splitk_kernel: rows issued before the activation prep, rows in
// flight after it (4096 x 14336 on MI355X, us a launch: 2 / 2 9.80, 2 / 4
// 9.72, 2 / 3 9.81, 1 / 2 10.30, 1 / 3 9.95, 1 / 4 9.87; 3 / 3 10.9 and 4 / 4
// 12.6: weight loads ahead of the prep delay every CU's activation; with the
// leaner dot and prep code since: 1 / 4 9.04, 2 / 4 8.88-8.91, 3 / 4 10.1)
constexpr int Q4K_SPLIT_PRE = 2, Q4K_SPLIT_AHEAD = 4;

// Q4_K rows of at most 64 units (K <= 4096): lane u takes unit u of R rows
// per wave (rows r0 + wv + r * NW; EPI_SWIGLU: row pairs 2j, 2j + 1 in one
// wave, pair j = wv + (r / 2) * NW of the workgroup's); each activation record
// is read from LDS once for the R rows.
template <int R, int NW, int PRO = PRO_NONE, int EPI = EPI_STORE>
__global__ __launch_bounds__(NW * 64) void gemv_q4k_fused_kernel(const uint8_t* __restrict__ W, int n,
                                                            int nsb, int rpw,
                                                            const float* __restrict__ X,
                                                            float* __restrict__ Y, KqFuse fz) {
    extern __shared__ i32x4 lds4[];
    constexpr bool PAIRS = (EPI == EPI_SWIGLU || EPI == EPI_ROPE_KV);
    static_assert(!PAIRS || R % 2 == 0, "row pairs need an even row count per wave");
    static_assert(R >= 1 && R <= 8, "rows per wave");
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int r0 = blockIdx.x * rpw;
    const int rend = min(n, r0 + rpw);
    const int nb = nsb * 8, nunits = nsb * 4;
    const float* x = X + (size_t)blockIdx.y * fz.xstride;
    float* y = Y + (size_t)blockIdx.y * fz.ystride;
    const uint32_t row_bytes = (uint32_t)nsb * Q4_K_BYTES;
    constexpr int PI = (16 + NW - 1) / NW;  // nb * 8 = 16 * units <= 1024 float4 pieces
    f32x4 xv[PI], gv[PI];
    __builtin_amdgcn_s_setprio(2);  // the prep ahead of other workgroups' streams
    load_prep_xg<NW, PI, PRO>(x, fz.g, nb, xv, gv);
    auto row_of = [&](int r) {
        if constexpr (PAIRS) return r0 + 2 * (wv + (r >> 1) * NW) + (r & 1);
        return r0 + wv + r * NW;
    };

    // rows issued Q4K_AHEAD at a time, as in gemv_q4k_splitk_kernel, into a
    // ring of NS load slots (row r in slot r % NS: the slot of row r + P0 is
    // that of row r - 1, consumed before it is issued).  With more than four
    // rows the later rows' offsets and each row's finished sum pass through
    // empty volatile asm statements, which keep their order: row r + P0 is
    // issued after row r - 1's arithmetic, so that the loads are not all
    // hoisted to the top (registers).
    const int u = lane;
    const bool uok = u < nunits;
    constexpr int P0 = R < Q4K_AHEAD ? R : Q4K_AHEAD;
    constexpr int NS = R < P0 + 1 ? R : P0 + 1;
    u32x4 hdr[NS], qa[NS], qb[NS];
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(W, (uint32_t)n * row_bytes);
    auto mat_row = [&](int lin) {
        if constexpr (EPI == EPI_ROPE_KV) return rope_row(lin, fz.hd);
        return lin;
    };
    auto issue = [&](int r) {
        const int row = row_of(r);
        uint32_t off = (row < rend && uok)
                           ? (uint32_t)mat_row(row) * row_bytes + (uint32_t)(u >> 2) * Q4_K_BYTES
                           : RSRC_OOB;
        if (R > 4 && r >= P0) asm volatile("" : "+v"(off));
        const uint32_t q = off + 16 + 32 * (u & 3);
        hdr[r % NS] = buf_load_b128(rs, off);
        qa[r % NS] = buf_load_b128(rs, q);
        qb[r % NS] = buf_load_b128(rs, q + 16);
    };
#pragma unroll
    for (int r = 0; r < P0; r++) issue(r);
    wait_prep_x<P0 * 3>();  // header + two 16-byte nibble loads per row
    after_wait<PI>(xv);
    if constexpr (PRO == PRO_RMSNORM) {
        after_wait<PI>(gv);
        rmsnorm_pieces<NW, PI>(xv, gv, fz.eps, nb, reinterpret_cast<float*>(lds4) + nb * 32);
    }
    prep_float_lds<NW, PI, false>(xv, nb, reinterpret_cast<int*>(lds4));
    __syncthreads();
    __builtin_amdgcn_s_setprio(0);
    if (row_of(0) >= rend) return;  // wave-uniform; the wave has no rows

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    if (uok) {
        const int sb = u >> 2, c = u & 3;
        const RF x1 = read_rf(lds4, nb, sb * 8 + 2 * c);
        const RF x2 = read_rf(lds4, nb, sb * 8 + 2 * c + 1);
        const Q4kSel qs = q4k_sel(c);
        const float s2h = x2.S * 0.0625f;  // the high nibbles enter as 16 (h - 8)
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (r + P0 < R) issue(r + P0);
            __builtin_amdgcn_sched_barrier(0);
            // row r's data enter the arithmetic here and not earlier (keeps the
            // compiler from hoisting every row's scale work above the first dot)
            const int sl = r % NS;
            asm volatile("" : "+v"(hdr[sl]), "+v"(qa[sl]), "+v"(qb[sl]));
            const uint32_t raw[8] = {qa[sl].x, qa[sl].y, qa[sl].z, qa[sl].w, qb[sl].x, qb[sl].y, qb[sl].z, qb[sl].w};
            // low nibbles as bytes 0..15; high nibbles h in place as the signed
            // bytes 16 (h - 8) (one bitop3 a word), with sum h x = sum 16 (h - 8)
            // x / 16 + 8 sum x
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                lo[k] = raw[k] & NIB;
                hi[k] = (raw[k] & ~NIB) ^ 0x80808080u;
            }
            const float d = h2f(hdr[sl].x & 0xFFFFu);
            const float dmin = h2f(hdr[sl].x >> 16);
            const uint32_t sm = q4k_scales4(hdr[sl], qs);
            // element value (d*sc)*q - (dmin*mn)   (parser.rs:577-587)
            const float d1 = d * (float)(sm & 0xFFu), m1 = dmin * (float)((sm >> 16) & 0xFFu);
            const float d2 = d * (float)((sm >> 8) & 0xFFu), m2 = dmin * (float)(sm >> 24);
            float a = acc[r];
            a = fmaf(d1 * x1.S, dot3z(lo, x1), a);
            a = fmaf(-m1, x1.xsum, a);
            a = fmaf(d2 * s2h, dot3z(hi, x2), a);
            a = fmaf(fmaf(8.0f, d2, -m2), x2.xsum, a);
            acc[r] = a;
            if constexpr (R > 4) asm volatile("" : "+v"(acc[r]));  // row r done before row r + P0 + 1 issues
            __builtin_amdgcn_sched_barrier(0);  // one row at a time, in load order
        }
    }
    // rows past rend hold 0 (their loads read zeros); they are not stored.
    // Rows 0-3 and 4-7 are reduced as two sets (pairs never straddle them).
    auto store = [&](float s, int sh, int rbase) {
        if constexpr (PAIRS) {
            // rows r (even) and r + 1 (gate and up; RoPE partners) sit in
            // adjacent lane groups
            const float s2 = __shfl_down(s, 1 << sh);
            if ((lane & ((2 << sh) - 1)) == 0) {
                const int g = row_of(rbase + (lane >> sh));
                if (g + 1 < rend) {
                    if constexpr (EPI == EPI_SWIGLU) y[g >> 1] = swiglu1(s, s2);
                    else rope_kv_pair(fz, mat_row(g), s, s2, y);
                }
            }
        } else if ((lane & ((1 << sh) - 1)) == 0) {
            const int row = row_of(rbase + (lane >> sh));
            if (row < rend) {
                if constexpr (EPI == EPI_RESIDUAL) y[row] = s + y[row];
                else y[row] = s;
            }
        }
    };
    constexpr int R0 = R < 4 ? R : 4;
    float a0[R0];
#pragma unroll
    for (int r = 0; r < R0; r++) a0[r] = acc[r];
    store(wave_reduce_rows<R0>(a0), reduce_span_log2<R0>(), 0);
    if constexpr (R > 4) {
        float a1[R - 4];
#pragma unroll
        for (int r = 0; r < R - 4; r++) a1[r] = acc[4 + r];
        store(wave_reduce_rows<R - 4>(a1), reduce_span_log2<R - 4>(), 4);
    }
}

// Q4_K rows longer than 64 units: K is split over the waves of a workgroup so
// that every wave can keep R rows in registers and read each activation
// record from LDS once for all of them.  Wave w takes K slice ks = w % KS
// (units ks * ups .. + ups - 1, one per lane, ups <= 64) of rows
// r0 + rg + r * RG, rg = w / KS, r < R; the KS slice sums of a row are added
// in a fixed order at the end, through LDS.
template <int R, int KS, int NW, int PRO = PRO_NONE, int EPI = EPI_STORE>
__global__ __launch_bounds__(NW * 64) void gemv_q4k_splitk_kernel(const uint8_t* __restrict__ W, int n, int nsb,
                                                                  int ups, const float* __restrict__ X,
                                                                  float* __restrict__ Y, KqFuse fz) {
    static_assert(NW % KS == 0, "slices per workgroup");
    constexpr int RG = NW / KS;  // row groups
    constexpr int RPW = RG * R;  // rows per workgroup
    extern __shared__ i32x4 lds4[];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int ks = wv % KS, rg = wv / KS;
    const int r0 = blockIdx.x * RPW;
    const int rend = min(n, r0 + RPW);
    const int nb = nsb * 8, nunits = nsb * 4;
    const float* x = X + (size_t)blockIdx.y * fz.xstride;
    float* y = Y + (size_t)blockIdx.y * fz.ystride;
    const uint32_t row_bytes = (uint32_t)nsb * Q4_K_BYTES;
    constexpr int PI = (KS * 16 + NW - 1) / NW;  // nb * 8 = 16 * units <= 1024 * KS float4 pieces
    f32x4 xv[PI], gv[PI];
    __builtin_amdgcn_s_setprio(2);  // the prep ahead of other workgroups' streams
    load_prep_xg<NW, PI, PRO>(x, fz.g, nb, xv, gv);
    // every wave's x loads enter the CU's memory pipeline ahead of any
    // wave's weight loads (an execution barrier only: no wait for the
    // loads); 4096 x 14336: 10.6 -> 9.9 us a launch (the 4096-column and
    // Q6_K kernels: no gain)
    __builtin_amdgcn_s_barrier();

    const int u = ks * ups + lane;
    const bool uok = lane < ups && u < nunits;
    // Rows are loaded Q4K_AHEAD at a time: row r + Q4K_AHEAD is issued when
    // row r's arithmetic starts, so each wave's loads arrive in the order they
    // are used and the arithmetic overlaps the stream.  No control flow around
    // the loads (empty slots load nothing through an out-of-range offset).
    u32x4 hdr[R], qa[R], qb[R];
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(W, (uint32_t)n * row_bytes);
    auto issue = [&](int r) {
        const int row = r0 + rg + r * RG;
        const int mrow = (EPI == EPI_ROPE_KV) ? rope_row(row, fz.hd) : row;
        const uint32_t off =
            (row < rend && uok) ? (uint32_t)mrow * row_bytes + (uint32_t)(u >> 2) * Q4_K_BYTES : RSRC_OOB;
        const uint32_t q = off + 16 + 32 * (u & 3);
        hdr[r] = buf_load_b128(rs, off);
        qa[r] = buf_load_b128(rs, q);
        qb[r] = buf_load_b128(rs, q + 16);
    };
    // P0 rows issued before the prep, AH rows in flight after it
    constexpr int P0 = R < Q4K_SPLIT_PRE ? R : Q4K_SPLIT_PRE;
    constexpr int AH = R < Q4K_SPLIT_AHEAD ? R : Q4K_SPLIT_AHEAD;
    static_assert(P0 <= AH, "rows before the prep");
#pragma unroll
    for (int r = 0; r < P0; r++) issue(r);
    wait_prep_x<P0 * 3>();  // header + two 16-byte nibble loads per row
    after_wait<PI>(xv);
    if constexpr (PRO == PRO_RMSNORM) {
        after_wait<PI>(gv);
        rmsnorm_pieces<NW, PI>(xv, gv, fz.eps, nb, reinterpret_cast<float*>(lds4) + nb * 32);
    }
    prep_float_lds<NW, PI, false>(xv, nb, reinterpret_cast<int*>(lds4));
    __syncthreads();
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int r = P0; r < AH; r++) issue(r);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    if (uok) {
        const int sb = u >> 2, c = u & 3;
        const RF x1 = read_rf(lds4, nb, sb * 8 + 2 * c);
        const RF x2 = read_rf(lds4, nb, sb * 8 + 2 * c + 1);
        const Q4kSel qs = q4k_sel(c);
        const float s2h = x2.S * 0.0625f;  // the high nibbles enter as 16 (h - 8)
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (r + AH < R) issue(r + AH);
            __builtin_amdgcn_sched_barrier(0);
            // row r's data enter the arithmetic here and not earlier (keeps the
            // compiler from hoisting every row's scale work above the first dot)
            asm volatile("" : "+v"(hdr[r]), "+v"(qa[r]), "+v"(qb[r]));
            const uint32_t raw[8] = {qa[r].x, qa[r].y, qa[r].z, qa[r].w, qb[r].x, qb[r].y, qb[r].z, qb[r].w};
            // low nibbles as bytes 0..15; high nibbles h in place as the signed
            // bytes 16 (h - 8) (one bitop3 a word), with sum h x = sum 16 (h - 8)
            // x / 16 + 8 sum x
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                lo[k] = raw[k] & NIB;
                hi[k] = (raw[k] & ~NIB) ^ 0x80808080u;
            }
            const float d = h2f(hdr[r].x & 0xFFFFu);
            const float dmin = h2f(hdr[r].x >> 16);
            const uint32_t sm = q4k_scales4(hdr[r], qs);
            // element value (d*sc)*q - (dmin*mn)   (parser.rs:577-587)
            const float d1 = d * (float)(sm & 0xFFu), m1 = dmin * (float)((sm >> 16) & 0xFFu);
            const float d2 = d * (float)((sm >> 8) & 0xFFu), m2 = dmin * (float)(sm >> 24);
            float a = acc[r];
            a = fmaf(d1 * x1.S, dot3z(lo, x1), a);
            a = fmaf(-m1, x1.xsum, a);
            a = fmaf(d2 * s2h, dot3z(hi, x2), a);
            a = fmaf(fmaf(8.0f, d2, -m2), x2.xsum, a);
            acc[r] = a;
            // one row at a time, in load order: row r's arithmetic runs while
            // the loads of rows r + 1 .. are still arriving
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // rows of empty slots hold 0 (their loads read zeros): no masking needed
    const float s = wave_reduce_rows<R>(acc);
    constexpr int SH = reduce_span_log2<R>();
    // [KS][RPW] slice sums over the start of the records, once every wave has read them
    float* red = reinterpret_cast<float*>(lds4);
    __syncthreads();
    if ((lane & ((1 << SH) - 1)) == 0) red[ks * RPW + rg + (lane >> SH) * RG] = s;
    __syncthreads();
    store_slices<KS, RPW, NW, EPI>(red, r0, n, y, fz);
}

// ---- Q6_K (float mode) ------------------------------------------------------------------
// A unit is one 32-element column of a super-block (Q6KUnit): K / 32 units a
// row.  K is split over KS waves of the workgroup as in gemv_q4k_splitk_kernel:
// wave w takes units ks * ups .. + ups - 1 (one per lane, ups <= 64) of R rows
// of each row group (RG = NW / KS waves share a slice; a group is RG * R rows).
// A workgroup converts x once and then walks the row groups blockIdx.x,
// blockIdx.x + gridDim.x, ...: the loads of the next group's first rows are
// issued while the current group's last rows are computed.  The KS slice sums
// of a row are added in a fixed order through LDS (two buffers, one barrier a
// group).
constexpr int Q6K_AHEAD = 2;  // rows whose loads are in flight ahead of the arithmetic

template <int R, int KS, int NW, int PRO = PRO_NONE, int EPI = EPI_STORE>
__global__ __launch_bounds__(NW * 64) void gemv_q6k_splitk_kernel(const uint8_t* __restrict__ W, int n, int nsb,
                                                                  int ups, const float* __restrict__ X,
                                                                  float* __restrict__ Y, KqFuse fz) {
    static_assert(NW % KS == 0, "slices per workgroup");
    constexpr int RG = NW / KS;  // waves per slice
    constexpr int RPW = RG * R;  // rows per group
    extern __shared__ i32x4 lds4[];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int ks = wv % KS, rg = wv / KS;
    const int ngroups = (n + RPW - 1) / RPW;
    const int nb = nsb * 8;  // units = 32-element columns
    const float* x = X + (size_t)blockIdx.y * fz.xstride;
    float* y = Y + (size_t)blockIdx.y * fz.ystride;
    const uint32_t row_bytes = (uint32_t)nsb * Q6_K_BYTES;
    constexpr int PI = (KS * 8 + NW - 1) / NW;  // nb * 8 <= 512 * KS float4 pieces
    f32x4 xv[PI], gv[PI];
    __builtin_amdgcn_s_setprio(2);  // the prep ahead of other workgroups' streams
    load_prep_xg<NW, PI, PRO>(x, fz.g, nb, xv, gv);

    const int u = ks * ups + lane;
    const bool uok = lane < ups && u < nb;
    // eight loads a row: two nine-dword windows (ql, qh), the scale pair, d;
    // empty slots read zeros through out-of-range offsets
    u32x4 l0[R], l1[R], h0[R], h1[R];
    uint32_t l2[R], h2[R], scw[R], dw[R];
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(W, (uint32_t)n * row_bytes);
    auto block_of = [&](int grp, int r) {  // byte offset of the unit's super-block in row r of group grp
        const int row = grp * RPW + rg + r * RG;
        const int mrow = (EPI == EPI_ROPE_KV) ? rope_row(row, fz.hd) : row;
        return (uint32_t)mrow * row_bytes + (uint32_t)(u >> 3) * Q6_K_BYTES;
    };
    // slot r <- row r of group grp
    auto issue = [&](int grp, int r) {
        const int row = grp * RPW + rg + r * RG;
        const bool live = row < n && grp < ngroups && uok;
        const Q6KUnit g = q6k_unit(block_of(grp, r), u & 7);
        const uint32_t bl = live ? (g.ql & ~3u) : RSRC_OOB, bh = live ? (g.qh & ~3u) : RSRC_OOB;
        l0[r] = buf_load_b128(rs, bl);
        l1[r] = buf_load_b128(rs, bl + 16);
        l2[r] = buf_load_b32(rs, bl + 32);
        h0[r] = buf_load_b128(rs, bh);
        h1[r] = buf_load_b128(rs, bh + 16);
        h2[r] = buf_load_b32(rs, bh + 32);
        scw[r] = buf_load_b16(rs, live ? g.sc : RSRC_OOB);
        dw[r] = buf_load_b16(rs, live ? g.d : RSRC_OOB);
    };
    constexpr int P0 = R < Q6K_AHEAD ? R : Q6K_AHEAD;
    const int tcol = u & 3;  // column within the half
    int grp = blockIdx.x;
#pragma unroll
    for (int r = 0; r < P0; r++) issue(grp, r);
    wait_prep_x<P0 * 8>();  // eight weight loads per row
    after_wait<PI>(xv);
    if constexpr (PRO == PRO_RMSNORM) {
        after_wait<PI>(gv);
        rmsnorm_pieces<NW, PI>(xv, gv, fz.eps, nb, reinterpret_cast<float*>(lds4) + nb * 32);
    }
    prep_float_lds<NW, PI, true>(xv, nb, reinterpret_cast<int*>(lds4));  // q6k_offsets reads the digit sums
    __syncthreads();
    __builtin_amdgcn_s_setprio(0);

    // the records are read once; the slice sums then go to LDS past them
    RF xr{};
    int off[6] = {0, 0, 0, 0, 0, 0};
    if (uok) {
        xr = read_rf(lds4, nb, u);
        q6k_offsets(xr, off);
    }
    float* red = reinterpret_cast<float*>(lds4) + (size_t)nb * 32;  // [2][KS][RPW]
    constexpr int SH = reduce_span_log2<R>();
    for (int it = 0; grp < ngroups; grp += gridDim.x, it ^= 1) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
        for (int r = 0; r < R; r++) {
            // keep P0 rows in flight, running into the next group (into slots
            // already consumed: the next group's rows are issued after row r's
            // arithmetic, since with P0 == R the slot is r's own)
            if (r + P0 < R) issue(grp, r + P0);
            __builtin_amdgcn_sched_barrier(0);
            // row r's data enter the arithmetic here and not earlier
            asm volatile("" : "+v"(l0[r]), "+v"(l1[r]), "+v"(l2[r]), "+v"(h0[r]), "+v"(h1[r]), "+v"(h2[r]),
                         "+v"(scw[r]), "+v"(dw[r]));
            if (uok) {
                const uint32_t wl[9] = {l0[r].x, l0[r].y, l0[r].z, l0[r].w, l1[r].x, l1[r].y, l1[r].z, l1[r].w, l2[r]};
                const uint32_t wh[9] = {h0[r].x, h0[r].y, h0[r].z, h0[r].w, h1[r].x, h1[r].y, h1[r].z, h1[r].w, h2[r]};
                uint32_t q[8];
                // the ql / qh runs share the block's dword alignment
                q6k_codes(wl, wh, q6k_sel(block_of(grp, r)), tcol, q);
                const int sc0 = (int)(int8_t)(scw[r] & 0xFFu), sc1 = (int)(int8_t)((scw[r] >> 8) & 0xFFu);
                const float f = q6k_dot(q, xr, off, sc0, sc1);
                acc[r] = fmaf(h2f(dw[r]) * xr.S, f, acc[r]);
            }
            if (r + P0 >= R) issue(grp + gridDim.x, r + P0 - R);
            __builtin_amdgcn_sched_barrier(0);  // one row at a time, in load order
        }
        // rows of empty slots hold 0 (d reads as zero): no masking needed
        const float sum = wave_reduce_rows<R>(acc);
        float* rb = red + it * (KS * RPW);
        if ((lane & ((1 << SH) - 1)) == 0) rb[ks * RPW + rg + (lane >> SH) * RG] = sum;
        __syncthreads();  // (the other buffer was last read before this barrier)
        store_slices<KS, RPW, NW, EPI>(rb, grp * RPW, n, y, fz);
    }
}

int g_num_cus = 0;

}  // namespace

int device_cu_count() {
    if (g_num_cus == 0) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            cus > 0)
            g_num_cus = cus;
        else
            g_num_cus = 256;
    }
    return g_num_cus;
}

namespace {

int num_cus() { return device_cu_count(); }

// Columns per lane (CPL) x rows per wave (R) <= 8 keeps the block windows
// within the VGPR budget.
int cpl_for(int nb) { return nb <= 128 ? 2 : nb <= 256 ? 4 : 8; }

struct Cfg {
    int nw;   // waves per workgroup
    int rpw;  // rows per workgroup
    int r;    // rows per wave (template R)
};

// Spread the rows over about `wg_per_cu` workgroups per CU with at most rmax
// rows per wave.
Cfg pick_cfg(int n, int nw, int rmax, int wg_per_cu) {
    const int target = num_cus() * wg_per_cu;
    int rpw = (n + target - 1) / target;
    if (rpw > rmax * nw) rpw = rmax * nw;
    if (rpw < 1) rpw = 1;
    int r = (rpw + nw - 1) / nw;
    r = r <= 1 ? 1 : r <= 2 ? 2 : r <= 3 ? 3 : 4;
    return Cfg{nw, rpw, r};
}

template <int WT, bool NATIVE, int CPL, bool EVEN, int NW, int PRO = PRO_NONE, int RES = EPI_STORE>
void launch_nw(const uint8_t* w, int n, int nb, const float* x, size_t m, float* y, hipStream_t s,
               const Cfg& c, size_t lds, const Fuse& fz) {
    const dim3 grid((unsigned)((n + c.rpw - 1) / c.rpw), (unsigned)m), block(NW * 64);
    constexpr int RMAX = 8 / CPL;
    const int rpw = c.rpw;
    if constexpr (RES == EPI_SWIGLU || RES == EPI_ROPE_KV) {
        // even row counts only (row pairs); RMAX 1 is rejected by the caller
        if constexpr (RMAX >= 4) {
            if constexpr (RES == EPI_SWIGLU) {
                if (c.r >= 8) {
                    launch_kernel((gemv_fused_kernel<WT, NATIVE, 8, CPL, EVEN, NW, PRO, RES>), grid, block, lds, s, w, n, nb, rpw, x, y, fz);
                    return;
                }
            }
            if (c.r >= 4)
                launch_kernel((gemv_fused_kernel<WT, NATIVE, 4, CPL, EVEN, NW, PRO, RES>), grid, block, lds, s, w, n, nb, rpw, x, y, fz);
            else
                launch_kernel((gemv_fused_kernel<WT, NATIVE, 2, CPL, EVEN, NW, PRO, RES>), grid, block, lds, s, w, n, nb, rpw, x, y, fz);
        } else if constexpr (RMAX >= 2) {
            launch_kernel((gemv_fused_kernel<WT, NATIVE, 2, CPL, EVEN, NW, PRO, RES>), grid, block, lds, s, w, n, nb, rpw, x, y, fz);
        }
        return;
    } else if (c.r >= 8 && RMAX >= 4 && RES == EPI_STORE)
        launch_kernel((gemv_fused_kernel<WT, NATIVE, (RES == EPI_STORE && RMAX >= 4 ? 8 : 1), CPL, EVEN, NW, PRO, RES>), grid, block, lds, s, w, n, nb, rpw, x, y, fz);
    else if (c.r <= 1 || RMAX == 1)
        launch_kernel((gemv_fused_kernel<WT, NATIVE, 1, CPL, EVEN, NW, PRO, RES>), grid, block, lds, s, w, n, nb, rpw, x, y, fz);
    else if (c.r <= 2 || RMAX == 2)
        launch_kernel((gemv_fused_kernel<WT, NATIVE, (RMAX >= 2 ? 2 : 1), CPL, EVEN, NW, PRO, RES>), grid, block, lds, s, w, n, nb, rpw, x, y, fz);
    else if (c.r <= 3)
        launch_kernel((gemv_fused_kernel<WT, NATIVE, (RMAX >= 4 ? 3 : 1), CPL, EVEN, NW, PRO, RES>), grid, block, lds, s, w, n, nb, rpw, x, y, fz);
    else
        launch_kernel((gemv_fused_kernel<WT, NATIVE, (RMAX >= 4 ? 4 : 1), CPL, EVEN, NW, PRO, RES>), grid, block, lds, s, w, n, nb, rpw, x, y, fz);
}

template <int WT, bool NATIVE, int CPL, bool EVEN>
void launch_even(const uint8_t* w, int n, int nb, const float* x, size_t m, float* y,
                 hipStream_t s, const Cfg& c, size_t lds) {
    Fuse fz{};
    fz.xstride = nb * 32;
    if (c.nw == 4) launch_nw<WT, NATIVE, CPL, EVEN, 4>(w, n, nb, x, m, y, s, c, lds, fz);
    else if (c.nw == 8) launch_nw<WT, NATIVE, CPL, EVEN, 8>(w, n, nb, x, m, y, s, c, lds, fz);
    else launch_nw<WT, NATIVE, CPL, EVEN, 16>(w, n, nb, x, m, y, s, c, lds, fz);
}

template <int WT, bool NATIVE, int CPL>
void launch_wt(const uint8_t* w, int n, int nb, const float* x, size_t m, float* y,
               hipStream_t s, const Cfg& c, size_t lds) {
    if ((nb & 1) == 0 || WT == (int)WType::Q4_1)
        launch_even<WT, NATIVE, CPL, true>(w, n, nb, x, m, y, s, c, lds);
    else
        launch_even<WT, NATIVE, CPL, false>(w, n, nb, x, m, y, s, c, lds);
}

template <int WT, bool NATIVE>
void launch_cpl(const uint8_t* w, int n, int nb, const float* x, size_t m, float* y,
                hipStream_t s, size_t lds, int nw, int wg_per_cu) {
    const int cpl = cpl_for(nb);
    const Cfg c = pick_cfg(n, nw, 8 / cpl, wg_per_cu);
    switch (cpl) {
        case 2: launch_wt<WT, NATIVE, 2>(w, n, nb, x, m, y, s, c, lds); break;
        case 4: launch_wt<WT, NATIVE, 4>(w, n, nb, x, m, y, s, c, lds); break;
        default: launch_wt<WT, NATIVE, 8>(w, n, nb, x, m, y, s, c, lds); break;
    }
}

// Rows of more than 64 units (K > 4096): K split over 2 or 4 waves of a
// 16-wave workgroup, 4 rows per wave (gemv_q4k_splitk_kernel).
template <int KS, int PRO, int EPI>
void launch_q4k_splitk(const uint8_t* w, int n, int nsb, const float* x, size_t m, float* y, hipStream_t s,
                       size_t lds, const KqFuse& fz) {
    constexpr int NW = 16, R = 4, RPW = NW / KS * R;
    const int units = nsb * 4, ups = (units + KS - 1) / KS;
    const dim3 grid((unsigned)((n + RPW - 1) / RPW), (unsigned)m), block(NW * 64);
    launch_kernel((gemv_q4k_splitk_kernel<R, KS, NW, PRO, EPI>), grid, block, lds, s, w, n, nsb, ups, x, y, fz);
}

template <int R, int PRO, int EPI>
void launch_q4k_r(const uint8_t* w, int n, int nsb, const float* x, size_t m, float* y, hipStream_t s,
                  size_t lds, int rpw, const KqFuse& fz) {
    constexpr int NW = 8;
    const dim3 grid((unsigned)((n + rpw - 1) / rpw), (unsigned)m), block(NW * 64);
    launch_kernel((gemv_q4k_fused_kernel<R, NW, PRO, EPI>), grid, block, lds, s, w, n, nsb, rpw, x, y, fz);
}

// Rows of at most 64 units (K <= 4096): 8-wave workgroups, two per CU, all
// of them in one round: rows spread evenly, up to 8 a wave (whole row pairs
// for EPI_SWIGLU).
template <int PRO, int EPI>
void launch_q4k_small(const uint8_t* w, int n, int nsb, const float* x, size_t m, float* y, hipStream_t s,
                      size_t lds, const KqFuse& fz) {
    constexpr int NW = 8;
    const int slots = 2 * num_cus();
    int rpw = (n + slots - 1) / slots;
    if (EPI == EPI_SWIGLU || EPI == EPI_ROPE_KV) rpw += rpw & 1;
    if (rpw > 8 * NW) rpw = 8 * NW;
    const int r = (rpw + NW - 1) / NW;
    if constexpr (EPI == EPI_SWIGLU || EPI == EPI_ROPE_KV) {
        if (r <= 2) launch_q4k_r<2, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz);
        else if (r <= 4) launch_q4k_r<4, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz);
        else if (r <= 6) launch_q4k_r<6, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz);
        else launch_q4k_r<8, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz);
    } else {
        switch (r) {
            case 1: launch_q4k_r<1, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz); break;
            case 2: launch_q4k_r<2, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz); break;
            case 3: launch_q4k_r<3, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz); break;
            case 4: launch_q4k_r<4, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz); break;
            case 5: launch_q4k_r<5, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz); break;
            case 6: launch_q4k_r<6, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz); break;
            case 7: launch_q4k_r<7, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz); break;
            default: launch_q4k_r<8, PRO, EPI>(w, n, nsb, x, m, y, s, lds, rpw, fz); break;
        }
    }
}

template <int PRO, int EPI>
void launch_q4k(const uint8_t* w, int n, int nsb, const float* x, size_t m, float* y, hipStream_t s, size_t lds,
                const KqFuse& fz) {
    // longer rows: K split over 2 or 4 waves of a 16-wave workgroup, one per CU
    const int units = nsb * 4;  // <= 256 (K <= 16384)
    if (units <= 64) launch_q4k_small<PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
    else if (units <= 128) launch_q4k_splitk<2, PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
    else launch_q4k_splitk<4, PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
}

// Q6_K: 16-wave workgroups, K split over KS = 1, 2, 4 or 8 waves (at most 64
// units a wave), one workgroup per CU walking the row groups.
template <int KS, int R, int PRO, int EPI>
void launch_q6k_ks_r(const uint8_t* w, int n, int nsb, const float* x, size_t m, float* y, hipStream_t s,
                     size_t lds, const KqFuse& fz) {
    constexpr int NW = 16, RPW = NW / KS * R;
    const int units = nsb * 8, ups = (units + KS - 1) / KS;
    // one workgroup per CU, each walking its share of the row groups
    const int groups = (n + RPW - 1) / RPW;
    const int wgs = groups < num_cus() ? groups : num_cus();
    const dim3 grid((unsigned)wgs, (unsigned)m), block(NW * 64);
    lds += (size_t)2 * KS * RPW * sizeof(float);  // slice sums after the records
    launch_kernel((gemv_q6k_splitk_kernel<R, KS, 16, PRO, EPI>), grid, block, lds, s, w, n, nsb, ups, x, y, fz);
}
template <int KS, int PRO, int EPI>
void launch_q6k_ks(const uint8_t* w, int n, int nsb, const float* x, size_t m, float* y, hipStream_t s,
                   size_t lds, const KqFuse& fz) {
    // R rows a wave a group: 4 when every CU gets at least one group of them
    const long rg = 16 / KS;
    if ((n + rg * 4 - 1) / (rg * 4) >= num_cus()) launch_q6k_ks_r<KS, 4, PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
    else if ((n + rg * 2 - 1) / (rg * 2) >= num_cus()) launch_q6k_ks_r<KS, 2, PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
    else launch_q6k_ks_r<KS, 1, PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
}
template <int PRO, int EPI>
void launch_q6k(const uint8_t* w, int n, int nsb, const float* x, size_t m, float* y, hipStream_t s, size_t lds,
                const KqFuse& fz) {
    const int units = nsb * 8;  // <= 512 (K <= 16384)
    if (units <= 64) launch_q6k_ks<1, PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
    else if (units <= 128) launch_q6k_ks<2, PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
    else if (units <= 256) launch_q6k_ks<4, PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
    else launch_q6k_ks<8, PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
}

template <int PRO, int EPI>
void launch_kq(WType t, const uint8_t* w, int n, int nsb, const float* x, size_t m, float* y, hipStream_t s,
               size_t lds, const KqFuse& fz) {
    if (t == WType::Q6_K) launch_q6k<PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
    else launch_q4k<PRO, EPI>(w, n, nsb, x, m, y, s, lds, fz);
}

// Decoder fusion: Q4_0 float mode, nb even.  8-wave workgroups, two per CU;
// rows longer than 4096 (their x, re-read by every workgroup, is long): one
// 16-wave workgroup per CU.
template <int PRO, int RES>
void launch_q4_0_fused_ex(const uint8_t* w, int n, int nb, const float* x, size_t m, float* y,
                          hipStream_t s, size_t lds, const Fuse& fz) {
    const int cpl = cpl_for(nb);
    constexpr int Q = (int)WType::Q4_0;
    if (RES != EPI_SWIGLU && RES != EPI_ROPE_KV && cpl == 8) {
        const Cfg c16 = pick_cfg(n, 16, 1, 1);
        launch_nw<Q, false, 8, true, 16, PRO, RES>(w, n, nb, x, m, y, s, c16, lds, fz);
        return;
    }
    Cfg c = pick_cfg(n, 8, 8 / cpl, 2);
    if (RES == EPI_SWIGLU || RES == EPI_ROPE_KV) {
        // whole row pairs per wave: R even, a workgroup takes NW * R rows
        // (two pairs a wave where the columns allow; measured on MI355X in the
        // 7B decode step, also for the 6144-row q/k/v launch)
        c.r = (8 / cpl >= 4) ? 4 : 2;
        c.rpw = 8 * c.r;
    }
    // Matrices taller than one round of two 8-wave workgroups a CU at 4 rows
    // a wave (the 28672-row gate/up, the 32000-row lm_head): 8 rows a wave, so
    // every workgroup is resident from the start and prepares x once.
    if ((RES == EPI_SWIGLU || RES == EPI_STORE) && cpl == 2 && n > num_cus() * 2 * 8 * 4) {
        c.r = 8;
        c.rpw = 64;
    }
    switch (cpl) {
        case 2: launch_nw<Q, false, 2, true, 8, PRO, RES>(w, n, nb, x, m, y, s, c, lds, fz); break;
        case 4: launch_nw<Q, false, 4, true, 8, PRO, RES>(w, n, nb, x, m, y, s, c, lds, fz); break;
        default: launch_nw<Q, false, 8, true, 8, PRO, RES>(w, n, nb, x, m, y, s, c, lds, fz); break;
    }
}

}  // namespace

hipError_t launch_gemv_q4_0_fused_ex(const uint8_t* w, size_t n, size_t k, const float* x, size_t xstride,
                                     size_t m, float* y, int prologue, const float* g, float eps,
                                     int epilogue, hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    const int nb = (int)(k / QK);
    if (nb == 0 || (nb & 1) || k > fused_max_k(WType::Q4_0) || ((uintptr_t)x & 15) || (xstride & 3) ||
        (uint64_t)n * nb * Q4_0_BYTES > FUSED_MAX_WEIGHT_BYTES || m > 4)
        return hipErrorInvalidValue;
    Fuse fz{};
    fz.g = g;
    fz.eps = eps;
    fz.xstride = (int)xstride;
    const size_t lds = (size_t)8 * 16 * nb;
    const int ni = (int)n;
    if (epilogue == EPI_SWIGLU && ((n & 1) || cpl_for(nb) > 4)) return hipErrorInvalidValue;
    if (epilogue == EPI_ROPE_KV) return hipErrorInvalidValue;  // launch_gemv_q4_0_rope_kv
    if (prologue == PRO_RMSNORM && epilogue == EPI_STORE)
        launch_q4_0_fused_ex<PRO_RMSNORM, EPI_STORE>(w, ni, nb, x, m, y, s, lds, fz);
    else if (prologue == PRO_RMSNORM && epilogue == EPI_SWIGLU)
        launch_q4_0_fused_ex<PRO_RMSNORM, EPI_SWIGLU>(w, ni, nb, x, m, y, s, lds, fz);
    else if (prologue == PRO_NONE && epilogue == EPI_RESIDUAL)
        launch_q4_0_fused_ex<PRO_NONE, EPI_RESIDUAL>(w, ni, nb, x, m, y, s, lds, fz);
    else if (prologue == PRO_SWIGLU && epilogue == EPI_RESIDUAL)
        launch_q4_0_fused_ex<PRO_SWIGLU, EPI_RESIDUAL>(w, ni, nb, x, m, y, s, lds, fz);
    else if (prologue == PRO_NONE && epilogue == EPI_STORE)
        launch_q4_0_fused_ex<PRO_NONE, EPI_STORE>(w, ni, nb, x, m, y, s, lds, fz);
    else if (prologue == PRO_NONE && epilogue == EPI_SWIGLU)
        launch_q4_0_fused_ex<PRO_NONE, EPI_SWIGLU>(w, ni, nb, x, m, y, s, lds, fz);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_gemv_q4_0_rope_kv(const uint8_t* w, size_t n, size_t k, const float* x, size_t m, float* y,
                                    const float* g, float eps, const int* pos, const float* cos_t,
                                    const float* sin_t, void* kc, void* vc, int n_heads, int n_kv, int hd,
                                    const int* kv_table, bool kv_f16, hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    const int nb = (int)(k / QK);
    if (nb == 0 || (nb & 1) || cpl_for(nb) > 4 || ((uintptr_t)x & 15) || m > 4 || (hd & 1) ||
        n != (size_t)(n_heads + 2 * n_kv) * hd || (uint64_t)n * nb * Q4_0_BYTES > FUSED_MAX_WEIGHT_BYTES)
        return hipErrorInvalidValue;
    Fuse fz{};
    fz.g = g;
    fz.eps = eps;
    fz.xstride = (int)k;
    fz.pos = pos;
    fz.cos_t = cos_t;
    fz.sin_t = sin_t;
    fz.kc = kc;
    fz.vc = vc;
    fz.n_heads = n_heads;
    fz.n_kv = n_kv;
    fz.hd = hd;
    fz.kv_table = kv_table;
    fz.kv_f16 = kv_f16 ? 1 : 0;
    launch_q4_0_fused_ex<PRO_RMSNORM, EPI_ROPE_KV>(w, (int)n, nb, x, m, y, s, (size_t)8 * 16 * nb, fz);
    return hipGetLastError();
}

hipError_t launch_qkv_attention(const uint8_t* w, size_t n, size_t k, const float* x, float* y, const float* g,
                                float eps, const int* pos, const float* cos_t, const float* sin_t, void* kc, void* vc,
                                const int* kv_table, int n_heads, int n_kv, int hd, bool kv_f16, float* att_part,
                                int nspan, int spans, int* att_cnt, float* att_out, uint64_t* xch, int* err,
                                const uint8_t* wo, size_t n_o, float* x_res, uint64_t* oxch, hipStream_t s,
                                const uint8_t* wd, size_t k_d, const float* h, uint64_t* xx) {
    const int nb = (int)(k / QK);
    const int cpl = cpl_for(nb);
    // the q/k/v launch's shape (launch_q4_0_fused_ex, EPI_ROPE_KV): row pairs, R rows a wave, 8 waves
    const int r = (8 / cpl >= 4) ? 4 : 2, rpw = 8 * r;
    if (k == 0 || nb == 0 || (nb & 1) || cpl > 4 || ((uintptr_t)x & 15) || (hd & 1) || hd % rpw ||
        n_kv <= 0 || n_heads % n_kv || n != (size_t)(n_heads + 2 * n_kv) * hd ||
        (uint64_t)n * nb * Q4_0_BYTES > FUSED_MAX_WEIGHT_BYTES || xch == nullptr || err == nullptr)
        return hipErrorInvalidValue;
    // the coalesced K/V layout of the fused attention: 16-byte pieces, at most 16 a row
    if (!((kv_f16 && (hd == 128 || hd == 64)) || (!kv_f16 && hd == 64))) return hipErrorInvalidValue;
    Fuse fz{};
    fz.g = g;
    fz.eps = eps;
    fz.xstride = (int)k;
    fz.pos = pos;
    fz.cos_t = cos_t;
    fz.sin_t = sin_t;
    fz.kc = kc;
    fz.vc = vc;
    fz.n_heads = n_heads;
    fz.n_kv = n_kv;
    fz.hd = hd;
    fz.kv_table = kv_table;
    fz.kv_f16 = kv_f16 ? 1 : 0;
    fz.xch = xch;
    const int n_gemv = (int)((n + rpw - 1) / rpw);
    if (spans < 1 || spans > nspan) return hipErrorInvalidValue;
    // o projection (optional): K = n_heads * hd in 32-element blocks, at most
    // two block columns a lane and one activation piece a thread
    OProj op{};
    int n_ow = 0;
    const int nb_o = n_heads * hd / QK;
    if (wo) {
        if ((n_heads * hd) % QK || nb_o > 128 || (nb_o & 1) || n_o == 0 || x_res == nullptr || oxch == nullptr ||
            (uint64_t)n_o * nb_o * Q4_0_BYTES > FUSED_MAX_WEIGHT_BYTES)
            return hipErrorInvalidValue;
        op.w = wo;
        op.n = (int)n_o;
        op.nb = nb_o;
        op.x = x_res;
        op.xch = oxch;
        n_ow = (int)((n_o + 8 * O_ROWS_PER_WAVE - 1) / (8 * O_ROWS_PER_WAVE));
    }
    // the previous layer's down projection (optional, with the o projection):
    // k rows of W_down over k_d columns (32-element blocks, an even count of
    // at most 512), h its SwiGLU row; the new x goes through xx ([k] tagged
    // words) to the q/k/v and o workgroups, which then read no x from memory
    DownPart dp{};
    size_t lds_d = 0;
    if (wd) {
        const int nb_d = (int)(k_d / QK);
        if (!wo || k_d == 0 || k_d % QK || (nb_d & 1) || nb_d > 8 * 64 || h == nullptr || xx == nullptr ||
            ((uintptr_t)h & 15) || (uint64_t)k * nb_d * Q4_0_BYTES > FUSED_MAX_WEIGHT_BYTES)
            return hipErrorInvalidValue;
        dp.w = wd;
        dp.n = (int)k;
        dp.nb = nb_d;
        dp.rpw = 8 * DOWN_R;
        dp.n_wg = (int)((k + dp.rpw - 1) / dp.rpw);
        dp.h = h;
        dp.x = x_res;
        dp.fz.xstride = (int)k_d;
        dp.fz.pos = pos;
        dp.fz.xout = xx;
        fz.xin = xx;
        fz.err = err;
        op.xin = xx;
        lds_d = (size_t)8 * 16 * nb_d;
    }
    const int n_att = n_heads * spans;
    const dim3 grid((unsigned)(dp.n_wg + n_gemv + n_att + n_ow)), block(512);
    // attention: q | per-wave contexts | current k | current v (f32); records of q/k/v's, o's and down's x
    const size_t lds = std::max({(size_t)8 * 16 * nb, (size_t)8 * 16 * nb_o,
                                 (size_t)(3 + ATT_WAVES) * hd * sizeof(float), lds_d});
    hipError_t attr = hipSuccess;
    auto go = [&](auto kv_tag, auto hd_tag, auto r_tag) {
        using KV = decltype(kv_tag);
        constexpr int HD = decltype(hd_tag)::value, R = decltype(r_tag)::value, CPL = R == 4 ? 2 : 4;
        AttArgs<KV> aa{};
        aa.qkv = y;
        aa.qkv_dim = (int)n;
        aa.pos_dev = pos;
        aa.kc = reinterpret_cast<const KV*>(kc);
        aa.vc = reinterpret_cast<const KV*>(vc);
        aa.kv_table = kv_table;
        aa.n_heads = n_heads;
        aa.n_kv = n_kv;
        aa.hd_rt = hd;
        aa.scale = sqrtf((float)hd);
        aa.part = att_part;
        aa.nspan = nspan;
        aa.counters = att_cnt;
        aa.out = att_out;
        aa.xch = xch;
        aa.oxch = wo ? oxch : nullptr;
        aa.err = err;
        if (wd) {
            const auto kern = qkv_attention_kernel<KV, HD, R, CPL, true>;
            if (lds > 65536 &&
                (attr = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                            (int)lds)) != hipSuccess)
                return;
            launch_kernel(kern, grid, block, lds, s, w, (int)n, nb, rpw, x, y, fz, aa, n_gemv, n_att, op, dp);
        } else {
            launch_kernel(qkv_attention_kernel<KV, HD, R, CPL, false>, grid, block, lds, s, w, (int)n, nb, rpw, x, y,
                          fz, aa, n_gemv, n_att, op, dp);
        }
    };
    using I64 = std::integral_constant<int, 64>;
    using I128 = std::integral_constant<int, 128>;
    using R4 = std::integral_constant<int, 4>;
    using R2 = std::integral_constant<int, 2>;
    if (kv_f16) {
        if (hd == 128) { if (r == 4) go(_Float16{}, I128{}, R4{}); else go(_Float16{}, I128{}, R2{}); }
        else { if (r == 4) go(_Float16{}, I64{}, R4{}); else go(_Float16{}, I64{}, R2{}); }
    } else {
        if (r == 4) go(0.0f, I64{}, R4{}); else go(0.0f, I64{}, R2{});
    }
    if (attr != hipSuccess) return attr;
    return hipGetLastError();
}

// Largest K the fused kernels take (records for all of K live in LDS and a
// lane holds at most 8 columns of blocks in registers).
size_t fused_max_k(WType t) { return t == WType::Q4_K ? 16384 : 16384; }

hipError_t launch_gemv_fused(WType t, bool native, const uint8_t* w, size_t n, size_t k,
                             const float* x, size_t m, float* y, hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    const int nb = (int)(k / QK);
    const size_t lds = (size_t)(native ? 3 : 8) * 16 * (nb > 0 ? nb : 1);
    const int ni = (int)n;
    if ((uint64_t)n * (k / block_elems(t)) * block_bytes(t) > FUSED_MAX_WEIGHT_BYTES)
        return hipErrorInvalidValue;  // weight windows use 32-bit buffer offsets
    // int4-record float GEMVs and Q8_0 float: 8-wave workgroups, two per CU
    // (the prep runs on half as many lanes per workgroup but overlaps the
    // other workgroup's stream; Q8_0 4096 x 4096: 5.95 -> 5.75 us a step);
    // everything else one 16-wave workgroup per CU.
    // Rows of more than 256 columns (K > 8192) run one row per wave in any case:
    // one 16-wave workgroup per CU (Q4_0 4096 x 14336: 11.1 -> 9.6 us).
    // Q8_0 float rows of at most 128 blocks (two columns a lane): one 4-wave
    // workgroup per CU, 4 rows a wave (4096 x 4096: 6.11 -> 5.83 us, swept
    // over 4 / 8 / 16 waves x 1-6 workgroups per CU).
    const bool i4 = !native && (t == WType::Q4_0 || t == WType::Q4_1) && cpl_for(nb) < 8;
    const bool q8_narrow = t == WType::Q8_0 && !native && cpl_for(nb) == 2;
    const bool two = i4 || (t == WType::Q8_0 && !native && cpl_for(nb) < 8);
    const int nw = q8_narrow ? 4 : two ? 8 : 16, wg_per_cu = q8_narrow ? 1 : two ? 2 : 1;
    if (t == WType::Q6_K || t == WType::Q4_K) {
        if (native) return hipErrorInvalidValue;
        KqFuse fz{};
        fz.xstride = (int)k;
        fz.ystride = ni;
        launch_kq<PRO_NONE, EPI_STORE>(t, w, ni, (int)(k / QK_K), x, m, y, s, lds, fz);
        return hipGetLastError();
    }
    if (native) {
        if (t == WType::Q4_1) launch_cpl<(int)WType::Q4_1, true>(w, ni, nb, x, m, y, s, lds, nw, wg_per_cu);
        else launch_cpl<(int)WType::Q4_0, true>(w, ni, nb, x, m, y, s, lds, nw, wg_per_cu);
    } else if (t == WType::Q4_1) {
        launch_cpl<(int)WType::Q4_1, false>(w, ni, nb, x, m, y, s, lds, nw, wg_per_cu);
    } else if (t == WType::Q8_0) {
        launch_cpl<(int)WType::Q8_0, false>(w, ni, nb, x, m, y, s, lds, nw, wg_per_cu);
    } else {
        launch_cpl<(int)WType::Q4_0, false>(w, ni, nb, x, m, y, s, lds, nw, wg_per_cu);
    }
    return hipGetLastError();
}

hipError_t launch_gemv_kquant_ex(WType t, const uint8_t* w, size_t n, size_t k, const float* x, size_t xstride,
                                 size_t m, float* y, size_t ystride, int prologue, const float* g, float eps,
                                 int epilogue, hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    if ((t != WType::Q4_K && t != WType::Q6_K) || k == 0 || k % QK_K || k > fused_max_k(t) || m > 4 ||
        ((uintptr_t)x & 15) || (xstride & 3) || xstride < k || xstride > INT32_MAX || ystride > INT32_MAX ||
        (prologue == PRO_RMSNORM && (g == nullptr || ((uintptr_t)g & 15))) ||
        (uint64_t)n * (k / QK_K) * block_bytes(t) > FUSED_MAX_WEIGHT_BYTES)
        return hipErrorInvalidValue;
    if (epilogue == EPI_SWIGLU ? (n & 1) || ystride < n / 2 : ystride < n) return hipErrorInvalidValue;
    KqFuse fz{};
    fz.g = g;
    fz.eps = eps;
    fz.xstride = (int)xstride;
    fz.ystride = (int)ystride;
    const int ni = (int)n, nsb = (int)(k / QK_K);
    // records plus the RMSNorm partials (one float a wave) after them
    const size_t lds = (size_t)8 * 16 * (k / QK) + 16 * sizeof(float);
    if (prologue == PRO_NONE && epilogue == EPI_STORE)
        launch_kq<PRO_NONE, EPI_STORE>(t, w, ni, nsb, x, m, y, s, lds, fz);
    else if (prologue == PRO_RMSNORM && epilogue == EPI_STORE)
        launch_kq<PRO_RMSNORM, EPI_STORE>(t, w, ni, nsb, x, m, y, s, lds, fz);
    else if (prologue == PRO_NONE && epilogue == EPI_RESIDUAL)
        launch_kq<PRO_NONE, EPI_RESIDUAL>(t, w, ni, nsb, x, m, y, s, lds, fz);
    else if (prologue == PRO_RMSNORM && epilogue == EPI_SWIGLU)
        launch_kq<PRO_RMSNORM, EPI_SWIGLU>(t, w, ni, nsb, x, m, y, s, lds, fz);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_gemv_kquant_rope_kv(WType t, const uint8_t* w, size_t n, size_t k, const float* x, size_t m,
                                      size_t row0, float* y, size_t ystride, const float* g, float eps,
                                      const int* pos, const float* cos_t, const float* sin_t, void* kc, void* vc,
                                      int n_heads, int n_kv, int hd, int head0, const int* kv_table, bool kv_f16,
                                      hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    // heads head0 .. head0 + n / hd - 1 of [q | k | v]; q heads only from head0 = 0
    if ((t != WType::Q4_K && t != WType::Q6_K) || k == 0 || k % QK_K || k > fused_max_k(t) || m > 4 ||
        ((uintptr_t)x & 15) || k > INT32_MAX || ystride < n || ystride > INT32_MAX || row0 > INT32_MAX ||
        g == nullptr || ((uintptr_t)g & 15) || hd <= 0 || (hd & 1) || n % (size_t)hd != 0 ||
        (head0 != 0 && head0 < n_heads) || head0 < 0 || (size_t)head0 + n / hd > (size_t)(n_heads + 2 * n_kv) ||
        (uint64_t)n * (k / QK_K) * block_bytes(t) > FUSED_MAX_WEIGHT_BYTES)
        return hipErrorInvalidValue;
    KqFuse fz{};
    fz.g = g;
    fz.eps = eps;
    fz.xstride = (int)k;
    fz.ystride = (int)ystride;
    fz.pos = pos;
    fz.row0 = (int)row0;
    fz.cos_t = cos_t;
    fz.sin_t = sin_t;
    fz.kc = kc;
    fz.vc = vc;
    fz.n_heads = n_heads;
    fz.n_kv = n_kv;
    fz.hd = hd;
    fz.kv_table = kv_table;
    fz.kv_f16 = kv_f16 ? 1 : 0;
    fz.head0 = head0;
    const size_t lds = (size_t)8 * 16 * (k / QK) + 16 * sizeof(float);
    launch_kq<PRO_RMSNORM, EPI_ROPE_KV>(t, w, (int)n, (int)(k / QK_K), x, m, y, s, lds, fz);
    return hipGetLastError();
}

}  // namespace rdl
