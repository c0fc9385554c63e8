// gemv.hip -- batch-1 decode GEMV, y = W x, straight from GGUF blocks in HBM.
//
// Reference semantics (paths relative to the rust-deeplearning root):
//   Q8_0 float   matmul_f32_q8         rustml/quant/main/src/core/quantize.rs:201-260
//   Q4_0 float   matmul_f32_q4         quantize.rs:265-320
//   Q4_0 native  matmul_f32_q4_native  quantize.rs:326-394 (int32 block dots, :383-384)
//   Q4_1 float   matmul_f32_q4_1       quantize.rs:429-495
//   Q4_1 native  matmul_f32_q4_1_native quantize.rs:501-572
//   Q4_K float   dequantize_q4k (rustml/gguf/main/src/core/parser.rs:549-593) + F32 GEMV
//   Q6_K float   dequantize_q6k (parser.rs:510-547) + F32 GEMV
//
// Mapping (wave-level, no LDS):
//   * one wave owns R consecutive weight rows for one activation row;
//   * lane l owns the 32-element columns l, l+64, ... (K/32 = 128 at K=4096,
//     448 at K=14336: 2 or 7 columns per lane); the prepared activation record
//     of a column is loaded once and reused for all R rows;
//   * a lane reads its 18/20/34-byte block with a dword-aligned 16-byte load
//     plus one or two dwords; 64 lanes read 64 consecutive blocks of a row, so
//     every load instruction covers one contiguous ~1.1-2.2 KB span;
//   * the block is realigned in registers with v_perm_b32 and dotted with the
//     activation digits on v_dot4_i32_i8; the int32 results are exact;
//   * the R row partials are summed across the wave with a transpose
//     reduction (R values, log2(64) exchange steps).
#include <algorithm>
#include "rdl_device.hpp"
#include "rdl_internal.hpp"

namespace rdl {

namespace {

constexpr int GEMV_THREADS = 256;  // 4 waves
constexpr int WAVES = GEMV_THREADS / 64;
constexpr uint32_t SEL_EVEN = 0x05040302u;  // bytes 2..5 of {w[k+1]:w[k]}
constexpr uint32_t SEL_ODD = 0x07060504u;   // bytes 4..7 (= w[k+1])
constexpr uint32_t NIB = 0x0F0F0F0Fu;

// ---- prepared-activation views ---------------------------------------------

struct XF {  // float mode, one 32-element column
    i32x4 a0, a1, b0, b1, c0, c1;
    float S;
    int sa, sb, sc;
    float xsum;
};
__device__ __forceinline__ XF load_xf(const FloatRec* r) {
    const i32x4* p = reinterpret_cast<const i32x4*>(r);
    XF x;
    x.a0 = p[0];
    x.a1 = p[1];
    x.b0 = p[2];
    x.b1 = p[3];
    x.c0 = p[4];
    x.c1 = p[5];
    i32x4 m = p[6];
    x.S = as_f32(m.x);
    x.sa = m.y;
    x.sb = m.z;
    x.sc = m.w;
    x.xsum = as_f32(p[7].x);
    return x;
}
struct XN {  // native mode: Q8_0 codes of the column
    i32x4 q0, q1;
    float scale;
    int qsum;
};
__device__ __forceinline__ XN load_xn(const NativeRec* r) {
    const i32x4* p = reinterpret_cast<const i32x4*>(r);
    XN x;
    x.q0 = p[0];
    x.q1 = p[1];
    i32x4 m = p[2];
    x.scale = as_f32(m.x);
    x.qsum = m.y;
    return x;
}

// Three-digit dot of 8 weight dwords (bytes in [-128,127] or nibbles 0..15)
// against digit dwords d0 (elements 0..15) and d1 (16..31); returns
// A + (B + C/256)/256 given the int32 accumulators' initial values.
__device__ __forceinline__ float dot3(const uint32_t (&w)[8], const XF& x, int ia, int ib,
                                      int ic) {
    int A = ia, B = ib, C = ic;
    A = dot4(w[0], x.a0.x, A); A = dot4(w[1], x.a0.y, A); A = dot4(w[2], x.a0.z, A); A = dot4(w[3], x.a0.w, A);
    A = dot4(w[4], x.a1.x, A); A = dot4(w[5], x.a1.y, A); A = dot4(w[6], x.a1.z, A); A = dot4(w[7], x.a1.w, A);
    B = dot4(w[0], x.b0.x, B); B = dot4(w[1], x.b0.y, B); B = dot4(w[2], x.b0.z, B); B = dot4(w[3], x.b0.w, B);
    B = dot4(w[4], x.b1.x, B); B = dot4(w[5], x.b1.y, B); B = dot4(w[6], x.b1.z, B); B = dot4(w[7], x.b1.w, B);
    C = dot4(w[0], x.c0.x, C); C = dot4(w[1], x.c0.y, C); C = dot4(w[2], x.c0.z, C); C = dot4(w[3], x.c0.w, C);
    C = dot4(w[4], x.c1.x, C); C = dot4(w[5], x.c1.y, C); C = dot4(w[6], x.c1.z, C); C = dot4(w[7], x.c1.w, C);
    float t = fmaf((float)C, 1.0f / 256.0f, (float)B);
    return fmaf(t, 1.0f / 256.0f, (float)A);
}

__device__ __forceinline__ int dot1(const uint32_t (&w)[8], const XN& x, int acc) {
    acc = dot4(w[0], x.q0.x, acc); acc = dot4(w[1], x.q0.y, acc);
    acc = dot4(w[2], x.q0.z, acc); acc = dot4(w[3], x.q0.w, acc);
    acc = dot4(w[4], x.q1.x, acc); acc = dot4(w[5], x.q1.y, acc);
    acc = dot4(w[6], x.q1.z, acc); acc = dot4(w[7], x.q1.w, acc);
    return acc;
}

// ---- raw block windows -------------------------------------------------------

template <int WT>
__device__ constexpr size_t block_bytes_dev() {
    return WT == (int)WType::Q8_0 ? Q8_0_BYTES : WT == (int)WType::Q4_1 ? Q4_1_BYTES : Q4_0_BYTES;
}

struct Win5 {  // 20 bytes from a dword-aligned base (Q4_0, Q4_1)
    uint32_t w[5];
    uint32_t sel;  // realignment selector
    uint32_t dsh;  // bit offset of the f16 scale inside w[0]
};
struct Win9 {  // 36 bytes from a dword-aligned base (Q8_0)
    uint32_t w[9];
    uint32_t sel;
    uint32_t dsh;
};

// The window may extend 2 bytes past the block; for the last block of the
// buffer those 2 bytes lie past its end, so the tail word is then read as a
// 16-bit load (the 2 bytes beyond are never used).
__device__ __forceinline__ uint32_t load_tail(const uint8_t* p, size_t addr_end, size_t wbytes) {
    if (addr_end <= wbytes) return *reinterpret_cast<const uint32_t*>(p);
    return (uint32_t)*reinterpret_cast<const uint16_t*>(p);
}

__device__ __forceinline__ void load_win5(const uint8_t* __restrict__ W, size_t off, size_t wbytes,
                                          Win5& b) {
    const size_t base = off & ~(size_t)3;
    const uint8_t* p = W + base;
    u32x4a4 v = *reinterpret_cast<const u32x4a4*>(p);
    b.w[0] = v.x; b.w[1] = v.y; b.w[2] = v.z; b.w[3] = v.w;
    b.w[4] = load_tail(p + 16, base + 20, wbytes);
    const bool odd = (off & 2) != 0;
    b.sel = odd ? SEL_ODD : SEL_EVEN;
    b.dsh = odd ? 16u : 0u;
}
__device__ __forceinline__ void load_win9(const uint8_t* __restrict__ W, size_t off, size_t wbytes,
                                          Win9& b) {
    const size_t base = off & ~(size_t)3;
    const uint8_t* p = W + base;
    u32x4a4 v0 = *reinterpret_cast<const u32x4a4*>(p);
    u32x4a4 v1 = *reinterpret_cast<const u32x4a4*>(p + 16);
    b.w[0] = v0.x; b.w[1] = v0.y; b.w[2] = v0.z; b.w[3] = v0.w;
    b.w[4] = v1.x; b.w[5] = v1.y; b.w[6] = v1.z; b.w[7] = v1.w;
    b.w[8] = load_tail(p + 32, base + 36, wbytes);
    const bool odd = (off & 2) != 0;
    b.sel = odd ? SEL_ODD : SEL_EVEN;
    b.dsh = odd ? 16u : 0u;
}

// Q4_0: nibble dwords lo (elements 0..15) and hi (16..31) from a window.
__device__ __forceinline__ void q4_0_unpack(const Win5& b, uint32_t (&q)[8], float& d) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t n = perm(b.w[k + 1], b.w[k], b.sel);
        q[k] = n & NIB;
        q[k + 4] = (n >> 4) & NIB;
    }
    d = h2f((b.w[0] >> b.dsh) & 0xFFFFu);
}
// Q4_1: block base is 20*g, always dword aligned.
__device__ __forceinline__ void q4_1_unpack(const Win5& b, uint32_t (&q)[8], float& d, float& m) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        q[k] = b.w[k + 1] & NIB;
        q[k + 4] = (b.w[k + 1] >> 4) & NIB;
    }
    d = h2f(b.w[0] & 0xFFFFu);
    m = h2f(b.w[0] >> 16);
}
__device__ __forceinline__ void q8_0_unpack(const Win9& b, uint32_t (&q)[8], float& d) {
#pragma unroll
    for (int k = 0; k < 8; k++) q[k] = perm(b.w[k + 1], b.w[k], b.sel);
    d = h2f((b.w[0] >> b.dsh) & 0xFFFFu);
}

// ---- wave reduction of R row partials ----------------------------------------
// After the call, lane l holds the full sum of row (l >> (6 - log2 R)).
template <int R>
__device__ __forceinline__ float wave_reduce_rows(float (&v)[R], int lane) {
    int count = R;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        if (count > 1) {
            const int half = count / 2;
            const bool upper = (lane & o) != 0;
#pragma unroll
            for (int i = 0; i < R / 2; i++) {
                if (i < half) {
                    float keep = upper ? v[half + i] : v[i];
                    float send = upper ? v[i] : v[half + i];
                    v[i] = keep + __shfl_xor(send, o);
                }
            }
            count = half;
        } else {
            v[0] += __shfl_xor(v[0], o);
        }
    }
    return v[0];
}

template <int R>
__device__ __forceinline__ void store_rows(float (&acc)[R], int lane, int row0, int n,
                                           float* __restrict__ y) {
    float s = wave_reduce_rows<R>(acc, lane);
    constexpr int LOG2R = (R >= 16) ? 4 : (R >= 8) ? 3 : (R >= 4) ? 2 : (R >= 2) ? 1 : 0;
    constexpr int SPAN = 64 >> LOG2R;
    if ((lane & (SPAN - 1)) == 0) {
        const int row = row0 + (lane >> (6 - LOG2R));
        if (row < n) y[row] = s;
    }
}

// ---- kernels -----------------------------------------------------------------

// Q4_0 / Q8_0 / Q4_1 in float mode: per-block int digit dots, f32 combine.
template <int R, int WT>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_float_kernel(
    const uint8_t* __restrict__ W, int n, int nb, const FloatRec* __restrict__ X,
    float* __restrict__ Y) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * WAVES + (threadIdx.x >> 6);
    const int row0 = wave * R;
    if (row0 >= n) return;
    const FloatRec* xr = X + (size_t)blockIdx.y * nb;
    float* yr = Y + (size_t)blockIdx.y * n;
    const size_t wbytes = (size_t)n * nb * block_bytes_dev<WT>();
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int col = lane; col < nb; col += 64) {
        if (WT == (int)WType::Q8_0) {
            Win9 blk[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = min(row0 + r, n - 1);
                load_win9(W, ((size_t)row * nb + col) * Q8_0_BYTES, wbytes, blk[r]);
            }
            const XF x = load_xf(xr + col);
#pragma unroll
            for (int r = 0; r < R; r++) {
                uint32_t q[8];
                float d;
                q8_0_unpack(blk[r], q, d);
                acc[r] = fmaf(x.S * d, dot3(q, x, 0, 0, 0), acc[r]);
            }
        } else {
            constexpr size_t BB = (WT == (int)WType::Q4_1) ? Q4_1_BYTES : Q4_0_BYTES;
            Win5 blk[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = min(row0 + r, n - 1);
                load_win5(W, ((size_t)row * nb + col) * BB, wbytes, blk[r]);
            }
            const XF x = load_xf(xr + col);
            if (WT == (int)WType::Q4_0) {
                const int ia = -8 * x.sa, ib = -8 * x.sb, ic = -8 * x.sc;
#pragma unroll
                for (int r = 0; r < R; r++) {
                    uint32_t q[8];
                    float d;
                    q4_0_unpack(blk[r], q, d);
                    acc[r] = fmaf(x.S * d, dot3(q, x, ia, ib, ic), acc[r]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    uint32_t q[8];
                    float d, m;
                    q4_1_unpack(blk[r], q, d, m);
                    acc[r] = fmaf(x.S * d, dot3(q, x, 0, 0, 0), fmaf(m, x.xsum, acc[r]));
                }
            }
        }
    }
    store_rows<R>(acc, lane, row0, n, yr);
}

// Q4_0 / Q4_1 native mode: exact int32 block dots against Q8_0 activations.
template <int R, int WT>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_native_kernel(
    const uint8_t* __restrict__ W, int n, int nb, const NativeRec* __restrict__ X,
    float* __restrict__ Y) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * WAVES + (threadIdx.x >> 6);
    const int row0 = wave * R;
    if (row0 >= n) return;
    const NativeRec* xr = X + (size_t)blockIdx.y * nb;
    float* yr = Y + (size_t)blockIdx.y * n;
    constexpr size_t BB = (WT == (int)WType::Q4_1) ? Q4_1_BYTES : Q4_0_BYTES;
    const size_t wbytes = (size_t)n * nb * BB;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    for (int col = lane; col < nb; col += 64) {
        Win5 blk[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(row0 + r, n - 1);
            load_win5(W, ((size_t)row * nb + col) * BB, wbytes, blk[r]);
        }
        const XN x = load_xn(xr + col);
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t q[8];
            if (WT == (int)WType::Q4_0) {
                float d;
                q4_0_unpack(blk[r], q, d);
                // dot_q4q8_block = sum (q-8)*q8 = sum q*q8 - 8*sum q8 (exact)
                const int id = dot1(q, x, -8 * x.qsum);
                // reference: dot += (int_dot as f32) * q8_scale * w_scale
                acc[r] += ((float)id * x.scale) * d;
            } else {
                float d, m;
                q4_1_unpack(blk[r], q, d, m);
                const int ud = dot1(q, x, 0);
                // reference: dot += q8_scale * (d * unsigned_dot + m * q8_sum)
                acc[r] += x.scale * (d * (float)ud + m * (float)x.qsum);
            }
        }
    }
    store_rows<R>(acc, lane, row0, n, yr);
}

// Q4_K float mode.  A unit is one 32-byte chunk of a super-block's nibbles
// (two 32-element sub-blocks: lo nibbles = sub-block 2c, hi = 2c+1,
// parser.rs:574-589); lane l owns units l, l+64, ...
__device__ __forceinline__ void q4k_scale_min(const u32x4& h, int c, int& sc1, int& mn1, int& sc2,
                                              int& mn2) {
    // scales_raw = header bytes 4..15 = h.y, h.z, h.w; s[k] = byte k.
    const uint64_t s03 = h.y, s47 = h.z, s811 = h.w;
    const uint32_t j1 = 2 * c;  // sub-blocks j1, j1+1
    if (c < 2) {
        // j < 4: sc = s[j] & 63, mn = s[j+4] & 63        (parser.rs:565-566)
        sc1 = (int)((s03 >> (8 * j1)) & 63);
        sc2 = (int)((s03 >> (8 * (j1 + 1))) & 63);
        mn1 = (int)((s47 >> (8 * j1)) & 63);
        mn2 = (int)((s47 >> (8 * (j1 + 1))) & 63);
    } else {
        // j >= 4, i = j-4: sc = ((s[i]>>6)&3) | ((s[i+8]&0xF)<<2),
        //                  mn = ((s[i+4]>>6)&3) | ((s[i+8]>>4)<<2)   (parser.rs:567-568)
        const uint32_t i1 = j1 - 4;
        const uint32_t si1 = (uint32_t)(s03 >> (8 * i1)), si2 = (uint32_t)(s03 >> (8 * (i1 + 1)));
        const uint32_t ti1 = (uint32_t)(s47 >> (8 * i1)), ti2 = (uint32_t)(s47 >> (8 * (i1 + 1)));
        const uint32_t ui1 = (uint32_t)(s811 >> (8 * i1)), ui2 = (uint32_t)(s811 >> (8 * (i1 + 1)));
        sc1 = (int)(((si1 >> 6) & 3) | ((ui1 & 0xF) << 2));
        sc2 = (int)(((si2 >> 6) & 3) | ((ui2 & 0xF) << 2));
        mn1 = (int)(((ti1 >> 6) & 3) | (((ui1 >> 4) & 0xF) << 2));
        mn2 = (int)(((ti2 >> 6) & 3) | (((ui2 >> 4) & 0xF) << 2));
    }
}

template <int R>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_q4k_kernel(const uint8_t* __restrict__ W,
                                                                int n, int nsb,
                                                                const FloatRec* __restrict__ X,
                                                                float* __restrict__ Y) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * WAVES + (threadIdx.x >> 6);
    const int row0 = wave * R;
    if (row0 >= n) return;
    const int nunits = nsb * 4;
    const FloatRec* xr = X + (size_t)blockIdx.y * nsb * 8;
    float* yr = Y + (size_t)blockIdx.y * n;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    for (int u = lane; u < nunits; u += 64) {
        const int sb = u >> 2, c = u & 3;
        u32x4 hdr[R], qa[R], qb[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(row0 + r, n - 1);
            const uint8_t* p = W + ((size_t)row * nsb + sb) * Q4_K_BYTES;
            hdr[r] = *reinterpret_cast<const u32x4*>(p);
            qa[r] = *reinterpret_cast<const u32x4*>(p + 16 + 32 * c);
            qb[r] = *reinterpret_cast<const u32x4*>(p + 32 + 32 * c);
        }
        const XF x1 = load_xf(xr + sb * 8 + 2 * c);
        const XF x2 = load_xf(xr + sb * 8 + 2 * c + 1);
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t lo[8], hi[8];
            const uint32_t raw[8] = {qa[r].x, qa[r].y, qa[r].z, qa[r].w,
                                     qb[r].x, qb[r].y, qb[r].z, qb[r].w};
#pragma unroll
            for (int k = 0; k < 8; k++) {
                lo[k] = raw[k] & NIB;
                hi[k] = (raw[k] >> 4) & NIB;
            }
            const float d = h2f(hdr[r].x & 0xFFFFu);
            const float dmin = h2f(hdr[r].x >> 16);
            int sc1, mn1, sc2, mn2;
            q4k_scale_min(hdr[r], c, sc1, mn1, sc2, mn2);
            // reference element: (d*sc)*q - (dmin*mn)   (parser.rs:577-587)
            const float d1 = d * (float)sc1, m1 = dmin * (float)mn1;
            const float d2 = d * (float)sc2, m2 = dmin * (float)mn2;
            float a = acc[r];
            a = fmaf(d1 * x1.S, dot3(lo, x1, 0, 0, 0), a);
            a = fmaf(-m1, x1.xsum, a);
            a = fmaf(d2 * x2.S, dot3(hi, x2, 0, 0, 0), a);
            a = fmaf(-m2, x2.xsum, a);
            acc[r] = a;
        }
    }
    store_rows<R>(acc, lane, row0, n, yr);
}

// Q6_K float mode.  A unit is one 32-element column of a super-block (the
// Q6KUnit layout); lane l owns units l, l+64, ...
template <int R>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_q6k_kernel(const uint8_t* __restrict__ W,
                                                                int n, int nsb,
                                                                const FloatRec* __restrict__ X,
                                                                float* __restrict__ Y) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * WAVES + (threadIdx.x >> 6);
    const int row0 = wave * R;
    if (row0 >= n) return;
    const int nunits = nsb * 8;
    const FloatRec* xr = X + (size_t)blockIdx.y * nunits;
    float* yr = Y + (size_t)blockIdx.y * n;
    const size_t row_bytes = (size_t)nsb * Q6_K_BYTES;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    for (int u = lane; u < nunits; u += 64) {
        const XF x = load_xf(xr + u);
        int off[6];
        q6k_offsets(x, off);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(row0 + r, n - 1);
            // block offsets fit 32 bits: the launcher bounds the matrix below 2 GiB
            const Q6KUnit g = q6k_unit((uint32_t)(row * row_bytes + (size_t)(u >> 3) * Q6_K_BYTES), u & 7);
            uint32_t wl[9], wh[9];
            const u32x4a4* pl = reinterpret_cast<const u32x4a4*>(W + (g.ql & ~3u));
            const u32x4a4* ph = reinterpret_cast<const u32x4a4*>(W + (g.qh & ~3u));
            const u32x4a4 l0 = pl[0], l1 = pl[1], h0 = ph[0], h1 = ph[1];
            wl[0] = l0.x; wl[1] = l0.y; wl[2] = l0.z; wl[3] = l0.w;
            wl[4] = l1.x; wl[5] = l1.y; wl[6] = l1.z; wl[7] = l1.w;
            wh[0] = h0.x; wh[1] = h0.y; wh[2] = h0.z; wh[3] = h0.w;
            wh[4] = h1.x; wh[5] = h1.y; wh[6] = h1.z; wh[7] = h1.w;
            // the ninth dword stays inside the block (the runs end at or before byte 192)
            wl[8] = *reinterpret_cast<const uint32_t*>(W + (g.ql & ~3u) + 32);
            wh[8] = *reinterpret_cast<const uint32_t*>(W + (g.qh & ~3u) + 32);
            uint32_t q[8];
            q6k_codes(wl, wh, q6k_sel(g.ql), g.t, q);
            const uint32_t scw = *reinterpret_cast<const uint16_t*>(W + g.sc);
            const float d = h2f(*reinterpret_cast<const uint16_t*>(W + g.d));
            const float f = q6k_dot(q, x, off, (int)(int8_t)(scw & 0xFF), (int)(int8_t)(scw >> 8));
            acc[r] = fmaf(d * x.S, f, acc[r]);
        }
    }
    store_rows<R>(acc, lane, row0, n, yr);
}

// int32 block partials of the native Q4_0 path, one thread per (row, block).
__global__ __launch_bounds__(256) void q4_0_block_dots_kernel(const uint8_t* __restrict__ W,
                                                              int n, int nb,
                                                              const NativeRec* __restrict__ X,
                                                              int32_t* __restrict__ P) {
    const size_t gid = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (size_t)n * nb) return;
    const int col = (int)(gid % nb);
    Win5 b;
    load_win5(W, gid * Q4_0_BYTES, (size_t)n * nb * Q4_0_BYTES, b);
    uint32_t q[8];
    float d;
    q4_0_unpack(b, q, d);
    const XN x = load_xn(X + col);
    P[gid] = dot1(q, x, -8 * x.qsum);
}

// Tensor::to_f32 rows (tensor.rs:535-639), dequantize_q4k (parser.rs:549-593) and
// dequantize_q6k (parser.rs:510-547): one thread per 32 elements (for Q4_K one
// of the eight sub-blocks of a super-block, for Q6_K one of its eight columns).
// Every product below is exact in f32 (f16 scale x 4- or 6-bit integer; for
// Q6_K f16 x int8 x 6-bit code, at most 24 significant bits), so each output
// has the reference's single rounding.
template <int WT>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t* __restrict__ W,
                                                           int nb, const int32_t* __restrict__ rows,
                                                           int n_rows, float* __restrict__ out) {
    const size_t gid = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (size_t)n_rows * nb) return;
    const int r = (int)(gid / nb), b = (int)(gid % nb);
    const size_t g = (size_t)rows[r] * nb + b;
    float* o = out + gid * QK;
    if (WT == (int)WType::Q6_K) {
        // column j of super-block g / 8 (parser.rs:525-541): (d * scale) * (code - 32)
        const uint8_t* p = W + (g / 8) * Q6_K_BYTES;
        const int j = (int)(g % 8), half = j >> 2, t = j & 3;
        const float d = h2f(p[208] | (p[209] << 8));
        const uint8_t* ql = p + 64 * half + 32 * (t & 1);
        const uint8_t* qh = p + 128 + 32 * half;
        const int8_t* sc = reinterpret_cast<const int8_t*>(p + 192 + 8 * half + 2 * t);
        for (int l = 0; l < 32; l++) {
            const int code = ((ql[l] >> (4 * (t >> 1))) & 0xF) | (((qh[l] >> (2 * t)) & 3) << 4);
            o[l] = d * (float)sc[l >> 4] * (float)(code - 32);
        }
    } else if (WT == (int)WType::Q4_K) {
        // sub-block j of super-block g / 8: chunk c = j / 2 of the nibble bytes,
        // low nibbles for even j, high for odd (parser.rs:571-590)
        const uint8_t* p = W + (g / 8) * Q4_K_BYTES;
        const int j = (int)(g % 8);
        const float d = h2f(p[0] | (p[1] << 8)), dmin = h2f(p[2] | (p[3] << 8));
        const uint8_t* sb = p + 4;
        int sc, mn;  // parser.rs:562-569
        if (j < 4) {
            sc = sb[j] & 63;
            mn = sb[j + 4] & 63;
        } else {
            sc = (sb[j - 4] >> 6) | ((sb[j + 4] & 0xF) << 2);
            mn = (sb[j] >> 6) | ((sb[j + 4] >> 4) << 2);
        }
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        const uint8_t* q = p + 16 + 32 * (j >> 1);
        const int sh = (j & 1) * 4;
        for (int l = 0; l < 32; l++) o[l] = d1 * (float)((q[l] >> sh) & 0xF) - m1;
    } else if (WT == (int)WType::Q8_0) {
        const uint8_t* p = W + g * Q8_0_BYTES;
        const float s = h2f(p[0] | (p[1] << 8));
        for (int j = 0; j < 32; j++) o[j] = s * (float)(int8_t)p[2 + j];
    } else if (WT == (int)WType::Q4_1) {
        const uint8_t* p = W + g * Q4_1_BYTES;
        const float d = h2f(p[0] | (p[1] << 8)), m = h2f(p[2] | (p[3] << 8));
        for (int j = 0; j < 16; j++) {
            const uint8_t v = p[4 + j];
            o[j] = d * (float)(v & 0x0F) + m;
            o[j + 16] = d * (float)(v >> 4) + m;
        }
    } else {
        const uint8_t* p = W + g * Q4_0_BYTES;
        const float s = h2f(p[0] | (p[1] << 8));
        for (int j = 0; j < 16; j++) {
            const uint8_t v = p[2 + j];
            o[j] = s * (float)((int)(v & 0x0F) - 8);
            o[j + 16] = s * (float)((int)(v >> 4) - 8);
        }
    }
}

// Rows per wave: enough waves to cover every SIMD about twice, at most 8 rows.
int pick_rows(size_t n) {
    const size_t target_waves = 2048;
    size_t r = n / target_waves;
    if (r >= 8) return 8;
    if (r >= 4) return 4;
    if (r >= 2) return 2;
    return 1;
}

template <int R>
hipError_t launch_r(WType t, bool native, const uint8_t* w, size_t n, size_t k, const void* xrec,
                    size_t m, float* y, hipStream_t s) {
    const size_t waves = (n + R - 1) / R;
    const dim3 grid((unsigned)((waves + WAVES - 1) / WAVES), (unsigned)m);
    const dim3 block(GEMV_THREADS);
    const int ni = (int)n;
    if (t == WType::Q4_K) {
        launch_kernel((gemv_q4k_kernel<R>), grid, block, 0, s, w, ni, (int)(k / QK_K),
                           (const FloatRec*)xrec, y);
        return hipGetLastError();
    }
    if (t == WType::Q6_K) {
        if ((uint64_t)n * (k / QK_K) * Q6_K_BYTES >= ((uint64_t)1 << 32)) return hipErrorInvalidValue;
        launch_kernel((gemv_q6k_kernel<R>), grid, block, 0, s, w, ni, (int)(k / QK_K),
                           (const FloatRec*)xrec, y);
        return hipGetLastError();
    }
    const int nb = (int)(k / QK);
    if (native && t == WType::Q4_0) {
        launch_kernel((gemv_native_kernel<R, (int)WType::Q4_0>), grid, block, 0, s, w, ni, nb,
                           (const NativeRec*)xrec, y);
    } else if (native && t == WType::Q4_1) {
        launch_kernel((gemv_native_kernel<R, (int)WType::Q4_1>), grid, block, 0, s, w, ni, nb,
                           (const NativeRec*)xrec, y);
    } else if (t == WType::Q4_0) {
        launch_kernel((gemv_float_kernel<R, (int)WType::Q4_0>), grid, block, 0, s, w, ni, nb,
                           (const FloatRec*)xrec, y);
    } else if (t == WType::Q4_1) {
        launch_kernel((gemv_float_kernel<R, (int)WType::Q4_1>), grid, block, 0, s, w, ni, nb,
                           (const FloatRec*)xrec, y);
    } else {
        launch_kernel((gemv_float_kernel<R, (int)WType::Q8_0>), grid, block, 0, s, w, ni, nb,
                           (const FloatRec*)xrec, y);
    }
    return hipGetLastError();
}

// y[i][j] += bias[j] over m rows of n: Linear::forward's output.add(bias)
// (linear.rs:172-176), one f32 add an element.
__global__ __launch_bounds__(256) void bias_add_kernel(float* __restrict__ y, const float* __restrict__ bias,
                                                       uint32_t n, uint32_t total) {
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) y[i] += bias[i % n];
}

}  // namespace

hipError_t launch_gemv(WType t, bool native, const uint8_t* w, size_t n, size_t k,
                       const void* xrec, size_t m, float* y, hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    switch (pick_rows(n)) {
        case 8: return launch_r<8>(t, native, w, n, k, xrec, m, y, s);
        case 4: return launch_r<4>(t, native, w, n, k, xrec, m, y, s);
        case 2: return launch_r<2>(t, native, w, n, k, xrec, m, y, s);
        default: return launch_r<1>(t, native, w, n, k, xrec, m, y, s);
    }
}

hipError_t launch_q4_0_block_dots(const uint8_t* w, size_t n, size_t k, const NativeRec* rec,
                                  int32_t* partials, hipStream_t s) {
    const size_t total = n * (k / QK);
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(q4_0_block_dots_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       s, w, (int)n, (int)(k / QK), rec, partials);
    return hipGetLastError();
}

hipError_t launch_bias_add(float* y, const float* bias, size_t m, size_t n, hipStream_t s) {
    const size_t total = m * n;
    if (total == 0) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(bias_add_kernel, dim3(blocks), dim3(256), 0, s, y, bias, (uint32_t)n, (uint32_t)total);
    return hipGetLastError();
}

hipError_t launch_dequant_rows(WType t, const uint8_t* w, size_t n, size_t k, const int32_t* rows,
                               size_t n_rows, float* out, hipStream_t s) {
    (void)n;
    const size_t total = n_rows * (k / QK);
    if (total == 0) return hipSuccess;
    const dim3 grid((unsigned)((total + 255) / 256));
    const int nb = (int)(k / QK);
    if (t == WType::Q4_K)
        hipLaunchKernelGGL((dequant_rows_kernel<(int)WType::Q4_K>), grid, dim3(256), 0, s, w, nb,
                           rows, (int)n_rows, out);
    else if (t == WType::Q6_K)
        hipLaunchKernelGGL((dequant_rows_kernel<(int)WType::Q6_K>), grid, dim3(256), 0, s, w, nb,
                           rows, (int)n_rows, out);
    else if (t == WType::Q8_0)
        hipLaunchKernelGGL((dequant_rows_kernel<(int)WType::Q8_0>), grid, dim3(256), 0, s, w, nb,
                           rows, (int)n_rows, out);
    else if (t == WType::Q4_1)
        hipLaunchKernelGGL((dequant_rows_kernel<(int)WType::Q4_1>), grid, dim3(256), 0, s, w, nb,
                           rows, (int)n_rows, out);
    else
        hipLaunchKernelGGL((dequant_rows_kernel<(int)WType::Q4_0>), grid, dim3(256), 0, s, w, nb,
                           rows, (int)n_rows, out);
    return hipGetLastError();
}

}  // namespace rdl
