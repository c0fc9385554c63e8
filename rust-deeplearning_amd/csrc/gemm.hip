// gemm.hip -- prefill GEMM for GGUF Q4_0 weights on the gfx950 matrix cores:
// Y[m, n] = X[m, k] . W[n, k]^T, the many-token case of matmul_f32_q4
// (quantize.rs:265-320; one f32 block dot per (row, column, block), summed
// over the blocks) and of matmul_f32_q4_native (quantize.rs:326-394; exact
// int32 block dots of the Q8_0-quantized x, times both block scales).
//
// Numerics.  One MFMA K step (16x16x32) is one 32-element block, so each
// block's dot leaves the matrix cores whole and the block scale d is applied
// in f32 afterwards; the weight operand is the exact (q - 8).
//  * float: each x row is scaled by a power of two 2^-e (row max ->
//    [2^14, 2^15)) and split into x_hi = f16(x') and x_lo = f16(x' - x_hi)
//    (about 22 significant bits together); per block two f16 MFMAs (x_hi,
//    x_lo) with f32 accumulation give the block dot, acc += d * dot, and
//    y = 2^e * acc;
//  * native: x is quantize_row_q8_0's int8 codes; per block one int8 MFMA
//    gives the exact int32 dot_q4q8_block (simd.rs:562-581) and
//    acc += (float)dot * (s_x * d).
//
// Operand layouts of v_mfma_f32_16x16x32_f16 / v_mfma_i32_16x16x32_i8 (checked
// on gfx950): lane l holds A[l % 16][8 (l / 16) .. +7] and
// B[8 (l / 16) .. +7][l % 16]; the result C[4 (l / 16) + t][l % 16], t < 4.
// A rows are weight rows j, B columns are x rows i, so a lane ends with
// y[i][j .. j+3] for one i.
//
// Tiling: a workgroup of WJ x WI x KS waves owns a TJ x TI output tile
// (TJ = WJ * FJ * 16 weight rows, TI = WI * FI * 16 x rows); the KS waves of
// one (wj, wi) split each chunk's blocks and their sums are added at the end.
// Chunks of CB = KB * KS blocks are staged into LDS, double-buffered: Q4_0
// blocks realigned to 16 nibble bytes + their f16 d, and the x tiles (f16
// hi / lo, or int8 codes + f32 scales); all global loads are raw buffer
// loads whose out-of-range slots (rows past n or m, blocks past nb) read zeros.
#include <algorithm>
#include <type_traits>

#include "rdl_device.hpp"
#include "rdl_internal.hpp"

namespace rdl {

namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---- x preparation: per-row power-of-two scale, f16 hi / lo split ---------------
constexpr int XPREP_THREADS = 256;

__global__ __launch_bounds__(XPREP_THREADS) void gemm_xprep_kernel(const float* __restrict__ X, int k,
                                                                   _Float16* __restrict__ XH,
                                                                   _Float16* __restrict__ XL,
                                                                   int* __restrict__ XE) {
    __shared__ float red[XPREP_THREADS / 64];
    const int row = blockIdx.x;
    const float* x = X + (size_t)row * k;
    float amax = 0.0f;
    bool bad = false;
    for (int c = threadIdx.x; c < k; c += XPREP_THREADS) {
        const float v = x[c];
        bad |= !isfinite(v);
        amax = fmaxf(amax, fabsf(v));
    }
    if (bad) amax = __builtin_inff();
    // wave max, then across the four waves
    amax = max8_f32(amax);
    amax = fmaxf(amax, dpp_f32<DPP_ROW_MIRROR>(amax));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // e: amax * 2^-e in [2^14, 2^15); non-finite or zero rows keep e = 0
    int e = 0;
    if (amax > 0.0f && isfinite(amax)) e = ilogbf(amax) - 14;
    if (threadIdx.x == 0) XE[row] = e;
    for (int c = threadIdx.x; c < k; c += XPREP_THREADS) {
        const float v = ldexpf(x[c], -e);
        const _Float16 h = (_Float16)v;
        XH[(size_t)row * k + c] = h;
        XL[(size_t)row * k + c] = (_Float16)(v - (float)h);
    }
}

// The same split with each row's values held in registers between the max
// and the conversion (k <= 4 * 4 * XPREP_FAST_THREADS): one global read.
constexpr int XPREP_FAST_THREADS = 1024;
__global__ __launch_bounds__(XPREP_FAST_THREADS) void gemm_xprep_fast_kernel(const float* __restrict__ X, int k,
                                                                             _Float16* __restrict__ XH,
                                                                             _Float16* __restrict__ XL,
                                                                             int* __restrict__ XE) {
    constexpr int NT = XPREP_FAST_THREADS, NV = 4;
    __shared__ float red[NT / 64];
    const int row = blockIdx.x;
    const float* x = X + (size_t)row * k;
    f32x4 v[NV];
    const int k4 = k >> 2;  // k % 32 == 0
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int p = threadIdx.x + j * NT;
        v[j] = p < k4 ? reinterpret_cast<const f32x4*>(x)[p] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    float amax = 0.0f;
    bool bad = false;
#pragma unroll
    for (int j = 0; j < NV; j++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
            bad |= !isfinite(v[j][t]);
            amax = fmaxf(amax, fabsf(v[j][t]));
        }
    if (bad) amax = __builtin_inff();
    amax = max8_f32(amax);
    amax = fmaxf(amax, dpp_f32<DPP_ROW_MIRROR>(amax));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) amax = fmaxf(amax, red[w]);
    // e: amax * 2^-e in [2^14, 2^15); non-finite or zero rows keep e = 0
    int e = 0;
    if (amax > 0.0f && isfinite(amax)) e = ilogbf(amax) - 14;
    if (threadIdx.x == 0) XE[row] = e;
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int p = threadIdx.x + j * NT;
        if (p < k4) {
            h4 hv, lv;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const float s = ldexpf(v[j][t], -e);
                hv[t] = (_Float16)s;
                lv[t] = (_Float16)(s - (float)hv[t]);
            }
            reinterpret_cast<h4*>(XH + (size_t)row * k)[p] = hv;
            reinterpret_cast<h4*>(XL + (size_t)row * k)[p] = lv;
        }
    }
}

// ---- GEMM ------------------------------------------------------------------------
// LDS row strides, padded so that the 16 rows a fragment read touches fall in
// distinct banks: nibble rows CB*16 + 8 bytes; x rows CB*64 + 16 bytes (f16)
// or CB*32 + 16 bytes (int8 codes).
template <int CB> struct Lds {
    static constexpr int WN_STRIDE = CB * 16 + 8;   // bytes per weight row (nibbles)
    static constexpr int X_STRIDE = CB * 64 + 16;   // bytes per x row (f16 x CB*32)
    static constexpr int XC_STRIDE = CB * 32 + 16;  // bytes per x row (int8 codes)
};

// 8 nibbles (two dwords of four) of a weight row as (q - 8): exact f16 values
// for the float product, signed bytes for the native one.
__device__ __forceinline__ half8_t q_f16(uint32_t n0, uint32_t n1) {
    const half2_t off = {(_Float16)1032.0f, (_Float16)1032.0f};
    constexpr uint32_t MAGIC = 0x64646464u;  // f16 0x64XX = 1024 + XX for XX < 16
    const half2_t q0 = __builtin_bit_cast(half2_t, perm(MAGIC, n0, 0x04010400u)) - off;
    const half2_t q1 = __builtin_bit_cast(half2_t, perm(MAGIC, n0, 0x04030402u)) - off;
    const half2_t q2 = __builtin_bit_cast(half2_t, perm(MAGIC, n1, 0x04010400u)) - off;
    const half2_t q3 = __builtin_bit_cast(half2_t, perm(MAGIC, n1, 0x04030402u)) - off;
    return half8_t{q0[0], q0[1], q1[0], q1[1], q2[0], q2[1], q3[0], q3[1]};
}
__device__ __forceinline__ long q_i8(uint32_t n0, uint32_t n1) {
    // per byte: (q + 128 - 8) ^ 128 = q - 8 as a signed byte, no borrow across bytes
    const uint32_t a = ((n0 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
    const uint32_t b = ((n1 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
    return (long)(((uint64_t)b << 32) | a);
}

template <bool NATIVE, int FJ, int FI, int WJ, int WI, int KS, int KB>
struct GemmCfg {
    static constexpr int NW = WJ * WI * KS;
    static constexpr int NT = NW * 64;
    static constexpr int TJ = WJ * FJ * 16;
    static constexpr int TI = WI * FI * 16;
    static constexpr int CB = KB * KS;                      // blocks per chunk
    static constexpr int WN_BYTES = TJ * Lds<CB>::WN_STRIDE;
    static constexpr int WD_BYTES = (TJ * CB * 2 + 15) & ~15;
    // float: x_hi and x_lo tiles; native: int8 codes and the f32 block scales
    static constexpr int X_BYTES = TI * (NATIVE ? Lds<CB>::XC_STRIDE : Lds<CB>::X_STRIDE);
    static constexpr int XS_BYTES = NATIVE ? TI * CB * 4 : 0;
    static constexpr int STAGE = WN_BYTES + WD_BYTES + (NATIVE ? X_BYTES + XS_BYTES : 2 * X_BYTES);
    static constexpr int STAGE_AL = (STAGE + 15) & ~15;
    static constexpr int WBLK = (TJ * CB + NT - 1) / NT;                          // weight blocks per thread
    static constexpr int XU = (TI * CB * (NATIVE ? 2 : 4) + NT - 1) / NT;          // 16-byte x units per thread
    static constexpr int XSU = NATIVE ? (TI * CB + NT - 1) / NT : 0;              // scale dwords per thread
    static constexpr int RED = (KS > 1) ? (KS - 1) * WJ * WI * FJ * FI * 64 * 16 : 0;
    // two staging buffers; the K-split sums reuse the same LDS at the end
    static constexpr int LDS = (2 * STAGE_AL > RED) ? 2 * STAGE_AL : RED;
};

// One chunk's global loads, held in registers until they are written to LDS.
template <int WBLK, int XU, int XSU>
struct Staged {
    uint32_t w[WBLK][5];
    u32x4 x0[XU], x1[XU];       // float: x_hi, x_lo; native: codes (x1 unused)
    uint32_t xs[XSU > 0 ? XSU : 1];
};

// Tile order: workgroups are dealt to the 8 XCDs round-robin (linear id % 8);
// give each XCD a contiguous run of tiles in row-major tile order, so the
// workgroups that share x rows share one L2.
__device__ __forceinline__ void tile_of(int nj, int ni, int& bx, int& by) {
    const int total = nj * ni, L = blockIdx.x;
    const int t = (total % 8 == 0) ? (L % 8) * (total / 8) + L / 8 : L;
    bx = t % nj;
    by = t / nj;
}

// NATIVE = false: X0 / X1 = x_hi / x_lo (f16 [m, k]), XE the row exponents.
// NATIVE = true:  X0 = Q8_0 codes (int8 [m, k]), X1 = their f32 block scales
// [m, nb] (quantize_row_q8_0); DUMP writes the int32 block dots to
// P[(i * n + j) * nb + b] instead of forming Y.
template <bool NATIVE, bool DUMP, int FJ, int FI, int WJ, int WI, int KS, int KB>
__global__ __launch_bounds__(WJ * WI * KS * 64) void gemm_q4_0_kernel(
    const uint8_t* __restrict__ W, int n, int nb, const void* __restrict__ X0, const void* __restrict__ X1,
    const int* __restrict__ XE, int m, float* __restrict__ Y, int32_t* __restrict__ P) {
    using C = GemmCfg<NATIVE, FJ, FI, WJ, WI, KS, KB>;
    constexpr int CB = C::CB;
    constexpr int XSTR = NATIVE ? Lds<CB>::XC_STRIDE : Lds<CB>::X_STRIDE;
    using S = Staged<C::WBLK, C::XU, C::XSU>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int ks = wave % KS;
    const int wi = (wave / KS) % WI;
    const int wj = wave / (KS * WI);
    int bx, by;
    tile_of((n + C::TJ - 1) / C::TJ, (m + C::TI - 1) / C::TI, bx, by);
    const int j0 = bx * C::TJ;
    const int i0 = by * C::TI;
    const int k = nb * 32;
    const uint32_t row_bytes = (uint32_t)nb * 18u;
    const uint32_t wbytes = (uint32_t)n * row_bytes;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(W, wbytes);
    const uint32_t xbytes = (uint32_t)m * (uint32_t)k * (NATIVE ? 1u : 2u);
    const __amdgpu_buffer_rsrc_t x0rs = make_rsrc(X0, xbytes);
    const __amdgpu_buffer_rsrc_t x1rs = make_rsrc(X1, NATIVE ? (uint32_t)m * (uint32_t)nb * 4u : xbytes);
    const int nchunks = (nb + CB - 1) / CB;

    // live == false (a chunk past the end) loads nothing through out-of-range
    // offsets: the loads are issued on every iteration, so the compiler's
    // wait counts before the LDS stores stay exact (no branch around them).
    auto load_chunk = [&](int c, S& r, bool live) {
#pragma unroll
        for (int u = 0; u < C::WBLK; u++) {
            const int idx = threadIdx.x + u * C::NT;
            const int jl = idx / CB, bl = idx % CB;
            const int j = j0 + jl, b = c * CB + bl;
            const uint32_t off = (live && idx < C::TJ * CB && j < n && b < nb)
                                     ? (uint32_t)j * row_bytes + (uint32_t)b * 18u
                                     : RSRC_OOB;
            const uint32_t base = off & ~3u;
            const u32x4 v = buf_load_b128(wrs, base);
            r.w[u][0] = v.x; r.w[u][1] = v.y; r.w[u][2] = v.z; r.w[u][3] = v.w;
            // the last block of an odd-sized matrix ends 2 bytes before its
            // window: its tail dword is read 2 bytes early and shifted when the
            // block is stored (not here: that would wait for the load now)
            const bool over = base < wbytes && base + 20u > wbytes;
            r.w[u][4] = buf_load_b32(wrs, over ? wbytes - 4u : base + 16u);
        }
        constexpr int UPR = CB * (NATIVE ? 2 : 4);  // 16-byte units per x row and chunk
#pragma unroll
        for (int u = 0; u < C::XU; u++) {
            const int idx = threadIdx.x + u * C::NT;
            const int il = idx / UPR, q = idx % UPR;
            const int i = i0 + il;
            const uint32_t kk = (uint32_t)c * CB * 32u + (uint32_t)q * (NATIVE ? 16u : 8u);  // element
            const uint32_t off = (live && idx < C::TI * UPR && i < m && kk < (uint32_t)k)
                                     ? ((uint32_t)i * (uint32_t)k + kk) * (NATIVE ? 1u : 2u)
                                     : RSRC_OOB;
            r.x0[u] = buf_load_b128(x0rs, off);
            if constexpr (!NATIVE) r.x1[u] = buf_load_b128(x1rs, off);
        }
        if constexpr (NATIVE) {
#pragma unroll
            for (int u = 0; u < C::XSU; u++) {
                const int idx = threadIdx.x + u * C::NT;
                const int il = idx / CB, bl = idx % CB;
                const int i = i0 + il, b = c * CB + bl;
                const uint32_t off = (live && idx < C::TI * CB && i < m && b < nb)
                                         ? ((uint32_t)i * (uint32_t)nb + (uint32_t)b) * 4u
                                         : RSRC_OOB;
                r.xs[u] = buf_load_b32(x1rs, off);
            }
        }
    };
    auto store_chunk = [&](int c, int buf, const S& r) {
        uint8_t* st = lds + buf * C::STAGE_AL;
        uint8_t* wn = st;
        uint16_t* wd = reinterpret_cast<uint16_t*>(st + C::WN_BYTES);
        uint8_t* x0s = st + C::WN_BYTES + C::WD_BYTES;
        uint8_t* x1s = x0s + C::X_BYTES;
#pragma unroll
        for (int u = 0; u < C::WBLK; u++) {
            const int idx = threadIdx.x + u * C::NT;
            if (idx < C::TJ * CB) {
                const int jl = idx / CB, bl = idx % CB;
                const int j = j0 + jl, b = c * CB + bl;
                const uint32_t off = (j < n && b < nb) ? (uint32_t)j * row_bytes + (uint32_t)b * 18u : RSRC_OOB;
                const uint32_t base = off & ~3u;
                const uint32_t w4 = (base < wbytes && base + 20u > wbytes) ? (r.w[u][4] >> 16) : r.w[u][4];
                // block g = j * nb + b starts at 18 g: 2 bytes past a dword when g is odd
                const bool odd = (((uint32_t)j * (uint32_t)nb + (uint32_t)b) & 1u) != 0;
                const uint32_t sel = odd ? 0x07060504u : 0x05040302u;
                const uint32_t dbits = odd ? (r.w[u][0] >> 16) : (r.w[u][0] & 0xFFFFu);
                // rows are 8-byte aligned (padded stride): two 8-byte stores
                uint2 lo, hi;
                lo.x = perm(r.w[u][1], r.w[u][0], sel);
                lo.y = perm(r.w[u][2], r.w[u][1], sel);
                hi.x = perm(r.w[u][3], r.w[u][2], sel);
                hi.y = perm(w4, r.w[u][3], sel);
                uint2* dst = reinterpret_cast<uint2*>(wn + jl * Lds<CB>::WN_STRIDE + bl * 16);
                dst[0] = lo;
                dst[1] = hi;
                wd[bl * C::TJ + jl] = (uint16_t)dbits;  // block-major: a lane's four rows are adjacent
            }
        }
        constexpr int UPR = CB * (NATIVE ? 2 : 4);
#pragma unroll
        for (int u = 0; u < C::XU; u++) {
            const int idx = threadIdx.x + u * C::NT;
            if (idx < C::TI * UPR) {
                const int il = idx / UPR, q = idx % UPR;
                *reinterpret_cast<u32x4*>(x0s + il * XSTR + q * 16) = r.x0[u];
                if constexpr (!NATIVE) *reinterpret_cast<u32x4*>(x1s + il * XSTR + q * 16) = r.x1[u];
            }
        }
        if constexpr (NATIVE) {
            uint32_t* xs = reinterpret_cast<uint32_t*>(x1s);
#pragma unroll
            for (int u = 0; u < C::XSU; u++) {
                const int idx = threadIdx.x + u * C::NT;
                if (idx < C::TI * CB) xs[(idx % CB) * C::TI + idx / CB] = r.xs[u];
            }
        }
    };

    f32x4 acc[FJ][FI];
#pragma unroll
    for (int a = 0; a < FJ; a++)
#pragma unroll
        for (int b = 0; b < FI; b++) acc[a][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int g = lane >> 4, r16 = lane & 15;
    // One MFMA K step is one Q4_0 block (32 elements): the block's dot comes
    // out whole and its scale d multiplies it in f32 (d need not fit f16).
    // Lane l holds A[l % 16][8 (l / 16) .. +7] (weight row, elements 8g..8g+7),
    // B[8 (l / 16) .. +7][l % 16] (x row) and C[4 (l / 16) + t][l % 16]: the
    // products of four weight rows 4g + t with one x row.
    auto compute_chunk = [&](int c, int buf) {
        const uint8_t* st = lds + buf * C::STAGE_AL;
        const uint8_t* wn = st;
        const uint16_t* wd = reinterpret_cast<const uint16_t*>(st + C::WN_BYTES);
        const uint8_t* x0s = st + C::WN_BYTES + C::WD_BYTES;
        const uint8_t* x1s = x0s + C::X_BYTES;
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const int bl = ks * KB + kb;  // this wave's block within the chunk
            typename std::conditional<NATIVE, long, half8_t>::type aq[FJ];
            f32x4 dv[FJ];
#pragma unroll
            for (int a = 0; a < FJ; a++) {
                const int jt = (wj * FJ + a) * 16;
                const uint2 nb8 = *reinterpret_cast<const uint2*>(wn + (jt + r16) * Lds<CB>::WN_STRIDE +
                                                                  bl * 16 + 8 * (g & 1));
                const uint32_t sh = (g >> 1) * 4;  // groups 2, 3: high nibbles
                const uint32_t n0 = (nb8.x >> sh) & 0x0F0F0F0Fu, n1 = (nb8.y >> sh) & 0x0F0F0F0Fu;
                if constexpr (NATIVE) aq[a] = q_i8(n0, n1);
                else aq[a] = q_f16(n0, n1);
                const uint2 dd = *reinterpret_cast<const uint2*>(wd + bl * C::TJ + jt + 4 * g);
                dv[a] = f32x4{h2f(dd.x & 0xFFFFu), h2f(dd.x >> 16), h2f(dd.y & 0xFFFFu), h2f(dd.y >> 16)};
            }
#pragma unroll
            for (int b = 0; b < FI; b++) {
                const int il = (wi * FI + b) * 16 + r16;
                if constexpr (NATIVE) {
                    const long bx = *reinterpret_cast<const long*>(x0s + il * XSTR + bl * 32 + g * 8);
                    const float sx = reinterpret_cast<const float*>(x1s)[bl * C::TI + il];
#pragma unroll
                    for (int a = 0; a < FJ; a++) {
                        typedef int i32x4_t __attribute__((ext_vector_type(4)));
                        const i32x4_t z = {0, 0, 0, 0};
                        const i32x4_t cv = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq[a], bx, z, 0, 0, 0);
                        if constexpr (DUMP) {
                            const int i = i0 + il, bg = c * CB + bl;
                            if (i < m && bg < nb) {
#pragma unroll
                                for (int t = 0; t < 4; t++) {
                                    const int j = j0 + (wj * FJ + a) * 16 + 4 * g + t;
                                    if (j < n) P[((size_t)i * n + j) * nb + bg] = cv[t];
                                }
                            }
                        } else {
                            // (int dot as f32) * (sx * d), summed over the blocks
#pragma unroll
                            for (int t = 0; t < 4; t++) acc[a][b][t] = fmaf((float)cv[t], sx * dv[a][t], acc[a][b][t]);
                        }
                    }
                } else {
                    const int xo = il * XSTR + bl * 64 + g * 16;
                    const half8_t bh = *reinterpret_cast<const half8_t*>(x0s + xo);
                    const half8_t bl8 = *reinterpret_cast<const half8_t*>(x1s + xo);
#pragma unroll
                    for (int a = 0; a < FJ; a++) {
                        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                        f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[a], bh, z, 0, 0, 0);
                        t = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[a], bl8, t, 0, 0, 0);
#pragma unroll
                        for (int u = 0; u < 4; u++) acc[a][b][u] = fmaf(dv[a][u], t[u], acc[a][b][u]);
                    }
                }
            }
        }
    };

    // Loads run two chunks ahead of the compute: register set P holds chunk
    // c + 2 while LDS buffer 1 - P receives chunk c + 1.
    S r0, r1;
    load_chunk(0, r0, true);
    load_chunk(1, r1, nchunks > 1);
    store_chunk(0, 0, r0);
    __syncthreads();
    for (int c = 0; c < nchunks; c += 2) {
        load_chunk(c + 2, r0, c + 2 < nchunks);
        compute_chunk(c, 0);
        if (c + 1 < nchunks) store_chunk(c + 1, 1, r1);
        __syncthreads();
        if (c + 1 >= nchunks) break;
        load_chunk(c + 3, r1, c + 3 < nchunks);
        compute_chunk(c + 1, 1);
        if (c + 2 < nchunks) store_chunk(c + 2, 0, r0);
        __syncthreads();
    }
    if constexpr (DUMP) return;

    // ---- K-split sums (waves ks > 0 hand their partials to ks == 0) ----
    if constexpr (KS > 1) {
        float* red = reinterpret_cast<float*>(lds);  // staging buffers are free now
        const int slot = wave / KS;                  // (wj, wi) pair
        if (ks > 0) {
#pragma unroll
            for (int a = 0; a < FJ; a++)
#pragma unroll
                for (int b = 0; b < FI; b++)
                    *reinterpret_cast<f32x4*>(
                        red + ((((slot * (KS - 1) + ks - 1) * FJ + a) * FI + b) * 64 + lane) * 4) = acc[a][b];
        }
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int s = 1; s < KS; s++)
#pragma unroll
            for (int a = 0; a < FJ; a++)
#pragma unroll
                for (int b = 0; b < FI; b++)
                    acc[a][b] += *reinterpret_cast<const f32x4*>(
                        red + ((((slot * (KS - 1) + s - 1) * FJ + a) * FI + b) * 64 + lane) * 4);
    }

    // ---- store: lane holds y[i][j .. j+3] ----
#pragma unroll
    for (int b = 0; b < FI; b++) {
        const int i = i0 + (wi * FI + b) * 16 + r16;
        if (i >= m) continue;
        const int e = NATIVE ? 0 : XE[i];
#pragma unroll
        for (int a = 0; a < FJ; a++) {
            const int j = j0 + (wj * FJ + a) * 16 + g * 4;
            float* yp = Y + (size_t)i * n + j;
            const f32x4 v = acc[a][b];
            if (j + 3 < n && ((n & 3) == 0)) {
                *reinterpret_cast<f32x4*>(yp) =
                    f32x4{ldexpf(v[0], e), ldexpf(v[1], e), ldexpf(v[2], e), ldexpf(v[3], e)};
            } else {
#pragma unroll
                for (int t = 0; t < 4; t++)
                    if (j + t < n) yp[t] = ldexpf(v[t], e);
            }
        }
    }
}

template <bool NATIVE, bool DUMP, int FJ, int FI, int WJ, int WI, int KS, int KB>
hipError_t launch_cfg(const uint8_t* w, int n, int nb, const void* x0, const void* x1, const int* xe, int m,
                      float* y, int32_t* p, hipStream_t s) {
    using C = GemmCfg<NATIVE, FJ, FI, WJ, WI, KS, KB>;
    auto kern = gemm_q4_0_kernel<NATIVE, DUMP, FJ, FI, WJ, WI, KS, KB>;
    static_assert(C::LDS >= C::RED, "K-split sums fit the staging LDS");
    static_assert(C::LDS <= 160 * 1024, "LDS per workgroup");
    if (C::LDS > 65536) {
        const hipError_t e = hipFuncSetAttribute((const void*)kern,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
    }
    const unsigned tiles = (unsigned)((n + C::TJ - 1) / C::TJ) * (unsigned)((m + C::TI - 1) / C::TI);
    launch_kernel(kern, dim3(tiles), dim3(C::NT), (size_t)C::LDS, s, w, n, nb, x0, x1, xe, m, y, p);
    return hipGetLastError();
}

// Tile choice: enough workgroups for the CUs, then the largest tile (fewest
// re-reads of x and W from L2).  M >= 256: swept on MI355X at M = 512 and
// 2048 over tile shapes, waves and chunk sizes, per mode (the native kernel
// stages half the x bytes and keeps fewer registers).
template <bool NATIVE, bool DUMP>
hipError_t launch_tiles(const uint8_t* w, int n, int nb, const void* x0, const void* x1, const int* xe, int m,
                        float* y, int32_t* p, hipStream_t s) {
    const int cus = device_cu_count();
    if (NATIVE) {
        if (m >= 1024) return launch_cfg<NATIVE, DUMP, 2, 2, 2, 2, 2, 2>(w, n, nb, x0, x1, xe, m, y, p, s);
        if (m >= 256) return launch_cfg<NATIVE, DUMP, 2, 4, 2, 2, 2, 2>(w, n, nb, x0, x1, xe, m, y, p, s);
    } else {
        if (m >= 1024) return launch_cfg<NATIVE, DUMP, 4, 4, 2, 2, 2, 1>(w, n, nb, x0, x1, xe, m, y, p, s);
        if (m >= 256) return launch_cfg<NATIVE, DUMP, 4, 2, 2, 2, 2, 2>(w, n, nb, x0, x1, xe, m, y, p, s);
    }
    if (m >= 48 && (size_t)((n + 31) / 32) * ((m + 63) / 64) >= (size_t)cus)
        return launch_cfg<NATIVE, DUMP, 2, 4, 1, 1, 4, 2>(w, n, nb, x0, x1, xe, m, y, p, s);
    if (m > 16) return launch_cfg<NATIVE, DUMP, 1, 2, 1, 1, 4, 2>(w, n, nb, x0, x1, xe, m, y, p, s);
    return launch_cfg<NATIVE, DUMP, 1, 1, 1, 1, 4, 8>(w, n, nb, x0, x1, xe, m, y, p, s);
}

}  // namespace

size_t gemm_scratch_bytes(size_t m, size_t k, bool native) {
    if (native)  // int8 codes and f32 block scales, 256-byte aligned pieces
        return ((m * k + 255) & ~(size_t)255) + ((m * (k / QK) * 4 + 255) & ~(size_t)255);
    // x_hi, x_lo (f16) and the row exponents
    const size_t xb = (m * k * 2 + 255) & ~(size_t)255;
    return 2 * xb + ((m * 4 + 255) & ~(size_t)255);
}

hipError_t launch_gemm_q4_0(const uint8_t* w, size_t n, size_t k, const float* x, size_t m, float* y,
                            void* scratch, hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    const size_t xb = (m * k * 2 + 255) & ~(size_t)255;
    _Float16* xh = reinterpret_cast<_Float16*>(scratch);
    _Float16* xl = reinterpret_cast<_Float16*>(reinterpret_cast<uint8_t*>(scratch) + xb);
    int* xe = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(scratch) + 2 * xb);
    if (k <= (size_t)16 * XPREP_FAST_THREADS)
        launch_kernel(gemm_xprep_fast_kernel, dim3((unsigned)m), dim3(XPREP_FAST_THREADS), 0, s, x, (int)k, xh, xl,
                      xe);
    else
        launch_kernel(gemm_xprep_kernel, dim3((unsigned)m), dim3(XPREP_THREADS), 0, s, x, (int)k, xh, xl, xe);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_tiles<false, false>(w, (int)n, (int)(k / QK), xh, xl, xe, (int)m, y, nullptr, s);
}

hipError_t launch_gemm_q4_0_native(const uint8_t* w, size_t n, size_t k, const float* x, size_t m, float* y,
                                   int32_t* partials, void* scratch, hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    int8_t* codes = reinterpret_cast<int8_t*>(scratch);
    float* scales = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(scratch) + ((m * k + 255) & ~(size_t)255));
    hipError_t e = launch_prep_native_codes(x, m, k, codes, scales, s);
    if (e != hipSuccess) return e;
    const int ni = (int)n, nb = (int)(k / QK), mi = (int)m;
    if (partials) return launch_tiles<true, true>(w, ni, nb, codes, scales, nullptr, mi, nullptr, partials, s);
    return launch_tiles<true, false>(w, ni, nb, codes, scales, nullptr, mi, y, nullptr, s);
}

}  // namespace rdl
