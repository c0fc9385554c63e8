// gemm.hip -- prefill GEMM for GGUF Q4_0 weights on the gfx950 matrix cores:
// Y[m, n] = X[m, k] . W[n, k]^T, the many-token case of matmul_f32_q4
// (quantize.rs:265-320; one f32 block dot per (row, column, block), summed
// over the blocks).
//
// Numerics (float mode).  Each weight element is (q - 8) * d with d an f16.
// d = d_hi + d_lo with d_hi = d's top 8 significant bits and d_lo the rest
// (<= 3 bits); |q - 8| has at most 3 significant bits, so (q - 8) * d_hi and
// (q - 8) * d_lo are exact f16 values.  Each x row is scaled by a power of two
// 2^-e (row max -> [2^14, 2^15)) and split into x_hi = f16(x') and
// x_lo = f16(x' - x_hi) (about 22 significant bits together).  Per 32-element
// block three f16 MFMAs with f32 accumulation form
//   A_hi.x_hi + A_hi.x_lo + A_lo.x_hi
// (the dropped A_lo.x_lo term is below 2^-19 of each product), and
// y = 2^e * acc.  The per-block scale d is inside the A operand, so the
// blocks accumulate straight into one f32 accumulator per output.
//
// Operand layouts of v_mfma_f32_16x16x32_f16 (checked on gfx950): lane l holds
// A[l % 16][8 (l / 16) .. +7] and B[8 (l / 16) .. +7][l % 16]; the result
// C[4 (l / 16) + t][l % 16], t < 4.  A rows are weight rows j, B columns are
// x rows i, so a lane ends with y[i][j .. j+3] for one i.
//
// Tiling: a workgroup of WJ x WI x KS waves owns a TJ x TI output tile
// (TJ = WJ * FJ * 16 weight rows, TI = WI * FI * 16 x rows); the KS waves of
// one (wj, wi) split each chunk's blocks and their sums are added at the end.
// Chunks of CB = 2 * KS blocks are staged into LDS, double-buffered: Q4_0
// blocks realigned to 16 nibble bytes + their f16 d, and the x_hi / x_lo
// tiles; all global loads are raw buffer loads whose out-of-range slots
// (rows past n or m, blocks past nb) read zeros.
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
// distinct banks: nibble rows CB*16 + 8 bytes, x rows CB*64 + 16 bytes.
template <int CB> struct Lds {
    static constexpr int WN_STRIDE = CB * 16 + 8;   // bytes per weight row (nibbles)
    static constexpr int X_STRIDE = CB * 64 + 16;   // bytes per x row (f16 x CB*32)
};

// 8 nibbles of (q - 8) as four f16 pairs times d_hi and d_lo.
__device__ __forceinline__ void a_fragment(uint32_t n0, uint32_t n1, uint32_t dbits, half8_t& ah,
                                           half8_t& al) {
    const uint32_t d_hi_bits = dbits & 0xFFF8u;
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)dbits);
    const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)d_hi_bits);
    const _Float16 dl = d - dh;  // exact: the bits d_hi dropped
    const half2_t vdh = {dh, dh}, vdl = {dl, dl}, off = {(_Float16)1032.0f, (_Float16)1032.0f};
    constexpr uint32_t MAGIC = 0x64646464u;  // f16 0x64XX = 1024 + XX for XX < 16
    const uint32_t p0 = perm(MAGIC, n0, 0x04010400u), p1 = perm(MAGIC, n0, 0x04030402u);
    const uint32_t p2 = perm(MAGIC, n1, 0x04010400u), p3 = perm(MAGIC, n1, 0x04030402u);
    const half2_t q0 = __builtin_bit_cast(half2_t, p0) - off;  // (q - 8), exact
    const half2_t q1 = __builtin_bit_cast(half2_t, p1) - off;
    const half2_t q2 = __builtin_bit_cast(half2_t, p2) - off;
    const half2_t q3 = __builtin_bit_cast(half2_t, p3) - off;
    const half2_t h0 = q0 * vdh, h1 = q1 * vdh, h2 = q2 * vdh, h3 = q3 * vdh;
    const half2_t l0 = q0 * vdl, l1 = q1 * vdl, l2 = q2 * vdl, l3 = q3 * vdl;
    ah = half8_t{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
    al = half8_t{l0[0], l0[1], l1[0], l1[1], l2[0], l2[1], l3[0], l3[1]};
}

template <int FJ, int FI, int WJ, int WI, int KS, int KB>
struct GemmCfg {
    static constexpr int NW = WJ * WI * KS;
    static constexpr int NT = NW * 64;
    static constexpr int TJ = WJ * FJ * 16;
    static constexpr int TI = WI * FI * 16;
    static constexpr int CB = KB * KS;                      // blocks per chunk
    static constexpr int WN_BYTES = TJ * Lds<CB>::WN_STRIDE;
    static constexpr int WD_BYTES = TJ * CB * 2;
    static constexpr int X_BYTES = TI * Lds<CB>::X_STRIDE;  // one of hi / lo
    static constexpr int STAGE = WN_BYTES + WD_BYTES + 2 * X_BYTES;
    static constexpr int STAGE_AL = (STAGE + 15) & ~15;
    static constexpr int LDS = 2 * STAGE_AL;
    static constexpr int WBLK = (TJ * CB + NT - 1) / NT;          // weight blocks per thread
    static constexpr int XU = (TI * CB * 4 + NT - 1) / NT;         // 16-byte x units per thread (each of hi, lo)
    static constexpr int RED = (KS > 1) ? (KS - 1) * WJ * WI * FJ * FI * 64 * 16 : 0;
};

// One chunk's global loads, held in registers until they are written to LDS.
template <int WBLK, int XU>
struct Staged {
    uint32_t w[WBLK][5];
    u32x4 xh[XU], xl[XU];
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

template <int FJ, int FI, int WJ, int WI, int KS, int KB>
__global__ __launch_bounds__(WJ * WI * KS * 64) void gemm_q4_0_f16_kernel(
    const uint8_t* __restrict__ W, int n, int nb, const _Float16* __restrict__ XH,
    const _Float16* __restrict__ XL, const int* __restrict__ XE, int m, float* __restrict__ Y) {
    using C = GemmCfg<FJ, FI, WJ, WI, KS, KB>;
    constexpr int CB = C::CB;
    using S = Staged<C::WBLK, C::XU>;
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
    const __amdgpu_buffer_rsrc_t xhrs = make_rsrc(XH, (uint32_t)m * (uint32_t)k * 2u);
    const __amdgpu_buffer_rsrc_t xlrs = make_rsrc(XL, (uint32_t)m * (uint32_t)k * 2u);
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
#pragma unroll
        for (int u = 0; u < C::XU; u++) {
            const int idx = threadIdx.x + u * C::NT;   // unit = 8 halfs
            const int il = idx / (CB * 4), q = idx % (CB * 4);
            const int i = i0 + il, kk = c * CB * 32 + q * 8;
            const uint32_t off = (live && idx < C::TI * CB * 4 && i < m && kk < k)
                                     ? ((uint32_t)i * (uint32_t)k + (uint32_t)kk) * 2u
                                     : RSRC_OOB;
            r.xh[u] = buf_load_b128(xhrs, off);
            r.xl[u] = buf_load_b128(xlrs, off);
        }
    };
    auto store_chunk = [&](int c, int buf, const S& r) {
        uint8_t* st = lds + buf * C::STAGE_AL;
        uint8_t* wn = st;
        uint16_t* wd = reinterpret_cast<uint16_t*>(st + C::WN_BYTES);
        uint8_t* xhs = st + C::WN_BYTES + C::WD_BYTES;
        uint8_t* xls = xhs + C::X_BYTES;
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
                wd[jl * CB + bl] = (uint16_t)dbits;
            }
        }
#pragma unroll
        for (int u = 0; u < C::XU; u++) {
            const int idx = threadIdx.x + u * C::NT;
            if (idx < C::TI * CB * 4) {
                const int il = idx / (CB * 4), q = idx % (CB * 4);
                *reinterpret_cast<u32x4*>(xhs + il * Lds<CB>::X_STRIDE + q * 16) = r.xh[u];
                *reinterpret_cast<u32x4*>(xls + il * Lds<CB>::X_STRIDE + q * 16) = r.xl[u];
            }
        }
    };

    f32x4 acc[FJ][FI];
#pragma unroll
    for (int a = 0; a < FJ; a++)
#pragma unroll
        for (int b = 0; b < FI; b++) acc[a][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int g = lane >> 4, r16 = lane & 15;
    auto compute_chunk = [&](int buf) {
        const uint8_t* st = lds + buf * C::STAGE_AL;
        const uint8_t* wn = st;
        const uint16_t* wd = reinterpret_cast<const uint16_t*>(st + C::WN_BYTES);
        const uint8_t* xhs = st + C::WN_BYTES + C::WD_BYTES;
        const uint8_t* xls = xhs + C::X_BYTES;
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const int bl = ks * KB + kb;  // this wave's block within the chunk
            half8_t ah[FJ], al[FJ];
#pragma unroll
            for (int a = 0; a < FJ; a++) {
                const int jl = (wj * FJ + a) * 16 + r16;
                const uint2 nb8 = *reinterpret_cast<const uint2*>(wn + jl * Lds<CB>::WN_STRIDE +
                                                                  bl * 16 + 8 * (g & 1));
                const uint32_t sh = (g >> 1) * 4;  // groups 2, 3: high nibbles
                a_fragment((nb8.x >> sh) & 0x0F0F0F0Fu, (nb8.y >> sh) & 0x0F0F0F0Fu, wd[jl * CB + bl],
                           ah[a], al[a]);
            }
#pragma unroll
            for (int b = 0; b < FI; b++) {
                const int il = (wi * FI + b) * 16 + r16;
                const int xo = il * Lds<CB>::X_STRIDE + bl * 64 + g * 16;
                const half8_t bh = *reinterpret_cast<const half8_t*>(xhs + xo);
                const half8_t bl8 = *reinterpret_cast<const half8_t*>(xls + xo);
#pragma unroll
                for (int a = 0; a < FJ; a++) {
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[a], bh, acc[a][b], 0, 0, 0);
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[a], bl8, acc[a][b], 0, 0, 0);
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[a], bh, acc[a][b], 0, 0, 0);
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
        compute_chunk(0);
        if (c + 1 < nchunks) store_chunk(c + 1, 1, r1);
        __syncthreads();
        if (c + 1 >= nchunks) break;
        load_chunk(c + 3, r1, c + 3 < nchunks);
        compute_chunk(1);
        if (c + 2 < nchunks) store_chunk(c + 2, 0, r0);
        __syncthreads();
    }

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
        const int e = XE[i];
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

template <int FJ, int FI, int WJ, int WI, int KS, int KB>
hipError_t launch_cfg(const uint8_t* w, int n, int nb, const _Float16* xh, const _Float16* xl,
                      const int* xe, int m, float* y, hipStream_t s) {
    using C = GemmCfg<FJ, FI, WJ, WI, KS, KB>;
    auto kern = gemm_q4_0_f16_kernel<FJ, FI, WJ, WI, KS, KB>;
    static_assert(C::LDS >= C::RED, "K-split sums fit the staging LDS");
    static_assert(C::LDS <= 160 * 1024, "LDS per workgroup");
    if (C::LDS > 65536) {
        const hipError_t e = hipFuncSetAttribute((const void*)kern,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
    }
    const unsigned tiles = (unsigned)((n + C::TJ - 1) / C::TJ) * (unsigned)((m + C::TI - 1) / C::TI);
    launch_kernel(kern, dim3(tiles), dim3(C::NT), (size_t)C::LDS, s, w, n, nb, xh, xl, xe, m, y);
    return hipGetLastError();
}

// Sets *flag when a Q4_0 block scale is finite with |d| > 4096 (its f16
// products (q - 8) * d could overflow in the GEMM's A operand).
__global__ __launch_bounds__(256) void q4_0_scale_scan_kernel(const uint8_t* __restrict__ W,
                                                             size_t nblocks, int* __restrict__ flag) {
    for (size_t g = (size_t)blockIdx.x * 256 + threadIdx.x; g < nblocks; g += (size_t)gridDim.x * 256) {
        const uint32_t a = *reinterpret_cast<const uint16_t*>(W + g * 18) & 0x7FFFu;
        if (a > 0x6C00u && a < 0x7C00u) *flag = 1;
    }
}

}  // namespace

hipError_t gemm_scales_ok(WType t, const uint8_t* w, size_t n, size_t k, bool* ok) {
    *ok = false;
    if (t != WType::Q4_0) return hipSuccess;
    const size_t nblocks = n * (k / QK);
    if (nblocks == 0) {
        *ok = true;
        return hipSuccess;
    }
    int* flag = nullptr;
    hipError_t e = hipMalloc(&flag, sizeof(int));
    if (e != hipSuccess) return e;
    int host = 0;
    e = hipMemset(flag, 0, sizeof(int));
    if (e == hipSuccess) {
        const unsigned grid = (unsigned)std::min<size_t>((nblocks + 255) / 256, 4096);
        hipLaunchKernelGGL(q4_0_scale_scan_kernel, dim3(grid), dim3(256), 0, nullptr, w, nblocks, flag);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(&host, flag, sizeof(int), hipMemcpyDeviceToHost);
    (void)hipFree(flag);
    *ok = (e == hipSuccess && host == 0);
    return e;
}

size_t gemm_scratch_bytes(size_t m, size_t k) {
    // x_hi, x_lo (f16) and the row exponents, 256-byte aligned pieces
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
    const int ni = (int)n, nb = (int)(k / QK), mi = (int)m;
    const int cus = device_cu_count();
    // Tile choice: enough workgroups for the CUs, then the largest tile
    // (fewest re-reads of x and W from L2).
    // (M >= 256: swept on MI355X at M = 512, 2048 over tile shape, waves and
    // chunk size; two-way K splits keep 8 waves a workgroup within the LDS)
    if (m >= 1024) return launch_cfg<4, 4, 2, 2, 2, 1>(w, ni, nb, xh, xl, xe, mi, y, s);
    if (m >= 256) return launch_cfg<2, 4, 2, 2, 2, 2>(w, ni, nb, xh, xl, xe, mi, y, s);
    if (m >= 48 && (size_t)((n + 31) / 32) * ((m + 63) / 64) >= (size_t)cus)
        return launch_cfg<2, 4, 1, 1, 4, 2>(w, ni, nb, xh, xl, xe, mi, y, s);
    if (m > 16) return launch_cfg<1, 2, 1, 1, 4, 2>(w, ni, nb, xh, xl, xe, mi, y, s);
    return launch_cfg<1, 1, 1, 1, 4, 8>(w, ni, nb, xh, xl, xe, mi, y, s);
}

}  // namespace rdl
