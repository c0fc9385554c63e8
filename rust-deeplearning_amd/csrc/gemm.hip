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

#include <atomic>
#include <mutex>
#include <vector>

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

// The split of a row held in registers (thread t: elements 4 (t + j NT) ..
// +3 of v[j], zeros past k): x' = x 2^-e, x_hi = f16(x'), x_lo = f16(x' -
// x_hi); XS (if not null): the f32 sum of x' over each 32-element block
// ([m, k / 32]; one block is 8 consecutive threads).
template <int NT, int NV>
__device__ __forceinline__ void split_store(const f32x4 (&v)[NV], int e, int row, int k, _Float16* __restrict__ XH,
                                            _Float16* __restrict__ XL, float* __restrict__ XS) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const int k4 = k >> 2;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int p = threadIdx.x + j * NT;
        h4 hv, lv;
        float bs = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float s = ldexpf(v[j][t], -e);
            hv[t] = (_Float16)s;
            lv[t] = (_Float16)(s - (float)hv[t]);
            bs += s;
        }
        if (p < k4) {
            reinterpret_cast<h4*>(XH + (size_t)row * k)[p] = hv;
            reinterpret_cast<h4*>(XL + (size_t)row * k)[p] = lv;
        }
        if (XS) {  // uniform: every thread of the launch takes the branch
            bs += __shfl_xor(bs, 1);
            bs += __shfl_xor(bs, 2);
            bs += __shfl_xor(bs, 4);
            if ((threadIdx.x & 7) == 0 && p < k4) XS[(size_t)row * (k >> 5) + (p >> 3)] = bs;
        }
    }
}

// The same split with each row's values held in registers between the max
// and the conversion (k <= 4 * 4 * XPREP_FAST_THREADS): one global read.
constexpr int XPREP_FAST_THREADS = 1024;
__global__ __launch_bounds__(XPREP_FAST_THREADS) void gemm_xprep_fast_kernel(const float* __restrict__ X, int k,
                                                                             _Float16* __restrict__ XH,
                                                                             _Float16* __restrict__ XL,
                                                                             int* __restrict__ XE,
                                                                             float* __restrict__ XS) {
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
    split_store<NT, NV>(v, e, row, k, XH, XL, XS);
}

// The fast split after a prologue on the row, for the decoder's prompt
// chunks (one launch instead of two):
// PRO 1: RMSNorm, x * (1 / sqrt(sum(x^2) / k + eps)) * g (ops.rs:688-751);
// PRO 2: SwiGLU of rows of 2k interleaved (gate_j, up_j) values,
//        silu(g) * u with silu(g) = g * (1 / (1 + exp(-g))) (ops.rs:441-446).
// The element arithmetic is the separate kernels'; only RMSNorm's sum of
// squares runs in another order.
template <int PRO>
__global__ __launch_bounds__(XPREP_FAST_THREADS) void gemm_xprep_pro_kernel(
    const float* __restrict__ X, int k, const float* __restrict__ g, float eps, _Float16* __restrict__ XH,
    _Float16* __restrict__ XL, int* __restrict__ XE, float* __restrict__ XS) {
    static_assert(PRO == 1 || PRO == 2, "RMSNorm or SwiGLU");
    constexpr int NT = XPREP_FAST_THREADS, NV = 4;
    __shared__ float red[NT / 64], red2[NT / 64];
    const int row = blockIdx.x;
    const int k4 = k >> 2;  // k % 32 == 0
    f32x4 v[NV];
    if constexpr (PRO == 2) {
        const f32x4* x = reinterpret_cast<const f32x4*>(X + (size_t)row * 2 * k);
        auto silu_mul = [](float gv, float uv) {
            const float sig = 1.0f / (1.0f + expf(-gv));
            return (gv * sig) * uv;
        };
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int p = threadIdx.x + j * NT;
            if (p < k4) {
                const f32x4 a = x[2 * p], b = x[2 * p + 1];
                v[j] = f32x4{silu_mul(a[0], a[1]), silu_mul(a[2], a[3]), silu_mul(b[0], b[1]), silu_mul(b[2], b[3])};
            } else {
                v[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    } else {
        const f32x4* x = reinterpret_cast<const f32x4*>(X + (size_t)row * k);
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int p = threadIdx.x + j * NT;
            v[j] = p < k4 ? x[p] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            ss += (v[j][0] * v[j][0] + v[j][1] * v[j][1]) + (v[j][2] * v[j][2] + v[j][3] * v[j][3]);
        }
        ss = sum8_f32(ss);
        ss += dpp_f32<DPP_ROW_MIRROR>(ss);
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        if ((threadIdx.x & 63) == 0) red2[threadIdx.x >> 6] = ss;
        __syncthreads();
        ss = red2[0];
#pragma unroll
        for (int w = 1; w < NT / 64; w++) ss += red2[w];
        const float inv = 1.0f / sqrtf(ss / (float)k + eps);
        const f32x4* g4 = reinterpret_cast<const f32x4*>(g);
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int p = threadIdx.x + j * NT;
            if (p < k4) v[j] = (v[j] * inv) * g4[p];
        }
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
    int e = 0;
    if (amax > 0.0f && isfinite(amax)) e = ilogbf(amax) - 14;
    if (threadIdx.x == 0) XE[row] = e;
    split_store<NT, NV>(v, e, row, k, XH, XL, XS);
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

// 8 codes (two dwords of four bytes) of a weight row as (q - Z), Z = 8 for
// nibbles, 32 for Q6_K's 6-bit codes, 128 for Q8_0's codes staged + 128:
// exact f16 values for the float product; signed bytes (q - 8) for the
// native one.
template <int Z = 8>
__device__ __forceinline__ half8_t q_f16(uint32_t n0, uint32_t n1) {
    const half2_t off = {(_Float16)(1024.0f + Z), (_Float16)(1024.0f + Z)};
    constexpr uint32_t MAGIC = 0x64646464u;  // f16 0x64XX = 1024 + XX (XX a byte)
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

// Weight formats of the LDS GEMM: GGUF Q4_0 blocks, Q4_K super-blocks taken
// as 32-element sub-blocks (value (d sc) q - dmin mn, parser.rs:549-593),
// Q6_K super-blocks taken as 32-element groups of two 16-element sub-blocks
// (value (d sc) (q - 32), parser.rs:510-547), Q8_0 blocks (value d q,
// tensor.rs:535-639) and Q4_1 blocks (value d q + m, quantize.rs:429-495).
constexpr int WF_Q4_0 = 0, WF_Q4_K = 1, WF_Q6_K = 2, WF_Q8_0 = 3, WF_Q4_1 = 4;
// staged as byte codes (32 a block) rather than nibbles; with f32 scale
// pairs a block rather than one f16 d; with x' block sums
constexpr bool wf_bytes(int wf) { return wf == WF_Q6_K || wf == WF_Q8_0; }
constexpr bool wf_pairs(int wf) { return wf == WF_Q4_K || wf == WF_Q6_K || wf == WF_Q4_1; }
constexpr bool wf_sums(int wf) { return wf == WF_Q4_K || wf == WF_Q4_1; }

template <bool NATIVE, int WF, int FJ, int FI, int WJ, int WI, int KS, int KB>
struct GemmCfg {
    static_assert(WF == WF_Q4_0 || !NATIVE, "native mode for Q4_0 only");
    static constexpr int NW = WJ * WI * KS;
    static constexpr int NT = NW * 64;
    static constexpr int TJ = WJ * FJ * 16;
    static constexpr int TI = WI * FI * 16;
    static constexpr int CB = KB * KS;                      // blocks per chunk
    // Q4_0 float mode, 128 x 128 tile: the weights staged as the MFMA's f16
    // (q - 8) operands, converted once a chunk by the staging threads rather
    // than by each of the WI waves that read a weight tile
    static constexpr bool AF16 = !NATIVE && WF == WF_Q4_0 && FJ * FI == 16;
    // weight rows: 16 nibble bytes a block (Q6_K, Q8_0: 32 codes as bytes;
    // AF16: 32 f16 operands, the x rows' stride), padded
    static constexpr int WNS = AF16 ? Lds<CB>::X_STRIDE : wf_bytes(WF) ? CB * 32 + 8 : Lds<CB>::WN_STRIDE;
    static constexpr int WN_BYTES = TJ * WNS;
    // Q4_0, Q8_0: the f16 d of each (row, block); Q4_K: f32 pairs {d sc,
    // 8 d sc - dmin mn}; Q6_K: {d sc0, d sc1} of the block's two sub-blocks;
    // Q4_1: {d, 8 d + m}
    static constexpr int WD_BYTES = wf_pairs(WF) ? TJ * CB * 8 : (TJ * CB * 2 + 15) & ~15;
    // float: x_hi and x_lo tiles (Q4_K: and the x block sums); native: int8
    // codes and the f32 block scales
    static constexpr int X_BYTES = TI * (NATIVE ? Lds<CB>::XC_STRIDE : Lds<CB>::X_STRIDE);
    static constexpr bool XSUMS = NATIVE || wf_sums(WF);
    static constexpr int XS_BYTES = XSUMS ? TI * CB * 4 : 0;
    static constexpr int STAGE = WN_BYTES + WD_BYTES + (NATIVE ? X_BYTES : 2 * X_BYTES) + XS_BYTES;
    static constexpr int STAGE_AL = (STAGE + 15) & ~15;
    static constexpr int WBLK = (TJ * CB + NT - 1) / NT;                          // weight blocks per thread
    // dwords a weight block's loads bring
    static constexpr int WWORDS = WF == WF_Q6_K ? 20 : WF == WF_Q4_K ? 12 : WF == WF_Q8_0 ? 9 : 5;
    static constexpr int XU = (TI * CB * (NATIVE ? 2 : 4) + NT - 1) / NT;          // 16-byte x units per thread
    static constexpr int XSU = XSUMS ? (TI * CB + NT - 1) / NT : 0;              // scale / sum dwords per thread
    static constexpr int RED = (KS > 1) ? (KS - 1) * WJ * WI * FJ * FI * 64 * 16 : 0;
    // two staging buffers; the K-split sums reuse the same LDS at the end
    static constexpr int LDS = (2 * STAGE_AL > RED) ? 2 * STAGE_AL : RED;
};

// One chunk's global loads, held in registers until they are written to LDS.
template <int WBLK, int WWORDS, int XU, int XSU>
struct Staged {
    uint32_t w[WBLK][WWORDS];
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

// 32-element sub-block j (0..7) of a Q4_K super-block: its 6-bit scale and
// min from the 12 scale bytes s[0..11] (header dwords s03, s47, s811), as
// the reference unpacks them (parser.rs:563-569).
__device__ __forceinline__ void q4k_sub_scale_min(uint32_t s03, uint32_t s47, uint32_t s811, int j, int& sc,
                                                  int& mn) {
    if (j < 4) {  // sc = s[j] & 63, mn = s[j + 4] & 63
        sc = (int)((s03 >> (8 * j)) & 63u);
        mn = (int)((s47 >> (8 * j)) & 63u);
    } else {      // i = j - 4: sc = (s[i] >> 6) | (s[i + 8] & 15) << 2, mn = (s[i + 4] >> 6) | (s[i + 8] >> 4) << 2
        const int i = j - 4;
        const uint32_t si = (s03 >> (8 * i)) & 0xFFu, ti = (s47 >> (8 * i)) & 0xFFu, ui = (s811 >> (8 * i)) & 0xFFu;
        sc = (int)((si >> 6) | ((ui & 15u) << 2));
        mn = (int)((ti >> 6) | ((ui >> 4) << 2));
    }
}

// NATIVE = false: X0 / X1 = x_hi / x_lo (f16 [m, k]), XE the row exponents.
// NATIVE = true:  X0 = Q8_0 codes (int8 [m, k]), X1 = their f32 block scales
// [m, nb] (quantize_row_q8_0); DUMP writes the int32 block dots to
// P[(i * n + j) * nb + b] instead of forming Y.
// WF = WF_Q4_K (float mode): W holds Q4_K super-blocks, nb counts their
// 32-element sub-blocks, and XS the sums of each row's scaled x' over each
// sub-block ([m, nb] f32).  A sub-block's nibbles are staged as a Q4_0
// block's, so the MFMAs give sum (q - 8) x'; with D = d sc and M = dmin mn
// the sub-block adds D sum (q - 8) x' + (8 D - M) sum x' = sum (D q - M) x'.
// WF = WF_Q6_K (float mode): W holds Q6_K super-blocks, nb counts their
// 32-element groups; a group's codes are staged as bytes, its two 16-element
// sub-blocks' scales D0 = d sc0, D1 = d sc1 in f32, and the MFMAs run once
// with the lanes of elements 16..31 zeroed and once with those of 0..15:
// the group adds D0 sum_0 (q - 32) x' + D1 sum_1 (q - 32) x'.
// WF = WF_Q8_0 (float mode): 34-byte blocks, 2-byte aligned; the int8 codes
// are staged as bytes + 128 and the f16 operand (b - 128) = q is exact; the
// block adds d sum q x'.
// WF = WF_Q4_1 (float mode): 20-byte blocks; nibbles staged as Q4_0's, and as
// for Q4_K the block adds d sum (q - 8) x' + (8 d + m) sum x'.
template <bool NATIVE, bool DUMP, int WF, int FJ, int FI, int WJ, int WI, int KS, int KB>
__global__ __launch_bounds__(WJ * WI * KS * 64) void gemm_q4_0_kernel(
    const uint8_t* __restrict__ W, int n, int nb, const void* __restrict__ X0, const void* __restrict__ X1,
    const int* __restrict__ XE, int m, float* __restrict__ Y, int32_t* __restrict__ P, int accy,
    const float* __restrict__ XS) {
    using C = GemmCfg<NATIVE, WF, FJ, FI, WJ, WI, KS, KB>;
    constexpr bool QK = WF == WF_Q4_K;
    constexpr bool Q6 = WF == WF_Q6_K;
    constexpr bool Q8 = WF == WF_Q8_0;
    constexpr bool Q41 = WF == WF_Q4_1;
    constexpr bool PAIRS = wf_pairs(WF), SUMS = wf_sums(WF);
    constexpr int CB = C::CB;
    constexpr int XSTR = NATIVE ? Lds<CB>::XC_STRIDE : Lds<CB>::X_STRIDE;
    using S = Staged<C::WBLK, C::WWORDS, C::XU, C::XSU>;
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
    // Q4_K: 144-byte super-blocks of 8 sub-blocks (nb % 8 == 0), rows 16-byte
    // aligned; Q6_K: 210-byte super-blocks of 8 groups, 2-byte aligned
    const uint32_t row_bytes = QK   ? (uint32_t)(nb / 8) * 144u
                               : Q6  ? (uint32_t)(nb / 8) * 210u
                               : Q8  ? (uint32_t)nb * 34u
                               : Q41 ? (uint32_t)nb * 20u
                                     : (uint32_t)nb * 18u;
    const uint32_t wbytes = (uint32_t)n * row_bytes;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(W, wbytes);
    const uint32_t xbytes = (uint32_t)m * (uint32_t)k * (NATIVE ? 1u : 2u);
    const __amdgpu_buffer_rsrc_t x0rs = make_rsrc(X0, xbytes);
    const __amdgpu_buffer_rsrc_t x1rs = make_rsrc(X1, NATIVE ? (uint32_t)m * (uint32_t)nb * 4u : xbytes);
    // per-(row, block) f32 x data: native's Q8_0 scales (X1), the x' sums (XS)
    const __amdgpu_buffer_rsrc_t xsrs = SUMS ? make_rsrc(XS, (uint32_t)m * (uint32_t)nb * 4u) : x1rs;
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
            if constexpr (QK) {
                // the super-block's 16-byte header (d, dmin, scales) and the 32
                // bytes whose low (even b) or high (odd b) nibbles are sub-block b
                const bool ok = live && idx < C::TJ * CB && j < n && b < nb;
                const uint32_t hoff = (uint32_t)j * row_bytes + (uint32_t)(b >> 3) * 144u;
                const uint32_t qoff = hoff + 16u + 32u * (uint32_t)((b & 7) >> 1);
                const u32x4 h = buf_load_b128(wrs, ok ? hoff : RSRC_OOB);
                const u32x4 q0 = buf_load_b128(wrs, ok ? qoff : RSRC_OOB);
                const u32x4 q1 = buf_load_b128(wrs, ok ? qoff + 16u : RSRC_OOB);
                r.w[u][0] = h.x; r.w[u][1] = h.y; r.w[u][2] = h.z; r.w[u][3] = h.w;
                r.w[u][4] = q0.x; r.w[u][5] = q0.y; r.w[u][6] = q0.z; r.w[u][7] = q0.w;
                r.w[u][8] = q1.x; r.w[u][9] = q1.y; r.w[u][10] = q1.z; r.w[u][11] = q1.w;
                continue;
            }
            if constexpr (Q8) {
                // 36 bytes from the dword below the block (it starts on a dword
                // or 2 bytes past one); the matrix's last block, when it starts
                // on a dword, ends 2 bytes into the window's last dword: that
                // dword is read 2 bytes early (shifted when stored)
                const bool ok = live && idx < C::TJ * CB && j < n && b < nb;
                const uint32_t al = ((uint32_t)j * row_bytes + (uint32_t)b * 34u) & ~3u;
                const uint32_t last = al + 32u > wbytes - 4u ? wbytes - 4u : al + 32u;
                const u32x4 v0 = buf_load_b128(wrs, ok ? al : RSRC_OOB);
                const u32x4 v1 = buf_load_b128(wrs, ok ? al + 16u : RSRC_OOB);
                r.w[u][0] = v0.x; r.w[u][1] = v0.y; r.w[u][2] = v0.z; r.w[u][3] = v0.w;
                r.w[u][4] = v1.x; r.w[u][5] = v1.y; r.w[u][6] = v1.z; r.w[u][7] = v1.w;
                r.w[u][8] = buf_load_b32(wrs, ok ? last : RSRC_OOB);
                continue;
            }
            if constexpr (Q41) {
                // d, m and the 16 nibble bytes: blocks start on a dword
                const bool ok = live && idx < C::TJ * CB && j < n && b < nb;
                const uint32_t base = (uint32_t)j * row_bytes + (uint32_t)b * 20u;
                const u32x4 v = buf_load_b128(wrs, ok ? base : RSRC_OOB);
                r.w[u][0] = v.x; r.w[u][1] = v.y; r.w[u][2] = v.z; r.w[u][3] = v.w;
                r.w[u][4] = buf_load_b32(wrs, ok ? base + 16u : RSRC_OOB);
                continue;
            }
            if constexpr (Q6) {
                // group b: half hh = (b / 4) % 2, t = b % 4 of super-block b / 8:
                // the 32 ql bytes whose low (t < 2) or high nibbles it takes, the
                // 32 qh bytes holding its 2-bit highs, its two scale bytes and d.
                // The super-block starts on a dword or 2 bytes past one: 36-byte
                // windows from the dword below, realigned when stored.
                const bool ok = live && idx < C::TJ * CB && j < n && b < nb;
                const uint32_t base = (uint32_t)j * row_bytes + (uint32_t)(b >> 3) * 210u;
                const uint32_t al = base & ~3u, hh = (uint32_t)(b >> 2) & 1u, t = (uint32_t)b & 3u;
                const uint32_t qlo = al + 64u * hh + 32u * (t & 1u), qho = al + 128u + 32u * hh;
                const uint32_t sco = (base + 192u + 8u * hh + 2u * t) & ~3u;
                // d's dword; the matrix's last super-block, starting on a dword,
                // ends 2 bytes into it: read 2 bytes early (the high half is d)
                const uint32_t dof0 = (base + 208u) & ~3u;
                const uint32_t dof = dof0 + 4u > wbytes ? wbytes - 4u : dof0;
                const u32x4 l0 = buf_load_b128(wrs, ok ? qlo : RSRC_OOB);
                const u32x4 l1 = buf_load_b128(wrs, ok ? qlo + 16u : RSRC_OOB);
                const uint32_t l2 = buf_load_b32(wrs, ok ? qlo + 32u : RSRC_OOB);
                const u32x4 h0 = buf_load_b128(wrs, ok ? qho : RSRC_OOB);
                const u32x4 h1 = buf_load_b128(wrs, ok ? qho + 16u : RSRC_OOB);
                const uint32_t h2 = buf_load_b32(wrs, ok ? qho + 32u : RSRC_OOB);
                r.w[u][0] = l0.x; r.w[u][1] = l0.y; r.w[u][2] = l0.z; r.w[u][3] = l0.w;
                r.w[u][4] = l1.x; r.w[u][5] = l1.y; r.w[u][6] = l1.z; r.w[u][7] = l1.w;
                r.w[u][8] = l2;
                r.w[u][9] = h0.x; r.w[u][10] = h0.y; r.w[u][11] = h0.z; r.w[u][12] = h0.w;
                r.w[u][13] = h1.x; r.w[u][14] = h1.y; r.w[u][15] = h1.z; r.w[u][16] = h1.w;
                r.w[u][17] = h2;
                r.w[u][18] = buf_load_b32(wrs, ok ? sco : RSRC_OOB);
                r.w[u][19] = buf_load_b32(wrs, ok ? dof : RSRC_OOB);
                continue;
            }
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
            r.w[u][C::WWORDS - 1] = buf_load_b32(wrs, over ? wbytes - 4u : base + 16u);
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
        if constexpr (C::XSUMS) {
#pragma unroll
            for (int u = 0; u < C::XSU; u++) {
                const int idx = threadIdx.x + u * C::NT;
                const int il = idx / CB, bl = idx % CB;
                const int i = i0 + il, b = c * CB + bl;
                const uint32_t off = (live && idx < C::TI * CB && i < m && b < nb)
                                         ? ((uint32_t)i * (uint32_t)nb + (uint32_t)b) * 4u
                                         : RSRC_OOB;
                r.xs[u] = buf_load_b32(xsrs, off);
            }
        }
    };
    auto store_chunk = [&](int c, int buf, const S& r) {
        uint8_t* st = lds + buf * C::STAGE_AL;
        uint8_t* wn = st;
        uint16_t* wd = reinterpret_cast<uint16_t*>(st + C::WN_BYTES);
        uint8_t* x0s = st + C::WN_BYTES + C::WD_BYTES;
        uint8_t* x1s = x0s + C::X_BYTES;
        uint8_t* xss = x0s + (NATIVE ? 1 : 2) * C::X_BYTES;
#pragma unroll
        for (int u = 0; u < C::WBLK; u++) {
            const int idx = threadIdx.x + u * C::NT;
            if constexpr (QK) {
                if (idx >= C::TJ * CB) continue;
                const int jl = idx / CB, bl = idx % CB;
                const int b = c * CB + bl;
                // sub-block element t is the nibble of byte t of the 32: stage
                // byte t = element t | element t + 16 << 4, a Q4_0 block's order
                const uint32_t sh = (b & 1) ? 4u : 0u;
                uint32_t q[8];
#pragma unroll
                for (int t = 0; t < 8; t++) q[t] = (r.w[u][4 + t] >> sh) & 0x0F0F0F0Fu;
                uint2* dst = reinterpret_cast<uint2*>(wn + jl * Lds<CB>::WN_STRIDE + bl * 16);
                dst[0] = uint2{q[0] | (q[4] << 4), q[1] | (q[5] << 4)};
                dst[1] = uint2{q[2] | (q[6] << 4), q[3] | (q[7] << 4)};
                // D = d sc and 8 D - M (M = dmin mn) in f32, block-major; rows or
                // sub-blocks past the matrix loaded zeros: D = 8 D - M = 0
                int sc, mn;
                q4k_sub_scale_min(r.w[u][1], r.w[u][2], r.w[u][3], b & 7, sc, mn);
                const float dd = h2f(r.w[u][0] & 0xFFFFu) * (float)sc;
                const float mm = h2f(r.w[u][0] >> 16) * (float)mn;
                float* wdf = reinterpret_cast<float*>(st + C::WN_BYTES);
                wdf[bl * C::TJ + jl] = dd;
                wdf[(CB + bl) * C::TJ + jl] = 8.0f * dd - mm;
            } else if constexpr (Q6) {
                if (idx >= C::TJ * CB) continue;
                const int jl = idx / CB, bl = idx % CB;
                const int j = j0 + jl, b = c * CB + bl;
                const uint32_t base = (uint32_t)j * row_bytes + (uint32_t)(b >> 3) * 210u;
                const uint32_t hh = (uint32_t)(b >> 2) & 1u, t = (uint32_t)b & 3u;
                const bool mis = (base & 2u) != 0;
                // codes q = (ql nibble) | (qh 2 bits) << 4, element l in byte l
                const uint32_t sh = 4u * (t >> 1), hs = 2u * t;
                uint32_t q[8];
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint32_t lo = mis ? perm(r.w[u][i + 1], r.w[u][i], 0x05040302u) : r.w[u][i];
                    const uint32_t hi = mis ? perm(r.w[u][i + 10], r.w[u][i + 9], 0x05040302u) : r.w[u][i + 9];
                    q[i] = ((lo >> sh) & 0x0F0F0F0Fu) | (((hi >> hs) & 0x03030303u) << 4);
                }
                uint2* dst = reinterpret_cast<uint2*>(wn + jl * C::WNS + bl * 32);
#pragma unroll
                for (int i = 0; i < 4; i++) dst[i] = uint2{q[2 * i], q[2 * i + 1]};
                // scales sc[8 hh + 2 t], sc[8 hh + 2 t + 1] (int8) and d; rows or
                // groups past the matrix loaded zeros: D0 = D1 = 0
                const uint32_t scw = r.w[u][18] >> (8u * ((base + 192u + 8u * hh + 2u * t) & 3u));
                const uint32_t dof0 = (base + 208u) & ~3u;
                const uint32_t dbits = dof0 + 4u > wbytes ? (r.w[u][19] >> 16)
                                                          : (r.w[u][19] >> (8u * ((base + 208u) & 3u))) & 0xFFFFu;
                const float d = h2f(dbits);
                float* wdf = reinterpret_cast<float*>(st + C::WN_BYTES);
                wdf[bl * C::TJ + jl] = d * (float)(int8_t)(scw & 0xFFu);
                wdf[(CB + bl) * C::TJ + jl] = d * (float)(int8_t)((scw >> 8) & 0xFFu);
            } else if constexpr (Q8) {
                if (idx >= C::TJ * CB) continue;
                const int jl = idx / CB, bl = idx % CB;
                const int j = j0 + jl, b = c * CB + bl;
                const uint32_t base = (uint32_t)j * row_bytes + (uint32_t)b * 34u, al = base & ~3u;
                const bool mis = (base & 2u) != 0;
                // the window's last dword, read 2 bytes early at the matrix's end
                const uint32_t w8 = al + 32u > wbytes - 4u ? r.w[u][8] >> 16 : r.w[u][8];
                // codes from byte 2 (block on a dword) or 4 of the window, + 128
                uint32_t q[8];
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint32_t hi = i == 7 ? w8 : r.w[u][i + 1];
                    q[i] = (mis ? hi : perm(hi, r.w[u][i], 0x05040302u)) ^ 0x80808080u;
                }
                uint2* dst = reinterpret_cast<uint2*>(wn + jl * C::WNS + bl * 32);
#pragma unroll
                for (int i = 0; i < 4; i++) dst[i] = uint2{q[2 * i], q[2 * i + 1]};
                // rows or blocks past the matrix loaded zeros: d = 0
                wd[bl * C::TJ + jl] = (uint16_t)(mis ? r.w[u][0] >> 16 : r.w[u][0] & 0xFFFFu);
            } else if constexpr (Q41) {
                if (idx >= C::TJ * CB) continue;
                const int jl = idx / CB, bl = idx % CB;
                // the 16 nibble bytes in a Q4_0 block's order; {d, 8 d + m} in f32
                uint2* dst = reinterpret_cast<uint2*>(wn + jl * Lds<CB>::WN_STRIDE + bl * 16);
                dst[0] = uint2{r.w[u][1], r.w[u][2]};
                dst[1] = uint2{r.w[u][3], r.w[u][4]};
                const float d = h2f(r.w[u][0] & 0xFFFFu), mm = h2f(r.w[u][0] >> 16);
                float* wdf = reinterpret_cast<float*>(st + C::WN_BYTES);
                wdf[bl * C::TJ + jl] = d;
                wdf[(CB + bl) * C::TJ + jl] = 8.0f * d + mm;
            } else if (idx < C::TJ * CB) {
                const int jl = idx / CB, bl = idx % CB;
                const int j = j0 + jl, b = c * CB + bl;
                const uint32_t off = (j < n && b < nb) ? (uint32_t)j * row_bytes + (uint32_t)b * 18u : RSRC_OOB;
                const uint32_t base = off & ~3u;
                const uint32_t wt = r.w[u][C::WWORDS - 1];
                const uint32_t w4 = (base < wbytes && base + 20u > wbytes) ? (wt >> 16) : wt;
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
                if constexpr (C::AF16) {
                    // elements 8 g .. 8 g + 7 at 16 g: the low nibbles of bytes
                    // 0-7, 8-15, then the high ones (rows or blocks past the
                    // matrix: codes -8 with d = 0)
                    constexpr uint32_t NIB = 0x0F0F0F0Fu;
                    half8_t* dst = reinterpret_cast<half8_t*>(wn + jl * C::WNS + bl * 64);
                    dst[0] = q_f16(lo.x & NIB, lo.y & NIB);
                    dst[1] = q_f16(hi.x & NIB, hi.y & NIB);
                    dst[2] = q_f16((lo.x >> 4) & NIB, (lo.y >> 4) & NIB);
                    dst[3] = q_f16((hi.x >> 4) & NIB, (hi.y >> 4) & NIB);
                } else {
                    uint2* dst = reinterpret_cast<uint2*>(wn + jl * Lds<CB>::WN_STRIDE + bl * 16);
                    dst[0] = lo;
                    dst[1] = hi;
                }
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
        if constexpr (C::XSUMS) {
            uint32_t* xs = reinterpret_cast<uint32_t*>(xss);
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
        const float* wdf = reinterpret_cast<const float*>(st + C::WN_BYTES);
        const uint8_t* x0s = st + C::WN_BYTES + C::WD_BYTES;
        const uint8_t* x1s = x0s + C::X_BYTES;
        const float* xss = reinterpret_cast<const float*>(x0s + (NATIVE ? 1 : 2) * C::X_BYTES);
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const int bl = ks * KB + kb;  // this wave's block within the chunk
            typename std::conditional<NATIVE, long, half8_t>::type aq[FJ];
            half8_t a1[Q6 ? FJ : 1];
            f32x4 dv[FJ], ev[FJ];
#pragma unroll
            for (int a = 0; a < FJ; a++) {
                const int jt = (wj * FJ + a) * 16;
                if constexpr (Q6) {
                    // lane group g: codes of elements 8 g .. 8 g + 7; aq keeps those
                    // of sub-block 0 (g < 2), a1 those of sub-block 1
                    const uint2 c8 = *reinterpret_cast<const uint2*>(wn + (jt + r16) * C::WNS + bl * 32 + 8 * g);
                    const half8_t q = q_f16<32>(c8.x, c8.y);
                    const half8_t zero = {};
                    aq[a] = g < 2 ? q : zero;
                    a1[a] = g < 2 ? zero : q;
                } else if constexpr (Q8) {
                    // lane group g: codes (+ 128) of elements 8 g .. 8 g + 7
                    const uint2 c8 = *reinterpret_cast<const uint2*>(wn + (jt + r16) * C::WNS + bl * 32 + 8 * g);
                    aq[a] = q_f16<128>(c8.x, c8.y);
                } else if constexpr (C::AF16) {
                    aq[a] = *reinterpret_cast<const half8_t*>(wn + (jt + r16) * C::WNS + bl * 64 + 16 * g);
                } else {
                    const uint2 nb8 = *reinterpret_cast<const uint2*>(wn + (jt + r16) * C::WNS + bl * 16 + 8 * (g & 1));
                    const uint32_t sh = (g >> 1) * 4;  // groups 2, 3: high nibbles
                    const uint32_t n0 = (nb8.x >> sh) & 0x0F0F0F0Fu, n1 = (nb8.y >> sh) & 0x0F0F0F0Fu;
                    if constexpr (NATIVE) aq[a] = q_i8(n0, n1);
                    else aq[a] = q_f16(n0, n1);
                }
                if constexpr (PAIRS) {
                    dv[a] = *reinterpret_cast<const f32x4*>(wdf + bl * C::TJ + jt + 4 * g);
                    ev[a] = *reinterpret_cast<const f32x4*>(wdf + (CB + bl) * C::TJ + jt + 4 * g);
                } else {
                    const uint2 dd = *reinterpret_cast<const uint2*>(wd + bl * C::TJ + jt + 4 * g);
                    dv[a] = f32x4{h2f(dd.x & 0xFFFFu), h2f(dd.x >> 16), h2f(dd.y & 0xFFFFu), h2f(dd.y >> 16)};
                }
            }
#pragma unroll
            for (int b = 0; b < FI; b++) {
                const int il = (wi * FI + b) * 16 + r16;
                if constexpr (NATIVE) {
                    const long bx = *reinterpret_cast<const long*>(x0s + il * XSTR + bl * 32 + g * 8);
                    const float sx = xss[bl * C::TI + il];
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
                    const float sx = SUMS ? xss[bl * C::TI + il] : 0.0f;
#pragma unroll
                    for (int a = 0; a < FJ; a++) {
                        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                        f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[a], bh, z, 0, 0, 0);
                        t = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[a], bl8, t, 0, 0, 0);
                        if constexpr (SUMS) {
#pragma unroll
                            for (int u = 0; u < 4; u++)
                                acc[a][b][u] = fmaf(dv[a][u], t[u], fmaf(ev[a][u], sx, acc[a][b][u]));
                        } else if constexpr (Q6) {
                            // t: elements 16..31 zeroed (sub-block 0); t1: 0..15 zeroed
                            f32x4 t1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[a], bh, z, 0, 0, 0);
                            t1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[a], bl8, t1, 0, 0, 0);
#pragma unroll
                            for (int u = 0; u < 4; u++)
                                acc[a][b][u] = fmaf(dv[a][u], t[u], fmaf(ev[a][u], t1[u], acc[a][b][u]));
                        } else {
#pragma unroll
                            for (int u = 0; u < 4; u++) acc[a][b][u] = fmaf(dv[a][u], t[u], acc[a][b][u]);
                        }
                    }
                }
            }
            if constexpr (!NATIVE && !SUMS && !Q6 && FI * FJ == 16 && KB == 1) {
                // the 128 x 128 tile: each tile's two MFMAs followed by four
                // VALU instructions (the previous tile's scale FMAs).  The
                // scheduler otherwise issues all 32 of a block's MFMAs first,
                // keeping every product live at once, and spills (256 -> 230
                // VGPRs, no scratch; M = 2048 309-313 -> 323-326 TFLOP/s; the
                // 128 x 64 tile measured 1-2 % slower with it)
#pragma unroll
                for (int p = 0; p < FI * FJ; p++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
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
            // accy: y += the product (the residual add, one rounding as x + y)
            if (j + 3 < n && ((n & 3) == 0)) {
                f32x4 r = f32x4{ldexpf(v[0], e), ldexpf(v[1], e), ldexpf(v[2], e), ldexpf(v[3], e)};
                if (accy) r = *reinterpret_cast<const f32x4*>(yp) + r;
                *reinterpret_cast<f32x4*>(yp) = r;
            } else {
#pragma unroll
                for (int t = 0; t < 4; t++)
                    if (j + t < n) yp[t] = accy ? yp[t] + ldexpf(v[t], e) : ldexpf(v[t], e);
            }
        }
    }
}

// ---- XCD placement ----------------------------------------------------------------------
// MI355X deals the workgroups of a launch round-robin to its 8 XCDs (each
// with its own L2): workgroup b runs on XCD (b + o) % 8, o fixed for the
// launch.  The x-tile GEMM relies on it to keep a strip's K-slices, which
// share b % 8, in one L2 (plain partial stores, read back with non-temporal
// loads by the last slice); the probe below checks it once per device, and
// the kernel falls back to agent-coherent stores and loads where it does not
// hold.
__global__ void xcd_probe_kernel(int* __restrict__ out) {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    if (threadIdx.x == 0) out[blockIdx.x] = (int)(x & 0xF);
}

namespace {
constexpr int XCD_COUNT = 8;
constexpr int MAX_DEVICES = 64;
std::mutex xcd_mu;
int xcd_state[MAX_DEVICES] = {};             // per device: 0 unknown, 1 rotation, 2 not
std::atomic<bool> combine_coherent{false};  // testing switch: every combine coherent
}  // namespace

// True when, on the current device, every launch deals its workgroups
// round-robin to the 8 XCDs from some starting XCD: workgroup b on XCD (b +
// o) % 8.  The starting XCD o depends on the hardware queue (measured on
// MI355X: 6, 7, 0, 0, 7, 6 for six streams, each the same on every launch,
// also with two queues' launches in flight together), so what the probe
// checks -- on a private stream, 2 x CUs workgroups recording their XCC id
// -- is the rotation, not o = 0.  Under it all workgroups with one b % 8 share
// an XCD, which is all the XCD-local combine needs.  Probed once per device,
// never while `s` is being captured into a graph (that call takes the
// coherent combine); false while the testing switch asks for the coherent
// combine.
bool xcd_round_robin(hipStream_t s) {
    if (combine_coherent.load()) return false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return false;
    std::lock_guard<std::mutex> lock(xcd_mu);
    if (xcd_state[dev]) return xcd_state[dev] == 1;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (s && hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) return false;
    const int nwg = 2 * device_cu_count();
    int* d = nullptr;
    hipStream_t ps = nullptr;
    bool ok = hipStreamCreateWithFlags(&ps, hipStreamNonBlocking) == hipSuccess &&
              hipMalloc(&d, nwg * sizeof(int)) == hipSuccess;
    std::vector<int> h(nwg, -1);
    if (ok) {
        hipLaunchKernelGGL(xcd_probe_kernel, dim3(nwg), dim3(64), 0, ps, d);
        ok = hipGetLastError() == hipSuccess && hipStreamSynchronize(ps) == hipSuccess &&
             hipMemcpy(h.data(), d, nwg * sizeof(int), hipMemcpyDeviceToHost) == hipSuccess;
    }
    for (int b = 0; ok && b < nwg; b++) ok = h[b] == (h[0] + b) % XCD_COUNT;
    if (d) (void)hipFree(d);
    if (ps) (void)hipStreamDestroy(ps);
    xcd_state[dev] = ok ? 1 : 2;
    return ok;
}

// ---- skinny GEMM (m <= GEMM_SMALL_M) ----------------------------------------------
// With few x rows, x is the costly operand: a workgroup that owns a strip of
// W over the whole of K must read and split all of x, and the split alone
// (about ten VALU operations an element) then outweighs the weight stream.
// Here a workgroup owns R weight rows over one K-slice: the grid is
// ceil(n / R) strips x S slices, S chosen to fill the CUs, so each x element
// is split by ceil(n / R) workgroups instead of n / 16.  Per chunk of KCB
// blocks of its slice:
//  1. the whole workgroup loads the chunk's x (coalesced) and splits it into
//     LDS: per (row, block) e = ilogb(max |x|) - 14 (0 for an all-zero or
//     non-finite block), x' = x 2^-e, x_hi = f16(x'), x_lo = f16(x' - x_hi)
//     (0 where x' is infinite), and the f32 scale 2^e;
//  2. wave (wr, wk) multiplies its JT row tiles (16 weight rows each) over its
//     KBW blocks of the chunk, x tiles from LDS: per (tile, block) two f16
//     MFMAs on the exact (q - 8) give the block dot, scaled by d 2^e in f32.
//     Its weight loads for the next chunk are in flight meanwhile.
// The WK waves of a row group are summed in wave order through LDS.  With
// S > 1 each workgroup publishes its strip partial, waits for the stores to
// complete, and counts itself on the strip's counter; the last of the S sums
// all S partials in slice order (the same bits whichever workgroup finishes
// last) and resets the counter to 0 for the next launch.  Where the probed
// placement holds (xcd_round_robin) a strip's slices share one XCD and the
// partials stay in its L2 (plain stores, non-temporal loads); elsewhere
// agent-coherent (sc1) stores and loads.
constexpr int SK_WAVES = 8;

template <int MT, int JT, int WR>
struct SkCfg {
    static constexpr int NT = SK_WAVES * 64;
    static constexpr int WK = SK_WAVES / WR;          // waves splitting a chunk's blocks
    static constexpr int R = 16 * JT * WR;            // weight rows per workgroup
    static constexpr int MP = 16 * MT;                // x rows held in LDS
    static constexpr int KCB = MT == 1 ? 32 : MT == 2 ? 16 : 8;  // blocks per chunk
    static constexpr int KBW = KCB / WK;              // blocks per wave and chunk
    static constexpr int XROW = KCB * 64 + 16;        // LDS bytes per x row of f16 (padded)
    static constexpr int X_BYTES = MP * XROW;
    static constexpr int SC_BYTES = KCB * MP * 4;     // block scales [block][row]
    static constexpr int D_BYTES = SK_WAVES * JT * KBW * 16 * 4;
    static constexpr int STAGE = 2 * X_BYTES + SC_BYTES + D_BYTES;
    static constexpr int UNITS = WR * MT * JT * 64;   // f32x4 outputs per workgroup
    static constexpr int UPT = (UNITS + NT - 1) / NT; // per thread
    static constexpr int RED = SK_WAVES * MT * JT * 64 * 16;
    static constexpr int LDS = STAGE > RED ? STAGE : RED;
    static constexpr int XU = (MP * KCB * 4 + NT - 1) / NT;  // 8-element x pieces per thread and chunk
    static_assert(XU <= 4, "x pieces held in registers");
    static_assert(KBW * WK == KCB, "chunk blocks split evenly over the waves");
};

// Cache policy bits of buffer loads / stores (gfx950): nt (non-temporal: no
// stale L1 line), sc1 (device scope: written through / read from the
// device's coherence point).
constexpr int CPOL_NT = 2, CPOL_SC1 = 16;

// EVEN: nb and the slice length even, so every chunk's first block starts on a
// dword and a lane's weight words sit at fixed offsets from one base.
template <int MT, int JT, int WR, bool EVEN, bool LOCAL>
__global__ __launch_bounds__(SK_WAVES * 64) void gemm_q4_0_skinny_kernel(
    const uint8_t* __restrict__ W, int n, int nb, const float* __restrict__ X, int m, float* __restrict__ Y, int S,
    int kbs, float* __restrict__ part, int* __restrict__ cnt) {
    using C = SkCfg<MT, JT, WR>;
    constexpr int KBW = C::KBW, KCB = C::KCB, MP = C::MP;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int last_sh;
    uint8_t* xh_s = lds;
    uint8_t* xl_s = lds + C::X_BYTES;
    float* sc_s = reinterpret_cast<float*>(lds + 2 * C::X_BYTES);
    float* d_s = reinterpret_cast<float*>(lds + 2 * C::X_BYTES + C::SC_BYTES);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r = lane & 15, h = g & 1;
    const int wr = wave / C::WK, wk = wave % C::WK;
    // LOCAL: strip st's slices share b % 8 = st % 8, so one XCD (one L2), as in the x-tile kernel
    int strip, ks;
    if constexpr (LOCAL) {
        const int xcd = (int)blockIdx.x % XCD_COUNT, i = (int)blockIdx.x / XCD_COUNT;
        strip = (i / S) * XCD_COUNT + xcd;
        ks = i % S;
    } else {
        strip = (int)blockIdx.x / S;
        ks = (int)blockIdx.x % S;
    }
    if (strip * C::R >= n) return;  // grid rounded up to whole XCD rounds (whole workgroup)
    const int j0 = strip * C::R;
    const int kb0 = min(nb, ks * kbs), kb1 = min(nb, kb0 + kbs);
    const int nchunks = (kb1 - kb0 + KCB - 1) / KCB;  // workgroup-uniform
    const uint32_t k = (uint32_t)nb * 32u;
    const uint32_t row_bytes = (uint32_t)nb * 18u;
    const uint32_t wbytes = (uint32_t)n * row_bytes;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(W, wbytes);
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(X, (uint32_t)m * k * 4u);
    float* dw = d_s + wave * (JT * KBW * 16);

    struct WRegs { uint32_t w[JT][KBW][3]; };
    // the wave's weight bytes of chunk c: for row j and block b, lane (g, r)
    // holds the 12 dword-aligned bytes holding its 8 nibble bytes (and, for
    // h == 0, the block's d)
    auto load_w = [&](int c, WRegs& R) {
        if constexpr (EVEN) {
            // block b0 + q of row j starts at j row_bytes + 18 b0 + 18 q, on a
            // dword for even q and 2 bytes past one for odd q; rows >= n fall
            // past the buffer (zeros), blocks past the slice get d = 0 below
            const uint32_t bc = (uint32_t)(kb0 + c * KCB + wk * KBW);
#pragma unroll
            for (int jt = 0; jt < JT; jt++) {
                const uint32_t base =
                    (uint32_t)(j0 + (wr * JT + jt) * 16 + r) * row_bytes + bc * 18u + 8u * (uint32_t)h;
#pragma unroll
                for (int q = 0; q < KBW; q++) {
                    const auto v = __builtin_amdgcn_raw_buffer_load_b96(wrs, (int)(base + 18u * q - 2u * (q & 1)), 0, 0);
                    R.w[jt][q][0] = v[0], R.w[jt][q][1] = v[1], R.w[jt][q][2] = v[2];
                }
            }
            return;
        }
#pragma unroll
        for (int jt = 0; jt < JT; jt++) {
            const int j = j0 + (wr * JT + jt) * 16 + r;
#pragma unroll
            for (int q = 0; q < KBW; q++) {
                const int b = kb0 + c * KCB + wk * KBW + q;
                const uint32_t boff = (uint32_t)j * row_bytes + (uint32_t)b * 18u;
                const uint32_t a = (j < n && b < kb1) ? ((boff + 8u * h) & ~3u) : RSRC_OOB;
                const auto v = __builtin_amdgcn_raw_buffer_load_b96(wrs, (int)a, 0, 0);
                R.w[jt][q][0] = v[0], R.w[jt][q][1] = v[1], R.w[jt][q][2] = v[2];
                // the matrix's last block when it ends 2 bytes into a dword:
                // that dword is out of range as a whole, its 2 bytes are not
                if (a < wbytes && a + 12u > wbytes) R.w[jt][q][2] = buf_load_b16(wrs, a + 8u);
            }
        }
    };
    // chunk c of x: the 8-element pieces of this thread (rows >= m and blocks
    // past the slice read as zero), loaded ahead of the chunk's weights so
    // that splitting them never waits for the weight stream
    struct XRegs { u32x4 v0[C::XU], v1[C::XU]; };
    auto load_x = [&](int c, XRegs& X) {
        const int cb0 = kb0 + c * KCB;
#pragma unroll
        for (int u = 0; u < C::XU; u++) {
            const int idx = tid + u * C::NT;
            const int row = idx / (KCB * 4), blk = (idx >> 2) % KCB, qt = idx & 3;
            const int b = cb0 + blk;
            const uint32_t off = (idx < MP * KCB * 4 && row < m && b < kb1)
                                     ? ((uint32_t)row * k + (uint32_t)b * 32u + (uint32_t)qt * 8u) * 4u
                                     : RSRC_OOB;
            X.v0[u] = buf_load_b128(xrs, off);
            X.v1[u] = buf_load_b128(xrs, off == RSRC_OOB ? RSRC_OOB : off + 16u);
        }
    };
    // the pieces split into LDS: x_hi = f16(x') rounded toward zero, x_lo =
    // f16(x' - x_hi) (x_hi + x_lo keeps about 22 significant bits either way)
    auto split_x = [&](const XRegs& X) {
#pragma unroll
        for (int u = 0; u < C::XU; u++) {
            const int idx = tid + u * C::NT;
            const int row = idx / (KCB * 4), blk = (idx >> 2) % KCB, qt = idx & 3;
            float xv[8];
            uint32_t amax = 0;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t bits = e < 4 ? X.v0[u][e] : X.v1[u][e - 4];
                xv[e] = __builtin_bit_cast(float, bits);
                amax = max(amax, bits & 0x7FFFFFFFu);
            }
            // the four lanes of a block are adjacent (idx = tid + u * NT)
            amax = max(amax, (uint32_t)dpp_i32<DPP_QUAD_XOR1>((int)amax));
            amax = max(amax, (uint32_t)dpp_i32<DPP_QUAD_XOR2>((int)amax));
            int ex = 0;
            if (amax != 0 && amax < 0x7F800000u)
                ex = (amax >= 0x00800000u ? (int)(amax >> 23) - 127 : (31 - (int)__builtin_clz(amax)) - 149) - 14;
            // an infinite x keeps its sign through the product: x_lo = 0 for a
            // block holding one (inf - inf would be NaN)
            const bool fin = amax < 0x7F800000u;
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float a = ldexpf(xv[e], -ex), b = ldexpf(xv[e + 1], -ex);
                const h2 hp = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(a, b));
                const h2 lp = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(a - (float)hp[0], b - (float)hp[1]));
                hw[e / 2] = __builtin_bit_cast(uint32_t, hp);
                lw[e / 2] = fin ? __builtin_bit_cast(uint32_t, lp) : 0u;
            }
            if (idx < MP * KCB * 4) {
                *reinterpret_cast<u32x4*>(xh_s + row * C::XROW + blk * 64 + qt * 16) = u32x4{hw[0], hw[1], hw[2], hw[3]};
                *reinterpret_cast<u32x4*>(xl_s + row * C::XROW + blk * 64 + qt * 16) = u32x4{lw[0], lw[1], lw[2], lw[3]};
                if (qt == 0) sc_s[blk * MP + row] = ldexpf(1.0f, ex);
            }
        }
    };

    f32x4 acc[MT][JT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int jt = 0; jt < JT; jt++) acc[t][jt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    WRegs wreg;
    XRegs xreg;
    auto compute = [&](int c) {
        WRegs& R = wreg;
        half8_t aq[JT][KBW];
#pragma unroll
        for (int jt = 0; jt < JT; jt++) {
            const uint32_t j = (uint32_t)(j0 + (wr * JT + jt) * 16 + r);
#pragma unroll
            for (int q = 0; q < KBW; q++) {
                const int b = kb0 + c * KCB + wk * KBW + q;
                const bool odd = EVEN ? (q & 1) != 0  // the block starts 2 bytes into a dword
                                      : ((j * row_bytes + (uint32_t)b * 18u) & 2u) != 0;
                const uint32_t lo = odd ? R.w[jt][q][1] : perm(R.w[jt][q][1], R.w[jt][q][0], 0x05040302u);
                const uint32_t hi = odd ? R.w[jt][q][2] : perm(R.w[jt][q][2], R.w[jt][q][1], 0x05040302u);
                const uint32_t sh = (g >> 1) * 4;
                aq[jt][q] = q_f16((lo >> sh) & 0x0F0F0F0Fu, (hi >> sh) & 0x0F0F0F0Fu);
                if (g == 0) {
                    const float d = h2f(odd ? R.w[jt][q][0] >> 16 : R.w[jt][q][0] & 0xFFFFu);
                    dw[(jt * KBW + q) * 16 + r] = (!EVEN || b < kb1) ? d : 0.0f;
                }
            }
        }
        // the raw registers are free: the next chunk's x, then its weights,
        // load during this chunk's products
        if (c + 1 < nchunks) {
            load_x(c + 1, xreg);
            load_w(c + 1, R);
        }
#pragma unroll
        for (int t = 0; t < MT; t++) {
#pragma unroll
            for (int q = 0; q < KBW; q++) {
                const int qa = wk * KBW + q;
                const int xo = (16 * t + r) * C::XROW + qa * 64 + g * 16;
                const half8_t bh = *reinterpret_cast<const half8_t*>(xh_s + xo);
                const half8_t bl = *reinterpret_cast<const half8_t*>(xl_s + xo);
                const float sx = sc_s[qa * MP + 16 * t + r];
#pragma unroll
                for (int jt = 0; jt < JT; jt++) {
                    const f32x4 dv = *reinterpret_cast<const f32x4*>(dw + (jt * KBW + q) * 16 + 4 * g);
                    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                    f32x4 cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[jt][q], bh, z, 0, 0, 0);
                    cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[jt][q], bl, cc, 0, 0, 0);
#pragma unroll
                    for (int u = 0; u < 4; u++) acc[t][jt][u] = fmaf(dv[u] * sx, cc[u], acc[t][jt][u]);
                }
            }
        }
    };

    // chunks: x split into LDS, then the products
    if (nchunks > 0) {
        load_x(0, xreg);
        load_w(0, wreg);
    }
    for (int c = 0; c < nchunks; c++) {
        split_x(xreg);
        __syncthreads();  // the chunk's x is in LDS
        compute(c);
        __syncthreads();  // every wave is done with the chunk's LDS
    }

    // wave sums of each row group, in wave order
    f32x4* red = reinterpret_cast<f32x4*>(lds);
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int jt = 0; jt < JT; jt++) red[((wave * MT + t) * JT + jt) * 64 + lane] = acc[t][jt];
    __syncthreads();
    // unit u = ((wr * MT + t) * JT + jt) * 64 + l: y[16 t + l % 16][row tile (wr JT + jt), 4 (l / 16) ..]
    f32x4 own[C::UPT];
#pragma unroll
    for (int p = 0; p < C::UPT; p++) {
        const int u = tid + p * C::NT;
        if (u >= C::UNITS) break;
        const int ln = u & 63, tj = u >> 6, jt = tj % JT, t = (tj / JT) % MT, wru = tj / (JT * MT);
        f32x4 sum = red[(((wru * C::WK) * MT + t) * JT + jt) * 64 + ln];
        for (int w = 1; w < C::WK; w++) sum += red[(((wru * C::WK + w) * MT + t) * JT + jt) * 64 + ln];
        own[p] = sum;
    }
    if (S > 1) {
        // the strip's partials: LOCAL into this XCD's L2 (plain stores), else
        // written through to the device's coherence point (sc1)
        const __amdgpu_buffer_rsrc_t prs = make_rsrc(part + (size_t)strip * S * C::UNITS * 4,
                                                     (uint32_t)S * C::UNITS * 16u);
#pragma unroll
        for (int p = 0; p < C::UPT; p++) {
            const int u = tid + p * C::NT;
            if (u < C::UNITS)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, own[p]), prs,
                                                       (int)(((uint32_t)ks * C::UNITS + u) * 16u), 0,
                                                       LOCAL ? 0 : CPOL_SC1);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partials have completed
        __syncthreads();
        if (tid == 0) {
            // LOCAL: the strip's slices all run on this XCD (one b % 8), so the
            // count lives in its L2: an L2 atomic, not a device-scope one
            // written through past it (M = 16: 10.9 -> 10.6 us a call)
            const int old = __hip_atomic_fetch_add(cnt + strip, 1, __ATOMIC_RELAXED,
                                                   LOCAL ? __HIP_MEMORY_SCOPE_WORKGROUP : __HIP_MEMORY_SCOPE_AGENT);
            last_sh = old == S - 1;
            if (old == S - 1)
                __hip_atomic_store(cnt + strip, 0, __ATOMIC_RELAXED,
                                   LOCAL ? __HIP_MEMORY_SCOPE_WORKGROUP : __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last_sh) return;
#pragma unroll
        for (int p = 0; p < C::UPT; p++) {
            const int u = tid + p * C::NT;
            if (u >= C::UNITS) break;
            // every slice's partial in flight together (groups of 8, branch-free:
            // slots past S or of this slice read zeros), then added in slice
            // order; LOCAL reads the L2 with non-temporal loads, else sc1
            f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int s0 = 0; s0 < S; s0 += 8) {
                f32x4 v[8];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const int sl = s0 + q;
                    const uint32_t off = (sl < S && sl != ks) ? ((uint32_t)sl * C::UNITS + u) * 16u : RSRC_OOB;
                    v[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, (int)off, 0,
                                                                                            LOCAL ? CPOL_NT : CPOL_SC1));
                }
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const int sl = s0 + q;
                    const f32x4 t = sl == ks ? own[p] : v[q];
                    if (sl < S) sum = sl == 0 ? t : sum + t;
                }
            }
            own[p] = sum;
        }
    }
#pragma unroll
    for (int p = 0; p < C::UPT; p++) {
        const int u = tid + p * C::NT;
        if (u >= C::UNITS) break;
        const int ln = u & 63, tj = u >> 6, jt = tj % JT, t = (tj / JT) % MT, wru = tj / (JT * MT);
        const int i = 16 * t + (ln & 15);
        const int j = j0 + (wru * JT + jt) * 16 + 4 * (ln >> 4);
        if (i >= m) continue;
        float* yp = Y + (size_t)i * n + j;
        if (j + 3 < n && (n & 3) == 0) {
            *reinterpret_cast<f32x4*>(yp) = own[p];
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++)
                if (j + c < n) yp[c] = own[p][c];
        }
    }
}

// ---- x-tile GEMM for m <= 64: K-slices joined through a strip counter -----------
// MT = ceil(m / 16) x tiles of 16 rows.  A workgroup of 8 waves owns 128
// weight rows (a 16-row tile a wave) over one K-slice of at most KB blocks;
// the grid is ceil(n / 128) strips x S slices, S chosen for about one
// workgroup per CU, so each x element is split by n / 128 workgroups and a
// workgroup streams 128 rows x KB blocks of W against 16 MT x KB blocks of x
// (n = k = 4096, m = 16: 36 KB of W and 32 KB of x).  Per workgroup:
//  1. every load at once: the wave's weight windows (one 12-byte window a
//     lane and block, the B operand of the MFMA) and the x tiles (8-element
//     pieces, coalesced);
//  2. x split into LDS as in the skinny kernel above (per (row, block) scale
//     2^e, x_hi + x_lo in f16);
//  3. per block and x tile two v_mfma_f32_16x16x32_f16 with x as the A
//     operand, so the lane's output column is its own weight row and its
//     block scale d is in its own window (or its partner's, l ^ 16, through a
//     permlane swap), decoded once for all tiles; acc += d * 2^e * dot in f32
//     (4 x rows a lane and tile);
//  4. the S slices of a strip meet through a counter: each writes its 16 MT x
//     128 partial, waits for the stores, counts itself on the strip's counter,
//     and the last of the S adds all partials in slice order (the same bits
//     whichever finishes last), resets the counter and stores Y.  Where the
//     workgroup placement is the probed round-robin (xcd_round_robin), a
//     strip's slices are put on one XCD and the partials stay in its L2:
//     plain 16-byte stores (acknowledged by the L2), read back with
//     non-temporal loads, which do not return a stale L1 line; measured at M =
//     16, the partial stores and their reads took 2.4 + 3.7 us as agent-coherent
//     (write-through) traffic.  Elsewhere agent-coherent stores and loads.
// Against the skinny kernel above (M = 32 / 48 / 64: 74 / 95 / 107 TFLOP/s)
// this shape runs 80 / 99 / 113; the skinny kernel remains for calls that
// give no partial buffer and a slice longer than the LDS allows.
constexpr int XT_WAVES = 8;
constexpr int XT_ROWS = 16 * XT_WAVES;  // weight rows per workgroup
constexpr int XT_UNITS = XT_WAVES * 64;  // f32x4 partial units per workgroup and x tile (16 x rows x 128 weight rows)

template <int KB, int MT>
struct XtCfg {
    static constexpr int NT = XT_WAVES * 64;
    static constexpr int XR = 16 * MT;                 // x rows (MT tiles of 16)
    static constexpr int XROW = KB * 64 + 16;          // LDS bytes per x row of f16 (padded)
    static constexpr int X_BYTES = XR * XROW;
    static constexpr int SC_BYTES = KB * XR * 4;       // block scales [block][x row]
    static constexpr int LDS = 2 * X_BYTES + SC_BYTES;
    static constexpr int XU = (XR * KB * 4 + NT - 1) / NT;  // 8-element x pieces per thread
    static constexpr int UNITS = XT_UNITS * MT;      // f32x4 partial units per workgroup
    static_assert(XU <= 8, "x pieces held in registers");
};

// EVEN: nb and the slice length even, so every slice's first block starts on a
// dword and a lane's weight windows sit at fixed offsets from one base.
template <int KB, int MT, bool EVEN, bool LOCAL>
__global__ __launch_bounds__(XT_WAVES * 64) void gemm_q4_0_xtile_kernel(
    const uint8_t* __restrict__ W, int n, int nb, const float* __restrict__ X, int m, float* __restrict__ Y, int S,
    int kbs, float* __restrict__ part, int* __restrict__ cnt) {
    using C = XtCfg<KB, MT>;
    constexpr int XR = C::XR, UNITS = C::UNITS;
    __shared__ int last_sh;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t* xh_s = lds;
    uint8_t* xl_s = lds + C::X_BYTES;
    float* sc_s = reinterpret_cast<float*>(lds + 2 * C::X_BYTES);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r = lane & 15, h = g & 1;
    // local: strip st's slices are the workgroups b with b % 8 = st % 8, which
    // run on one XCD (a rotation of b % 8, probed) and share its L2; otherwise
    // strips are consecutive slices
    int strip, ks;
    if constexpr (LOCAL) {
        const int xcd = (int)blockIdx.x % XCD_COUNT, i = (int)blockIdx.x / XCD_COUNT;
        strip = (i / S) * XCD_COUNT + xcd;
        ks = i % S;
    } else {
        strip = (int)blockIdx.x / S;
        ks = (int)blockIdx.x % S;
    }
    if (strip * XT_ROWS >= n) return;  // grid rounded up to whole XCD rounds (whole workgroup)
    const int kb0 = min(nb, ks * kbs), kb1 = min(nb, kb0 + kbs);
    const uint32_t k = (uint32_t)nb * 32u;
    const uint32_t row_bytes = (uint32_t)nb * 18u;
    const uint32_t wbytes = (uint32_t)n * row_bytes;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(W, wbytes);
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(X, (uint32_t)m * k * 4u);
    const int j = strip * XT_ROWS + wave * 16 + r;  // the lane's weight row (output column)

    // 1. loads: x pieces first, then the weight windows
    u32x4 xa[C::XU], xb[C::XU];
#pragma unroll
    for (int u = 0; u < C::XU; u++) {
        const int idx = tid + u * C::NT;
        const int row = idx / (KB * 4), blk = (idx >> 2) % KB, qt = idx & 3;
        const int b = kb0 + blk;
        const uint32_t off = (idx < XR * KB * 4 && row < m && b < kb1)
                                 ? ((uint32_t)row * k + (uint32_t)b * 32u + (uint32_t)qt * 8u) * 4u
                                 : RSRC_OOB;
        xa[u] = buf_load_b128(xrs, off);
        xb[u] = buf_load_b128(xrs, off == RSRC_OOB ? RSRC_OOB : off + 16u);
    }
    uint32_t wv[KB][3];
    if constexpr (EVEN) {
        // block kb0 + q of row j starts at j row_bytes + 18 kb0 + 18 q, on a
        // dword for even q and 2 bytes past one for odd q; rows >= n fall
        // past the buffer (zeros), blocks past the slice get d = 0 below
        const uint32_t base = (uint32_t)j * row_bytes + (uint32_t)kb0 * 18u + 8u * (uint32_t)h;
#pragma unroll
        for (int q = 0; q < KB; q++) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b96(wrs, (int)(j < n ? base + 18u * q - 2u * (q & 1) : RSRC_OOB), 0, 0);
            wv[q][0] = v[0], wv[q][1] = v[1], wv[q][2] = v[2];
        }
    } else {
#pragma unroll
        for (int q = 0; q < KB; q++) {
            const int b = kb0 + q;
            const uint32_t boff = (uint32_t)j * row_bytes + (uint32_t)b * 18u;
            const uint32_t a = (j < n && b < kb1) ? ((boff + 8u * h) & ~3u) : RSRC_OOB;
            const auto v = __builtin_amdgcn_raw_buffer_load_b96(wrs, (int)a, 0, 0);
            wv[q][0] = v[0], wv[q][1] = v[1], wv[q][2] = v[2];
            // the matrix's last block when it ends 2 bytes into a dword
            if (a < wbytes && a + 12u > wbytes) wv[q][2] = buf_load_b16(wrs, a + 8u);
        }
    }

    // 2. x split into LDS (x_hi = f16(x 2^-e) toward zero, x_lo = f16(rest))
#pragma unroll
    for (int u = 0; u < C::XU; u++) {
        const int idx = tid + u * C::NT;
        const int row = idx / (KB * 4), blk = (idx >> 2) % KB, qt = idx & 3;
        float xv[8];
        uint32_t amax = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t bits = e < 4 ? xa[u][e] : xb[u][e - 4];
            xv[e] = __builtin_bit_cast(float, bits);
            amax = max(amax, bits & 0x7FFFFFFFu);
        }
        amax = max(amax, (uint32_t)dpp_i32<DPP_QUAD_XOR1>((int)amax));  // the four lanes of a block
        amax = max(amax, (uint32_t)dpp_i32<DPP_QUAD_XOR2>((int)amax));
        int ex = 0;
        if (amax != 0 && amax < 0x7F800000u)
            ex = (amax >= 0x00800000u ? (int)(amax >> 23) - 127 : (31 - (int)__builtin_clz(amax)) - 149) - 14;
        const bool fin = amax < 0x7F800000u;  // an infinite x keeps x_lo = 0 (no inf - inf)
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const float a = ldexpf(xv[e], -ex), b = ldexpf(xv[e + 1], -ex);
            const h2 hp = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(a, b));
            const h2 lp = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(a - (float)hp[0], b - (float)hp[1]));
            hw[e / 2] = __builtin_bit_cast(uint32_t, hp);
            lw[e / 2] = fin ? __builtin_bit_cast(uint32_t, lp) : 0u;
        }
        if (idx < XR * KB * 4) {
            *reinterpret_cast<u32x4*>(xh_s + row * C::XROW + blk * 64 + qt * 16) = u32x4{hw[0], hw[1], hw[2], hw[3]};
            *reinterpret_cast<u32x4*>(xl_s + row * C::XROW + blk * 64 + qt * 16) = u32x4{lw[0], lw[1], lw[2], lw[3]};
            if (qt == 0) sc_s[blk * XR + row] = ldexpf(1.0f, ex);
        }
    }
    __syncthreads();

    // 3. products: lane (g, r) holds Y[x rows 16 t + 4g .. + 3][weight row j]
    // for each x tile t
    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < KB; q++) {
        const int b = kb0 + q;
        const bool odd = EVEN ? (q & 1) != 0 : (((uint32_t)j * row_bytes + (uint32_t)b * 18u) & 2u) != 0;
        const uint32_t lo = odd ? wv[q][1] : perm(wv[q][1], wv[q][0], 0x05040302u);
        const uint32_t hi = odd ? wv[q][2] : perm(wv[q][2], wv[q][1], 0x05040302u);
        const uint32_t sh = (uint32_t)(g >> 1) * 4u;
        const half8_t bq = q_f16((lo >> sh) & 0x0F0F0F0Fu, (hi >> sh) & 0x0F0F0F0Fu);
        // d: in the window of the lanes with h == 0; lanes with h == 1 take
        // their partner's (l ^ 16) through a permlane swap
        const uint32_t dbits = odd ? wv[q][0] >> 16 : wv[q][0] & 0xFFFFu;
        const auto sw = __builtin_amdgcn_permlane16_swap(dbits, dbits, false, false);
        const uint32_t other = (sw[0] == dbits) ? sw[1] : sw[0];
        const uint32_t dsel = h ? other : dbits;
        const float d = (b < kb1) ? h2f(dsel) : 0.0f;
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int xo = (16 * t + r) * C::XROW + q * 64 + g * 16;
            const half8_t ah = *reinterpret_cast<const half8_t*>(xh_s + xo);
            const half8_t al = *reinterpret_cast<const half8_t*>(xl_s + xo);
            const f32x4 s4 = *reinterpret_cast<const f32x4*>(sc_s + q * XR + 16 * t + 4 * g);
            const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
            f32x4 cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq, z, 0, 0, 0);
            cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq, cc, 0, 0, 0);
#pragma unroll
            for (int u = 0; u < 4; u++) acc[t][u] = fmaf(d * s4[u], cc[u], acc[t][u]);
        }
    }

    // 4. slices of the strip: partials, counter, the last one adds them
    if (S > 1) {
        // the strip's partials: LOCAL into this XCD's L2 (plain stores), else
        // written through to the device's coherence point (sc1)
        const __amdgpu_buffer_rsrc_t prs = make_rsrc(part + (size_t)strip * S * UNITS * 4,
                                                     (uint32_t)S * UNITS * 16u);
#pragma unroll
        for (int t = 0; t < MT; t++)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[t]), prs,
                                                   (int)(((uint32_t)ks * UNITS + t * XT_UNITS + tid) * 16u), 0,
                                                   LOCAL ? 0 : CPOL_SC1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial has completed
        __syncthreads();
        if (tid == 0) {
            // LOCAL: the strip's slices all run on this XCD (one b % 8), so the
            // count lives in its L2: an L2 atomic, not a device-scope one
            // written through past it (M = 16: 10.9 -> 10.6 us a call)
            const int old = __hip_atomic_fetch_add(cnt + strip, 1, __ATOMIC_RELAXED,
                                                   LOCAL ? __HIP_MEMORY_SCOPE_WORKGROUP : __HIP_MEMORY_SCOPE_AGENT);
            last_sh = old == S - 1;
            if (old == S - 1)
                __hip_atomic_store(cnt + strip, 0, __ATOMIC_RELAXED,
                                   LOCAL ? __HIP_MEMORY_SCOPE_WORKGROUP : __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last_sh) return;
        // every slice's partial in flight together (groups of 8, branch-free:
        // slots past S or of this slice read zeros), then added in slice order;
        // LOCAL reads the L2 with non-temporal loads (no stale L1 line), else sc1
#pragma unroll
        for (int t = 0; t < MT; t++) {
            f32x4 tot = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int s0 = 0; s0 < S; s0 += 8) {
                f32x4 v[8];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const int sl = s0 + q;
                    const uint32_t off =
                        (sl < S && sl != ks) ? ((uint32_t)sl * UNITS + t * XT_UNITS + tid) * 16u : RSRC_OOB;
                    v[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, (int)off, 0,
                                                                                            LOCAL ? CPOL_NT : CPOL_SC1));
                }
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const int sl = s0 + q;
                    const f32x4 tv = sl == ks ? acc[t] : v[q];
                    if (sl < S) tot = sl == 0 ? tv : tot + tv;
                }
            }
            acc[t] = tot;
        }
    }
    if (j < n) {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = 16 * t + 4 * g + u;
                if (i < m) Y[(size_t)i * n + j] = acc[t][u];
            }
    }
}

// Launch plan of the x-tile kernel: 128-row strips, S K-slices of kbs
// blocks (even when nb is) for about one workgroup per CU, KB the template
// bound of kbs (8, 16 or 32; at most 16 with more than one x tile, for the
// LDS).  ok = false (the skinny kernel runs) when a slice would exceed that.
struct XtPlan {
    int strips, S, kbs, KB;
    bool even, ok;
};
inline XtPlan xtile_plan(size_t n, int nb, int mt = 1) {
    // LDS per workgroup: 2 * 16 mt * (64 KB + 16) + 64 KB mt bytes; at most 16
    // blocks a slice when mt > 1
    const int kmax = mt > 1 ? 16 : 32;
    XtPlan p{};
    p.strips = (int)((n + XT_ROWS - 1) / XT_ROWS);
    const int S = std::max(1, (device_cu_count() + p.strips / 2) / p.strips);
    p.kbs = std::max(1, (nb + S - 1) / S);
    p.kbs = std::min(p.kbs, kmax);
    p.even = nb % 2 == 0;
    if (p.even) p.kbs += p.kbs & 1;
    p.S = std::max(1, (nb + p.kbs - 1) / p.kbs);  // no empty slices
    p.KB = p.kbs <= 8 ? 8 : p.kbs <= 16 ? 16 : 32;
    p.ok = p.kbs <= kmax;
    return p;
}

template <int KB, int MT, bool EVEN, bool LOCAL>
hipError_t launch_xtile_cfg(const uint8_t* w, int n, int nb, const float* x, int m, float* y, const XtPlan& p,
                           float* part, int* cnt, hipStream_t s) {
    using C = XtCfg<KB, MT>;
    static_assert(C::LDS <= 160 * 1024, "LDS per workgroup");
    auto kern = gemm_q4_0_xtile_kernel<KB, MT, EVEN, LOCAL>;
    if (C::LDS > 65536) {
        static const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                        C::LDS);  // once per kernel and process
        if (e != hipSuccess) return e;
    }
    const int strips = LOCAL ? (p.strips + XCD_COUNT - 1) / XCD_COUNT * XCD_COUNT : p.strips;
    launch_kernel(kern, dim3((unsigned)(strips * p.S)), dim3(C::NT), (size_t)C::LDS, s, w, n, nb, x, m, y, p.S,
                  p.kbs, part, cnt);
    return hipGetLastError();
}

hipError_t launch_xtile(const uint8_t* w, int n, int nb, const float* x, int m, float* y, float* part, int* cnt,
                       hipStream_t s) {
    const int mt = (m + 15) / 16;
    if (mt < 1 || mt > 4) return hipErrorInvalidValue;
    XtPlan p = xtile_plan((size_t)n, nb, mt);
    if (!part || !cnt) {  // no partial buffer or counters: one slice
        p.S = 1;
        p.kbs = nb;
        p.KB = nb <= 8 ? 8 : nb <= 16 ? 16 : 32;
        p.ok = nb <= (mt > 1 ? 16 : 32);
    }
    if (!p.ok) return hipErrorInvalidValue;  // the caller takes the other kernel
    const bool local = p.S > 1 && xcd_round_robin(s);
    auto go = [&](auto kb_tag, auto mt_tag, auto even_tag) {
        constexpr int KB = decltype(kb_tag)::value, MT = decltype(mt_tag)::value;
        constexpr bool EVEN = decltype(even_tag)::value;
        return local ? launch_xtile_cfg<KB, MT, EVEN, true>(w, n, nb, x, m, y, p, part, cnt, s)
                     : launch_xtile_cfg<KB, MT, EVEN, false>(w, n, nb, x, m, y, p, part, cnt, s);
    };
    using T = std::true_type;
    using F = std::false_type;
    using K8 = std::integral_constant<int, 8>;
    using K16 = std::integral_constant<int, 16>;
    using K32 = std::integral_constant<int, 32>;
    auto by_kb = [&](auto mt_tag, auto even_tag) {
        constexpr int MT = decltype(mt_tag)::value;
        if constexpr (MT == 1) {
            return p.KB == 8 ? go(K8{}, mt_tag, even_tag) : p.KB == 16 ? go(K16{}, mt_tag, even_tag)
                                                                        : go(K32{}, mt_tag, even_tag);
        } else {
            return p.KB == 8 ? go(K8{}, mt_tag, even_tag) : go(K16{}, mt_tag, even_tag);
        }
    };
    auto by_mt = [&](auto even_tag) {
        switch (mt) {
            case 1: return by_kb(std::integral_constant<int, 1>{}, even_tag);
            case 2: return by_kb(std::integral_constant<int, 2>{}, even_tag);
            case 3: return by_kb(std::integral_constant<int, 3>{}, even_tag);
            default: return by_kb(std::integral_constant<int, 4>{}, even_tag);
        }
    };
    return p.even ? by_mt(T{}) : by_mt(F{});
}

// Launch plan of the skinny GEMM for (m, n, nb): the template shape by m, the
// number of K-slices S (a grid of about one workgroup per CU; S = 1 when the
// strips alone fill the CUs or no partial buffer is given) and the blocks per
// slice.
struct SkPlan {
    int mt, R, strips, S, kbs, units;
    bool even;  // nb and kbs even (EVEN kernels)
};
inline SkPlan skinny_plan(size_t m, size_t n, int nb, bool can_split) {
    SkPlan p{};
    p.mt = (int)((m + 15) / 16);
    const int jt = 4, wr = p.mt >= 3 ? 2 : 1;
    p.R = 16 * jt * wr;
    p.units = wr * p.mt * jt * 64;
    p.strips = (int)((n + p.R - 1) / p.R);
    int S = can_split ? (device_cu_count() + p.strips / 2) / p.strips : 1;
    S = std::max(1, std::min(S, std::min(16, nb)));
    p.kbs = (nb + S - 1) / S;
    p.even = nb % 2 == 0;
    if (p.even) p.kbs += p.kbs & 1;
    p.S = (nb + p.kbs - 1) / p.kbs;  // no empty slices
    return p;
}

template <int MT, int JT, int WR, bool EVEN, bool LOCAL>
hipError_t launch_skinny_cfg(const uint8_t* w, int n, int nb, const float* x, int m, float* y, const SkPlan& p,
                             float* part, int* cnt, hipStream_t s) {
    using C = SkCfg<MT, JT, WR>;
    static_assert(C::LDS <= 160 * 1024, "LDS per workgroup");
    auto kern = gemm_q4_0_skinny_kernel<MT, JT, WR, EVEN, LOCAL>;
    if (C::LDS > 65536) {
        static const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                        C::LDS);  // once per kernel and process
        if (e != hipSuccess) return e;
    }
    const int strips = LOCAL ? (p.strips + XCD_COUNT - 1) / XCD_COUNT * XCD_COUNT : p.strips;
    launch_kernel(kern, dim3((unsigned)(strips * p.S)), dim3(C::NT), (size_t)C::LDS, s, w, n, nb, x, m, y, p.S,
                  p.kbs, part, cnt);
    return hipGetLastError();
}

hipError_t launch_skinny(const uint8_t* w, int n, int nb, const float* x, int m, float* y, float* part, int* cnt,
                         hipStream_t s) {
    const SkPlan p = skinny_plan((size_t)m, (size_t)n, nb, part != nullptr && cnt != nullptr);
    const bool local = p.S > 1 && xcd_round_robin(s);
    auto go = [&](auto mt_tag, auto even_tag) {
        constexpr int MT = decltype(mt_tag)::value;
        constexpr bool EVEN = decltype(even_tag)::value;
        constexpr int WR = MT >= 3 ? 2 : 1;
        return local ? launch_skinny_cfg<MT, 4, WR, EVEN, true>(w, n, nb, x, m, y, p, part, cnt, s)
                     : launch_skinny_cfg<MT, 4, WR, EVEN, false>(w, n, nb, x, m, y, p, part, cnt, s);
    };
    using M1 = std::integral_constant<int, 1>;
    using M2 = std::integral_constant<int, 2>;
    using M3 = std::integral_constant<int, 3>;
    using M4 = std::integral_constant<int, 4>;
    using T = std::true_type;
    using F = std::false_type;
    if (p.even) return p.mt == 1 ? go(M1{}, T{}) : p.mt == 2 ? go(M2{}, T{}) : p.mt == 3 ? go(M3{}, T{}) : go(M4{}, T{});
    return p.mt == 1 ? go(M1{}, F{}) : p.mt == 2 ? go(M2{}, F{}) : p.mt == 3 ? go(M3{}, F{}) : go(M4{}, F{});
}

template <bool NATIVE, bool DUMP, int WF, int FJ, int FI, int WJ, int WI, int KS, int KB>
hipError_t launch_cfg(const uint8_t* w, int n, int nb, const void* x0, const void* x1, const int* xe, int m,
                      float* y, int32_t* p, hipStream_t s, int accy, const float* xs) {
    using C = GemmCfg<NATIVE, WF, FJ, FI, WJ, WI, KS, KB>;
    auto kern = gemm_q4_0_kernel<NATIVE, DUMP, WF, FJ, FI, WJ, WI, KS, KB>;
    static_assert(C::LDS >= C::RED, "K-split sums fit the staging LDS");
    static_assert(C::LDS <= 160 * 1024, "LDS per workgroup");
    if (C::LDS > 65536) {
        static const hipError_t e = hipFuncSetAttribute((const void*)kern,
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
    }
    const unsigned tiles = (unsigned)((n + C::TJ - 1) / C::TJ) * (unsigned)((m + C::TI - 1) / C::TI);
    launch_kernel(kern, dim3(tiles), dim3(C::NT), (size_t)C::LDS, s, w, n, nb, x0, x1, xe, m, y, p, accy, xs);
    return hipGetLastError();
}

// Tile choice: enough workgroups for the CUs, then the largest tile (fewest
// re-reads of x and W from L2).  M >= 256: swept on MI355X at M = 512 and
// 2048 over tile shapes, waves and chunk sizes, per mode (the native kernel
// stages half the x bytes and keeps fewer registers).
// WF_Q4_K: the float shapes, 128 x 64 tiles of one block a wave (or 64 x 64)
// in place of the 128-row ones; xs the x' block sums.  WF_Q6_K: shapes of at
// most 64 x 64.  (Their staged headers or codes, scale pairs and masked
// operands hold more registers: the larger tiles spill.)
template <bool NATIVE, bool DUMP, int WF = WF_Q4_0>
hipError_t launch_tiles(const uint8_t* w, int n, int nb, const void* x0, const void* x1, const int* xe, int m,
                        float* y, int32_t* p, hipStream_t s, int accy = 0, const float* xs = nullptr) {
    const int cus = device_cu_count();
    if constexpr (WF == WF_Q4_K || WF == WF_Q4_1 || WF == WF_Q8_0) {
        // Q4_0's shapes, with 128 x 64 tiles of one block a wave a chunk (or
        // 64 x 64) where it takes its 128-row ones, which spill with Q4_K's
        // staged headers and scale pairs (7B gate/up at 128 rows: 194 us
        // spilling, 165 us in 64 x 64 tiles, 136 us in these)
        if (m >= 128 && (size_t)((n + 127) / 128) * ((m + 63) / 64) >= (size_t)cus)
            return launch_cfg<NATIVE, DUMP, WF, 4, 2, 2, 2, 2, 1>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
        if (m >= 128 && (size_t)((n + 63) / 64) * ((m + 63) / 64) >= (size_t)cus)
            return launch_cfg<NATIVE, DUMP, WF, 2, 2, 2, 2, 2, 2>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
    }
    if constexpr (WF == WF_Q6_K) {
        const size_t t64 = (size_t)((n + 63) / 64) * ((m + 63) / 64);
        if (m >= 48 && t64 >= (size_t)cus)
            return launch_cfg<NATIVE, DUMP, WF, 2, 2, 2, 2, 2, 2>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
        // 32 x 64 tiles of 8 waves (K split over 4) where they fill the CUs
        // (7B down at 128 rows: 121 us with K over 2 waves, 113 us), else
        // 32 x 16 of 4
        if (m >= 48 && (size_t)((n + 31) / 32) * ((m + 63) / 64) >= (size_t)cus)
            return launch_cfg<NATIVE, DUMP, WF, 2, 2, 1, 2, 4, 1>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
        if (m > 16) return launch_cfg<NATIVE, DUMP, WF, 1, 2, 1, 1, 4, 2>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
        return launch_cfg<NATIVE, DUMP, WF, 1, 1, 1, 1, 4, 4>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
    } else {
        if constexpr (NATIVE) {
            if (m >= 1024) return launch_cfg<NATIVE, DUMP, WF, 2, 2, 2, 2, 2, 2>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
            if (m >= 256) return launch_cfg<NATIVE, DUMP, WF, 2, 4, 2, 2, 2, 2>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
        } else if constexpr (WF == WF_Q4_0) {
            if (m >= 1024) return launch_cfg<NATIVE, DUMP, WF, 4, 4, 2, 2, 2, 1>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
            // 128 x 128 tiles from m = 128 where they fill three quarters of
            // the CUs (the 7B prefill's 28672-row gate/up GEMM at 128 rows: 224
            // tiles, 110 us against 119 us in 128 x 64 tiles); 128 x 64 tiles from
            // m = 256, and from m = 128 where they alone fill the CUs (prefill
            // 15.7 -> 12.3 ms; taken for every matrix: 14.9 ms)
            if (m >= 128 && m < 256 && 4 * (size_t)((n + 127) / 128) * ((m + 127) / 128) >= 3 * (size_t)cus)
                return launch_cfg<NATIVE, DUMP, WF, 4, 4, 2, 2, 2, 1>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
            if (m >= 256 || (m >= 128 && (size_t)((n + 127) / 128) * ((m + 63) / 64) >= (size_t)cus))
                return launch_cfg<NATIVE, DUMP, WF, 4, 2, 2, 2, 2, 2>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
        }
        const size_t t32 = (size_t)((n + 31) / 32) * ((m + 63) / 64);  // 32 x 64 tiles
        if (m >= 48 && t32 >= (size_t)cus) {
            if constexpr (!NATIVE) {
                // 8 waves a tile; 64 x 64 tiles when 32-row ones overflow a round
                // (us at 128 rows, 4096 x 4096 / 4096 x 14336 / 6144 x 4096: 4-wave
                // 32 x 64 tiles 37.2 / 106.5 / 66.0, 8-wave 30.3 / 89.1 / 51.5,
                // 64 x 64 38.7 / 112.9 / 40.0)
                if (t32 > (size_t)cus) {
                    // (the other formats' scale pairs, sums or byte codes: chunks of
                    // 4 blocks fit the LDS)
                    if constexpr (WF != WF_Q4_0)
                        return launch_cfg<NATIVE, DUMP, WF, 2, 4, 2, 1, 4, 1>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
                    else
                        return launch_cfg<NATIVE, DUMP, WF, 2, 4, 2, 1, 4, 2>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
                }
                return launch_cfg<NATIVE, DUMP, WF, 2, 2, 1, 2, 4, 2>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
            }
            return launch_cfg<NATIVE, DUMP, WF, 2, 4, 1, 1, 4, 2>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
        }
        if (m > 16) return launch_cfg<NATIVE, DUMP, WF, 1, 2, 1, 1, 4, 2>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
        if constexpr (wf_bytes(WF))  // (byte codes: chunks of 16 blocks fit the LDS)
            return launch_cfg<NATIVE, DUMP, WF, 1, 1, 1, 1, 4, 4>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
        else
            return launch_cfg<NATIVE, DUMP, WF, 1, 1, 1, 1, 4, 8>(w, n, nb, x0, x1, xe, m, y, p, s, accy, xs);
    }
}

}  // namespace

void set_combine_coherent(bool on) { combine_coherent.store(on); }
bool combine_is_coherent() { return combine_coherent.load(); }

bool combine_local_now() {
    if (combine_coherent.load()) return false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return false;
    std::lock_guard<std::mutex> lock(xcd_mu);
    return xcd_state[dev] == 1;
}

__global__ void zero_i32_kernel(int* __restrict__ p, int n) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) p[i] = 0;
}

hipError_t launch_zero_counters(int* counters, size_t count, hipStream_t s) {
    if (count == 0) return hipSuccess;
    launch_kernel(zero_i32_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, counters, (int)count);
    return hipGetLastError();
}

size_t gemm_counter_count(size_t n, size_t) { return (n + 63) / 64 + 1; }  // a counter per strip of 64 (or 128) rows

size_t gemm_scratch_bytes(size_t m, size_t n, size_t k, bool native) {
    if (!native && m >= 1 && m <= GEMM_XTILE_M) {  // the K-slice partials of the x-tile kernel
        const int mt = (int)((m + 15) / 16);
        const XtPlan p = xtile_plan(n, (int)(k / QK), mt);
        if (p.ok) return p.S > 1 ? ((size_t)p.strips * p.S * XT_UNITS * mt * 16 + 255) & ~(size_t)255 : 0;
    }
    if (!native && m <= GEMM_SMALL_M) {  // the K-slice partials of the skinny GEMM
        if (m == 0 || n == 0) return 0;
        const SkPlan p = skinny_plan(m, n, (int)(k / QK), true);
        return p.S > 1 ? ((size_t)p.strips * p.S * p.units * 16 + 255) & ~(size_t)255 : 0;
    }
    if (native)  // int8 codes and f32 block scales, 256-byte aligned pieces
        return ((m * k + 255) & ~(size_t)255) + ((m * (k / QK) * 4 + 255) & ~(size_t)255);
    // x_hi, x_lo (f16) and the row exponents
    const size_t xb = (m * k * 2 + 255) & ~(size_t)255;
    return 2 * xb + ((m * 4 + 255) & ~(size_t)255);
}

size_t gemm_tiles_scratch_bytes(size_t m, size_t k) {
    // the float layout (x_hi, x_lo, exponents) and the x' sums of each 32-element block
    const size_t xb = (m * k * 2 + 255) & ~(size_t)255;
    return 2 * xb + ((m * 4 + 255) & ~(size_t)255) + ((m * (k / QK) * 4 + 255) & ~(size_t)255);
}

hipError_t launch_gemm_q4_0(const uint8_t* w, size_t n, size_t k, const float* x, size_t m, float* y,
                            void* scratch, int* counters, hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    if (m <= GEMM_XTILE_M) {
        float* part = reinterpret_cast<float*>(scratch);  // the K-slice partials
        const hipError_t e = launch_xtile(w, (int)n, (int)(k / QK), x, (int)m, y, part, counters, s);
        if (e != hipErrorInvalidValue) return e;
    }
    if (m <= GEMM_SMALL_M) {
        float* part = reinterpret_cast<float*>(scratch);  // the K-slice partials
        return launch_skinny(w, (int)n, (int)(k / QK), x, (int)m, y, part, counters, s);
    }
    const size_t xb = (m * k * 2 + 255) & ~(size_t)255;
    _Float16* xh = reinterpret_cast<_Float16*>(scratch);
    _Float16* xl = reinterpret_cast<_Float16*>(reinterpret_cast<uint8_t*>(scratch) + xb);
    int* xe = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(scratch) + 2 * xb);
    if (k <= (size_t)16 * XPREP_FAST_THREADS)
        launch_kernel(gemm_xprep_fast_kernel, dim3((unsigned)m), dim3(XPREP_FAST_THREADS), 0, s, x, (int)k, xh, xl,
                      xe, (float*)nullptr);
    else
        launch_kernel(gemm_xprep_kernel, dim3((unsigned)m), dim3(XPREP_THREADS), 0, s, x, (int)k, xh, xl, xe);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_tiles<false, false>(w, (int)n, (int)(k / QK), xh, xl, xe, (int)m, y, nullptr, s);
}

hipError_t launch_gemm_tiles_ex(WType t, const uint8_t* w, size_t n, size_t k, const float* x, size_t m, float* y,
                                void* scratch, int pro, const float* g, float eps, bool accumulate, hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    const bool q40 = t == WType::Q4_0;
    if ((!q40 && t != WType::Q4_K && t != WType::Q6_K && t != WType::Q8_0 && t != WType::Q4_1) || k == 0 ||
        k % block_elems(t) != 0 || (pro < 0 || pro > 2) || (pro == 1 && !g))
        return hipErrorInvalidValue;
    // Q4_0's m <= GEMM_XTILE_M rows belong to the x-tile kernel; the x' block
    // sums and the prologues come from the one-read x prep (k <= 16384)
    if ((q40 && m <= GEMM_XTILE_M) || ((!q40 || pro != 0) && k > (size_t)16 * XPREP_FAST_THREADS))
        return hipErrorInvalidValue;
    const bool sums = t == WType::Q4_K || t == WType::Q4_1;
    // 32-bit buffer offsets, out-of-range slots at RSRC_OOB
    const size_t wb = n * (k / block_elems(t)) * block_bytes(t);
    if (wb > FUSED_MAX_WEIGHT_BYTES || m * k * 2 > FUSED_MAX_WEIGHT_BYTES) return hipErrorInvalidValue;
    const size_t xb = (m * k * 2 + 255) & ~(size_t)255;
    _Float16* xh = reinterpret_cast<_Float16*>(scratch);
    _Float16* xl = reinterpret_cast<_Float16*>(reinterpret_cast<uint8_t*>(scratch) + xb);
    int* xe = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(scratch) + 2 * xb);
    float* xs = sums ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(scratch) + 2 * xb +
                                                ((m * 4 + 255) & ~(size_t)255))
                     : nullptr;
    const dim3 grid((unsigned)m);
    if (pro == 1)
        launch_kernel(gemm_xprep_pro_kernel<1>, grid, dim3(XPREP_FAST_THREADS), 0, s, x, (int)k, g, eps, xh, xl, xe,
                      xs);
    else if (pro == 2)
        launch_kernel(gemm_xprep_pro_kernel<2>, grid, dim3(XPREP_FAST_THREADS), 0, s, x, (int)k, g, eps, xh, xl, xe,
                      xs);
    else if (k <= (size_t)16 * XPREP_FAST_THREADS)
        launch_kernel(gemm_xprep_fast_kernel, grid, dim3(XPREP_FAST_THREADS), 0, s, x, (int)k, xh, xl, xe, xs);
    else
        launch_kernel(gemm_xprep_kernel, grid, dim3(XPREP_THREADS), 0, s, x, (int)k, xh, xl, xe);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int accy = accumulate ? 1 : 0;
    const int ni = (int)n, nb = (int)(k / QK), mi = (int)m;
    switch (t) {
        case WType::Q4_K: return launch_tiles<false, false, WF_Q4_K>(w, ni, nb, xh, xl, xe, mi, y, nullptr, s, accy, xs);
        case WType::Q6_K: return launch_tiles<false, false, WF_Q6_K>(w, ni, nb, xh, xl, xe, mi, y, nullptr, s, accy);
        case WType::Q8_0: return launch_tiles<false, false, WF_Q8_0>(w, ni, nb, xh, xl, xe, mi, y, nullptr, s, accy);
        case WType::Q4_1: return launch_tiles<false, false, WF_Q4_1>(w, ni, nb, xh, xl, xe, mi, y, nullptr, s, accy, xs);
        default: return launch_tiles<false, false>(w, ni, nb, xh, xl, xe, mi, y, nullptr, s, accy);
    }
}

hipError_t launch_gemm_typed(WType t, const uint8_t* w, size_t n, size_t k, const float* x, size_t m, float* y,
                             void* scratch, hipStream_t s) {
    if (t == WType::Q4_0) return hipErrorInvalidValue;  // launch_gemm_q4_0
    return launch_gemm_tiles_ex(t, w, n, k, x, m, y, scratch, 0, nullptr, 0.0f, false, s);
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
