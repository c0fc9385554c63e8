// llama.hip -- batch-1 Llama-style decoder (include/rdl_llama.h): the rustml
// decode loop with every activation on the device and the Q4_0 Linears on
// this library's fused GEMV (one or a few rows) and matrix-core GEMM (prompt
// chunks).
//
// Per layer (TransformerBlock::forward_with_cache, transformer_block.rs:297-356,
// standard pre-norm branch):
//   xn  = rms_norm(x, attn_norm)                    ops.rs:688-751
//   qkv = xn . [Wq; Wk; Wv]^T                       one launch over the
//                                                    row-concatenated weights
//   rope(q), rope(k) at start_pos; k, v -> cache    attention.rs:393-399, rope.rs:134-200
//   att = softmax(q k^T / sqrt(hd) + causal) v      attention.rs:401-446, head h reads
//                                                    KV head h / (n_heads / n_kv)
//   x  += att . Wo^T
//   xn  = rms_norm(x, ffn_norm)
//   gu  = xn . [Wgate; Wup]^T
//   h   = silu(gate) * up                           feed_forward.rs:138-150, ops.rs:441-446
//   x  += h . Wdown^T
// then rms_norm(x, norm) . Wout^T on the last row, argmax (sampling.rs:8-18).
// The cache position lives in device memory, so a decode step has no host
// dependency and is captured once as a HIP graph and replayed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <string>
#include <cmath>
#include <cstring>
#include <type_traits>
#include <vector>

#include "../../include/rdl_gguf.h"
#include "../../include/rdl_llama.h"
#include "attention.hpp"
#include "rdl_device.hpp"
#include "rdl_internal.hpp"

namespace rdl {
namespace {

constexpr int NT = 256;  // threads of the element-wise / reduction kernels

// Sum over a 256-thread block, returned to every thread.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// rms = sqrt(sum(x^2) / d + eps); out = x * (1 / rms) * g   (ops.rs:688-751)
__global__ __launch_bounds__(NT) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ g,
                                                     int d, float eps, float* __restrict__ out) {
    __shared__ float red[NT / 64];
    // d % 4 == 0: float4 per thread, RN of them issued before any use
    constexpr int RN = 8;
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4* xr = reinterpret_cast<const f4*>(x + (size_t)blockIdx.x * d);
    const f4* g4 = reinterpret_cast<const f4*>(g);
    f4* o = reinterpret_cast<f4*>(out + (size_t)blockIdx.x * d);
    const int d4 = d / 4;
    float ss = 0.0f;
    for (int c0 = 0; c0 < d4; c0 += RN * NT) {
        f4 v[RN];
#pragma unroll
        for (int r = 0; r < RN; r++) {
            const int c = c0 + r * NT + threadIdx.x;
            v[r] = (c < d4) ? xr[c] : f4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int r = 0; r < RN; r++) ss += (v[r].x * v[r].x + v[r].y * v[r].y) + (v[r].z * v[r].z + v[r].w * v[r].w);
    }
    ss = block_sum(ss, red);
    const float rms = sqrtf(ss / (float)d + eps);
    const float inv = 1.0f / rms;
    for (int c0 = 0; c0 < d4; c0 += RN * NT) {
        f4 v[RN], gv[RN];
#pragma unroll
        for (int r = 0; r < RN; r++) {
            const int c = c0 + r * NT + threadIdx.x;
            v[r] = (c < d4) ? xr[c] : f4{0.0f, 0.0f, 0.0f, 0.0f};
            gv[r] = (c < d4) ? g4[c] : f4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int r = 0; r < RN; r++) {
            const int c = c0 + r * NT + threadIdx.x;
            if (c < d4) o[c] = (v[r] * inv) * gv[r];
        }
    }
}

// RoPE (half-split pairs (i, i + hd/2), rope.rs:134-200) of q and k at
// positions pos..pos+m-1, then k and v into the cache (KVCache::update,
// kv_cache.rs:94-106; paged layout: kv_row).
template <typename KV>
__global__ void rope_kv_kernel(float* __restrict__ qkv, int qkv_dim, const int* __restrict__ pos_dev,
                               const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                               int n_heads, int n_kv, int hd, KV* __restrict__ kc, KV* __restrict__ vc,
                               const int* __restrict__ kv_table) {
    const int s = blockIdx.y, head = blockIdx.x, i = threadIdx.x, half = hd >> 1;
    const int pos = *pos_dev + s;
    float* row = qkv + (size_t)s * qkv_dim;
    const float c = cos_t[(size_t)pos * half + i], sn = sin_t[(size_t)pos * half + i];
    if (head < n_heads) {
        float* q = row + head * hd;
        const float x1 = q[i], x2 = q[half + i];
        q[i] = x1 * c - x2 * sn;
        q[half + i] = x1 * sn + x2 * c;
    } else {
        const int kvh = head - n_heads;
        const float* k = row + n_heads * hd + kvh * hd;
        const float* v = row + (n_heads + n_kv) * hd + kvh * hd;
        const float x1 = k[i], x2 = k[half + i];
        KV* kd = kc + kv_row(kv_table, n_kv, kvh, pos, hd);
        KV* vd = vc + kv_row(kv_table, n_kv, kvh, pos, hd);
        kd[i] = (KV)(x1 * c - x2 * sn);
        kd[half + i] = (KV)(x1 * sn + x2 * c);
        vd[i] = (KV)v[i];
        vd[half + i] = (KV)v[half + i];
    }
}

// Decode attention: attention.hpp (attention_body); the launch here serves
// every row count and position (prefill chunks, eager decode steps, the
// captured decode graph).
template <typename KV, int HD>
__global__ __launch_bounds__(64 * ATT_WAVES) void attention_kernel(AttArgs<KV> a) {
    extern __shared__ float sm[];
    attention_body<KV, HD, false>(blockIdx.x, blockIdx.y, blockIdx.z, sm, a);
}

// A prompt chunk of at least PREFILL_ATT_ALL_ROWS rows takes the kernel below
// at any length, one of PREFILL_ATT_MIN_ROWS .. that while its rows see at
// most PREFILL_ATT_MAX_PAGES cache pages (keys / 64); it walks a row's pages
// in turn, so short chunks at long lengths keep the per-row kernel, which
// spreads a row's pages over workgroups.  MI355X, 7B Q4_0, 2040-token prompt
// (per-row kernel / this one at every length): chunks of 128 rows 245 / 179 ms,
// 32 rows 410 / 384 ms, 16 rows 677 / 734 ms, 8 rows 1220 / 1435 ms.
constexpr size_t PREFILL_ATT_ALL_ROWS = 32, PREFILL_ATT_MIN_ROWS = 8, PREFILL_ATT_MAX_PAGES = 8;
constexpr size_t PREFILL_ATT_MFMA_MIN_ROWS = 32;

// Attention of a prompt chunk (m > 1 rows at positions *pos .. *pos + m - 1,
// keys already in the cache): one wave a query row, 8 consecutive rows of one
// head a workgroup.  The workgroup copies each cache page (64 keys) it needs
// into LDS once, with coalesced 16-byte loads issued while the waves work on
// the page before, and its waves read it from there: lane j scores key p0 + j against q (LDS broadcast), then the page's
// max, an online rescale of the running (max M, sum L, context o) and the
// weighted V rows, lane l owning dims HD / 64 * l ..; at the end o / L.  K
// rows sit 16 bytes apart from a multiple of the bank width in LDS, so the 64
// lanes' reads of 64 rows spread over the banks.  The same f32 arithmetic as
// attention_kernel per term (scores / sqrt(hd), exp(score - max),
// attention.rs:414-441); the running max replaces the chunk combine, so sums
// round in another order.
template <typename KV, int HD>
__global__ __launch_bounds__(512) void prefill_attention_kernel(AttArgs<KV> a, int m) {
    static_assert(HD % 64 == 0 && HD <= 256, "head dims a lane");
    constexpr int DPL = HD / 64;
    constexpr int V = 16 / (int)sizeof(KV);  // cache elements a 16-byte load
    constexpr int KROW = HD + V;             // K row stride in LDS (elements)
    constexpr int PIECES = KV_PAGE * HD / V;  // 16-byte pieces of a page
    constexpr int PER = (PIECES + 511) / 512;
    typedef KV kvv __attribute__((ext_vector_type(V)));
    __shared__ __attribute__((aligned(16))) float qsh[8][HD];
    __shared__ __attribute__((aligned(16))) KV ks[KV_PAGE * KROW];
    __shared__ __attribute__((aligned(16))) KV vs[KV_PAGE * HD];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n_heads = a.n_heads, n_kv = a.n_kv, G = n_heads / n_kv;
    // the G query heads of a KV head on one XCD (block b on XCD b % 8)
    const int h = ((int)blockIdx.x % n_kv) * G + (int)blockIdx.x / n_kv;
    const int kvh = h / G;
    const int s0 = (int)blockIdx.y * 8, s = s0 + w;
    const int pos0 = *a.pos_dev;
    const int tmax = pos0 + min(s0 + 8, m);  // keys of the group's last row
    const int t = pos0 + s + 1;              // keys 0 .. t - 1 of this row
    const bool live = s < m;                 // wave-uniform
    if (live) {
        const float* q = a.qkv + (size_t)s * a.qkv_dim + (size_t)h * HD;
#pragma unroll
        for (int c = 0; c < DPL; c++) qsh[w][lane + 64 * c] = q[lane + 64 * c];
    }
    float M = -__builtin_inff(), L = 0.0f, o[DPL];
#pragma unroll
    for (int c = 0; c < DPL; c++) o[c] = 0.0f;
    // this thread's pieces of the page at p0 (rows of it that any wave reads)
    kvv kr[PER], vr[PER];
    auto fetch = [&](int p0) {
        const int nv = min(KV_PAGE, tmax - p0);
        const size_t page = kv_row(a.kv_table, n_kv, kvh, p0, HD);
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int pc = threadIdx.x + 512 * i;
            if (pc < nv * (HD / V)) {
                kr[i] = *reinterpret_cast<const kvv*>(a.kc + page + (size_t)pc * V);
                vr[i] = *reinterpret_cast<const kvv*>(a.vc + page + (size_t)pc * V);
            }
        }
    };
    fetch(0);
    for (int p0 = 0; p0 < tmax; p0 += KV_PAGE) {
        const int nv = min(KV_PAGE, tmax - p0);  // rows of the page any wave reads
        __syncthreads();  // the previous page's reads are done
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int pc = threadIdx.x + 512 * i;
            if (pc < nv * (HD / V)) {
                const int r = pc / (HD / V), c = pc % (HD / V);
                *reinterpret_cast<kvv*>(ks + r * KROW + c * V) = kr[i];
                *reinterpret_cast<kvv*>(vs + pc * V) = vr[i];
            }
        }
        __syncthreads();
        if (p0 + KV_PAGE < tmax) fetch(p0 + KV_PAGE);  // in flight during this page
        if (live && p0 < t) {
            const int nvalid = min(KV_PAGE, t - p0);  // <= nv
            // score of key p0 + lane (a key past the row re-reads the last one)
            const KV* krow = ks + min(lane, nvalid - 1) * KROW;
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < HD / V; i++) {
                const kvv k = *reinterpret_cast<const kvv*>(krow + i * V);
#pragma unroll
                for (int e = 0; e < V; e++) acc += qsh[w][i * V + e] * (float)k[e];
            }
            const bool valid = lane < nvalid;
            const float sc = valid ? acc / a.scale : -__builtin_inff();
            const float Mn = fmaxf(M, wave_max(sc));
            const float corr = expf(M - Mn);  // 0 on the first page
            const float e = valid ? expf(sc - Mn) : 0.0f;
            L = L * corr + wave_sum(e);
#pragma unroll
            for (int c = 0; c < DPL; c++) o[c] *= corr;
            // weighted V rows; rows past the row's keys re-read the last
            // valid one with weight 0 (rows past nv were not copied)
#pragma unroll
            for (int j = 0; j < KV_PAGE; j++) {
                const float ej = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), j));
                const KV* vrow = vs + min(j, nvalid - 1) * HD + DPL * lane;
#pragma unroll
                for (int c = 0; c < DPL; c++) o[c] += ej * (float)vrow[c];
            }
            M = Mn;
        }
    }
    if (!live) return;
    float* out = a.out + (size_t)s * n_heads * HD + (size_t)h * HD + DPL * lane;
    const float invL = 1.0f / L;
#pragma unroll
    for (int c = 0; c < DPL; c++) out[c] = o[c] * invL;
}

// The same attention on the matrix cores, for an f16 cache: a workgroup of 4
// waves takes 16 consecutive rows of one head and walks the cache pages
// their rows need, staged in LDS as above (K rows, V transposed: the MFMA
// operands read 8 consecutive keys of one dim).  Per page:
//  1. scores: wave w forms S[16 rows][keys 16w .. 16w + 15] with
//     v_mfma_f32_16x16x32_f16, q as the A operand; q rows are scaled by a
//     power of two (row max into [2^14, 2^15)) and split into f16 hi + lo,
//     so hi * k + lo * k (f16 k exact) carries about 22 significant bits of
//     q, products exact and sums in f32;
//  2. softmax: wave w takes rows 4w .. 4w + 3, a lane a key: scores / sqrt(hd)
//     (attention.rs:414-415), page max, online rescale of the running
//     (max, sum), weights exp(score - max) split into f16 hi + lo;
//  3. context: wave w forms O[16 rows][HD / 4 dims] += P V, after scaling O
//     by the rows' rescale factors, with the weights as the A operand.
// At the end o / sum.  Keys past a row's length weigh 0; cache rows past the
// ones copied are zeros in LDS (finite, so 0 * v stays 0).
template <int HD>
__global__ __launch_bounds__(256) void prefill_attention_mfma_kernel(AttArgs<_Float16> a, int m) {
    static_assert(HD % 64 == 0 && HD <= 256, "16-dim output tiles, 4 waves");
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int KST = HD / 32;            // MFMA K steps over the head dims
    constexpr int OT = HD / 64;             // 16-dim output tiles a wave
    constexpr int KR = HD + 8;              // LDS row strides (elements): 16 bytes
    constexpr int VR = KV_PAGE + 8;         // past a multiple of the bank period
    constexpr int PR = KV_PAGE + 8;
    constexpr int SR = KV_PAGE + 4;
    constexpr int PPR = HD / 8;             // 16-byte pieces a cache row
    constexpr int PER = KV_PAGE * PPR / 256;
    __shared__ __attribute__((aligned(16))) _Float16 ks[KV_PAGE * KR];
    __shared__ __attribute__((aligned(16))) _Float16 vt[HD * VR];
    __shared__ __attribute__((aligned(16))) _Float16 ph[16 * PR];
    __shared__ __attribute__((aligned(16))) _Float16 pl[16 * PR];
    __shared__ __attribute__((aligned(16))) float ss[16 * SR];
    __shared__ int rexp[16];
    __shared__ float rcorr[16], rsum[16];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    const int n_heads = a.n_heads, n_kv = a.n_kv, G = n_heads / n_kv;
    const int h = ((int)blockIdx.x % n_kv) * G + (int)blockIdx.x / n_kv;
    const int kvh = h / G;
    const int s0 = (int)blockIdx.y * 16;
    const int pos0 = *a.pos_dev;
    const int tmax = pos0 + min(s0 + 16, m);  // keys of the group's last row
    const float* qh0 = a.qkv + (size_t)h * HD;

    // row exponents: wave w takes rows 4w .. 4w + 3
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 4 * w + i, s = s0 + r;
        float mx = 0.0f;
        if (s < m)
#pragma unroll
            for (int c = 0; c < HD / 64; c++) mx = fmaxf(mx, fabsf(qh0[(size_t)s * a.qkv_dim + lane + 64 * c]));
        mx = wave_max(mx);
        int e = 0;
        if (mx > 0.0f) {
            frexpf(mx, &e);  // mx = f * 2^e, f in [0.5, 1)
            e -= 15;
        }
        if (lane == 0) rexp[r] = e;
    }
    __syncthreads();
    // A operands of the scores: row r16, dims 32k + 8g .. + 7, hi and lo
    h8 qhi[KST], qlo[KST];
    {
        const int s = s0 + r16, e = rexp[r16];
#pragma unroll
        for (int k = 0; k < KST; k++) {
            float4 q0 = {0.0f, 0.0f, 0.0f, 0.0f}, q1 = q0;
            if (s < m) {
                const float4* qp = reinterpret_cast<const float4*>(qh0 + (size_t)s * a.qkv_dim + 32 * k + 8 * g);
                q0 = qp[0];
                q1 = qp[1];
            }
            const float qv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float v = ldexpf(qv[u], -e);
                const _Float16 hi = (_Float16)v;
                qhi[k][u] = hi;
                qlo[k][u] = (_Float16)(v - (float)hi);
            }
        }
    }
    f4 o[OT];
#pragma unroll
    for (int t = 0; t < OT; t++) o[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    float Mr[4], Lr[4];  // running max / sum of rows 4w + i (every lane)
#pragma unroll
    for (int i = 0; i < 4; i++) {
        Mr[i] = -__builtin_inff();
        Lr[i] = 0.0f;
    }
    // this thread's pieces of the page at p0 (zeros for rows past the group's
    // keys).  K: piece pc = key * PPR + c.  V: a wave's 64 pieces are 16 keys x
    // 4 consecutive pieces, so its transposed 2-byte stores fall on different
    // banks for different keys.
    h8 kr[PER], vr[PER];
    auto vpiece = [&](int idx, int& key, int& c) {
        c = (idx >> 4) % PPR;
        key = (idx & 15) + 16 * ((idx >> 4) / PPR);
    };
    auto fetch = [&](int p0) {
        const int nv = min(KV_PAGE, tmax - p0);
        const size_t page = kv_row(a.kv_table, n_kv, kvh, p0, HD);
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int pc = threadIdx.x + 256 * i;
            int vk, vc;
            vpiece(pc, vk, vc);
            kr[i] = pc / PPR < nv ? *reinterpret_cast<const h8*>(a.kc + page + (size_t)pc * 8) : h8{};
            vr[i] = vk < nv ? *reinterpret_cast<const h8*>(a.vc + page + (size_t)vk * HD + vc * 8) : h8{};
        }
    };
    fetch(0);
    for (int p0 = 0; p0 < tmax; p0 += KV_PAGE) {
        __syncthreads();  // the previous page's LDS reads are done
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int pc = threadIdx.x + 256 * i;
            *reinterpret_cast<h8*>(ks + (pc / PPR) * KR + (pc % PPR) * 8) = kr[i];
            int vk, vc;
            vpiece(pc, vk, vc);
#pragma unroll
            for (int u = 0; u < 8; u++) vt[(vc * 8 + u) * VR + vk] = vr[i][u];
        }
        __syncthreads();
        if (p0 + KV_PAGE < tmax) fetch(p0 + KV_PAGE);  // in flight during this page
        // 1. scores of keys 16w .. 16w + 15: lane holds S[4g + t][16w + r16]
        f4 sacc = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < KST; k++) {
            const h8 b = *reinterpret_cast<const h8*>(ks + (16 * w + r16) * KR + 32 * k + 8 * g);
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qhi[k], b, sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qlo[k], b, sacc, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < 4; t++) ss[(4 * g + t) * SR + 16 * w + r16] = sacc[t];
        __syncthreads();
        // 2. softmax of rows 4w .. 4w + 3 over the page, a lane a key
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 4 * w + i, s = s0 + r;
            const bool valid = s < m && p0 + lane < pos0 + s + 1;
            const float sc = valid ? ldexpf(ss[r * SR + lane], rexp[r]) / a.scale : -__builtin_inff();
            const float Mn = fmaxf(Mr[i], wave_max(sc));
            const float corr = Mn == -__builtin_inff() ? 1.0f : expf(Mr[i] - Mn);  // a row past m: no keys
            const float e = valid ? expf(sc - Mn) : 0.0f;
            Lr[i] = Lr[i] * corr + wave_sum(e);
            Mr[i] = Mn;
            const _Float16 hi = (_Float16)e;
            ph[r * PR + lane] = hi;
            pl[r * PR + lane] = (_Float16)(e - (float)hi);
            if (lane == 0) rcorr[r] = corr;
        }
        __syncthreads();
        // 3. context: lane holds O[4g + t][(w OT + j) 16 + r16]
        {
            float cr[4];
#pragma unroll
            for (int t = 0; t < 4; t++) cr[t] = rcorr[4 * g + t];
#pragma unroll
            for (int j = 0; j < OT; j++)
#pragma unroll
                for (int t = 0; t < 4; t++) o[j][t] *= cr[t];
#pragma unroll
            for (int kk = 0; kk < KV_PAGE / 32; kk++) {
                const h8 pa = *reinterpret_cast<const h8*>(ph + r16 * PR + 32 * kk + 8 * g);
                const h8 pb = *reinterpret_cast<const h8*>(pl + r16 * PR + 32 * kk + 8 * g);
#pragma unroll
                for (int j = 0; j < OT; j++) {
                    const int d0 = (w * OT + j) * 16;
                    const h8 vb = *reinterpret_cast<const h8*>(vt + (d0 + r16) * VR + 32 * kk + 8 * g);
                    o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, o[j], 0, 0, 0);
                    o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pb, vb, o[j], 0, 0, 0);
                }
            }
        }
    }
    if (lane == 0)
#pragma unroll
        for (int i = 0; i < 4; i++) rsum[4 * w + i] = Lr[i];
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int r = 4 * g + t, s = s0 + r;
        if (s >= m) continue;
        const float invL = 1.0f / rsum[r];
        float* out = a.out + (size_t)s * n_heads * HD + (size_t)h * HD;
#pragma unroll
        for (int j = 0; j < OT; j++) out[(w * OT + j) * 16 + r16] = o[j][t] * invL;
    }
}

// x += y (Tensor::add_inplace, ops.rs:276-289)
__global__ void add_kernel(float* __restrict__ x, const float* __restrict__ y, size_t n) {
    const size_t i = (size_t)blockIdx.x * NT + threadIdx.x;
    if (i < n) x[i] = x[i] + y[i];
}

// h = silu(gate) * up, silu(g) = g * (1 / (1 + exp(-g)))   (ops.rs:441-446);
// gu rows hold (gate_j, up_j) at 2j, 2j + 1 (the interleaved Wgu rows)
__global__ void swiglu_kernel(const float* __restrict__ gu, int ffn, size_t n, float* __restrict__ h) {
    const size_t i = (size_t)blockIdx.x * NT + threadIdx.x;
    if (i >= n) return;
    const size_t s = i / ffn, j = i % ffn;
    const float g = gu[s * 2 * ffn + 2 * j], u = gu[s * 2 * ffn + 2 * j + 1];
    const float sig = 1.0f / (1.0f + expf(-g));
    h[i] = (g * sig) * u;
}

// The same over separate [rows, ffn] gate and up buffers.
__global__ void swiglu2_kernel(const float* __restrict__ g, const float* __restrict__ u, size_t n,
                               float* __restrict__ h) {
    const size_t i = (size_t)blockIdx.x * NT + threadIdx.x;
    if (i >= n) return;
    const float gv = g[i];
    const float sig = 1.0f / (1.0f + expf(-gv));
    h[i] = (gv * sig) * u[i];
}

// One greedy sampling step in one launch: argmax of the logits with the first
// maximum winning (strict >, NaN never wins; an all-NaN / -inf row gives 0,
// sampling.rs:8-18), the token written for the next step and to
// out_tokens[*step] (then *step + 1), the position advanced by `advance`
// (KVCache::advance, kv_cache.rs:112-114), and the sampled token's embedding
// row dequantized into x (Embedding::forward, embedding.rs:50-76, on the Q4_0
// table as Tensor::to_f32 computes it: d * (q - 8)) for the next step (emb
// NULL: no embedding, the next forward reads the token id).
constexpr int SAMPLE_NT = 1024;
__global__ __launch_bounds__(SAMPLE_NT) void sample_kernel(const float* __restrict__ logits, int vocab,
                                                           int* __restrict__ token, int* __restrict__ out_tokens,
                                                           int* __restrict__ step, int* __restrict__ pos,
                                                           int advance, const uint8_t* __restrict__ emb, int dim,
                                                           float* __restrict__ x) {
    __shared__ float bv[SAMPLE_NT / 64];
    __shared__ int bi[SAMPLE_NT / 64];
    __shared__ int win;
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int VU = 8;  // float4 loads in flight per thread
    // the step counter is read with the logits, not after the reduction
    const int st = threadIdx.x == 0 ? *step : 0;
    float best = -__builtin_inff();
    int idx = 0x7FFFFFFF;
    const int n4 = vocab >> 2;
    const f4* l4 = reinterpret_cast<const f4*>(logits);
    // each thread visits its indices in increasing order
    for (int base = 0; base < n4; base += SAMPLE_NT * VU) {
        f4 v[VU];
#pragma unroll
        for (int j = 0; j < VU; j++) {
            const int p = base + (int)threadIdx.x + j * SAMPLE_NT;
            v[j] = p < n4 ? l4[p] : f4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int j = 0; j < VU; j++) {
            const int p = base + (int)threadIdx.x + j * SAMPLE_NT;
            if (p < n4)
#pragma unroll
                for (int t = 0; t < 4; t++)
                    if (v[j][t] > best) {
                        best = v[j][t];
                        idx = 4 * p + t;
                    }
        }
    }
    for (int i = 4 * n4 + (int)threadIdx.x; i < vocab; i += SAMPLE_NT) {
        const float v = logits[i];
        if (v > best) {
            best = v;
            idx = i;
        }
    }
    // (value, index) reduction: larger value, then smaller index
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int oi = __shfl_xor(idx, o);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = best;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < SAMPLE_NT / 64; w++)
            if (bv[w] > best || (bv[w] == best && bi[w] < idx)) {
                best = bv[w];
                idx = bi[w];
            }
        if (idx == 0x7FFFFFFF) idx = 0;
        token[0] = idx;
        out_tokens[st] = idx;
        *step = st + 1;
        if (advance) *pos += advance;
        win = idx;
    }
    __syncthreads();
    if (!emb) return;
    const uint8_t* row = emb + (size_t)win * (dim / 32) * Q4_0_BYTES;
    for (int e = threadIdx.x; e < dim; e += SAMPLE_NT) {
        const uint8_t* blk = row + (e >> 5) * Q4_0_BYTES;
        const int j = e & 31;
        const float d = h2f(blk[0] | (blk[1] << 8));
        const uint8_t v = blk[2 + (j & 15)];
        x[e] = d * (float)((int)(j < 16 ? (v & 0x0F) : (v >> 4)) - 8);
    }
}

// KVCache::advance (kv_cache.rs:112-114)
__global__ void advance_kernel(int* pos, int by) {
    if (threadIdx.x == 0) *pos += by;
}
__global__ void set_int_kernel(int* p, int v) {
    if (threadIdx.x == 0) *p = v;
}

// ---- synthetic weights --------------------------------------------------------------
__device__ __forceinline__ uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Q4_0 blocks: 16 random nibble bytes, d = f16(|N(0, sigma)| / 8) (Box-Muller).
__global__ void fill_q4_0_kernel(uint8_t* __restrict__ w, size_t nblocks, uint64_t seed, float sigma) {
    const size_t g = (size_t)blockIdx.x * NT + threadIdx.x;
    if (g >= nblocks) return;
    uint64_t st = seed ^ (g * 0xD1B54A32D192ED03ull);
    const uint64_t a = splitmix64(st), b = splitmix64(st), c = splitmix64(st);
    const float u1 = ((float)(c >> 40) + 1.0f) * 0x1p-24f;  // (0, 1]
    const float u2 = (float)((c >> 16) & 0xFFFFFFu) * 0x1p-24f;
    const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2);
    const uint32_t d = f2h_rne(fabsf(z) * sigma / 8.0f);
    uint16_t* p = reinterpret_cast<uint16_t*>(w + g * Q4_0_BYTES);  // blocks are 2-byte aligned
    p[0] = (uint16_t)d;
    for (int i = 0; i < 4; i++) p[1 + i] = (uint16_t)(a >> (16 * i));
    for (int i = 0; i < 4; i++) p[5 + i] = (uint16_t)(b >> (16 * i));
}
__global__ void fill_f32_kernel(float* __restrict__ p, size_t n, float v) {
    const size_t i = (size_t)blockIdx.x * NT + threadIdx.x;
    if (i < n) p[i] = v;
}

unsigned blocks_for(size_t n) { return (unsigned)((n + NT - 1) / NT); }

}  // namespace

// ---- the model -------------------------------------------------------------------------
struct LlamaModel {
    rdl_llama_config cfg{};
    int q_dim = 0, kv_dim = 0, qkv_dim = 0;
    size_t row_q4(int k) const { return (size_t)(k / QK) * Q4_0_BYTES; }

    struct Mat {
        uint8_t* dev = nullptr;
        int n = 0, k = 0;
        WType type = WType::Q4_0;
        size_t row_bytes() const { return (size_t)(k / block_elems(type)) * block_bytes(type); }
        size_t bytes() const { return (size_t)n * row_bytes(); }
    };
    struct Layer {
        // q/k/v rows concatenated and gate/up rows interleaved when the parts
        // share a GGUF type; otherwise the parts stand alone (split_*), q and
        // k still concatenated in qk when theirs agree (qk_joint: llama.cpp's
        // Q4_K_M files give only attn_v another type)
        Mat qkv, o, gu, down;
        Mat q, k, v, gate, up, qk;
        bool split_qkv = false, split_gu = false, qk_joint = false;
        bool fused = false;  // Q4_0 throughout: the fused launches serve m <= 4 rows
        // Linear::use_native_q4 of the layer's Q4_0 / Q4_1 Linears
        // (TransformerBlock::set_native_q4_matmul): activations quantized to
        // Q8_0, int32 block dots (matmul_f32_q4_native / _q4_1_native)
        bool native = false;
        float* attn_norm = nullptr;
        float* ffn_norm = nullptr;
    };
    std::vector<Layer> layers;
    Mat emb, out;
    float* final_norm = nullptr;
    void* kc = nullptr;  // [layer][page][kv_head][KV_PAGE][hd] (paged, kv_row)
    void* vc = nullptr;
    int* kv_table = nullptr;  // [n_pages]: physical page of each logical page
    int n_pages = 0;
    float *cos_t = nullptr, *sin_t = nullptr;
    std::vector<float> cos_h, sin_h;
    // activations for up to max_batch rows
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *gu = nullptr, *hb = nullptr,
          *logits = nullptr;
    float* part_tmp = nullptr;  // [max_batch][qkv_dim]: split q/k/v rows before they join qkv
    int *tokens = nullptr, *pos = nullptr, *step = nullptr, *out_tokens = nullptr;
    size_t out_cap = 0;
    void* gemm_scratch = nullptr;
    int* gemm_cnt = nullptr;  // the skinny GEMMs' strip counters (zero between launches)
    float* att_part = nullptr;  // [max_batch][n_heads][spans of max_seq][hd + 2]
    int* att_cnt = nullptr;     // [max_batch][n_heads] finished-chunk counters (zero between launches)
    int att_nspan = 0;
    // decode steps: attention fused into the q/k/v launch (fused layers, one
    // row), and the previous fused layer's down projection too (fused_down,
    // off by default: on the 7B shape that launch, 24.6 us, took longer than
    // the down GEMV and the fused launch apart, 8.6 + 14.5 us, because its
    // one workgroup a CU leaves no room for q/k/v workgroups to stream their
    // weights while the down projection runs)
    bool fused_attention = true;
    bool fused_down = false;
    // [layer][xch_stride()] exchange of the fused decode launch: the q/k/v
    // values, the attention outputs, then the layer's input x when the
    // previous layer's down projection runs in the launch (zero on an empty cache)
    uint64_t* att_xch = nullptr;
    size_t xch_stride() const { return (size_t)qkv_dim + q_dim + cfg.dim; }
    int* att_err = nullptr;  // set by a fused launch whose wait ran out
    rdl_llama_path_counts path{};  // attention launches enqueued, by kernel
    hipStream_t stream = nullptr;
    hipGraphExec_t decode_exec = nullptr;
    hipGraph_t decode_graph = nullptr;
    hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
    float prefill_ms = 0.0f, decode_ms = 0.0f;
    size_t host_pos = 0;  // mirror of *pos
    std::vector<void*> allocs;

    ~LlamaModel() {
        if (decode_exec) (void)hipGraphExecDestroy(decode_exec);
        if (decode_graph) (void)hipGraphDestroy(decode_graph);
        for (hipEvent_t e : ev)
            if (e) (void)hipEventDestroy(e);
        if (stream) (void)hipStreamDestroy(stream);
        for (void* p : allocs) (void)hipFree(p);
    }

    hipError_t alloc(void** p, size_t bytes) {
        hipError_t e = hipMalloc(p, bytes ? bytes : 16);
        if (e == hipSuccess) allocs.push_back(*p);
        return e;
    }
    template <typename T>
    hipError_t alloc_t(T** p, size_t count) {
        return alloc(reinterpret_cast<void**>(p), count * sizeof(T));
    }
    size_t kv_elem() const { return cfg.kv_f16 ? 2 : 4; }
    size_t kv_layer_elems() const { return (size_t)n_pages * cfg.n_kv_heads * KV_PAGE * cfg.head_dim; }

    // y[m, mat.n] = x[m, mat.k] . W^T on the model's stream; native: the
    // Linear's use_native_q4 (Q4_0 / Q4_1 weights only, as in linear.rs:119-153)
    hipError_t linear(const Mat& w, const float* xin, size_t m, float* y, bool native = false) {
        native = native && (w.type == WType::Q4_0 || w.type == WType::Q4_1);
        if (m <= 4) return launch_gemv_fused(w.type, native, w.dev, w.n, w.k, xin, m, y, stream);
        if (w.type == WType::Q4_0)
            return native ? launch_gemm_q4_0_native(w.dev, w.n, w.k, xin, m, y, nullptr, gemm_scratch, stream)
                          : launch_gemm_q4_0(w.dev, w.n, w.k, xin, m, y, gemm_scratch, gemm_cnt, stream);
        if (kgemm(w, m, native)) {
            const hipError_t e = launch_gemm_typed(w.type, w.dev, w.n, w.k, xin, m, y, gemm_scratch, stream);
            if (e != hipErrorInvalidValue) return e;
        }
        // rows four at a time through the fused GEMV (other types, or scales
        // beyond the GEMM's range)
        for (size_t r = 0; r < m; r += 4) {
            const size_t mr = (m - r < 4) ? m - r : 4;
            hipError_t e = launch_gemv_fused(w.type, native, w.dev, w.n, w.k, xin + r * w.k, mr,
                                             y + r * w.n, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }

    // Attention chunks to launch for m rows starting at the current position
    // (capture_any_pos: the launch is recorded once for every position).
    bool capture_any_pos = false;
    int chunks_needed(size_t m) const {  // workgroups of ATT_SPAN keys
        const size_t upto = capture_any_pos ? (size_t)cfg.max_seq : host_pos + m;
        return (int)((upto + ATT_SPAN - 1) / ATT_SPAN);
    }

    void* kv_layer(void* base, int l) const {
        return reinterpret_cast<uint8_t*>(base) + (size_t)l * kv_layer_elems() * kv_elem();
    }

    // RoPE + cache write (unless the qkv launch did it), then attention.
    template <typename KV>
    hipError_t layer_attention(int l, size_t m, bool rope = true) {
        KV* kcl = reinterpret_cast<KV*>(kv_layer(kc, l));
        KV* vcl = reinterpret_cast<KV*>(kv_layer(vc, l));
        const int hd = cfg.head_dim;
        if (rope)
            hipLaunchKernelGGL(rope_kv_kernel<KV>, dim3(cfg.n_heads + cfg.n_kv_heads, (unsigned)m), dim3(hd / 2), 0,
                               stream, qkv, qkv_dim, pos, cos_t, sin_t, cfg.n_heads, cfg.n_kv_heads, hd, kcl, vcl,
                               kv_table);
        const float scale = sqrtf((float)hd);
        // a prompt chunk whose rows see few pages: a wave a row
        const size_t pages = (host_pos + m + KV_PAGE - 1) / KV_PAGE;
        if constexpr (std::is_same<KV, _Float16>::value) {
            if (m >= PREFILL_ATT_MFMA_MIN_ROWS && !capture_any_pos && (hd == 64 || hd == 128 || hd == 256)) {
                AttArgs<KV> pa{};
                pa.qkv = qkv;
                pa.qkv_dim = qkv_dim;
                pa.pos_dev = pos;
                pa.kc = kcl;
                pa.vc = vcl;
                pa.kv_table = kv_table;
                pa.n_heads = cfg.n_heads;
                pa.n_kv = cfg.n_kv_heads;
                pa.hd_rt = hd;
                pa.scale = scale;
                pa.out = att;
                auto pk = (hd == 128) ? prefill_attention_mfma_kernel<128>
                        : (hd == 64)  ? prefill_attention_mfma_kernel<64>
                                      : prefill_attention_mfma_kernel<256>;
                hipLaunchKernelGGL(pk, dim3(cfg.n_heads, (unsigned)((m + 15) / 16)), dim3(256), 0, stream, pa, (int)m);
                path.prefill_mfma++;
                return hipGetLastError();
            }
        }
        if ((m >= PREFILL_ATT_ALL_ROWS || (m >= PREFILL_ATT_MIN_ROWS && pages <= PREFILL_ATT_MAX_PAGES)) &&
            !capture_any_pos &&
            (hd == 64 || hd == 128 || hd == 256)) {
            AttArgs<KV> pa{};
            pa.qkv = qkv;
            pa.qkv_dim = qkv_dim;
            pa.pos_dev = pos;
            pa.kc = kcl;
            pa.vc = vcl;
            pa.kv_table = kv_table;
            pa.n_heads = cfg.n_heads;
            pa.n_kv = cfg.n_kv_heads;
            pa.hd_rt = hd;
            pa.scale = scale;
            pa.out = att;
            auto pk = (hd == 128) ? prefill_attention_kernel<KV, 128>
                    : (hd == 64)  ? prefill_attention_kernel<KV, 64>
                                  : prefill_attention_kernel<KV, 256>;
            hipLaunchKernelGGL(pk, dim3(cfg.n_heads, (unsigned)((m + 7) / 8)), dim3(512), 0, stream, pa, (int)m);
            path.prefill_rows++;
            return hipGetLastError();
        }
        // chunks that can hold keys for these rows (every chunk of the cache
        // when the launch is captured for replay at any position)
        const int nz = chunks_needed(m);
        const dim3 grid(cfg.n_heads, (unsigned)m, (unsigned)nz);
        const size_t lds = (size_t)(1 + ATT_WAVES) * hd * sizeof(float);
        auto kern = (hd == 128) ? attention_kernel<KV, 128>
                  : (hd == 64)  ? attention_kernel<KV, 64>
                  : (hd == 256) ? attention_kernel<KV, 256>
                                : attention_kernel<KV, 0>;
        AttArgs<KV> aa{};
        aa.qkv = qkv;
        aa.qkv_dim = qkv_dim;
        aa.pos_dev = pos;
        aa.kc = kcl;
        aa.vc = vcl;
        aa.kv_table = kv_table;
        aa.n_heads = cfg.n_heads;
        aa.n_kv = cfg.n_kv_heads;
        aa.hd_rt = hd;
        aa.scale = scale;
        aa.part = att_part;
        aa.nspan = att_nspan;
        aa.counters = att_cnt;
        aa.out = att;
        hipLaunchKernelGGL(kern, grid, dim3(64 * ATT_WAVES), lds, stream, aa);
        path.attention++;
        return hipGetLastError();
    }

    // x += h . Wdown^T of fused layer l (h: its SwiGLU rows in hb)
    hipError_t layer_down(int l, size_t m) {
        const Layer& L = layers[l];
        return launch_gemv_q4_0_fused_ex(L.down.dev, L.down.n, cfg.ffn_dim, hb, cfg.ffn_dim, m, x, 0, nullptr,
                                         0.0f, 1, stream);
    }

    // One layer through the fused Q4_0 launches (m <= 4): RMSNorm, RoPE + KV,
    // SwiGLU and the residual adds ride in the GEMV launches (prologue /
    // epilogue of the fused GEMV): five launches, three in a decode step
    // (q/k/v, attention and o in one launch), two when the previous layer's
    // down projection joins that launch.  pending: a fused layer whose down
    // projection has not run yet (its SwiGLU rows in hb), or -1; this call
    // runs it and may leave its own layer's pending instead.
    hipError_t layer_fused(int l, size_t m, int& pending) {
        const int d = cfg.dim;
        const float eps = cfg.norm_eps;
        Layer& L = layers[l];
        hipError_t e;
        if (m == 1 && fused_attention) {
            // q/k/v, RoPE + cache, the attention over the cache and the o
            // projection with its residual add in one launch (led by the
            // pending down projection, whose new x reaches q/k/v and o through
            // the exchange)
            uint64_t* xl = att_xch + (size_t)l * xch_stride();
            for (int chain = pending >= 0 ? 1 : 0; chain >= 0; chain--) {
                e = launch_qkv_attention(L.qkv.dev, L.qkv.n, d, x, qkv, L.attn_norm, eps, pos, cos_t, sin_t,
                                         kv_layer(kc, l), kv_layer(vc, l), kv_table, cfg.n_heads, cfg.n_kv_heads,
                                         cfg.head_dim, cfg.kv_f16 != 0, att_part, att_nspan, chunks_needed(1),
                                         att_cnt, att, xl, att_err, L.o.dev, L.o.n, x, xl + qkv_dim, stream,
                                         chain ? layers[pending].down.dev : nullptr, cfg.ffn_dim, hb,
                                         xl + qkv_dim + q_dim);
                if (e == hipErrorInvalidValue) {
                    (void)hipGetLastError();
                    if (chain) {  // a shape the joint launch does not take: the down on its own first
                        if ((e = layer_down(pending, m)) != hipSuccess) return e;
                        pending = -1;
                    }
                    continue;
                }
                if (e != hipSuccess) return e;
                path.fused_decode++;
                if (chain) {
                    path.fused_down++;
                    pending = -1;
                }
                return layer_fused_tail(l, m, true, pending);
            }
        }
        if (pending >= 0) {
            if ((e = layer_down(pending, m)) != hipSuccess) return e;
            pending = -1;
        }
        // q = rope(rms_norm(x) . Wq^T); k, v -> cache (RoPE on k) in the same launch
        e = launch_gemv_q4_0_rope_kv(L.qkv.dev, L.qkv.n, d, x, m, qkv, L.attn_norm, eps, pos, cos_t,
                                                sin_t, kv_layer(kc, l), kv_layer(vc, l), cfg.n_heads, cfg.n_kv_heads,
                                                cfg.head_dim, kv_table, cfg.kv_f16 != 0, stream);
        if (e != hipSuccess) return e;
        e = cfg.kv_f16 ? layer_attention<_Float16>(l, m, false) : layer_attention<float>(l, m, false);
        if (e != hipSuccess) return e;
        return layer_fused_tail(l, m, false, pending);
    }

    // o (unless o_done), gate/up and down of a fused layer (after its
    // attention); the down projection is left pending (for the next layer's
    // fused decode launch) when that layer can take it
    hipError_t layer_fused_tail(int l, size_t m, bool o_done, int& pending) {
        const int d = cfg.dim;
        const float eps = cfg.norm_eps;
        Layer& L = layers[l];
        hipError_t e;
        // x += att . Wo^T
        if (!o_done) {
            e = launch_gemv_q4_0_fused_ex(L.o.dev, L.o.n, q_dim, att, q_dim, m, x, 0, nullptr, 0.0f, 1, stream);
            if (e != hipSuccess) return e;
        }
        // h = silu(gate) * up with [gate; up] = rms_norm(x) . Wgu^T (rows interleaved)
        e = launch_gemv_q4_0_fused_ex(L.gu.dev, L.gu.n, d, x, d, m, hb, 1, L.ffn_norm, eps, 2, stream);
        if (e != hipSuccess) return e;
        // x += h . Wdown^T, now or in the next layer's launch
        if (m == 1 && fused_attention && fused_down && l + 1 < cfg.n_layers && layers[l + 1].fused &&
            !layers[l + 1].native) {
            pending = l;
            return hipSuccess;
        }
        return layer_down(l, m);
    }

    static bool kquant(const Mat& w) { return w.type == WType::Q4_K || w.type == WType::Q6_K; }
    // Q4_K / Q6_K / Q8_0 products of m >= KQ_GEMM_MIN_M rows, and Q4_1 ones
    // outside native mode, run on the LDS tile GEMM
    static bool kgemm(const Mat& w, size_t m, bool native = false) {
        const bool typed = kquant(w) || w.type == WType::Q8_0 || (w.type == WType::Q4_1 && !native);
        return typed && m >= KQ_GEMM_MIN_M && w.k % (int)block_elems(w.type) == 0 && w.k <= 16384;
    }
    // the K-quant GEMVs with the decoder's steps folded into their launches
    static bool kfold(const Mat& w, size_t m) { return kquant(w) && !kgemm(w, m); }

    // y rows (ystride floats apart) = epilogue(W . prologue(x rows)) through the
    // K-quant decoder fusion, four rows a launch
    hipError_t kq_linear(const Mat& w, const float* xin, size_t xstride, size_t m, float* y, size_t ystride,
                         int pro, const float* g, int epi) {
        for (size_t r = 0; r < m; r += 4) {
            const size_t mr = (m - r < 4) ? m - r : 4;
            hipError_t e = launch_gemv_kquant_ex(w.type, w.dev, w.n, w.k, xin + r * xstride, xstride, mr,
                                                 y + r * ystride, ystride, pro, g, cfg.norm_eps, epi, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }

    // One layer of any resident types, any row count (m > 4 Q4_0 rows and
    // m >= KQ_GEMM_MIN_M rows of the other types take the GEMMs).  Q4_K / Q6_K matrices on
    // the GEMVs fold the RMSNorm in front of them, the residual add after o /
    // down, the SwiGLU of combined gate/up rows and the RoPE + cache write of
    // combined q/k/v rows into their GEMV launches; the other types run
    // separate norm / add / SwiGLU / RoPE launches.
    hipError_t layer_plain(int l, size_t m) {
        const int d = cfg.dim, f = cfg.ffn_dim;
        Layer& L = layers[l];
        hipError_t e;
        auto rmsnorm = [&](const float* g) {
            hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)m), dim3(NT), 0, stream, x, g, d, cfg.norm_eps, xn);
        };
        // ---- q, k, v -> qkv rows ----
        const Mat* parts[3] = {&L.qkv, nullptr, nullptr};
        int cols[3] = {0, q_dim, q_dim + kv_dim};
        int np = 1;
        if (L.split_qkv && L.qk_joint) {
            parts[0] = &L.qk, parts[1] = &L.v;
            cols[1] = q_dim + kv_dim;
            np = 2;
        } else if (L.split_qkv) {
            parts[0] = &L.q, parts[1] = &L.k, parts[2] = &L.v;
            np = 3;
        }
        // Q4_0 (m > GEMM_XTILE_M) and other prompt chunks (m >= KQ_GEMM_MIN_M) on the LDS tile GEMM
        // fold the RMSNorms, the SwiGLU and the residual adds into the GEMMs'
        // x splits and stores (hipErrorInvalidValue: a shape they do not take,
        // nothing launched, the separate launches below run instead)
        // (native layers keep their Linears' own products: no folding)
        auto q4t = [&](const Mat& w) {
            return !L.native && ((m > GEMM_XTILE_M && w.type == WType::Q4_0) || kgemm(w, m));
        };
        auto kfold_m = [&](const Mat& w) { return kfold(w, m); };
        const bool nat = L.native;
        bool qkv_done = false;
        if (np == 1 && q4t(L.qkv)) {
            e = launch_gemm_tiles_ex(L.qkv.type, L.qkv.dev, L.qkv.n, L.qkv.k, x, m, qkv, gemm_scratch, 1,
                                     L.attn_norm, cfg.norm_eps, false, stream);
            if (e != hipSuccess && e != hipErrorInvalidValue) return e;
            qkv_done = e == hipSuccess;
        }
        bool want_xn = false;
        for (int i = 0; i < np; i++) want_xn |= !kfold_m(*parts[i]);
        if (want_xn && !qkv_done) rmsnorm(L.attn_norm);
        // a K-quant [Wq; Wk; Wv] (or K-quant [Wq; Wk] and Wv, two launches)
        // also applies RoPE and writes the cache
        const bool rope_fused = !qkv_done && ((np == 1 && kfold_m(L.qkv)) ||
                                              (np == 2 && kfold_m(L.qk) && kfold_m(L.v)));
        for (size_t r = 0; rope_fused && r < m; r += 4) {
            const size_t mr = (m - r < 4) ? m - r : 4;
            for (int i = 0; i < np; i++) {
                const Mat& w = *parts[i];
                e = launch_gemv_kquant_rope_kv(w.type, w.dev, w.n, d, x + r * d, mr, r, qkv + r * qkv_dim + cols[i],
                                               qkv_dim, L.attn_norm, cfg.norm_eps, pos, cos_t, sin_t,
                                               kv_layer(kc, l), kv_layer(vc, l), cfg.n_heads, cfg.n_kv_heads,
                                               cfg.head_dim, cols[i] / cfg.head_dim, kv_table, cfg.kv_f16 != 0,
                                               stream);
                if (e != hipSuccess) return e;
            }
        }
        for (int i = 0; i < np && !rope_fused && !qkv_done; i++) {
            const Mat& w = *parts[i];
            if (kfold_m(w)) {
                e = kq_linear(w, x, d, m, qkv + cols[i], qkv_dim, GEMV_PRO_RMSNORM, L.attn_norm, GEMV_EPI_STORE);
            } else if (np == 1 || m == 1) {  // whole rows, or one row: in place
                e = linear(w, xn, m, qkv + cols[i], nat);
            } else {  // [m, part] rows, then strided into the [m, qkv_dim] rows
                if ((e = linear(w, xn, m, part_tmp, nat)) != hipSuccess) return e;
                const size_t wb = (size_t)w.n * sizeof(float);
                e = hipMemcpy2DAsync(qkv + cols[i], (size_t)qkv_dim * sizeof(float), part_tmp, wb, wb, m,
                                     hipMemcpyDeviceToDevice, stream);
            }
            if (e != hipSuccess) return e;
        }
        e = cfg.kv_f16 ? layer_attention<_Float16>(l, m, !rope_fused) : layer_attention<float>(l, m, !rope_fused);
        if (e != hipSuccess) return e;
        // ---- x += att . Wo^T ----
        e = q4t(L.o) ? launch_gemm_tiles_ex(L.o.type, L.o.dev, L.o.n, L.o.k, att, m, x, gemm_scratch, 0, nullptr,
                                            0.0f, true, stream)
                     : hipErrorInvalidValue;
        if (e != hipSuccess && e != hipErrorInvalidValue) return e;
        if (e == hipSuccess) {
        } else if (kfold_m(L.o)) {
            e = kq_linear(L.o, att, q_dim, m, x, d, GEMV_PRO_NONE, nullptr, GEMV_EPI_RESIDUAL);
            if (e != hipSuccess) return e;
        } else {
            if ((e = linear(L.o, att, m, xn, nat)) != hipSuccess) return e;
            hipLaunchKernelGGL(add_kernel, dim3(blocks_for(m * d)), dim3(NT), 0, stream, x, xn, m * d);
        }
        // ---- h = silu(gate) * up ----
        const size_t nf = m * (size_t)f;
        // gu_raw: gu holds the interleaved gate / up rows and the down GEMM's
        // x split forms h from them
        bool gu_raw = false;
        if (!L.split_gu && q4t(L.gu) && q4t(L.down)) {
            e = launch_gemm_tiles_ex(L.gu.type, L.gu.dev, L.gu.n, L.gu.k, x, m, gu, gemm_scratch, 1, L.ffn_norm,
                                     cfg.norm_eps, false, stream);
            if (e != hipSuccess && e != hipErrorInvalidValue) return e;
            gu_raw = e == hipSuccess;
        }
        if (gu_raw) {
        } else if (!L.split_gu && kfold_m(L.gu)) {
            e = kq_linear(L.gu, x, d, m, hb, f, GEMV_PRO_RMSNORM, L.ffn_norm, GEMV_EPI_SWIGLU);
            if (e != hipSuccess) return e;
        } else if (!L.split_gu) {
            rmsnorm(L.ffn_norm);
            if ((e = linear(L.gu, xn, m, gu, nat)) != hipSuccess) return e;
            hipLaunchKernelGGL(swiglu_kernel, dim3(blocks_for(nf)), dim3(NT), 0, stream, gu, f, nf, hb);
        } else {
            if (!kfold_m(L.gate) || !kfold_m(L.up)) rmsnorm(L.ffn_norm);
            const Mat* gp[2] = {&L.gate, &L.up};
            for (int i = 0; i < 2; i++) {
                float* yo = gu + i * nf;
                e = kfold_m(*gp[i]) ? kq_linear(*gp[i], x, d, m, yo, f, GEMV_PRO_RMSNORM, L.ffn_norm, GEMV_EPI_STORE)
                                   : linear(*gp[i], xn, m, yo, nat);
                if (e != hipSuccess) return e;
            }
            hipLaunchKernelGGL(swiglu2_kernel, dim3(blocks_for(nf)), dim3(NT), 0, stream, gu, gu + nf, nf, hb);
        }
        // ---- x += h . Wdown^T ----
        if (gu_raw) {
            e = launch_gemm_tiles_ex(L.down.type, L.down.dev, L.down.n, L.down.k, gu, m, x, gemm_scratch, 2, nullptr,
                                     0.0f, true, stream);
            if (e != hipSuccess && e != hipErrorInvalidValue) return e;
            if (e == hipErrorInvalidValue) {  // the SwiGLU on its own, then the product
                hipLaunchKernelGGL(swiglu_kernel, dim3(blocks_for(nf)), dim3(NT), 0, stream, gu, f, nf, hb);
                if ((e = linear(L.down, hb, m, xn, nat)) != hipSuccess) return e;
                hipLaunchKernelGGL(add_kernel, dim3(blocks_for(m * d)), dim3(NT), 0, stream, x, xn, m * d);
            }
        } else if (kfold_m(L.down)) {
            e = kq_linear(L.down, hb, f, m, x, d, GEMV_PRO_NONE, nullptr, GEMV_EPI_RESIDUAL);
            if (e != hipSuccess) return e;
        } else {
            if ((e = linear(L.down, hb, m, xn, nat)) != hipSuccess) return e;
            hipLaunchKernelGGL(add_kernel, dim3(blocks_for(m * d)), dim3(NT), 0, stream, x, xn, m * d);
        }
        return hipGetLastError();
    }

    bool fused_shapes = false;  // the model's shapes meet the fused launches' rules
    bool sample_embeds = false; // Q4_0 embedding table: sample_kernel writes the next x

    // forward_with_cache_pass over m rows whose token ids are in `tokens`, the
    // last row's logits into `logits`.  embed: x from the token ids (otherwise
    // x already holds the rows, as sample_kernel leaves them); advance: the
    // position moves on by m here.
    hipError_t forward(size_t m, bool embed = true, bool advance = true) {
        const int d = cfg.dim;
        const float eps = cfg.norm_eps;
        hipError_t e = hipSuccess;
        if (embed && (e = launch_dequant_rows(emb.type, emb.dev, emb.n, emb.k, tokens, m, x, stream)) != hipSuccess)
            return e;
        int pending = -1;  // a fused layer whose down projection has not run yet
        for (int l = 0; l < cfg.n_layers; l++) {
            if (m <= 4 && layers[l].fused && !layers[l].native) {
                e = layer_fused(l, m, pending);
            } else {
                if (pending >= 0 && (e = layer_down(pending, m)) != hipSuccess) return e;
                pending = -1;
                e = layer_plain(l, m);
            }
            if (e != hipSuccess) return e;
        }
        if (pending >= 0 && (e = layer_down(pending, m)) != hipSuccess) return e;
        // logits = rms_norm(x_last, norm) . Wout^T (the norm fused into the GEMV for Q4_0, Q4_K, Q6_K)
        if (fused_shapes && out.type == WType::Q4_0) {
            e = launch_gemv_q4_0_fused_ex(out.dev, out.n, d, x + (m - 1) * d, d, 1, logits, 1, final_norm, eps, 0,
                                          stream);
        } else if (kquant(out)) {
            e = kq_linear(out, x + (m - 1) * d, d, 1, logits, out.n, GEMV_PRO_RMSNORM, final_norm, GEMV_EPI_STORE);
        } else {
            hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(NT), 0, stream, x + (m - 1) * d, final_norm, d, eps, xn);
            e = linear(out, xn, 1, logits);
        }
        if (e != hipSuccess) return e;
        if (advance) hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, stream, pos, (int)m);
        return hipGetLastError();
    }

    // argmax of `logits` -> token, out_tokens, step; position += advance; the
    // token's embedding row -> x (the input of the next decode step)
    void sample(int advance) {
        hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(SAMPLE_NT), 0, stream, logits, cfg.vocab, tokens, out_tokens,
                           step, pos, advance, sample_embeds ? emb.dev : nullptr, cfg.dim, x);
    }

    // One greedy decode step: the last token (its embedding in x when the
    // sampling launch wrote it) -> logits -> sample: the next token (and its
    // embedding, and the position advance, when the table is Q4_0).
    hipError_t decode_step() {
        hipError_t e = forward(1, !sample_embeds, !sample_embeds);
        if (e != hipSuccess) return e;
        sample(sample_embeds ? 1 : 0);
        return hipGetLastError();
    }
};

}  // namespace rdl

struct rdl_llama {
    rdl::LlamaModel m;
};

using rdl::api_fail;
using rdl::api_ok;

namespace {

bool valid_config(const rdl_llama_config& c) {
    return c.dim > 0 && c.n_layers > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.head_dim > 0 &&
           c.head_dim % 2 == 0 && c.head_dim <= 256 && c.n_heads % c.n_kv_heads == 0 && c.ffn_dim > 0 &&
           c.vocab > 0 && c.max_seq > 0 && c.max_seq <= 65536 && c.max_batch > 0 && c.dim % 32 == 0 && c.ffn_dim % 32 == 0 &&
           (c.n_heads * c.head_dim) % 32 == 0 && c.dim <= 16384 && c.ffn_dim <= 16384 &&
           c.n_heads * c.head_dim <= 16384;
}

// Where a weight slot's bytes go: `rows` rows of row_bytes, at dst with row
// pitch dpitch (the gate and up rows interleave in one matrix).
struct SlotTarget {
    uint8_t* dst = nullptr;
    size_t row_bytes = 0, rows = 0, dpitch = 0;
    rdl::LlamaModel::Mat* mat = nullptr;  // quantized matrix to rescan after the copy
    bool q4 = false;                      // Q4_0 rows (else f32 norm weights)
    size_t bytes() const { return row_bytes * rows; }
};

rdl_status slot_target(rdl::LlamaModel& M, int32_t slot, int32_t layer, SlotTarget* t) {
    const rdl_llama_config& c = M.cfg;
    const bool per_layer = slot >= RDL_LLAMA_ATTN_NORM && slot <= RDL_LLAMA_W_DOWN;
    if (per_layer && (layer < 0 || layer >= c.n_layers))
        return api_fail(RDL_ERR_INVALID_DATA, "layer %d out of range", layer);
    auto q4 = [&](rdl::LlamaModel::Mat& w, int row0, int rows, int interleave = 1) {
        const size_t rb = w.row_bytes();
        t->mat = &w;
        t->q4 = true;
        t->row_bytes = rb;
        t->rows = (size_t)rows;
        t->dpitch = rb * interleave;
        t->dst = w.dev + (size_t)row0 * rb;
    };
    auto f32 = [&](float* p) {
        t->dst = reinterpret_cast<uint8_t*>(p);
        t->row_bytes = t->dpitch = (size_t)c.dim * 4;
        t->rows = 1;
    };
    switch (slot) {
        case RDL_LLAMA_TOKEN_EMBEDDING: q4(M.emb, 0, c.vocab); t->mat = nullptr; break;  // no GEMM over it
        case RDL_LLAMA_OUTPUT: q4(M.out, 0, c.vocab); break;
        case RDL_LLAMA_FINAL_NORM: f32(M.final_norm); break;
        case RDL_LLAMA_ATTN_NORM: f32(M.layers[layer].attn_norm); break;
        case RDL_LLAMA_FFN_NORM: f32(M.layers[layer].ffn_norm); break;
        case RDL_LLAMA_WQ: {
            auto& L = M.layers[layer];
            L.split_qkv ? (L.qk_joint ? q4(L.qk, 0, M.q_dim) : q4(L.q, 0, M.q_dim)) : q4(L.qkv, 0, M.q_dim);
            break;
        }
        case RDL_LLAMA_WK: {
            auto& L = M.layers[layer];
            L.split_qkv ? (L.qk_joint ? q4(L.qk, M.q_dim, M.kv_dim) : q4(L.k, 0, M.kv_dim))
                        : q4(L.qkv, M.q_dim, M.kv_dim);
            break;
        }
        case RDL_LLAMA_WV: {
            auto& L = M.layers[layer];
            L.split_qkv ? q4(L.v, 0, M.kv_dim) : q4(L.qkv, M.q_dim + M.kv_dim, M.kv_dim);
            break;
        }
        case RDL_LLAMA_WO: q4(M.layers[layer].o, 0, c.dim); break;
        case RDL_LLAMA_W_GATE: {  // even rows of the interleaved [gate; up]
            auto& L = M.layers[layer];
            L.split_gu ? q4(L.gate, 0, c.ffn_dim) : q4(L.gu, 0, c.ffn_dim, 2);
            break;
        }
        case RDL_LLAMA_W_UP: {  // odd rows
            auto& L = M.layers[layer];
            L.split_gu ? q4(L.up, 0, c.ffn_dim) : q4(L.gu, 1, c.ffn_dim, 2);
            break;
        }
        case RDL_LLAMA_W_DOWN: q4(M.layers[layer].down, 0, c.dim); break;
        default: return api_fail(RDL_ERR_INVALID_DATA, "unknown weight slot %d", slot);
    }
    return api_ok();
}


// After a synchronized call: a fused attention launch whose wait for its q/k/v
// workgroups ran out (which a correct launch never does) left the flag set.
rdl_status check_fused(rdl::LlamaModel& M) {
    int err = 0;
    HIP_TRY(hipMemcpy(&err, M.att_err, sizeof(int), hipMemcpyDeviceToHost));
    if (!err) return RDL_OK;
    HIP_TRY(hipMemset(M.att_err, 0, sizeof(int)));
    HIP_TRY(hipMemset(M.att_xch, 0, (size_t)M.cfg.n_layers * M.xch_stride() * sizeof(uint64_t)));
    return api_fail(RDL_ERR_HIP, "fused decode attention: a wait for the q/k/v workgroups ran out");
}

}  // namespace

extern "C" {

rdl_status rdl_llama_create(const rdl_llama_config* cfg, rdl_llama** out) {
    return rdl_llama_create_typed(cfg, nullptr, out);
}

rdl_status rdl_llama_create_typed(const rdl_llama_config* cfg, const int32_t* types, rdl_llama** out) {
    if (!cfg || !out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    *out = nullptr;
    if (!valid_config(*cfg))
        return api_fail(RDL_ERR_INVALID_DATA,
                        "unsupported config (dim, ffn_dim, heads*head_dim multiples of 32 and <= 16384; "
                        "head_dim even <= 256; n_heads %% n_kv_heads == 0)");
    const int32_t od = cfg->output_dtype == 0 ? RDL_DTYPE_Q4_0 : cfg->output_dtype;
    const int q_dim = cfg->n_heads * cfg->head_dim;
    // the GGUF type of every matrix: types[layer * RDL_LLAMA_SLOTS + slot],
    // model-level slots in layer 0's row; 0 = Q4_0 (the output: output_dtype)
    auto type_of = [&](int slot, int layer) -> int32_t {
        const int32_t t = types ? types[(size_t)layer * RDL_LLAMA_SLOTS + slot] : 0;
        if (t != 0) return t;
        return slot == RDL_LLAMA_OUTPUT ? od : RDL_DTYPE_Q4_0;
    };
    auto in_features = [&](int slot) {
        return slot == RDL_LLAMA_WO ? q_dim : slot == RDL_LLAMA_W_DOWN ? cfg->ffn_dim : cfg->dim;
    };
    for (int l = 0; l < cfg->n_layers; l++)
        for (int slot = 0; slot < RDL_LLAMA_SLOTS; slot++) {
            const bool model_slot =
                slot == RDL_LLAMA_TOKEN_EMBEDDING || slot == RDL_LLAMA_FINAL_NORM || slot == RDL_LLAMA_OUTPUT;
            if (slot == RDL_LLAMA_ATTN_NORM || slot == RDL_LLAMA_FFN_NORM || slot == RDL_LLAMA_FINAL_NORM ||
                (model_slot && l > 0))
                continue;
            const int32_t t = type_of(slot, l);
            if (t != RDL_DTYPE_Q4_0 && t != RDL_DTYPE_Q8_0 && t != RDL_DTYPE_Q4_1 && t != RDL_DTYPE_Q4_K &&
                t != RDL_DTYPE_Q6_K)
                return api_fail(RDL_ERR_UNSUPPORTED, "slot %d layer %d: type %d (Q4_0, Q8_0, Q4_1, Q4_K or Q6_K)",
                                slot, l, t);
            if ((t == RDL_DTYPE_Q4_K || t == RDL_DTYPE_Q6_K) && in_features(slot) % rdl::QK_K != 0)
                return api_fail(RDL_ERR_UNSUPPORTED, "slot %d layer %d: a K-quant matrix needs in_features %% 256 "
                                "== 0 (%d)", slot, l, in_features(slot));
        }
    rdl_status st = rdl::api_require_device();
    if (st != RDL_OK) return st;
    rdl_llama* h = new rdl_llama();
    rdl::LlamaModel& M = h->m;
    M.cfg = *cfg;
    M.cfg.output_dtype = type_of(RDL_LLAMA_OUTPUT, 0);
    M.out.type = (rdl::WType)M.cfg.output_dtype;
    M.emb.type = (rdl::WType)type_of(RDL_LLAMA_TOKEN_EMBEDDING, 0);
    M.sample_embeds = M.emb.type == rdl::WType::Q4_0;
    const rdl_llama_config& c = M.cfg;
    M.q_dim = c.n_heads * c.head_dim;
    M.kv_dim = c.n_kv_heads * c.head_dim;
    M.qkv_dim = M.q_dim + 2 * M.kv_dim;
    auto mat = [&](rdl::LlamaModel::Mat& w, int n, int k, int32_t t = RDL_DTYPE_Q4_0) -> hipError_t {
        w.n = n;
        w.k = k;
        w.type = (rdl::WType)t;
        return M.alloc(reinterpret_cast<void**>(&w.dev), w.bytes() + 64);
    };
    auto fail_free = [&](hipError_t e) {
        delete h;
        return api_fail(RDL_ERR_HIP, "allocation failed: %s", hipGetErrorString(e));
    };
    hipError_t e = hipStreamCreateWithFlags(&M.stream, hipStreamNonBlocking);
    if (e != hipSuccess) return fail_free(e);
    for (auto& ev : M.ev)
        if ((e = hipEventCreate(&ev)) != hipSuccess) return fail_free(e);
    M.layers.resize(c.n_layers);
    bool any_split_qkv = false;
    for (int l = 0; l < c.n_layers; l++) {
        rdl::LlamaModel::Layer& L = M.layers[l];
        const int32_t tq = type_of(RDL_LLAMA_WQ, l), tk = type_of(RDL_LLAMA_WK, l), tv = type_of(RDL_LLAMA_WV, l);
        const int32_t tg = type_of(RDL_LLAMA_W_GATE, l), tu = type_of(RDL_LLAMA_W_UP, l);
        L.split_qkv = tq != tk || tq != tv;
        L.split_gu = tg != tu;
        any_split_qkv |= L.split_qkv;
        L.qk_joint = L.split_qkv && tq == tk;
        if (L.qk_joint) {
            if ((e = mat(L.qk, M.q_dim + M.kv_dim, c.dim, tq)) != hipSuccess) return fail_free(e);
            if ((e = mat(L.v, M.kv_dim, c.dim, tv)) != hipSuccess) return fail_free(e);
        } else if (L.split_qkv) {
            if ((e = mat(L.q, M.q_dim, c.dim, tq)) != hipSuccess) return fail_free(e);
            if ((e = mat(L.k, M.kv_dim, c.dim, tk)) != hipSuccess) return fail_free(e);
            if ((e = mat(L.v, M.kv_dim, c.dim, tv)) != hipSuccess) return fail_free(e);
        } else if ((e = mat(L.qkv, M.qkv_dim, c.dim, tq)) != hipSuccess) {
            return fail_free(e);
        }
        if ((e = mat(L.o, c.dim, M.q_dim, type_of(RDL_LLAMA_WO, l))) != hipSuccess) return fail_free(e);
        if (L.split_gu) {
            if ((e = mat(L.gate, c.ffn_dim, c.dim, tg)) != hipSuccess) return fail_free(e);
            if ((e = mat(L.up, c.ffn_dim, c.dim, tu)) != hipSuccess) return fail_free(e);
        } else if ((e = mat(L.gu, 2 * c.ffn_dim, c.dim, tg)) != hipSuccess) {
            return fail_free(e);
        }
        if ((e = mat(L.down, c.dim, c.ffn_dim, type_of(RDL_LLAMA_W_DOWN, l))) != hipSuccess) return fail_free(e);
        if ((e = M.alloc_t(&L.attn_norm, c.dim)) != hipSuccess) return fail_free(e);
        if ((e = M.alloc_t(&L.ffn_norm, c.dim)) != hipSuccess) return fail_free(e);
    }
    if ((e = mat(M.emb, c.vocab, c.dim, (int32_t)M.emb.type)) != hipSuccess) return fail_free(e);
    if ((e = mat(M.out, c.vocab, c.dim, (int32_t)M.out.type)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.final_norm, c.dim)) != hipSuccess) return fail_free(e);
    M.n_pages = (c.max_seq + rdl::KV_PAGE - 1) / rdl::KV_PAGE;
    const size_t kv_bytes = (size_t)c.n_layers * M.kv_layer_elems() * M.kv_elem();
    if ((e = M.alloc(&M.kc, kv_bytes)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc(&M.vc, kv_bytes)) != hipSuccess) return fail_free(e);
    {  // identity page table: the layout of a contiguous cache
        std::vector<int> ident(M.n_pages);
        for (int p = 0; p < M.n_pages; p++) ident[p] = p;
        if ((e = M.alloc_t(&M.kv_table, M.n_pages)) != hipSuccess) return fail_free(e);
        if ((e = hipMemcpy(M.kv_table, ident.data(), ident.size() * sizeof(int), hipMemcpyHostToDevice)) != hipSuccess)
            return fail_free(e);
    }
    const size_t mb = c.max_batch;
    if ((e = M.alloc_t(&M.x, mb * c.dim)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.xn, mb * c.dim)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.qkv, mb * M.qkv_dim)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.att, mb * M.q_dim)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.gu, mb * 2 * c.ffn_dim)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.hb, mb * c.ffn_dim)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.logits, c.vocab)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.tokens, mb)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.pos, 1)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.step, 1)) != hipSuccess) return fail_free(e);
    M.out_cap = (size_t)c.max_seq + 1;
    if ((e = M.alloc_t(&M.out_tokens, M.out_cap)) != hipSuccess) return fail_free(e);
    // GEMM scratch for every chunk size and matrix shape the prefill runs
    size_t gsb = 0, nmax = 0;
    const size_t shapes[][2] = {{(size_t)M.qkv_dim, (size_t)c.dim}, {(size_t)c.dim, (size_t)M.q_dim},
                                {2 * (size_t)c.ffn_dim, (size_t)c.dim}, {(size_t)c.dim, (size_t)c.ffn_dim},
                                {(size_t)M.q_dim, (size_t)c.dim}, {(size_t)c.n_kv_heads * c.head_dim, (size_t)c.dim},
                                {(size_t)c.ffn_dim, (size_t)c.dim}};
    size_t gcc = 1;  // GEMM counters: the most any shape needs
    for (const auto& sh : shapes) {
        nmax = std::max(nmax, sh[0]);
        gcc = std::max(gcc, rdl::gemm_counter_count(sh[0], sh[1]));
        // every skinny shape (it depends on ceil(m / 16)) and the largest
        // chunk, in float and in native mode (rdl_llama_set_native_q4)
        for (size_t mm : {(size_t)1, (size_t)16, (size_t)32, (size_t)48, (size_t)64, mb})
            for (bool nat : {false, true})
                gsb = std::max(gsb, rdl::gemm_scratch_bytes(std::min(mm, mb), sh[0], sh[1], nat));
        // K-quant matrices on the tile GEMM (x' block sums beside the split)
        gsb = std::max(gsb, rdl::gemm_tiles_scratch_bytes(mb, sh[1]));
    }
    if ((e = M.alloc(&M.gemm_scratch, gsb)) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.gemm_cnt, gcc)) != hipSuccess) return fail_free(e);
    if ((e = hipMemset(M.gemm_cnt, 0, gcc * sizeof(int))) != hipSuccess)
        return fail_free(e);
    if (any_split_qkv && (e = M.alloc_t(&M.part_tmp, mb * M.qkv_dim)) != hipSuccess) return fail_free(e);
    // (row-pair epilogues need at most 4 columns per lane: dim <= 8192)
    M.fused_shapes = (c.dim / 32) % 2 == 0 && (M.q_dim / 32) % 2 == 0 && (c.ffn_dim / 32) % 2 == 0 &&
                     c.dim / 32 <= 256 &&
                     (uint64_t)2 * c.ffn_dim * (c.dim / 32) * rdl::Q4_0_BYTES <= rdl::FUSED_MAX_WEIGHT_BYTES &&
                     (uint64_t)c.vocab * (c.dim / 32) * rdl::Q4_0_BYTES <= rdl::FUSED_MAX_WEIGHT_BYTES;
    for (auto& L : M.layers)
        L.fused = M.fused_shapes && !L.split_qkv && !L.split_gu && L.qkv.type == rdl::WType::Q4_0 &&
                  L.o.type == rdl::WType::Q4_0 && L.gu.type == rdl::WType::Q4_0 && L.down.type == rdl::WType::Q4_0;
    M.att_nspan = (c.max_seq + rdl::ATT_SPAN - 1) / rdl::ATT_SPAN;
    if ((e = M.alloc_t(&M.att_part, mb * c.n_heads * (size_t)M.att_nspan * (c.head_dim + 2))) != hipSuccess)
        return fail_free(e);
    if ((e = M.alloc_t(&M.att_cnt, mb * c.n_heads)) != hipSuccess) return fail_free(e);
    if ((e = hipMemset(M.att_cnt, 0, mb * c.n_heads * sizeof(int))) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.att_xch, (size_t)c.n_layers * M.xch_stride())) != hipSuccess) return fail_free(e);
    if ((e = hipMemset(M.att_xch, 0, (size_t)c.n_layers * M.xch_stride() * sizeof(uint64_t))) != hipSuccess)
        return fail_free(e);
    if ((e = M.alloc_t(&M.att_err, 1)) != hipSuccess) return fail_free(e);
    if ((e = hipMemset(M.att_err, 0, sizeof(int))) != hipSuccess) return fail_free(e);
    // RoPEFreqs::new (rope.rs:93-108) in f32 with the C library's powf / cosf / sinf
    const int half = c.head_dim / 2;
    M.cos_h.resize((size_t)c.max_seq * half);
    M.sin_h.resize((size_t)c.max_seq * half);
    for (int p = 0; p < c.max_seq; p++)
        for (int i = 0; i < half; i++) {
            const float freq = 1.0f / powf(c.rope_theta, (2.0f * (float)i) / (float)c.head_dim);
            const float angle = (float)p * freq;
            M.cos_h[(size_t)p * half + i] = cosf(angle);
            M.sin_h[(size_t)p * half + i] = sinf(angle);
        }
    if ((e = M.alloc_t(&M.cos_t, M.cos_h.size())) != hipSuccess) return fail_free(e);
    if ((e = M.alloc_t(&M.sin_t, M.sin_h.size())) != hipSuccess) return fail_free(e);
    if ((e = hipMemcpy(M.cos_t, M.cos_h.data(), M.cos_h.size() * 4, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(M.sin_t, M.sin_h.data(), M.sin_h.size() * 4, hipMemcpyHostToDevice)) != hipSuccess)
        return fail_free(e);
    hipLaunchKernelGGL(rdl::set_int_kernel, dim3(1), dim3(64), 0, M.stream, M.pos, 0);
    if ((e = hipStreamSynchronize(M.stream)) != hipSuccess) return fail_free(e);
    *out = h;
    return api_ok();
}

rdl_status rdl_llama_free(rdl_llama* model) {
    delete model;
    return api_ok();
}

rdl_status rdl_llama_set_weight(rdl_llama* model, int32_t slot, int32_t layer, const void* bytes, size_t len) {
    if (!model || !bytes) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    rdl::LlamaModel& M = model->m;
    SlotTarget t;
    rdl_status st = slot_target(M, slot, layer, &t);
    if (st != RDL_OK) return st;
    if (len != t.bytes())
        return rdl::api_shape_fail(("slot " + std::to_string(slot) + " bytes").c_str(), {t.bytes()}, {len});
    HIP_TRY(hipMemcpy2D(t.dst, t.dpitch, bytes, t.row_bytes, t.row_bytes, t.rows, hipMemcpyHostToDevice));
    return api_ok();
}

rdl_status rdl_llama_init_random(rdl_llama* model, uint64_t seed) {
    if (!model) return api_fail(RDL_ERR_NULL_POINTER, "NULL model");
    rdl::LlamaModel& M = model->m;
    const rdl_llama_config& c = M.cfg;
    bool all_q4 = M.out.type == rdl::WType::Q4_0 && M.emb.type == rdl::WType::Q4_0;
    for (auto& L : M.layers) all_q4 &= L.fused || (!L.split_qkv && !L.split_gu && L.qkv.type == rdl::WType::Q4_0 &&
                                                  L.o.type == rdl::WType::Q4_0 && L.gu.type == rdl::WType::Q4_0 &&
                                                  L.down.type == rdl::WType::Q4_0);
    if (!all_q4) return api_fail(RDL_ERR_UNSUPPORTED, "synthetic weights are Q4_0: every matrix must be Q4_0");
    uint64_t tag = 0;
    auto fill_mat = [&](rdl::LlamaModel::Mat& w) {
        const size_t nblocks = (size_t)w.n * (w.k / rdl::QK);
        hipLaunchKernelGGL(rdl::fill_q4_0_kernel, dim3(rdl::blocks_for(nblocks)), dim3(rdl::NT), 0, M.stream,
                           w.dev, nblocks, seed * 0x100000001B3ull + (++tag) * 0x9E3779B97F4A7C15ull, 0.02f);
    };
    auto fill_ones = [&](float* p) {
        hipLaunchKernelGGL(rdl::fill_f32_kernel, dim3(rdl::blocks_for(c.dim)), dim3(rdl::NT), 0, M.stream, p,
                           (size_t)c.dim, 1.0f);
    };
    fill_mat(M.emb);
    for (auto& L : M.layers) {
        fill_mat(L.qkv);
        fill_mat(L.o);
        fill_mat(L.gu);
        fill_mat(L.down);
        fill_ones(L.attn_norm);
        fill_ones(L.ffn_norm);
    }
    fill_mat(M.out);
    fill_ones(M.final_norm);
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipStreamSynchronize(M.stream));
    return api_ok();
}

rdl_status rdl_llama_reset(rdl_llama* model) {
    if (!model) return api_fail(RDL_ERR_NULL_POINTER, "NULL model");
    rdl::LlamaModel& M = model->m;
    hipLaunchKernelGGL(rdl::set_int_kernel, dim3(1), dim3(64), 0, M.stream, M.pos, 0);
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipStreamSynchronize(M.stream));
    HIP_TRY(hipMemset(M.att_xch, 0, (size_t)M.cfg.n_layers * M.xch_stride() * sizeof(uint64_t)));
    HIP_TRY(hipMemset(M.att_err, 0, sizeof(int)));
    M.host_pos = 0;
    return api_ok();
}

rdl_status rdl_llama_position(const rdl_llama* model, size_t* out) {
    if (!model || !out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    *out = model->m.host_pos;
    return api_ok();
}

rdl_status rdl_llama_kv_pages(const rdl_llama* model, size_t* page_positions, size_t* n_pages) {
    if (!model) return api_fail(RDL_ERR_NULL_POINTER, "NULL model");
    if (page_positions) *page_positions = rdl::KV_PAGE;
    if (n_pages) *n_pages = (size_t)model->m.n_pages;
    return api_ok();
}

rdl_status rdl_llama_set_kv_page_table(rdl_llama* model, const int32_t* table, size_t n) {
    if (!model || !table) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    rdl::LlamaModel& M = model->m;
    if (n != (size_t)M.n_pages)
        return rdl::api_shape_fail("page table entries", {(size_t)M.n_pages}, {n});
    if (M.host_pos != 0)
        return api_fail(RDL_ERR_INVALID_DATA, "the page table can change only on an empty cache (position %zu)",
                        M.host_pos);
    std::vector<char> seen(n, 0);
    for (size_t p = 0; p < n; p++) {
        if (table[p] < 0 || (size_t)table[p] >= n || seen[table[p]])
            return api_fail(RDL_ERR_INVALID_DATA, "page table entry %zu = %d: not a permutation of 0..%zu", p,
                            table[p], n - 1);
        seen[table[p]] = 1;
    }
    HIP_TRY(hipMemcpy(M.kv_table, table, n * sizeof(int32_t), hipMemcpyHostToDevice));
    return api_ok();
}

rdl_status rdl_llama_forward(rdl_llama* model, const int32_t* tokens, size_t n, float* logits, size_t logits_len) {
    if (!model || !tokens || !logits) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    rdl::LlamaModel& M = model->m;
    const rdl_llama_config& c = M.cfg;
    if (n == 0 || n > (size_t)c.max_batch)
        return api_fail(RDL_ERR_SHAPE_MISMATCH, "%zu tokens: 1 .. max_batch (%d) per call", n, c.max_batch);
    if (logits_len < (size_t)c.vocab)
        return api_fail(RDL_ERR_SHAPE_MISMATCH, "logits length %zu < vocab %d", logits_len, c.vocab);
    if (M.host_pos + n > (size_t)c.max_seq)
        return api_fail(RDL_ERR_INVALID_DATA, "sequence length %zu exceeds maximum %d (start_pos=%zu)",
                        M.host_pos + n, c.max_seq, M.host_pos);
    for (size_t i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= c.vocab)
            return api_fail(RDL_ERR_INVALID_DATA, "token %d out of bounds for embedding with %d entries",
                            tokens[i], c.vocab);
    HIP_TRY(hipMemcpyAsync(M.tokens, tokens, n * 4, hipMemcpyHostToDevice, M.stream));
    HIP_TRY(M.forward(n));
    HIP_TRY(hipMemcpyAsync(logits, M.logits, (size_t)c.vocab * 4, hipMemcpyDeviceToHost, M.stream));
    HIP_TRY(hipStreamSynchronize(M.stream));
    rdl_status st = check_fused(M);
    if (st != RDL_OK) return st;
    M.host_pos += n;
    return api_ok();
}

rdl_status rdl_llama_generate_greedy(rdl_llama* model, const int32_t* prompt, size_t n_prompt, size_t n_gen,
                                     int32_t* out_tokens) {
    if (!model || (!prompt && n_prompt) || (!out_tokens && n_gen))
        return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    rdl::LlamaModel& M = model->m;
    const rdl_llama_config& c = M.cfg;
    if (n_prompt == 0) return api_fail(RDL_ERR_INVALID_DATA, "empty prompt");
    if (n_gen == 0) return api_ok();
    // the last sampled token is not fed back: positions used = prompt + n_gen - 1
    if (M.host_pos + n_prompt + n_gen - 1 > (size_t)c.max_seq)
        return api_fail(RDL_ERR_INVALID_DATA, "sequence length %zu exceeds maximum %d",
                        M.host_pos + n_prompt + n_gen - 1, c.max_seq);
    for (size_t i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= c.vocab)
            return api_fail(RDL_ERR_INVALID_DATA, "token %d out of bounds for embedding with %d entries",
                            prompt[i], c.vocab);
    hipLaunchKernelGGL(rdl::set_int_kernel, dim3(1), dim3(64), 0, M.stream, M.step, 0);
    HIP_TRY(hipEventRecord(M.ev[0], M.stream));
    // prefill in chunks; the last chunk's logits give the first token
    const size_t start = M.host_pos;
    for (size_t r = 0; r < n_prompt; r += (size_t)c.max_batch) {
        const size_t mr = std::min(n_prompt - r, (size_t)c.max_batch);
        HIP_TRY(hipMemcpyAsync(M.tokens, prompt + r, mr * 4, hipMemcpyHostToDevice, M.stream));
        const hipError_t fe = M.forward(mr);
        M.host_pos += mr;  // the device position advanced with the forward
        if (fe != hipSuccess) {
            M.host_pos = start;
            return api_fail(RDL_ERR_HIP, "prefill failed: %s", hipGetErrorString(fe));
        }
    }
    M.sample(0);  // the prefill advanced the position
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipEventRecord(M.ev[1], M.stream));
    if (n_gen > 1) {
        if (!M.decode_exec) {
            HIP_TRY(hipStreamBeginCapture(M.stream, hipStreamCaptureModeThreadLocal));
            M.capture_any_pos = true;
            const hipError_t ce = M.decode_step();
            M.capture_any_pos = false;
            hipGraph_t g = nullptr;
            const hipError_t ee = hipStreamEndCapture(M.stream, &g);
            HIP_TRY(ce);
            HIP_TRY(ee);
            M.decode_graph = g;
            HIP_TRY(hipGraphInstantiate(&M.decode_exec, g, nullptr, nullptr, 0));
        }
        for (size_t i = 1; i < n_gen; i++) HIP_TRY(hipGraphLaunch(M.decode_exec, M.stream));
    }
    HIP_TRY(hipEventRecord(M.ev[2], M.stream));
    HIP_TRY(hipMemcpyAsync(out_tokens, M.out_tokens, n_gen * 4, hipMemcpyDeviceToHost, M.stream));
    HIP_TRY(hipStreamSynchronize(M.stream));
    HIP_TRY(hipEventElapsedTime(&M.prefill_ms, M.ev[0], M.ev[1]));
    HIP_TRY(hipEventElapsedTime(&M.decode_ms, M.ev[1], M.ev[2]));
    rdl_status st = check_fused(M);
    if (st != RDL_OK) return st;
    M.host_pos += n_gen - 1;
    return api_ok();
}

rdl_status rdl_llama_set_fused_attention(rdl_llama* model, int32_t enable) {
    if (!model) return api_fail(RDL_ERR_NULL_POINTER, "NULL model");
    if (enable < 0 || enable > 2) return api_fail(RDL_ERR_INVALID_DATA, "fused-attention level %d (0, 1 or 2)", enable);
    rdl::LlamaModel& M = model->m;
    if (M.fused_attention != (enable != 0) || M.fused_down != (enable == 2)) {
        M.fused_attention = enable != 0;
        M.fused_down = enable == 2;
        // the captured decode step holds the other launches: capture again
        if (M.decode_exec) (void)hipGraphExecDestroy(M.decode_exec);
        if (M.decode_graph) (void)hipGraphDestroy(M.decode_graph);
        M.decode_exec = nullptr;
        M.decode_graph = nullptr;
    }
    return api_ok();
}

rdl_status rdl_llama_get_path_counts(const rdl_llama* model, rdl_llama_path_counts* out) {
    if (!model || !out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    *out = model->m.path;
    return api_ok();
}

rdl_status rdl_llama_set_native_q4(rdl_llama* model, int32_t layer, int32_t enable) {
    if (!model) return api_fail(RDL_ERR_NULL_POINTER, "NULL model");
    rdl::LlamaModel& M = model->m;
    if (layer < -1 || layer >= M.cfg.n_layers)
        return api_fail(RDL_ERR_INVALID_DATA, "layer %d outside -1 .. %d", layer, M.cfg.n_layers - 1);
    bool changed = false;
    for (int l = 0; l < M.cfg.n_layers; l++)
        if ((layer < 0 || l == layer) && M.layers[l].native != (enable != 0)) {
            M.layers[l].native = enable != 0;
            changed = true;
        }
    if (changed) {  // the captured decode step holds the other launches: capture again
        if (M.decode_exec) (void)hipGraphExecDestroy(M.decode_exec);
        if (M.decode_graph) (void)hipGraphDestroy(M.decode_graph);
        M.decode_exec = nullptr;
        M.decode_graph = nullptr;
    }
    return api_ok();
}

rdl_status rdl_llama_last_timing(const rdl_llama* model, float* prefill_ms, float* decode_ms) {
    if (!model || !prefill_ms || !decode_ms) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    *prefill_ms = model->m.prefill_ms;
    *decode_ms = model->m.decode_ms;
    return api_ok();
}

rdl_status rdl_llama_rope_tables(const rdl_llama* model, float* cos_out, float* sin_out, size_t len) {
    if (!model || !cos_out || !sin_out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    const rdl::LlamaModel& M = model->m;
    if (len != M.cos_h.size())
        return rdl::api_shape_fail("rope table floats", {M.cos_h.size()}, {len});
    memcpy(cos_out, M.cos_h.data(), len * 4);
    memcpy(sin_out, M.sin_h.data(), len * 4);
    return api_ok();
}

}  // extern "C"

// ---- loading from a GGUF file ------------------------------------------------
namespace {

// Tensor names of the Llama weight map (weight_map.rs:26-73) and the internal
// names from_pretrained asks for (model.rs:95-223), per slot.
struct SlotName {
    int slot;
    const char* gguf;      // model-level name, or the suffix after "blk.<i>."
    const char* internal;  // printf format with the layer index where per-layer
};
constexpr SlotName MODEL_NAMES[] = {
    {RDL_LLAMA_TOKEN_EMBEDDING, "token_embd.weight", "token_embedding.weight"},
    {RDL_LLAMA_FINAL_NORM, "output_norm.weight", "norm.weight"},
    {RDL_LLAMA_OUTPUT, "output.weight", "output.weight"},
};
// in the order from_pretrained loads a layer (model.rs:146-211)
constexpr SlotName LAYER_NAMES[] = {
    {RDL_LLAMA_WQ, "attn_q.weight", "layers.%d.attention.q_proj.weight"},
    {RDL_LLAMA_WK, "attn_k.weight", "layers.%d.attention.k_proj.weight"},
    {RDL_LLAMA_WV, "attn_v.weight", "layers.%d.attention.v_proj.weight"},
    {RDL_LLAMA_WO, "attn_output.weight", "layers.%d.attention.out_proj.weight"},
    {RDL_LLAMA_W_UP, "ffn_up.weight", "layers.%d.feed_forward.up_proj.weight"},
    {RDL_LLAMA_W_DOWN, "ffn_down.weight", "layers.%d.feed_forward.down_proj.weight"},
    {RDL_LLAMA_W_GATE, "ffn_gate.weight", "layers.%d.feed_forward.gate_proj.weight"},
    {RDL_LLAMA_ATTN_NORM, "attn_norm.weight", "layers.%d.attention_norm.weight"},
    {RDL_LLAMA_FFN_NORM, "ffn_norm.weight", "layers.%d.ffn_norm.weight"},
};

const char* ggml_name(int32_t t) {
    switch (t) {
        case 0: return "F32"; case 1: return "F16"; case 2: return "Q4_0"; case 3: return "Q4_1";
        case 6: return "Q5_0"; case 7: return "Q5_1"; case 8: return "Q8_0"; case 9: return "Q8_1";
        case 10: return "Q2K"; case 11: return "Q3K"; case 12: return "Q4K"; case 13: return "Q5K";
        case 14: return "Q6K"; case 15: return "Q8K";
    }
    return "?";
}

// The slot and layer a GGUF tensor name maps to (false: not a weight of the
// Llama map for n_layers layers; such tensors are ignored, as remap passes
// them through and from_pretrained never asks for them).
bool gguf_slot(const char* name, int n_layers, int* slot, int* layer) {
    for (const SlotName& m : MODEL_NAMES)
        if (strcmp(name, m.gguf) == 0) return *slot = m.slot, *layer = 0, true;
    if (strncmp(name, "blk.", 4) != 0) return false;
    const char* p = name + 4;
    // the decimal form format!("blk.{}", i) writes: no sign, no leading zero
    if (!(*p >= '0' && *p <= '9') || (p[0] == '0' && p[1] >= '0' && p[1] <= '9')) return false;
    long i = 0;
    while (*p >= '0' && *p <= '9') {
        i = i * 10 + (*p++ - '0');
        if (i >= n_layers) return false;
    }
    if (*p++ != '.') return false;
    for (const SlotName& l : LAYER_NAMES)
        if (strcmp(p, l.gguf) == 0) return *slot = l.slot, *layer = (int)i, true;
    return false;
}

std::string internal_name(const SlotName& s, int layer) {
    char buf[128];
    snprintf(buf, sizeof buf, s.internal, layer);
    return buf;
}

// Expected GGUF dims (innermost first) of a slot's tensor: {k, n} or {dim}.
void slot_dims(const rdl_llama_config& c, int slot, uint64_t d[2], uint32_t* nd) {
    const uint64_t q = (uint64_t)c.n_heads * c.head_dim, kv = (uint64_t)c.n_kv_heads * c.head_dim;
    *nd = 2;
    switch (slot) {
        case RDL_LLAMA_TOKEN_EMBEDDING:
        case RDL_LLAMA_OUTPUT: d[0] = c.dim, d[1] = c.vocab; return;
        case RDL_LLAMA_WQ: d[0] = c.dim, d[1] = q; return;
        case RDL_LLAMA_WK:
        case RDL_LLAMA_WV: d[0] = c.dim, d[1] = kv; return;
        case RDL_LLAMA_WO: d[0] = q, d[1] = c.dim; return;
        case RDL_LLAMA_W_GATE:
        case RDL_LLAMA_W_UP: d[0] = c.dim, d[1] = c.ffn_dim; return;
        case RDL_LLAMA_W_DOWN: d[0] = c.ffn_dim, d[1] = c.dim; return;
    }
    *nd = 1;
    d[0] = c.dim;
}

// Type and shape of one tensor against its slot.
rdl_status check_tensor(const rdl_llama_config& c, int slot, const rdl_gguf_tensor_info& ti) {
    const bool norm = slot == RDL_LLAMA_ATTN_NORM || slot == RDL_LLAMA_FFN_NORM || slot == RDL_LLAMA_FINAL_NORM;
    const int32_t t = ti.ggml_type;
    if (norm ? (t != 0 && t != 1)
             : (t != RDL_DTYPE_Q4_0 && t != RDL_DTYPE_Q8_0 && t != RDL_DTYPE_Q4_1 && t != RDL_DTYPE_Q4_K &&
                t != RDL_DTYPE_Q6_K))
        return api_fail(RDL_ERR_UNSUPPORTED, "tensor '%s' is %s; the decoder takes %s", ti.name, ggml_name(t),
                        norm ? "F32 or F16 norm weights" : "Q4_0, Q8_0, Q4_1, Q4_K or Q6_K matrices");
    uint64_t d[2];
    uint32_t nd = 0;
    slot_dims(c, slot, d, &nd);
    bool same = ti.n_dims == nd;
    for (uint32_t i = 0; same && i < nd; i++) same = ti.dims[i] == d[i];
    if (!same) {
        size_t want[2] = {(size_t)d[0], (size_t)d[1]}, got[4] = {};
        const size_t ng = std::min<size_t>(ti.n_dims, 4);
        for (size_t i = 0; i < ng; i++) got[i] = (size_t)ti.dims[i];
        return rdl::api_shape_fail((std::string("tensor '") + ti.name + "' dims").c_str(), want, nd, got, ng);
    }
    return api_ok();
}

// A present tensor's info by GGUF name (the last one of that name).
bool find_info(const rdl_gguf* g, const char* name, rdl_gguf_tensor_info* ti) {
    size_t i = 0;
    return rdl_gguf_find_tensor(g, name, &i) == RDL_OK && rdl_gguf_tensor_info_at(g, i, ti) == RDL_OK;
}

}  // namespace

extern "C" {

rdl_status rdl_llama_load_gguf(const rdl_gguf* g, const rdl_llama_gguf_options* opt, rdl_llama** out) {
    if (!g || !out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    *out = nullptr;
    rdl_gguf_model_config gc;
    rdl_status st = rdl_gguf_model_config_get(g, &gc);
    if (st != RDL_OK) return st;
    if (strcmp(gc.architecture, "gemma3") == 0)
        return api_fail(RDL_ERR_UNSUPPORTED, "architecture gemma3 (from_pretrained_gemma3) is not built");
    // gguf_config_to_model_config + ModelConfig::validate (gguf_bridge.rs:46-84, types.rs:794-826)
    const uint32_t n_kv = gc.has_n_kv_heads ? gc.n_kv_heads : gc.n_heads;
    const uint32_t max_seq = (opt && opt->max_seq > 0) ? (uint32_t)opt->max_seq : gc.max_seq_len;
    if (gc.dim == 0) return api_fail(RDL_ERR_INVALID_DATA, "dim must be > 0");
    if (gc.n_heads == 0) return api_fail(RDL_ERR_INVALID_DATA, "n_heads must be > 0");
    if (gc.dim % gc.n_heads != 0)
        return api_fail(RDL_ERR_INVALID_DATA, "dim (%u) must be divisible by n_heads (%u)", gc.dim, gc.n_heads);
    if (gc.vocab_size == 0) return api_fail(RDL_ERR_INVALID_DATA, "vocab_size must be > 0");
    if (gc.n_layers == 0) return api_fail(RDL_ERR_INVALID_DATA, "n_layers must be > 0");
    if (max_seq == 0) return api_fail(RDL_ERR_INVALID_DATA, "max_seq_len must be > 0");
    if (gc.has_n_kv_heads && gc.n_kv_heads == 0) return api_fail(RDL_ERR_INVALID_DATA, "n_kv_heads must be > 0");
    if (gc.n_heads % n_kv != 0)
        return api_fail(RDL_ERR_INVALID_DATA, "n_heads (%u) must be divisible by n_kv_heads (%u)", gc.n_heads, n_kv);
    if (gc.n_layers > 4096 || gc.n_heads > 4096 || gc.dim > (1u << 20) || max_seq > (1u << 20))
        return api_fail(RDL_ERR_UNSUPPORTED, "config beyond the decoder's limits");

    // Presence, in from_pretrained's order: the first missing weight is named.
    auto missing = [&](const SlotName& s, int layer) {
        return api_fail(RDL_ERR_NOT_FOUND, "Missing weight: %s", internal_name(s, layer).c_str());
    };
    rdl_gguf_tensor_info emb{}, outw{}, up0{};
    if (!find_info(g, MODEL_NAMES[0].gguf, &emb)) return missing(MODEL_NAMES[0], 0);
    for (uint32_t l = 0; l < gc.n_layers; l++)
        for (const SlotName& s : LAYER_NAMES) {
            char nm[96];
            snprintf(nm, sizeof nm, "blk.%u.%s", l, s.gguf);
            rdl_gguf_tensor_info ti;
            if (!find_info(g, nm, &ti)) {
                if (s.slot == RDL_LLAMA_W_GATE)  // FeedForward without gate: Activation::Silu MLP
                    return api_fail(RDL_ERR_UNSUPPORTED, "%s: the decoder is SwiGLU only (no gate weight)", nm);
                return missing(s, (int)l);
            }
        }
    rdl_gguf_tensor_info norm{};
    if (!find_info(g, MODEL_NAMES[1].gguf, &norm)) return missing(MODEL_NAMES[1], 0);
    if (!find_info(g, MODEL_NAMES[2].gguf, &outw)) return missing(MODEL_NAMES[2], 0);
    if (!find_info(g, "blk.0.ffn_up.weight", &up0)) return missing(LAYER_NAMES[4], 0);

    rdl_llama_config c{};
    c.dim = (int32_t)gc.dim;
    c.n_layers = (int32_t)gc.n_layers;
    c.n_heads = (int32_t)gc.n_heads;
    c.n_kv_heads = (int32_t)n_kv;
    c.head_dim = (int32_t)(gc.dim / gc.n_heads);  // MultiHeadAttention::from_weights: d_model / num_heads
    // the matrices fix the FFN width and vocabulary (Linear::from_weights takes their shapes)
    c.ffn_dim = up0.n_dims == 2 ? (int32_t)std::min<uint64_t>(up0.dims[1], INT32_MAX) : 0;
    c.vocab = outw.n_dims == 2 ? (int32_t)std::min<uint64_t>(outw.dims[1], INT32_MAX) : 0;
    c.max_seq = (int32_t)max_seq;
    c.norm_eps = gc.norm_eps;
    c.rope_theta = gc.rope_theta;
    c.kv_f16 = opt ? opt->kv_f16 : 1;
    c.max_batch = (opt && opt->max_batch > 0) ? opt->max_batch : 32;
    c.output_dtype = outw.ggml_type;

    // Type, shape and file bounds of every mapped tensor before allocating.
    const size_t nt = [&] { size_t n = 0; rdl_gguf_tensor_count(g, &n); return n; }();
    std::vector<std::pair<size_t, std::pair<int, int>>> plan;  // tensor index, (slot, layer)
    for (size_t i = 0; i < nt; i++) {
        rdl_gguf_tensor_info ti;
        if ((st = rdl_gguf_tensor_info_at(g, i, &ti)) != RDL_OK) return st;
        int slot = 0, layer = 0;
        if (strlen(ti.name) != ti.name_len || !gguf_slot(ti.name, c.n_layers, &slot, &layer)) continue;
        if ((st = check_tensor(c, slot, ti)) != RDL_OK) return st;
        const void* src = nullptr;
        uint64_t len = 0;
        if ((st = rdl_gguf_tensor_data(g, i, &src, &len)) != RDL_OK) return st;
        plan.push_back({i, {slot, layer}});
    }

    // the file's type for every matrix slot (the later of two same-named tensors)
    std::vector<int32_t> types((size_t)c.n_layers * RDL_LLAMA_SLOTS, 0);
    for (const auto& p : plan) {
        rdl_gguf_tensor_info ti;
        rdl_gguf_tensor_info_at(g, p.first, &ti);
        const int slot = p.second.first, layer = p.second.second;
        if (slot != RDL_LLAMA_ATTN_NORM && slot != RDL_LLAMA_FFN_NORM && slot != RDL_LLAMA_FINAL_NORM)
            types[(size_t)layer * RDL_LLAMA_SLOTS + slot] = ti.ggml_type;
    }
    rdl_llama* h = nullptr;
    if ((st = rdl_llama_create_typed(&c, types.data(), &h)) != RDL_OK) return st;
    rdl::LlamaModel& M = h->m;
    auto fail = [&](rdl_status s) {
        rdl_llama_free(h);
        return s;
    };
    rdl::Stager stage;
    std::vector<float> f32;
    for (const auto& p : plan) {
        const void* src = nullptr;
        uint64_t len = 0;
        rdl_gguf_tensor_info ti;
        rdl_gguf_tensor_info_at(g, p.first, &ti);
        rdl_gguf_tensor_data(g, p.first, &src, &len);
        SlotTarget t;
        if ((st = slot_target(M, p.second.first, p.second.second, &t)) != RDL_OK) return fail(st);
        if (ti.ggml_type == 1) {  // F16 norm weights: to f32 as Tensor::to_f32 does
            f32.resize((size_t)c.dim);
            const auto* hp = static_cast<const uint8_t*>(src);
            for (int j = 0; j < c.dim; j++) {
                _Float16 v;
                memcpy(&v, hp + 2 * j, 2);
                f32[j] = (float)v;
            }
            src = f32.data();
        }
        const hipError_t e = stage.copy2d(src, t.row_bytes, t.rows, t.dst, t.dpitch, M.stream);
        if (e != hipSuccess)
            return fail(api_fail(RDL_ERR_HIP, "upload of '%s' failed: %s", ti.name, hipGetErrorString(e)));
    }
    *out = h;
    return api_ok();
}

rdl_status rdl_llama_get_config(const rdl_llama* model, rdl_llama_config* out) {
    if (!model || !out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    *out = model->m.cfg;
    return api_ok();
}

}  // extern "C"
