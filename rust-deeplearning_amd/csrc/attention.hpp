// attention.hpp -- batch-1 decode attention over the paged KV cache
// (MultiHeadAttention::forward_with_cache, attention.rs:401-446), shared by
// the decoder's attention launch (llama.hip) and the q/k/v launch with the
// attention fused in (gemv_fused.hip).
#pragma once

#include "rdl_device.hpp"
#include "rdl_internal.hpp"

namespace rdl {
namespace att {

__device__ __forceinline__ float wave_sum(float v) {
    v = sum8_f32(v);
    v += dpp_f32<DPP_ROW_MIRROR>(v);
    v += __shfl_xor(v, 16);
    return v + __shfl_xor(v, 32);
}
__device__ __forceinline__ float wave_max(float v) {
    v = max8_f32(v);
    v = fmaxf(v, dpp_f32<DPP_ROW_MIRROR>(v));
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}

// Attention of query row s (position pos + s) and head h over the cached keys
// 0 .. pos + s (the causal mask of attention.rs:424-433 keeps exactly these):
// scores q.k / sqrt(hd), max-subtracted softmax (ops.rs:582-628), then the
// probability-weighted sum of the values.  Split over the keys in chunks of
// ATT_CHUNK: one wave per (head, row, chunk) forms the chunk's scores (one
// key's score per lane), its max m_c, sum l_c = sum exp(score - m_c) and the
// unnormalised context o_c = sum exp(score - m_c) v; the chunks are then
// combined as (sum_c exp(m_c - M) o_c) / (sum_c exp(m_c - M) l_c), M = max
// m_c (in LDS within a workgroup, see attention_kernel for several spans).
// Chunks past the row's length exit at once, so a launch sized for the cache
// capacity serves every position (the captured decode graph).
constexpr int ATT_CHUNK = 64;
static_assert(KV_PAGE % ATT_CHUNK == 0, "an attention chunk lies in one cache page");

// HD: head dim as a compile-time constant (64, 128, 256), so that all of a
// key row's loads are issued before its dot product; 0: runtime hd.
// A workgroup of ATT_WAVES waves covers ATT_WAVES chunks (ATT_SPAN keys):
// wave w forms chunk w's max m_w, sum l_w and unnormalised context o_w; the
// workgroup combines its chunks in LDS.  A row with more than ATT_SPAN keys
// uses several workgroups, and the last of them to finish combines their
// partials (device-scope counter, chunk order fixed: deterministic).
constexpr int ATT_WAVES = 8;
constexpr int ATT_SPAN = ATT_CHUNK * ATT_WAVES;

// One step of the transposed sum of N values over N lanes (lane index c within
// its group of N): the lane keeps the half of its values selected by bit HF
// of c and adds the partner lane's (c ^ HF) copy of that half.  After the
// steps HF = N/2, ..., 1, v[0] of lane c is the group's total of value c.
template <int HF, int N>
__device__ __forceinline__ void transposed_sum(float (&v)[N], int c) {
    if constexpr (HF >= 1) {
        const bool up = (c & HF) != 0;
#pragma unroll
        for (int j = 0; j < HF; j++) {
            const float send = up ? v[j] : v[j + HF];
            const float keep = up ? v[j + HF] : v[j];
            v[j] = keep + __shfl_xor(send, HF);
        }
        transposed_sum<HF / 2, N>(v, c);
    }
}

// Arguments of one attention launch.  Fused launches (FUSED, attention in
// the q/k/v launch): the q rows and the current position's cache rows come
// from workgroups of the same launch (written with agent-coherent stores).
// Each KV group has a PUB_SLOT-int slot of pub: the group's producer
// workgroups count themselves at PUB_COUNT, and the one that completes the
// count returns it to 0 and writes the launch's position + 1 at PUB_READY;
// the group's attention waves wait for that value.  Positions grow from
// launch to launch until the cache is emptied (which zeroes pub), so a value
// left by an earlier launch never matches.  Count and flag sit on separate
// 128-byte lines, and the consumers only read: no atomic of theirs queues
// behind the producers' adds.
constexpr int PUB_SLOT = 64, PUB_COUNT = 0, PUB_READY = 32;
template <typename KV>
struct AttArgs {
    const float* qkv;          // [rows][qkv_dim]: q heads | k heads | v heads
    int qkv_dim;
    const int* pos_dev;        // cache position of row 0
    const KV* kc;              // paged K pool of the layer
    const KV* vc;
    const int* kv_table;
    int n_heads, n_kv, hd_rt;
    float scale;               // sqrt(head_dim)
    float* part;               // [rows][n_heads][nspan][hd + 2] span partials
    int nspan;
    int* counters;             // [rows][n_heads] span counters
    float* out;                // [rows][n_heads * hd]
    const int* pub;            // FUSED: [n_kv][PUB_SLOT] count / ready slots
    int* err;                  // FUSED: set when a wait runs out (never in a correct launch)
};

// Coherent (agent-scope) loads of values another workgroup of the same launch
// published with coherent stores.
template <typename T>
__device__ __forceinline__ T ld_coh8(const T* p) {
    static_assert(sizeof(T) == 16, "16-byte pieces");
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    struct P { uint64_t a, b; } r{a, b};
    return __builtin_bit_cast(T, r);
}

// Bounded wait of one fused attention wave until its KV group's producers
// have marked the position ready (every lane reads the same word).
__device__ __forceinline__ void wave_wait_ready(const int* ready, int want, int* err) {
    int spins = 0;
    for (;;) {
        const int v = __builtin_amdgcn_readfirstlane(__hip_atomic_load(ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (v == want) break;
        __builtin_amdgcn_s_sleep(2);
        if (++spins > (1 << 20)) {  // about a second: only a broken launch gets here
            if ((threadIdx.x & 63) == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
    }
}

template <typename KV, int HD, bool FUSED>
__device__ __forceinline__ void attention_body(int bx, int by, int bz, float* __restrict__ sm, const AttArgs<KV>& a) {
    const float* __restrict__ qkv = a.qkv;
    const int qkv_dim = a.qkv_dim;
    const int* __restrict__ pos_dev = a.pos_dev;
    const KV* __restrict__ kc = a.kc;
    const KV* __restrict__ vc = a.vc;
    const int* __restrict__ kv_table = a.kv_table;
    const int n_heads = a.n_heads, n_kv = a.n_kv, hd_rt = a.hd_rt;
    const float scale = a.scale;
    float* __restrict__ part = a.part;
    const int nspan = a.nspan;
    int* __restrict__ counters = a.counters;
    float* __restrict__ out = a.out;

    // sm: q[hd] | o[ATT_WAVES][hd]
    __shared__ float ml[ATT_WAVES][2];
    __shared__ float wsc[1024];
    __shared__ int last;
    const int hd = HD ? HD : hd_rt;
    // Workgroups are dealt to the 8 XCDs round-robin by linear id; block b
    // serves head (b % n_kv) * G + b / n_kv, so the G query heads of a KV
    // head (blocks g, g + n_kv, ...) run on one XCD and share its L2.
    const int G = n_heads / n_kv;
    const int h = (bx % n_kv) * G + bx / n_kv;
    const int s = by, z = bz;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t = *pos_dev + s + 1;
    if (z * ATT_SPAN >= t) return;  // whole workgroup
    float* qs = sm;
    float* os = sm + hd;
    const int kvh = h / G;
    const float* q = qkv + (size_t)s * qkv_dim + h * hd;
    // V rows in pieces of 16 bytes: CPR lanes cover a row, one load covers
    // KG rows; load i of lane l is row KG i + l / CPR (when CPR <= 16)
    constexpr int V = 16 / sizeof(KV);
    constexpr int CPR = HD * (int)sizeof(KV) / 16;
    constexpr bool VPRE = HD > 0 && CPR <= 16 && 64 % (CPR > 0 ? CPR : 1) == 0;
    static_assert(!FUSED || VPRE, "the fused launch takes the coalesced K/V layout");
    if constexpr (!VPRE) {
        for (int d = threadIdx.x; d < hd; d += 64 * ATT_WAVES) qs[d] = q[d];
        __syncthreads();
    }
    const int p0 = z * ATT_SPAN + w * ATT_CHUNK;
    float mx = -__builtin_inff(), l = 0.0f;
    if (p0 < t) {  // wave-uniform
        const int p = p0 + lane;
        const bool valid = p < t;
        typedef KV kvv __attribute__((ext_vector_type(V)));
        // the chunk's 64 keys are one page of the cache: rows p0 .. p0 + 63
        // at kb / vb + (p - p0) * hd
        const size_t page = kv_row(kv_table, n_kv, kvh, p0, hd);
        const KV* vb = vc + page;
        const int nvalid = min(ATT_CHUNK, t - p0);
        constexpr int KG = VPRE ? 64 / (CPR > 0 ? CPR : 1) : 1;
        float acc = 0.0f;
        if constexpr (VPRE) {
            // K and V rows of the chunk in the same coalesced layout (load i of
            // lane l = piece l % CPR of row KG i + l / CPR), all in flight
            // before the query (which the previous launch wrote) is read: one
            // memory round trip.  Rows past the length re-read the last valid row.
            const KV* kb = kc + page;
            kvv kreg[CPR], vreg[CPR];
            const int vk = lane / CPR, pc = lane % CPR, ve = pc * V;
#pragma unroll
            for (int i = 0; i < CPR; i++) {
                const int j = min(KG * i + vk, nvalid - 1);
                kreg[i] = *reinterpret_cast<const kvv*>(kb + (size_t)j * hd + ve);
            }
#pragma unroll
            for (int i = 0; i < CPR; i++) {
                const int j = min(KG * i + vk, nvalid - 1);
                vreg[i] = *reinterpret_cast<const kvv*>(vb + (size_t)j * hd + ve);
            }
            float qv[V];
            if constexpr (FUSED) {
                // the rows before the current position are older launches'
                // stores (loaded above); the current row and q are this
                // launch's, published by the q/k/v workgroups: wait for them,
                // then read them coherently (rows past the length re-read the
                // current row, so they are reloaded too)
                wave_wait_ready(a.pub + (size_t)kvh * PUB_SLOT + PUB_READY, t, a.err);
                const int cur = t - 1 - p0;
#pragma unroll
                for (int i = 0; i < CPR; i++) {
                    if (min(KG * i + vk, nvalid - 1) == cur) {
                        kreg[i] = ld_coh8(reinterpret_cast<const kvv*>(kb + (size_t)cur * hd + ve));
                        vreg[i] = ld_coh8(reinterpret_cast<const kvv*>(vb + (size_t)cur * hd + ve));
                    }
                }
#pragma unroll
                for (int e = 0; e < V; e += 4) {
                    const float4 t4 = ld_coh8(reinterpret_cast<const float4*>(q + ve + e));
                    qv[e] = t4.x, qv[e + 1] = t4.y, qv[e + 2] = t4.z, qv[e + 3] = t4.w;
                }
            } else {
#pragma unroll
                for (int e = 0; e < V; e += 4) {
                    const float4 t4 = *reinterpret_cast<const float4*>(q + ve + e);
                    qv[e] = t4.x, qv[e + 1] = t4.y, qv[e + 2] = t4.z, qv[e + 3] = t4.w;
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the arithmetic
            // partial scores of the lane's CPR rows over its V dims, then a
            // transposed sum over the CPR lanes of the row group: after the
            // step of mask hf a lane keeps the half of its rows selected by
            // bit hf of its piece, so piece c ends with row KG c + vk's score.
            float ps[CPR];
#pragma unroll
            for (int i = 0; i < CPR; i++) {
                float a = 0.0f;
#pragma unroll
                for (int e = 0; e < V; e++) a += qv[e] * (float)kreg[i][e];
                ps[i] = a;
            }
            transposed_sum<CPR / 2, CPR>(ps, pc);
            const int key = KG * pc + vk;  // the row whose score this lane holds
            const bool kvalid = key < nvalid;
            const float sc = kvalid ? ps[0] / scale : -__builtin_inff();
            mx = wave_max(sc);
            const float e = kvalid ? expf(sc - mx) : 0.0f;
            l = wave_sum(e);
            float o[V];
#pragma unroll
            for (int c = 0; c < V; c++) o[c] = 0.0f;
#pragma unroll
            for (int i = 0; i < CPR; i++) {
                const float pj = __shfl(e, vk * CPR + i);  // row KG i + vk; rows past the length carry 0
#pragma unroll
                for (int c = 0; c < V; c++) o[c] += pj * (float)vreg[i][c];
            }
#pragma unroll
            for (int off = CPR; off < 64; off <<= 1)
#pragma unroll
                for (int c = 0; c < V; c++) o[c] += __shfl_xor(o[c], off);
            if (lane < CPR)
#pragma unroll
                for (int c = 0; c < V; c++) os[w * hd + ve + c] = o[c];
        } else {
            const KV* kr = kc + page + (size_t)(valid ? p - p0 : 0) * hd;
            if constexpr (HD > 0) {
                kvv kreg[HD / V];
#pragma unroll
                for (int i = 0; i < HD / V; i++) kreg[i] = *reinterpret_cast<const kvv*>(kr + i * V);
#pragma unroll
                for (int i = 0; i < HD / V; i++)
#pragma unroll
                    for (int e = 0; e < V; e++) acc += qs[i * V + e] * (float)kreg[i][e];
            } else {
                for (int d = 0; d < hd; d += V) {
                    const kvv kv = *reinterpret_cast<const kvv*>(kr + d);
#pragma unroll
                    for (int e = 0; e < V; e++) acc += qs[d + e] * (float)kv[e];
                }
            }
            const float sc = valid ? acc / scale : -__builtin_inff();
            mx = wave_max(sc);
            const float e = valid ? expf(sc - mx) : 0.0f;
            l = wave_sum(e);
            for (int d0 = 0; d0 < hd; d0 += 128) {
                const int d = d0 + 2 * lane;
                if (d < hd) {
                    float o0 = 0.0f, o1 = 0.0f;
                    // branch-free: a key past the row's length re-reads the last
                    // valid row with weight 0, so all row loads are in flight together
#pragma unroll
                    for (int j = 0; j < ATT_CHUNK; j++) {
                        const float ej =
                            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), j));
                        typedef KV kv2 __attribute__((ext_vector_type(2)));
                        const int pj = min(j, nvalid - 1);
                        const kv2 v2 = *reinterpret_cast<const kv2*>(vb + (size_t)pj * hd + d);
                        o0 += ej * (float)v2[0];
                        o1 += ej * (float)v2[1];
                    }
                    os[w * hd + d] = o0;
                    os[w * hd + d + 1] = o1;
                }
            }
        }
    }
    if (lane == 0) {
        ml[w][0] = mx;
        ml[w][1] = l;
    }
    __syncthreads();
    // combine this workgroup's chunks (inactive waves carry m = -inf, l = 0)
    const int nw = min(ATT_WAVES, (t - z * ATT_SPAN + ATT_CHUNK - 1) / ATT_CHUNK);
    float M = -__builtin_inff();
    for (int c = 0; c < nw; c++) M = fmaxf(M, ml[c][0]);
    float L = 0.0f;
    for (int c = 0; c < nw; c++) L += ml[c][1] * expf(ml[c][0] - M);
    const int nz = (t + ATT_SPAN - 1) / ATT_SPAN;
    float* o = out + (size_t)s * n_heads * hd + h * hd;
    if (nz == 1) {
        const float invL = 1.0f / L;
        for (int d = threadIdx.x; d < hd; d += 64 * ATT_WAVES) {
            float O = 0.0f;
            for (int c = 0; c < nw; c++) O += os[c * hd + d] * expf(ml[c][0] - M);
            o[d] = O * invL;
        }
        return;
    }
    // several workgroups: partial (M, L, O) to global, the last one combines.
    // Publication without cache maintenance: the partials are written with
    // agent-coherent stores (relaxed agent-scope atomic stores: global_store
    // ... sc1, written through to the device's coherence point) and every
    // wave waits for its own stores to complete (s_waitcnt vmcnt(0)) before
    // the barrier; thread 0's counter add follows the barrier, so a workgroup
    // that sees the count of nz - 1 others sees every other workgroup's stores
    // completed, and reads them with agent-coherent loads (relaxed agent-scope
    // atomic loads: global_load ... sc1, never served from a stale L1 / L2
    // line).  This is the sequence an agent-scope release / acquire pair
    // compiles to, minus the L2 writeback (buffer_wbl2) and invalidate
    // (buffer_inv) that only non-coherent stores and loads need -- and those
    // cost about 0.1 us a wave, serialized per XCD, on MI355X.
    float* po = part + (((size_t)s * n_heads + h) * nspan + z) * (hd + 2);
    for (int d = threadIdx.x; d < hd; d += 64 * ATT_WAVES) {
        float O = 0.0f;
        for (int c = 0; c < nw; c++) O += os[c * hd + d] * expf(ml[c][0] - M);
        __hip_atomic_store(po + 2 + d, O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x == 0) {
        __hip_atomic_store(po, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(po + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        int* cnt = counters + (size_t)s * n_heads + h;
        const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = (old == nz - 1);
        if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    const float* pb = part + ((size_t)s * n_heads + h) * nspan * (hd + 2);
    auto ld = [](const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    if (w == 0) {
        float MM = -__builtin_inff();
        for (int c = lane; c < nz; c += 64) MM = fmaxf(MM, ld(pb + (size_t)c * (hd + 2)));
        MM = wave_max(MM);
        float LL = 0.0f;
        for (int c = lane; c < nz; c += 64) {
            const float wgt = expf(ld(pb + (size_t)c * (hd + 2)) - MM);
            wsc[c] = wgt;
            LL += ld(pb + (size_t)c * (hd + 2) + 1) * wgt;
        }
        LL = wave_sum(LL);
        if (lane == 0) ml[0][1] = LL;
    }
    __syncthreads();
    const float invL = 1.0f / ml[0][1];
    for (int d = threadIdx.x; d < hd; d += 64 * ATT_WAVES) {
        float O = 0.0f;
        for (int c = 0; c < nz; c++) O += ld(pb + (size_t)c * (hd + 2) + 2 + d) * wsc[c];
        o[d] = O * invL;
    }
}

}  // namespace att
using att::AttArgs;
using att::attention_body;
using att::ATT_SPAN;
using att::ATT_WAVES;
using att::ATT_CHUNK;
using att::PUB_SLOT;
using att::PUB_COUNT;
using att::PUB_READY;
using att::wave_max;
using att::wave_sum;
}  // namespace rdl
