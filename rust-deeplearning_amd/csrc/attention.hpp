// attention.hpp -- batch-1 decode attention over the paged KV cache
// (MultiHeadAttention::forward_with_cache, attention.rs:401-446), shared by
// the decoder's attention launch (llama.hip) and the q/k/v launch with the
// attention fused in (gemv_fused.hip).
#pragma once

#include <type_traits>

#include "rdl_device.hpp"
#include "rdl_internal.hpp"

namespace rdl {
namespace att {

// v[l ^ 16] and v[l ^ 32] through gfx950's permlane swaps (no LDS round trip):
// each swap returns the lane's own value and its partner's, in some order.
__device__ __forceinline__ void pair16(float v, float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    const uint32_t lo = r[0], hi = r[1];
    a = __builtin_bit_cast(float, lo), b = __builtin_bit_cast(float, hi);
}
__device__ __forceinline__ void pair32(float v, float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    const uint32_t lo = r[0], hi = r[1];
    a = __builtin_bit_cast(float, lo), b = __builtin_bit_cast(float, hi);
}
// Sum / max over the 64 lanes, in every lane (both lanes of each pair form
// the same commutative result, so every lane holds the same bits).
__device__ __forceinline__ float wave_sum(float v) {
    v = sum8_f32(v);
    v += dpp_f32<DPP_ROW_MIRROR>(v);
    float a, b;
    pair16(v, a, b);
    v = a + b;
    pair32(v, a, b);
    return a + b;
}
__device__ __forceinline__ float wave_max(float v) {
    v = max8_f32(v);
    v = fmaxf(v, dpp_f32<DPP_ROW_MIRROR>(v));
    float a, b;
    pair16(v, a, b);
    v = fmaxf(a, b);
    pair32(v, a, b);
    return fmaxf(a, b);
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
// A workgroup of ATT_WAVES waves covers ATT_SPAN_WAVES chunks (ATT_SPAN
// keys): wave w < ATT_SPAN_WAVES forms chunk w's max m_w, sum l_w and
// unnormalised context o_w; the workgroup combines its chunks in LDS.  A row
// with more than ATT_SPAN keys uses several workgroups, and the last of them
// to finish combines their partials (device-scope counter, chunk order
// fixed: deterministic).
constexpr int ATT_WAVES = 8;
static_assert(ATT_WAVES <= 8, "the chunk combine reduces over one 8-lane group");
// (7B decode, 128-token prompt + 256 tokens: 827 tokens/s at 8 chunks a
// span; 815 at 4 and 786 at 2, whose cross-workgroup combine costs more than
// the halved K/V stream per CU saves)
constexpr int ATT_SPAN_WAVES = 8;
static_assert(ATT_SPAN_WAVES >= 1 && ATT_SPAN_WAVES <= ATT_WAVES, "chunks a workgroup");
constexpr int ATT_SPAN = ATT_CHUNK * ATT_SPAN_WAVES;

// One step of the transposed sum of N values over N lanes (lane index c within
// its aligned group of N <= 16): the lane keeps the half of its values
// selected by bit HF of c and adds the partner lane's copy of that half.  The
// partner is any lane of the group with the other value of bit HF and the same
// higher bits: row_mirror (15 - c), row_half_mirror (c ^ 7 within 8 lanes),
// quad_perm (c ^ 2, c ^ 1) -- DPP moves, no LDS round trip.  After the steps HF
// = N/2, ..., 1, v[0] of lane c is the group's total of value c.
template <int HF, int N>
__device__ __forceinline__ void transposed_sum(float (&v)[N], int c) {
    if constexpr (HF >= 1) {
        static_assert(HF <= 8, "groups of at most 16 lanes");
        constexpr int CTRL = HF == 8 ? DPP_ROW_MIRROR : HF == 4 ? DPP_ROW_HALF_MIRROR : HF == 2 ? DPP_QUAD_XOR2
                                                                                                   : DPP_QUAD_XOR1;
        const bool up = (c & HF) != 0;
#pragma unroll
        for (int j = 0; j < HF; j++) {
            const float send = up ? v[j] : v[j + HF];
            const float keep = up ? v[j + HF] : v[j];
            v[j] = keep + dpp_f32<CTRL>(send);
        }
        transposed_sum<HF / 2, N>(v, c);
    }
}

// Sum over each aligned group of N = 8 or 16 lanes, in every lane of the group.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(N == 8 || N == 16, "8- or 16-lane groups");
    v = sum8_f32(v);
    if constexpr (N == 16) v += dpp_f32<DPP_ROW_MIRROR>(v);
    return v;
}

// f(std::integral_constant<int, I>) for I = B .. E - 1, in order.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// Lane i of each 16-lane row, in every lane of the row (DPP row_newbcast).
template <int I>
__device__ __forceinline__ float row_bcast(float v) {
    return dpp_f32<0x150 + I>(v);
}

// Tagged exchange between the q/k/v workgroups and the attention workgroups
// of one fused launch: the value v of q/k/v row r for the token at cache
// position p is the 8-byte word (p + 1) << 32 | bits(v) at xch[r], written
// and read as single-copy-atomic agent-scope stores / loads (global_store /
// global_load ... sc1, served at the device's coherence point, never from a
// non-coherent L1 / L2 line).  A reader that sees the tag it expects therefore
// sees that launch's value, with no counter, fence or second read.  Tags grow
// from launch to launch on one exchange until the cache is emptied (which
// zeroes it), so a word left by an earlier launch never matches.
__device__ __forceinline__ void xch_put(uint64_t* p, float v, int tag) {
    const uint64_t word = ((uint64_t)(uint32_t)tag << 32) | __builtin_bit_cast(uint32_t, v);
    __hip_atomic_store(p, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t xch_get(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool xch_ok(uint64_t word, int tag) { return (uint32_t)(word >> 32) == (uint32_t)tag; }
__device__ __forceinline__ float xch_val(uint64_t word) { return __builtin_bit_cast(float, (uint32_t)word); }

// Arguments of one attention launch.  Fused launches (FUSED, attention in
// the q/k/v launch): head h's q row and its KV head's current k / v rows come
// from workgroups of the same launch through the exchange xch ([q heads | k
// heads | v heads] x hd tagged words, see xch_put).
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
    const uint64_t* xch;       // FUSED: the layer's exchange
    uint64_t* oxch;            // FUSED, when set: outputs as tagged words (tag t) here instead of out
    int* err;                  // FUSED: set when a wait runs out (never in a correct launch)
};

// Wave 0 of a fused attention workgroup: poll the exchange until head h's q
// row and, when the workgroup's span holds the current position (cur), the
// KV head's current k and v rows carry tag t; leave them in LDS: q as f32
// (qs), k and v in the cache's type (kn, vn), rounded as the cache writer
// rounds them.  Bounded: a wait that runs out sets *err (which a correct launch
// never does) and leaves what it last read.
template <typename KV, int HD>
__device__ __forceinline__ void wave_poll_exchange(const uint64_t* xq, const uint64_t* xk, const uint64_t* xv,
                                                   bool cur, int t, float* qs, KV* kn, KV* vn, int* err) {
    static_assert(HD == 64 || HD == 128, "one or two values a lane");
    constexpr int PER = HD / 64;
    const int d = (threadIdx.x & 63) * PER;
    uint64_t q[PER], k[PER], v[PER];
    for (int spins = 0;; spins++) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            q[i] = xch_get(xq + d + i);
            if (cur) {
                k[i] = xch_get(xk + d + i);
                v[i] = xch_get(xv + d + i);
            }
        }
#pragma unroll
        for (int i = 0; i < PER; i++) ok = ok && xch_ok(q[i], t) && (!cur || (xch_ok(k[i], t) && xch_ok(v[i], t)));
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
        if (spins > (1 << 16)) {  // tens of milliseconds: only a broken launch gets here
            if ((threadIdx.x & 63) == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int i = 0; i < PER; i++) {
        qs[d + i] = xch_val(q[i]);
        if (cur) {
            kn[d + i] = (KV)xch_val(k[i]);
            vn[d + i] = (KV)xch_val(v[i]);
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
    const bool active = w < ATT_SPAN_WAVES && p0 < t;  // wave-uniform
    float mx = -__builtin_inff(), l = 0.0f;
    typedef KV kvv __attribute__((ext_vector_type(V)));
    if constexpr (VPRE) {
        // K and V rows of the chunk in the same coalesced layout (load i of
        // lane l = piece l % CPR of row KG i + l / CPR), all in flight
        // before the query is read: one memory round trip.  The chunk's 64
        // keys are one page of the cache (rows p0 .. p0 + 63 at kb / vb +
        // (p - p0) * hd).  The row's last key t - 1 (row cr of its chunk)
        // does not take part in the loads: it is the one a fused launch
        // writes itself, and in every launch it enters the scores and the
        // context as an extra term (kcur, vcur: the lanes of row group cr % KG
        // hold its pieces), so the fused and the separate attention do the
        // same arithmetic.  Buffer loads over the rows before it: rows from
        // cr on read as zeros without touching memory (a masked key has a
        // finite V row and weight 0).
        constexpr int KG = 64 / CPR;
        const int cr = t - 1 - p0;  // the last key's row in this chunk (>= ATT_CHUNK: not in it)
        const bool here = cr < ATT_CHUNK;
        const int nvalid = active ? min(ATT_CHUNK, t - p0) : 0;
        const int nload = here ? cr : nvalid;
        const size_t page = active ? kv_row(kv_table, n_kv, kvh, p0, hd) : 0;
        const uint32_t row_bytes = (uint32_t)hd * (uint32_t)sizeof(KV);
        const __amdgpu_buffer_rsrc_t krs = make_rsrc(kc + page, (uint32_t)nload * row_bytes);
        const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vc + page, (uint32_t)nload * row_bytes);
        kvv kreg[CPR], vreg[CPR];
        kvv kcur{}, vcur{};
        const int vk = lane / CPR, pc = lane % CPR, ve = pc * V;
        const bool mine = here && vk == cr % KG;  // the lane holds a piece of the last key
        if (active) {
#pragma unroll
            for (int i = 0; i < CPR; i++)
                kreg[i] = __builtin_bit_cast(kvv, buf_load_b128(krs, (uint32_t)(KG * i + vk) * row_bytes + ve * sizeof(KV)));
#pragma unroll
            for (int i = 0; i < CPR; i++)
                vreg[i] = __builtin_bit_cast(kvv, buf_load_b128(vrs, (uint32_t)(KG * i + vk) * row_bytes + ve * sizeof(KV)));
            if constexpr (!FUSED) {  // the last key from the cache (the previous launch wrote it)
                const __amdgpu_buffer_rsrc_t k1 = make_rsrc(kc + page, (uint32_t)nvalid * row_bytes);
                const __amdgpu_buffer_rsrc_t v1 = make_rsrc(vc + page, (uint32_t)nvalid * row_bytes);
                const uint32_t off = mine ? (uint32_t)cr * row_bytes + ve * sizeof(KV) : RSRC_OOB;
                kcur = __builtin_bit_cast(kvv, buf_load_b128(k1, off));
                vcur = __builtin_bit_cast(kvv, buf_load_b128(v1, off));
            }
        }
        float qv[V];
        if constexpr (FUSED) {
            // The keys before the last are older launches' stores (loaded
            // above); q and the last key's k / v rows are this launch's: wave
            // 0 polls them from the exchange into LDS while the loads are in
            // flight.
            KV* kn = reinterpret_cast<KV*>(os + ATT_WAVES * hd);
            KV* vn = kn + hd;
            const bool cur = (t - 1) / ATT_SPAN == z;
            if (w == 0)
                wave_poll_exchange<KV, HD>(a.xch + (size_t)h * hd, a.xch + (size_t)(n_heads + kvh) * hd,
                                           a.xch + (size_t)(n_heads + n_kv + kvh) * hd, cur, t, qs, kn, vn, a.err);
            __syncthreads();
            if (active) {
#pragma unroll
                for (int e = 0; e < V; e += 4) {
                    const float4 t4 = *reinterpret_cast<const float4*>(qs + ve + e);
                    qv[e] = t4.x, qv[e + 1] = t4.y, qv[e + 2] = t4.z, qv[e + 3] = t4.w;
                }
                if (mine) {
                    kcur = *reinterpret_cast<const kvv*>(kn + ve);
                    vcur = *reinterpret_cast<const kvv*>(vn + ve);
                }
            }
        } else if (active) {
#pragma unroll
            for (int e = 0; e < V; e += 4) {
                const float4 t4 = *reinterpret_cast<const float4*>(q + ve + e);
                qv[e] = t4.x, qv[e + 1] = t4.y, qv[e + 2] = t4.z, qv[e + 3] = t4.w;
            }
        }
        if (active) {
            __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the arithmetic
            // partial scores of the lane's CPR rows over its V dims, then a
            // transposed sum over the CPR lanes of the row group: piece c ends
            // with row KG c + vk's score
            float ps[CPR];
#pragma unroll
            for (int i = 0; i < CPR; i++) {
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < V; e++) acc += qv[e] * (float)kreg[i][e];
                ps[i] = acc;
            }
            transposed_sum<CPR / 2, CPR>(ps, pc);
            // the last key: its partial over the lane's dims, summed over its
            // row group (zero elsewhere), joins the score of the lane that
            // holds row cr (lane lcur; its loaded row was zeros)
            const int lcur = (cr % KG) * CPR + cr / KG;
            float pcur = 0.0f;
#pragma unroll
            for (int e = 0; e < V; e++) pcur += qv[e] * (float)kcur[e];
            pcur = group_sum<CPR>(pcur);
            const int key = KG * pc + vk;  // the row whose score this lane holds
            const bool kvalid = key < nvalid;
            const float sc = kvalid ? (ps[0] + (here && lane == lcur ? pcur : 0.0f)) / scale : -__builtin_inff();
            mx = wave_max(sc);
            const float e = kvalid ? expf(sc - mx) : 0.0f;
            l = wave_sum(e);
            float o[V];
#pragma unroll
            for (int c = 0; c < V; c++) o[c] = 0.0f;
            // row KG i + vk's weight sits in piece i of the lane's row group
            // (rows past the length carry 0 and zero V rows)
            auto pv = [&](auto ic) {
                constexpr int i = decltype(ic)::value;
                float pj;
                if constexpr (CPR == 16) pj = row_bcast<i>(e);
                else pj = __shfl(e, vk * CPR + i);
#pragma unroll
                for (int c = 0; c < V; c++) o[c] += pj * (float)vreg[i][c];
            };
            static_for<0, CPR>(pv);
            if (here) {  // the last key's weight times its V piece (zero pieces elsewhere)
                const float pl = __shfl(e, lcur);
#pragma unroll
                for (int c = 0; c < V; c++) o[c] += pl * (float)vcur[c];
            }
            if constexpr (CPR == 16 && V == 8) {
                // sum over the 4 row groups (lanes l, l + 16, l + 32, l + 48)
                // with permlane swaps: lane l ends with values c0 = 2 (2 * 0 +
                // odd16) + hi32 and c1 = c0 + 4 of its piece
                float r[4];
#pragma unroll
                for (int m = 0; m < 4; m++) r[m] = fold32(o[2 * m], o[2 * m + 1]);
                const float s0 = fold16(r[0], r[1]), s1 = fold16(r[2], r[3]);
                const int c0 = 2 * ((lane >> 4) & 1) + (lane >> 5);
                os[w * hd + ve + c0] = s0;
                os[w * hd + ve + c0 + 4] = s1;
            } else {
#pragma unroll
                for (int off = CPR; off < 64; off <<= 1)
#pragma unroll
                    for (int c = 0; c < V; c++) o[c] += __shfl_xor(o[c], off);
                if (lane < CPR)
#pragma unroll
                    for (int c = 0; c < V; c++) os[w * hd + ve + c] = o[c];
            }
        }
    } else if (active) {
        const int p = p0 + lane;
        const bool valid = p < t;
        const size_t page = kv_row(kv_table, n_kv, kvh, p0, hd);
        const KV* vb = vc + page;
        const int nvalid = min(ATT_CHUNK, t - p0);
        float acc = 0.0f;
        {
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
    const int nw = min(ATT_SPAN_WAVES, (t - z * ATT_SPAN + ATT_CHUNK - 1) / ATT_CHUNK);
    const int nz = (t + ATT_SPAN - 1) / ATT_SPAN;
    if (nz == 1 && w * 64 >= hd) return;  // a wave with no outputs to form (whole wave)
    // lane c < nw forms chunk c's weight exp(m_c - M); the sums read the
    // weights back as scalars and add in chunk order
    const float mcl = lane < nw ? ml[min(lane, ATT_WAVES - 1)][0] : -__builtin_inff();
    const float M = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, max8_f32(mcl))));
    const float wcl = lane < nw ? expf(mcl - M) : 0.0f;
    float wc[ATT_WAVES];
#pragma unroll
    for (int c = 0; c < ATT_WAVES; c++) wc[c] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wcl), c));
    float L = 0.0f;
#pragma unroll
    for (int c = 0; c < ATT_WAVES; c++) L = c < nw ? L + ml[c][1] * wc[c] : L;
    float* o = out + (size_t)s * n_heads * hd + h * hd;
    auto chunk_sum = [&](int d) {
        float O = 0.0f;
#pragma unroll
        for (int c = 0; c < ATT_WAVES; c++) O = c < nw ? O + os[c * hd + d] * wc[c] : O;
        return O;
    };
    // output element d of the head: to out, or tagged to the o projection of
    // the same launch
    uint64_t* ox = (FUSED && a.oxch) ? a.oxch + (size_t)h * hd : nullptr;
    auto put = [&](int d, float v) {
        if (FUSED && ox) xch_put(ox + d, v, t);
        else o[d] = v;
    };
    if (nz == 1) {
        const float invL = 1.0f / L;
        for (int d = threadIdx.x; d < hd; d += 64 * ATT_WAVES) put(d, chunk_sum(d) * invL);
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
    for (int d = threadIdx.x; d < hd; d += 64 * ATT_WAVES)
        __hip_atomic_store(po + 2 + d, chunk_sum(d), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
        put(d, O * invL);
    }
}

}  // namespace att
using att::AttArgs;
using att::attention_body;
using att::ATT_SPAN;
using att::ATT_WAVES;
using att::ATT_CHUNK;
using att::xch_put;
using att::wave_max;
using att::wave_sum;
}  // namespace rdl
