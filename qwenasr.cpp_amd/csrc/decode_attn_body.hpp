// Split-K GQA decode attention (scores and values passes) as device functions, shared by the
// per-launch kernels (decode_attn.hip) and the persistent decode step (decode_persist.hip), so that both
// compute the same bits.  The design and the reference's arithmetic are described in decode_attn.hip.
// `bx`, `by` take the place of blockIdx.x (chunk * n_kv + KV head) and blockIdx.y (stream).  COH: the
// scores, chunk statistics, outputs and the new K/V row are written with agent-scope (write-through)
// stores, for workgroups of the same launch on other XCDs (coherent.hpp); inputs are plain loads.
#pragma once

#include "coherent.hpp"
#include "common.hpp"
#include "prep.hpp"

#include <cmath>
#include <cstdlib>

namespace qa {
namespace {

constexpr int kThreads = 256;   // 4 waves
constexpr int kRep = 2;         // query heads per KV head (Qwen3-ASR: 16 / 8)
constexpr int kMinChunk = 32;   // the workspace is laid out for the smallest chunk size
// Merge counters sit 256 bytes apart.  Device-scope atomics on one cache line are serialised (about
// 10 ns each whichever word of the line they hit), so counters packed 8 to a line made every
// participant of 8 units queue behind each other; one line per counter leaves only the participants
// of one unit in the queue.
constexpr int kCounterStride = 64;

struct alignas(16) SplitStat {
    float m;
    float pad;
    double s;
};

struct DecodeParams {
    const float * q;          // [S][q_stride] prepared q; fused mode: raw q|k|v rows [S][q_stride]
    void * cache;
    float * out;              // [S][out_stride]
    const int32_t * lens;     // attended length = lens[s] + lens_add, clamped to [0, max_len]
    float * scores;           // [S_cap][n_heads][score_stride]
    SplitStat * stats;        // [S_cap][n_heads][max_chunks]
    float * partial;          // [S_cap][n_kv][max_chunks][2][128]
    uint32_t * counters;      // [S_cap][n_kv][kCounterStride]
    const float * q_norm_w;   // fused mode only
    const float * k_norm_w;
    float eps;
    int32_t lens_add;
    int32_t q_stride, out_stride;
    int32_t n_heads, n_kv_heads, n_streams, max_seq, layer;
    int32_t max_len, max_chunks, score_stride;
    int32_t stat_chunk;       // positions per scores-kernel chunk (granularity of the statistics)
    float scale;
};

// The double sum of a SplitStat loaded as 16 raw bytes (m, pad, s).
__device__ inline double stat_sum(const float4 & raw) {
    const uint64_t lo = __float_as_uint(raw.z), hi = __float_as_uint(raw.w);
    return __longlong_as_double(static_cast<long long>((hi << 32) | lo));
}

// A chunk statistic for the values pass: agent-scope (write-through) stores with COH.
template <bool COH>
__device__ __forceinline__ void store_stat(SplitStat * dst, float m, double s) {
    if constexpr (COH) {
        st_u64<true>(reinterpret_cast<uint64_t *>(dst), static_cast<uint64_t>(__float_as_uint(m)));
        st_u64<true>(reinterpret_cast<uint64_t *>(dst) + 1, static_cast<uint64_t>(__double_as_longlong(s)));
    } else {
        SplitStat st;
        st.m = m;
        st.pad = 0.0f;
        st.s = s;
        *dst = st;
    }
}

struct Workspace {
    size_t scores, stats, partial, counters, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// Sized from the cache capacity (streams x max_seq), never from a call's length, so the offsets of
// the counters stay fixed for the lifetime of a workspace.
Workspace workspace_layout(int32_t n_streams, int32_t n_kv, int32_t max_seq) {
    const size_t chunks = (static_cast<size_t>(max_seq) + kMinChunk - 1) / kMinChunk;
    const size_t units = static_cast<size_t>(n_streams) * n_kv;
    Workspace w{};
    w.scores = 0;
    w.stats = align256(w.scores + sizeof(float) * units * kRep * chunks * kMinChunk);
    w.partial = align256(w.stats + sizeof(SplitStat) * units * kRep * chunks);
    w.counters = align256(w.partial + sizeof(float) * units * chunks * kRep * kHeadDim);
    w.total = align256(w.counters + sizeof(uint32_t) * units * kCounterStride);
    return w;
}

// 8 consecutive elements of a cache row: raw bits are loaded first (all loads in flight), converted
// to f32 when used.  Cache rows are read once per call, so they are loaded with the streaming
// (nontemporal) policy: they do not evict the scores, statistics and partials that the kernels write,
// which then stay in L2 until the end of the kernel instead of being written back between the reads
// (a microbenchmark of 32 KB one-shot workgroups: 6.35 -> 6.79 TB/s reading, 5.82 -> 6.41 TB/s with a
// 1 KB write per workgroup).
template <typename CT>
struct Slice;

template <>
struct Slice<_Float16> {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 x;
    __device__ inline void load(const _Float16 * p) { x = __builtin_nontemporal_load(reinterpret_cast<const h8 *>(p)); }
    __device__ inline void zero() {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = static_cast<_Float16>(0.0f);
    }
    __device__ inline float get(int i) const { return static_cast<float>(x[i]); }
    __device__ inline void set(int i, float v) { x[i] = static_cast<_Float16>(v); }
};

template <>
struct Slice<float> {
    float4 a, b;
    __device__ inline void load(const float * p) {
        typedef float f4v __attribute__((ext_vector_type(4)));
        const f4v lo = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(p));
        const f4v hi = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(p + 4));
        a = make_float4(lo[0], lo[1], lo[2], lo[3]);
        b = make_float4(hi[0], hi[1], hi[2], hi[3]);
    }
    __device__ inline void zero() {
        a = make_float4(0.f, 0.f, 0.f, 0.f);
        b = a;
    }
    __device__ inline float get(int i) const {
        switch (i) {
            case 0: return a.x; case 1: return a.y; case 2: return a.z; case 3: return a.w;
            case 4: return b.x; case 5: return b.y; case 6: return b.z; default: return b.w;
        }
    }
    __device__ inline void set(int i, float v) {
        switch (i) {
            case 0: a.x = v; break; case 1: a.y = v; break; case 2: a.z = v; break; case 3: a.w = v; break;
            case 4: b.x = v; break; case 5: b.y = v; break; case 6: b.z = v; break; default: b.w = v; break;
        }
    }
};

__device__ inline float round_f16(float x) { return static_cast<float>(static_cast<_Float16>(x)); }

// Probabilities are kept as f16 when V is f16 (the rounding the reference applies before PV), else f32.
template <bool R16>
struct PStore {
    typedef float type;
};
template <>
struct PStore<true> {
    typedef _Float16 type;
};

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Elements 2I, 2I + 1 of an f16 slice as one packed pair.
template <int I>
__device__ inline h2 pair_of(const Slice<_Float16> & s) {
    return __builtin_shufflevector(s.x, s.x, 2 * I, 2 * I + 1);
}

// DPP lane permutation of a float within rows of 16 lanes (VALU, no LDS round trip).
template <int CTRL>
__device__ inline float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// One reduce-scatter stage over the lane pairs of DPP pattern CTRL (an XOR of the lane index within
// 16 whose top set bit is BIT): of the N live values the lane keeps the half selected by its own BIT
// and adds the partner's copy of that half; with N == 1 the stage is a plain butterfly add.
template <int N, int CTRL, int BIT>
__device__ inline void rs_stage(float (&v)[16], int part) {
    if constexpr (N > 1) {
        const bool up = (part & BIT) != 0;
#pragma unroll
        for (int i = 0; i < N / 2; ++i) {
            const float send = up ? v[i] : v[i + N / 2];
            const float keep = up ? v[i + N / 2] : v[i];
            v[i] = keep + dpp<CTRL>(send);
        }
    } else {
        v[0] += dpp<CTRL>(v[0]);
    }
}

// Sums each of N values (N = 2, 4, 8 or 16) over the 16 lanes of a row group and leaves lane `part`
// with the full sum of value part / (16 / N).  Partners are lane XOR 15 (row_mirror), XOR 7
// (row_half_mirror), XOR 2 and XOR 1 (quad_perm): linearly independent masks, so the four stages
// cover all 16 lanes, and each stage pairs lanes that hold the same index subset.  A full butterfly
// per value would cost 4 shuffle-adds per value per lane; this costs N - 1 + (4 - log2 N).
template <int N>
__device__ inline float reduce_scatter16(const float (&in)[N], int part) {
    float v[16];
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = in[i];
    rs_stage<N, 0x140, 8>(v, part);
    rs_stage<(N > 1 ? N / 2 : 1), 0x141, 4>(v, part);
    rs_stage<(N > 2 ? N / 4 : 1), 0x4E, 2>(v, part);
    rs_stage<(N > 4 ? N / 8 : 1), 0xB1, 1>(v, part);
    return v[0];
}

__device__ inline void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ inline void publish(float * p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline int attended(const DecodeParams & p, int s) {
    return min(max(p.lens[s] + p.lens_add, 0), p.max_len);
}

template <typename CT, bool R16, int CHUNK, bool FUSED, bool COH>
__device__ __forceinline__ void decode_scores_body(const DecodeParams & p, const RopeTable & rope, int bx, int by) {
    // no contraction left to the compiler: the products that are fused are written as fma, so the per-launch
    // kernel and the persistent step (where inlining differs) compute the same bits
#pragma clang fp contract(off)
    constexpr int RPT = CHUNK / 16;   // rows per lane: 16 rows per workgroup pass
    const int g = bx % p.n_kv_heads;
    const int c = bx / p.n_kv_heads;
    const int s = by;
    const int L = attended(p, s);
    if (c * CHUNK >= L) return;                      // uniform for the whole workgroup

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int sub = lane >> 4;                        // row within the wave's 4-row group
    const int part = lane & 15;                       // 8-element slice of the row
    const int h0 = g * kRep;
    const int row0 = c * CHUNK + wave * (CHUNK / 4);  // each wave: CHUNK / 4 consecutive rows
    const int pos_new = L - 1;                        // fused mode: the token being appended
    const bool owner = FUSED && pos_new / CHUNK == c;

    CT * kc = static_cast<CT *>(p.cache) +
              cache_row_offset(p.layer, 0, s, g, 0, p.n_streams, p.n_kv_heads, p.max_seq);
    const CT * kb = kc + part * 8;

    // Every load of the workgroup is issued before the first use of any of them, the prologue's
    // inputs first: vector memory loads complete in issue order, so waiting for a prologue input never
    // waits for the K rows behind it, and the prologue runs while the K rows are in flight.
    // Fused mode: waves 0/1 load query head h0 + wave, wave 2 the new k row and wave 3 the new v row of
    // KV head g, each with its norm weight (every workgroup loads them; only the owner of the new
    // position uses waves 2/3).  Unfused mode: the prepared q slices of both heads.
    const float * row = p.q + static_cast<int64_t>(s) * p.q_stride;
    float pa = 0.0f, pb = 0.0f, wa = 0.0f, wb = 0.0f;
    double inv_freq = 0.0;
    float4 qv[4];
    if constexpr (FUSED) {
        const int q_dim = p.n_heads * kHeadDim;
        const float * src = wave < 2 ? row + (h0 + wave) * kHeadDim
                                     : row + q_dim + (wave == 2 ? 0 : p.n_kv_heads * kHeadDim) + g * kHeadDim;
        const float * w = wave < 2 ? p.q_norm_w : p.k_norm_w;
        pa = src[lane];
        pb = src[lane + 64];
        wa = w[lane];
        wb = w[lane + 64];
        inv_freq = rope.inv_freq[lane];   // kernel argument, indexed per lane: also a memory load
    } else {
        const float * qp = row + h0 * kHeadDim + part * 8;
        qv[0] = *reinterpret_cast<const float4 *>(qp);
        qv[1] = *reinterpret_cast<const float4 *>(qp + 4);
        qv[2] = *reinterpret_cast<const float4 *>(qp + kHeadDim);
        qv[3] = *reinterpret_cast<const float4 *>(qp + kHeadDim + 4);
    }
    // K rows.  Rows past the end re-read the last row instead of branching around the load (a branch
    // would split the loads with a wait); their scores are masked below.  In fused mode the new row
    // is not in the cache yet: its stale contents are loaded and replaced from LDS.
    Slice<CT> ks[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const int j = min(row0 + k * 4 + sub, L - 1);
        ks[k].load(kb + static_cast<int64_t>(j) * kHeadDim);
    }

    float q0[8], q1[8];
    if constexpr (FUSED) {
        __shared__ float s_q[kRep][kHeadDim];
        __shared__ float s_k[kHeadDim];
        if (wave < 2) {
            norm_rope_pair(pa, pb, wa, wb, p.eps, pos_new, inv_freq);
            s_q[wave][lane] = pa;
            s_q[wave][lane + 64] = pb;
        } else if (owner) {
            const bool is_k = wave == 2;
            if (is_k) norm_rope_pair(pa, pb, wa, wb, p.eps, pos_new, inv_freq);
            const CT ca = static_cast<CT>(pa), cb = static_cast<CT>(pb);
            const int64_t v_delta = cache_row_offset(0, 1, 0, 0, 0, p.n_streams, p.n_kv_heads, p.max_seq);
            CT * dst = kc + (is_k ? 0 : v_delta) + static_cast<int64_t>(pos_new) * kHeadDim;
            st_cache<COH>(dst + lane, ca);
            st_cache<COH>(dst + lane + 64, cb);
            if (is_k) {
                s_k[lane] = static_cast<float>(ca);
                s_k[lane + 64] = static_cast<float>(cb);
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            q0[i] = s_q[0][part * 8 + i];
            q1[i] = s_q[1][part * 8 + i];
        }
        if (owner) {
#pragma unroll
            for (int k = 0; k < RPT; ++k) {
                if (row0 + k * 4 + sub == pos_new) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) ks[k].set(i, s_k[part * 8 + i]);
                }
            }
        }
    } else {
        q0[0] = qv[0].x; q0[1] = qv[0].y; q0[2] = qv[0].z; q0[3] = qv[0].w;
        q0[4] = qv[1].x; q0[5] = qv[1].y; q0[6] = qv[1].z; q0[7] = qv[1].w;
        q1[0] = qv[2].x; q1[1] = qv[2].y; q1[2] = qv[2].z; q1[3] = qv[2].w;
        q1[4] = qv[3].x; q1[5] = qv[3].y; q1[6] = qv[3].z; q1[7] = qv[3].w;
    }
    if (R16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) { q0[i] = round_f16(q0[i]); q1[i] = round_f16(q1[i]); }
    }

    // partial dot products of this lane's 8 dims: v[2k + h] for row row0 + 4k + sub and head h
    float * sc0 = p.scores + (static_cast<int64_t>(s) * p.n_heads + h0) * p.score_stride;
    float * sc1 = sc0 + p.score_stride;
    float vdot[2 * RPT];
    // f16 cache: q (already rounded to f16) and K as f16 pairs on v_dot2_f32_f16: exact f16 products,
    // f32 sums -- the f16 dot type of the reference's mul_mat with f32 precision, in 8 instead of 24
    // VALU operations per row and head
    h2 qa2[4], qb2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        qa2[i] = h2{static_cast<_Float16>(q0[2 * i]), static_cast<_Float16>(q0[2 * i + 1])};
        qb2[i] = h2{static_cast<_Float16>(q1[2 * i]), static_cast<_Float16>(q1[2 * i + 1])};
    }
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        float a = 0.0f, b = 0.0f;
        if constexpr (R16) {
            const h2 k0 = pair_of<0>(ks[k]), k1 = pair_of<1>(ks[k]), k2 = pair_of<2>(ks[k]), k3 = pair_of<3>(ks[k]);
            a = __builtin_amdgcn_fdot2(k0, qa2[0], a, false);
            b = __builtin_amdgcn_fdot2(k0, qb2[0], b, false);
            a = __builtin_amdgcn_fdot2(k1, qa2[1], a, false);
            b = __builtin_amdgcn_fdot2(k1, qb2[1], b, false);
            a = __builtin_amdgcn_fdot2(k2, qa2[2], a, false);
            b = __builtin_amdgcn_fdot2(k2, qb2[2], b, false);
            a = __builtin_amdgcn_fdot2(k3, qa2[3], a, false);
            b = __builtin_amdgcn_fdot2(k3, qb2[3], b, false);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float kv = ks[k].get(i);
                a = fmaf(q0[i], kv, a);
                b = fmaf(q1[i], kv, b);
            }
        }
        vdot[2 * k] = a;
        vdot[2 * k + 1] = b;
    }
    // After the reduce-scatter lane `part` of row group `sub` holds the full score of value index
    // part / kDup, i.e. row row0 + 4 kk + sub and head hh; each score is then scaled, stored, and fed
    // to the statistics exactly once (kDup lanes hold a copy when 2 RPT < 16; only the first counts).
    // With more than 16 values per lane (RPT > 8) the first 16 are reduced as above and the remaining
    // NB in a second reduce-scatter, whose scores (value index 16 + part / kDupB) each lane also holds.
    constexpr int NA = 2 * RPT > 16 ? 16 : 2 * RPT;
    constexpr int NB = 2 * RPT - NA;
    static_assert(NB == 0 || NB == 2 || NB == 4 || NB == 8 || NB == 16, "rows per lane: 1, 2, 4, 8, 9, 10, 12 or 16");
    constexpr int kDup = 16 / NA;
    float va[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) va[i] = vdot[i];
    const float dot = reduce_scatter16<NA>(va, part);
    const int idx = part / kDup;
    const int kk = idx >> 1, hh = idx & 1;
    const int j = row0 + kk * 4 + sub;
    const bool valid = j < L;
    const bool primary = part % kDup == 0;
    const float x = valid ? dot * p.scale : -INFINITY;
    if (valid && primary) st_f<COH>((hh ? sc1 : sc0) + j, x);
    float x2 = -INFINITY;
    int hh2 = 0;
    bool use2 = false;
    if constexpr (NB > 0) {
        constexpr int kDupB = 16 / NB;
        float vb[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) vb[i] = vdot[NA + i];
        const float dot2 = reduce_scatter16<NB>(vb, part);
        const int idx2 = NA + part / kDupB;
        hh2 = idx2 & 1;
        const int j2 = row0 + (idx2 >> 1) * 4 + sub;
        const bool valid2 = j2 < L;
        use2 = valid2 && part % kDupB == 0;
        x2 = valid2 ? dot2 * p.scale : -INFINITY;
        if (use2) st_f<COH>((hh2 ? sc1 : sc0) + j2, x2);
    }

    __shared__ float s_max[kRep][4];
    __shared__ double s_sum[kRep][4];
    float m0, m1;
    if constexpr (NB > 0) {
        m0 = wave_max_lane63(fmaxf(hh == 0 ? x : -INFINITY, hh2 == 0 ? x2 : -INFINITY));
        m1 = wave_max_lane63(fmaxf(hh == 1 ? x : -INFINITY, hh2 == 1 ? x2 : -INFINITY));
    } else {
        m0 = wave_max_lane63(hh == 0 ? x : -INFINITY);
        m1 = wave_max_lane63(hh == 1 ? x : -INFINITY);
    }
    if (lane == kWave - 1) { s_max[0][wave] = m0; s_max[1][wave] = m1; }
    __syncthreads();
    m0 = fmaxf(fmaxf(s_max[0][0], s_max[0][1]), fmaxf(s_max[0][2], s_max[0][3]));
    m1 = fmaxf(fmaxf(s_max[1][0], s_max[1][1]), fmaxf(s_max[1][2], s_max[1][3]));
    // sum of expf(x - max) per head: f32 within the wave (at most 64 terms), double across waves
    const float e = valid && primary ? expf(x - (hh ? m1 : m0)) : 0.0f;
    float e0, e1;
    if constexpr (NB > 0) {
        const float f = use2 ? expf(x2 - (hh2 ? m1 : m0)) : 0.0f;
        e0 = wave_sum_lane63((hh == 0 ? e : 0.0f) + (hh2 == 0 ? f : 0.0f));
        e1 = wave_sum_lane63((hh == 1 ? e : 0.0f) + (hh2 == 1 ? f : 0.0f));
    } else {
        e0 = wave_sum_lane63(hh == 0 ? e : 0.0f);
        e1 = wave_sum_lane63(hh == 1 ? e : 0.0f);
    }
    if (lane == kWave - 1) { s_sum[0][wave] = e0; s_sum[1][wave] = e1; }
    __syncthreads();
    if (threadIdx.x < kRep) {
        const int h = threadIdx.x;
        store_stat<COH>(p.stats + (static_cast<int64_t>(s) * p.n_heads + h0 + h) * p.max_chunks + c,
                        h == 0 ? m0 : m1, (s_sum[h][0] + s_sum[h][1]) + (s_sum[h][2] + s_sum[h][3]));
    }
}

template <typename CT, bool R16, int CHUNK, int SR, int MB, bool COH>
__device__ __forceinline__ void decode_values_body(const DecodeParams & p, int bx, int by) {
    // no contraction left to the compiler: the products that are fused are written as fma, so the per-launch
    // kernel and the persistent step (where inlining differs) compute the same bits
#pragma clang fp contract(off)
    constexpr int RPT = CHUNK / 16;
    const int g = bx % p.n_kv_heads;
    const int c = bx / p.n_kv_heads;
    const int s = by;
    const int L = attended(p, s);
    const int n_chunks = (L + CHUNK - 1) / CHUNK;                   // values chunks = merge participants
    const int n_stats = (L + p.stat_chunk - 1) / p.stat_chunk;      // scores chunks
    if (c >= n_chunks) return;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int sub = lane >> 4;
    const int part = lane & 15;
    const int h0 = g * kRep;
    const int row0 = c * CHUNK + wave * (CHUNK / 4);

    // Loads are issued in the order statistics, scores, V rows, all before the first use of any of
    // them: vector memory loads complete in issue order, so the softmax normalisation below waits for
    // the statistics and scores only and runs while the V rows are in flight.  Out-of-range indices
    // re-read the last valid entry instead of branching around the load (a branch would split the
    // loads with a wait) and are masked where the value is used.
    // The first SR * 64 statistics of each head are held in registers (one 16-byte load each; SR is
    // chosen from the cache capacity so that this covers every call); longer prefixes loop over the
    // rest.
    const SplitStat * st0 = p.stats + (static_cast<int64_t>(s) * p.n_heads + h0) * p.max_chunks;
    const SplitStat * st1 = st0 + p.max_chunks;
    constexpr int kStatRegs = SR;
    float4 sa[kStatRegs], sb[kStatRegs];
#pragma unroll
    for (int u = 0; u < kStatRegs; ++u) {
        const int i = min(lane + u * kWave, n_stats - 1);
        sa[u] = *reinterpret_cast<const float4 *>(st0 + i);
        sb[u] = *reinterpret_cast<const float4 *>(st1 + i);
    }
    // Each lane loads the one score it turns into p below (the wave's CHUNK / 4 rows are row0 ..
    // row0 + RW - 1; lane -> row lane % RW, and for RW <= 32 head (lane / RW) & 1, so every (row, head)
    // probability is computed once, not by all 16 lanes that hold a slice of that row).
    constexpr int RW = CHUNK / 4;
    const float * sc0 = p.scores + (static_cast<int64_t>(s) * p.n_heads + h0) * p.score_stride;
    const float * sc1 = sc0 + p.score_stride;
    const int own = lane % RW;
    const int jr = row0 + own;
    const int jrc = min(jr, L - 1);
    const int hsel = RW >= kWave ? 0 : (lane / RW) & 1;
    float xs0, xs1 = 0.0f;
    if constexpr (RW >= kWave) {
        xs0 = sc0[jrc];
        xs1 = sc1[jrc];
    } else {
        xs0 = (hsel ? sc1 : sc0)[jrc];
    }
    const CT * vb = static_cast<const CT *>(p.cache) +
                    cache_row_offset(p.layer, 1, s, g, 0, p.n_streams, p.n_kv_heads, p.max_seq) + part * 8;
    Slice<CT> vs[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const int j = min(row0 + k * 4 + sub, L - 1);   // rows past the end get p = 0
        vs[k].load(vb + static_cast<int64_t>(j) * kHeadDim);
    }

    // global max and sum of both heads from the chunk statistics (every wave, redundantly); a repeated
    // entry leaves the max unchanged and is excluded from the sum
    float M0 = -INFINITY, M1 = -INFINITY;
#pragma unroll
    for (int u = 0; u < kStatRegs; ++u) {
        M0 = fmaxf(M0, sa[u].x);
        M1 = fmaxf(M1, sb[u].x);
    }
    for (int i = lane + kStatRegs * kWave; i < n_stats; i += kWave) {
        M0 = fmaxf(M0, st0[i].m);
        M1 = fmaxf(M1, st1[i].m);
    }
    M0 = wave_max_all(M0);
    M1 = wave_max_all(M1);
    // rescaled chunk sums, accumulated in double (the rescale factor in f32: its rounding is far below
    // the f32 resolution of the final 1 / sum)
    double S0 = 0.0, S1 = 0.0;
#pragma unroll
    for (int u = 0; u < kStatRegs; ++u) {
        if (lane + u * kWave < n_stats) {
            S0 = fma(stat_sum(sa[u]), static_cast<double>(expf(sa[u].x - M0)), S0);
            S1 = fma(stat_sum(sb[u]), static_cast<double>(expf(sb[u].x - M1)), S1);
        }
    }
    for (int i = lane + kStatRegs * kWave; i < n_stats; i += kWave) {
        S0 = fma(st0[i].s, static_cast<double>(expf(st0[i].m - M0)), S0);
        S1 = fma(st1[i].s, static_cast<double>(expf(st1[i].m - M1)), S1);
    }
    S0 = wave_sum_d_all(S0);
    S1 = wave_sum_d_all(S1);
    const float r0 = static_cast<float>(1.0 / S0);
    const float r1 = static_cast<float>(1.0 / S1);
    const bool row_valid = jr < L;

    // normalised probabilities of this lane's (row, head), rounded to f16 for an f16 V, shared in LDS.
    // Row k * 4 + sub of the wave is stored at sub * RPT + k, so the lanes of group `sub` read the pair
    // (k, k + 1) as one 32-bit word.
    typedef typename PStore<R16>::type PT;
    __shared__ __attribute__((aligned(16))) PT s_p[4][kRep][kWave];
    {
        const float Ma = hsel ? M1 : M0, ra = hsel ? r1 : r0;
        const float pa = row_valid ? expf(xs0 - Ma) * ra : 0.0f;
        const int slot = (own & 3) * RPT + (own >> 2);
        if constexpr (RW >= kWave) {
            const float pb = row_valid ? expf(xs1 - M1) * r1 : 0.0f;
            s_p[wave][0][slot] = static_cast<PT>(pa);
            s_p[wave][1][slot] = static_cast<PT>(pb);
        } else if (lane < kRep * RW) {
            s_p[wave][hsel][slot] = static_cast<PT>(pa);
        }
    }
    __syncthreads();
    float a0[8], a1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { a0[i] = 0.0f; a1[i] = 0.0f; }
    if constexpr (R16) {
        // pairs of rows on v_dot2_f32_f16: exact f16 products of p and V, f32 sums
#pragma unroll
        for (int k = 0; k < RPT; k += 2) {
            const h2 pa = *reinterpret_cast<const h2 *>(&s_p[wave][0][sub * RPT + k]);
            const h2 pb = *reinterpret_cast<const h2 *>(&s_p[wave][1][sub * RPT + k]);
            const h2 v0 = __builtin_shufflevector(vs[k].x, vs[k + 1].x, 0, 8);
            const h2 v1 = __builtin_shufflevector(vs[k].x, vs[k + 1].x, 1, 9);
            const h2 v2 = __builtin_shufflevector(vs[k].x, vs[k + 1].x, 2, 10);
            const h2 v3 = __builtin_shufflevector(vs[k].x, vs[k + 1].x, 3, 11);
            const h2 v4 = __builtin_shufflevector(vs[k].x, vs[k + 1].x, 4, 12);
            const h2 v5 = __builtin_shufflevector(vs[k].x, vs[k + 1].x, 5, 13);
            const h2 v6 = __builtin_shufflevector(vs[k].x, vs[k + 1].x, 6, 14);
            const h2 v7 = __builtin_shufflevector(vs[k].x, vs[k + 1].x, 7, 15);
            a0[0] = __builtin_amdgcn_fdot2(v0, pa, a0[0], false); a1[0] = __builtin_amdgcn_fdot2(v0, pb, a1[0], false);
            a0[1] = __builtin_amdgcn_fdot2(v1, pa, a0[1], false); a1[1] = __builtin_amdgcn_fdot2(v1, pb, a1[1], false);
            a0[2] = __builtin_amdgcn_fdot2(v2, pa, a0[2], false); a1[2] = __builtin_amdgcn_fdot2(v2, pb, a1[2], false);
            a0[3] = __builtin_amdgcn_fdot2(v3, pa, a0[3], false); a1[3] = __builtin_amdgcn_fdot2(v3, pb, a1[3], false);
            a0[4] = __builtin_amdgcn_fdot2(v4, pa, a0[4], false); a1[4] = __builtin_amdgcn_fdot2(v4, pb, a1[4], false);
            a0[5] = __builtin_amdgcn_fdot2(v5, pa, a0[5], false); a1[5] = __builtin_amdgcn_fdot2(v5, pb, a1[5], false);
            a0[6] = __builtin_amdgcn_fdot2(v6, pa, a0[6], false); a1[6] = __builtin_amdgcn_fdot2(v6, pb, a1[6], false);
            a0[7] = __builtin_amdgcn_fdot2(v7, pa, a0[7], false); a1[7] = __builtin_amdgcn_fdot2(v7, pb, a1[7], false);
        }
    } else {
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
            const float pa = s_p[wave][0][sub * RPT + k];
            const float pb = s_p[wave][1][sub * RPT + k];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float v = vs[k].get(i);
                a0[i] = fmaf(pa, v, a0[i]);
                a1[i] = fmaf(pb, v, a1[i]);
            }
        }
    }
    // reduce over the 16 row groups of the workgroup (4 per wave x 4 waves) in LDS: every lane stores
    // its 16 partial sums, then thread (head, dim) adds the 16 groups in a fixed order
    __shared__ __attribute__((aligned(16))) float s_o[4][4][kRep][kHeadDim];
    {
        float4 * o0 = reinterpret_cast<float4 *>(&s_o[wave][sub][0][part * 8]);
        float4 * o1 = reinterpret_cast<float4 *>(&s_o[wave][sub][1][part * 8]);
        o0[0] = make_float4(a0[0], a0[1], a0[2], a0[3]);
        o0[1] = make_float4(a0[4], a0[5], a0[6], a0[7]);
        o1[0] = make_float4(a1[0], a1[1], a1[2], a1[3]);
        o1[1] = make_float4(a1[4], a1[5], a1[6], a1[7]);
    }
    __syncthreads();
    const int hh = threadIdx.x >> 7;               // query head of the group this thread finishes
    const int d = threadIdx.x & (kHeadDim - 1);
    float o = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
#pragma unroll
        for (int r = 0; r < 4; ++r) o += s_o[w][r][hh][d];
    }
    float * out = p.out + static_cast<int64_t>(s) * p.out_stride + (h0 + hh) * kHeadDim + d;
    if (n_chunks == 1) {
        st_f<COH>(out, o);
        return;
    }

    const int64_t unit = static_cast<int64_t>(s) * p.n_kv_heads + g;
    float * part_base = p.partial + unit * p.max_chunks * (kRep * kHeadDim);
    publish(part_base + static_cast<int64_t>(c) * (kRep * kHeadDim) + threadIdx.x, o);
    // every wave's stores have completed before any wave passes the barrier; then count
    wait_vmem();
    __syncthreads();
    __shared__ int s_last;
    if (threadIdx.x == 0) {
        uint32_t * ctr = p.counters + unit * kCounterStride;
        const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == static_cast<uint32_t>(n_chunks - 1);
        if (s_last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;

    // Sum of the partials: thread t owns the float pair j = t % 128 of the 256-float state and the
    // chunks c = t / 128, t / 128 + 2, ...; 32 8-byte loads per thread in flight at once (chunks past
    // the end load nothing and add +0).  The two chunk groups are then added in LDS.  Fixed order, so
    // the result is deterministic.
    const int pair = threadIdx.x & 127;
    const int grp = threadIdx.x >> 7;
    const uint64_t * pp = reinterpret_cast<const uint64_t *>(part_base) + pair;
    constexpr int kStride = kRep * kHeadDim / 2;    // uint64 per chunk state
    constexpr int kBatch = MB;   // chosen from the capacity: one round of loads for every call
    float acc_lo = 0.0f, acc_hi = 0.0f;
    for (int i0 = grp; i0 < n_chunks; i0 += 2 * kBatch) {
        uint64_t v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int i = i0 + 2 * u;
            v[u] = i < n_chunks ? __hip_atomic_load(pp + static_cast<int64_t>(i) * kStride, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT)
                                : 0;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            acc_lo += __uint_as_float(static_cast<uint32_t>(v[u]));
            acc_hi += __uint_as_float(static_cast<uint32_t>(v[u] >> 32));
        }
    }
    __shared__ float s_acc[2][kRep * kHeadDim];
    s_acc[grp][2 * pair] = acc_lo;
    s_acc[grp][2 * pair + 1] = acc_hi;
    __syncthreads();
    st_f<COH>(out, s_acc[0][threadIdx.x] + s_acc[1][threadIdx.x]);
}

// Positions per workgroup of each kernel.  The scores kernel has no merge; its chunk trades workgroup
// count (dispatch and per-workgroup overhead) against the load size of one workgroup.  The values
// kernel's chunks are the merge participants of one (stream, KV head), so it uses chunks large enough
// to keep them at <= 16 per unit (every participant increments the same counter), or <= 32 where that
// still fits one workgroup per CU (below).  The choice depends on the cache layout only (capacity,
// streams, cache dtype), never on a call's length, so a captured decode step (grids sized by capacity)
// and an eager one (grids sized by the longest stream) run the same tiling and produce the same bits.
// QA_DECODE_CHUNK / QA_DECODE_VCHUNK override the choice (tuning).
struct Chunks {
    int scores, values;
};

// The scores kernel is instantiated for 32, 64, 128, 144, 160, 192 and 256 positions per workgroup, the
// values kernel for 32, 64, 128 and 256; any other override value is ignored.
int env_chunk(const char * name, bool values) {
    const char * e = std::getenv(name);
    const int v = e ? std::atoi(e) : 0;
    if (v == 32 || v == 64 || v == 128 || v == 256) return v;
    return !values && (v == 144 || v == 160 || v == 192) ? v : 0;
}

Chunks pick_chunks(const qa_kv_layout & layout) {
    static const int forced_s = env_chunk("QA_DECODE_CHUNK", false);
    static const int forced_v = env_chunk("QA_DECODE_VCHUNK", true);
    const int32_t capacity = layout.max_seq;
    Chunks ch{};
    // scores: the smallest chunk that keeps the grid at about one workgroup per CU, else 128 (measured
    // at batch 1: 32 is best up to ~1k positions, 64 at 2k, 128 from 4k on, 11.1 vs 12.2 us at 4186;
    // 128 also for 32 streams).  "About": at most 256 workgroups for f16 rows, whose pair time rises when
    // some CUs hold two (batch 1: 64 against 32 positions 8.07 vs 8.57 us at 1200, 128 against 64 8.62 vs
    // 9.13 at 2300 and 8.73 vs 9.26 at 2550); at most 320 for f32 rows, twice the bytes per position, where
    // more and smaller workgroups time the same or better (11.74-11.90 vs 12.24 us at 2500 for 32-64 against
    // 128 positions).  Where 128-position chunks would put a second workgroup on some CUs
    // (8 units: capacities 4097 to 6144), the smallest of 144, 160 and 192 that keeps one workgroup per
    // CU: the CUs holding two would set the time (measured at batch 1: 10.1 vs 10.5 us at 4186, 10.6 vs
    // 11.2 at 5000, 10.9 vs 11.4 at 6000).  From 6145 on 128 stays: at 8000 a 256-position chunk (one
    // workgroup per CU) times the same as 128 (about two on every CU).
    const int64_t units = static_cast<int64_t>(layout.n_streams) * layout.n_kv_heads;
    const bool f32 = layout.cache_type == QA_CACHE_F32;
    const int64_t fill = f32 ? 320 : 256;
    ch.scores = 128;
    for (int c = 32; c < 128; c *= 2) {
        if (units * ((capacity + c - 1) / c) <= fill) {
            ch.scores = c;
            break;
        }
    }
    if (ch.scores == 128 && units * ((capacity + 127) / 128) > 256) {
        for (const int c : {144, 160, 192}) {
            if (units * ((capacity + c - 1) / c) <= 256) {
                ch.scores = c;
                break;
            }
        }
    }
    if (forced_s) ch.scores = forced_s;
    // values: at most 16 participants per unit; then half that chunk (up to 32 participants) where the
    // grid still holds at most one workgroup per CU, for f32 caches and for f16 caches at 256 positions
    // (V rows of 64 KB per workgroup).  Measured at batch 1 (pair time, 28 rotated layer caches): f32
    // cache 8.27 against 8.81 us at 700 positions, 9.66 against 10.33 at 1500, 10.23 against 10.82 at
    // 2000, 11.45 against 13.13 at 2100, 13.60 against 15.42 at 3947; f16 cache 8.99 against 9.43 us at
    // 2100, 8.95 against 9.17 at 3000, 9.60 against 9.84 at 3947; f16 rows of 64-128 positions lost (7.98
    // against 8.25 us at 700, 8.37 against 8.55 at 2000), and so did 32 streams (config-4 shapes, 49.1
    // against 50.2 us), whose grid holds thousands of workgroups.
    int v = 32;
    while (v < 256 && (capacity + v - 1) / v > 16) v *= 2;
    const int half = v / 2;
    if (half >= 32 && (f32 || v == 256) && units * ((capacity + half - 1) / half) <= 256) v = half;
    ch.values = forced_v ? forced_v : v;
    if (ch.values < ch.scores) ch.values = ch.scores > 128 ? 256 : ch.scores;   // values chunks: 32 ... 256
    return ch;
}

// Statistics per head held in the values kernel's registers at the capacity: 64 per register slot,
// 1/2/4/8 slots.
inline int values_stat_regs(int32_t max_seq, int scores_chunk) {
    const int n_stats_cap = (max_seq + scores_chunk - 1) / scores_chunk;
    return n_stats_cap <= 64 ? 1 : n_stats_cap <= 128 ? 2 : n_stats_cap <= 256 ? 4 : 8;
}

// Merge loads per thread and round: the participants (values chunks at the capacity) split over two
// thread groups, so MB loads cover 2 MB participants in one round; fewer registers held means more
// workgroups in flight.
inline int values_merge_loads(int32_t max_seq, int values_chunk) {
    const int n_vchunks_cap = (max_seq + values_chunk - 1) / values_chunk;
    return n_vchunks_cap <= 16 ? 8 : n_vchunks_cap <= 32 ? 16 : 40;
}

// The workspace pointers and cache geometry of `p` for a cache `layout`; false if the workspace is
// smaller than the capacity needs.
inline bool set_workspace(DecodeParams & p, const qa_kv_layout & layout, void * workspace, size_t workspace_bytes) {
    const Workspace w = workspace_layout(layout.n_streams, layout.n_kv_heads, layout.max_seq);
    if (!workspace || workspace_bytes < w.total) return false;
    char * base = static_cast<char *>(workspace);
    p.scores = reinterpret_cast<float *>(base + w.scores);
    p.stats = reinterpret_cast<SplitStat *>(base + w.stats);
    p.partial = reinterpret_cast<float *>(base + w.partial);
    p.counters = reinterpret_cast<uint32_t *>(base + w.counters);
    p.n_kv_heads = layout.n_kv_heads;
    p.n_streams = layout.n_streams;
    p.max_seq = layout.max_seq;
    p.max_chunks = (layout.max_seq + kMinChunk - 1) / kMinChunk;
    p.score_stride = p.max_chunks * kMinChunk;
    return true;
}

}  // namespace
}  // namespace qa
