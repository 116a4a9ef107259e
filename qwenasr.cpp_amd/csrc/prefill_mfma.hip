// Causal prefill attention on CDNA4 f16 MFMA (v_mfma_f32_16x16x32_f16), for f16 KV caches.
//
// Replaces the prefill half of the cached layer graph (text-decoder.cpp:435-463 with T > 1 and the
// dense mask of 1729-1735): scores = mul_mat(K, q), soft_max_ext(scores, mask, 1/sqrt(d)),
// out = mul_mat(cont(V^T), p).  With f16 K/V the reference's GGML arithmetic rounds q to f16 before
// QK^T and the normalised probabilities to f16 before PV; both are exactly the f16 operands the MFMA
// takes, with f32 accumulation.
//
// Tiling.  A workgroup (8 waves) owns 128 query tokens of one stream and both query heads of one KV
// head: 256 query columns, every K/V byte of the head shared by both heads and by all 128 tokens.
// Wave w takes head 2g + w/4 and tokens [32 (w & 3), +32) as two blocks of 16 columns.  Per 64-key
// tile a wave computes S^T = K Q^T (keys x queries, 16x16 blocks, head dim in 4 steps of 32) for both
// blocks, each K fragment read from LDS once and used by the MFMAs of both blocks (likewise each V^T
// fragment in PV).  After the MFMA each lane holds 16 keys of one query column per block.
// (Measured at T = 3913: with 64 query tokens per workgroup the steps waited on the K/V tile loads,
// each CU pulling one 32 KB tile per step for every 128 columns; 128 tokens halve that traffic.)
//
// Exact GGML softmax needs the row max and sum before any PV, so the key tiles are walked twice, by two
// kernels over the same work items:
//   pass 1  S^T, a running max per lane and the sum of exp(s - max): 16 terms in f32 per tile and
//           lane, carried across tiles in double and rescaled when the lane's max grows; the 4 lanes
//           of a query column are combined at the end and the item's statistics stored;
//   pass 2  the statistics of the query tile's parts combined into M and S, S^T again,
//           p = f16(exp(s - M) / S), O^T += V^T P^T.
// exp(x * scale - m) is evaluated as exp2(x * (scale log2 e) - m (scale log2 e)), with log2 S folded
// into m in pass 2: one FMA and one v_exp_f32 per score.  Its rounding differs from the reference's
// expf(x - M) * (1 / S) by about 1e-6 relative, far below the f16 resolution of p (the reference's own
// CPU softmax uses a vectorised exp approximation as well).
// Only the diagonal tiles (keys past the first query of the workgroup) are masked, in a loop of their
// own; every other tile takes an unmasked path.
// P^T goes from the accumulator registers straight into the B operand of the PV MFMA: the PV k-index
// e of lane group j is mapped to key (e / 4) * 16 + j * 4 + e % 4 of the 32-key step, which is
// exactly the set of keys that lane already holds; V^T is read from LDS with the same mapping.
//
// LDS: two buffers of the K tile (row-major, 144-half rows) and of V^T (dims x keys in PV order,
// 80-half rows): one barrier per tile; the next tile's global loads are in registers while the current
// one is computed.  Both operands are read as 16-byte rows at conflict-free strides.  V^T is written as
// 2 keys x 1 dim per 4-byte store, transposed in registers from 2 rows of 8 dims.
// Work distribution: the longest query tiles are cut in two parts of the key range; every part (or
// uncut tile) of one KV head is a work item, pulled from that head's queue by the workgroups serving
// the head, longest first (see the work plan below).
#include "ops.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <type_traits>

namespace qa {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kBQ = 128;    // query tokens per workgroup
constexpr int kBK = 64;     // keys per tile
constexpr int kQB = 2;      // 16-column query blocks per wave
constexpr int kCols = 2 * kBQ;    // query columns per workgroup (both heads)
constexpr int kPfThreads = 512;   // 8 waves: wave w takes head 2g + w / 4 and query tokens 32 (w % 4) .. + 31
// Row strides: a 16-byte LDS read by 16 lanes of consecutive rows is conflict-free on gfx950 when the
// stride in dwords is 8 mod 16 (measured: 80, 112, 144 halfs conflict-free; 72, 88, 96, 136 halfs
// lose ~half the LDS cycles to bank conflicts).
constexpr int kKS = 144;    // K tile row stride (halfs): 128 dims + 16
constexpr int kVS = 80;     // V^T tile row stride (halfs): 64 keys + 16
constexpr float kLog2e = 1.4426950408889634f;
// Work plan.  Query tile qt attends key tiles [0, n_kt(qt)).  A tile with more than cap =
// ceil(n_kt_last / 2) key tiles is cut at key tile cap into two parts; every part (or uncut tile) is
// one work item.  Items are pulled from a queue per KV head by a grid that fits on the GPU at once, in
// about descending order of size (see item_of), so that every CU stays busy until the end: a grid of
// one workgroup per query tile lasts as long as the longest tile, about twice the average.
// Workspace: a fixed region (queue and merge counters) first, so that calls of any shape can share one
// workspace, then the statistics of every item and the partial outputs of the cut tiles.
constexpr int kPfCounterStride = 64;    // uint32 (256 bytes) per counter
constexpr int kPfMaxHeads = 8;          // KV heads (one queue each per pass)
constexpr int kPfMaxMerge = 8192;       // merge counters: one per (KV head, query tile)
constexpr int kPfCutUnits = 2048;       // (KV head, query tile) units up to which long tiles are cut
constexpr size_t kPfQueueBytes = 2 * kPfMaxHeads * kPfCounterStride * sizeof(uint32_t);
constexpr size_t kPfFixedBytes = kPfQueueBytes + static_cast<size_t>(kPfMaxMerge) * kPfCounterStride * sizeof(uint32_t);
constexpr size_t kPfOFloats = kQB * 8 * kPfThreads * 4;           // one part's O: 16 float4 per thread
// one part's O, then (single pass) each thread's running max and sum of its two query columns: a float pair
// (m, pad) and a double per block, 4 uint64 per thread
constexpr size_t kPfPartialFloats = kPfOFloats + kPfThreads * 8;

struct alignas(16) PrefillStat {
    float m;
    float pad;
    double s;
};

struct MfmaParams {
    const float * q;          // [T][q_stride], token t of the call
    const _Float16 * k;       // this layer/stream's K rows, head 0 position 0
    const _Float16 * v;
    float * out;              // [T][q_stride]
    int64_t head_stride;      // elements between KV heads (max_seq * 128)
    int32_t q_stride;
    int32_t n_past, n_tokens, n_kv, n_qt;
    int32_t cap;              // key tiles of the first part of a cut query tile
    int32_t qt_cut;           // first cut query tile (n_kt > cap); n_qt when none is cut
    int32_t n_items;          // work items per KV head: n_qt + (n_qt - qt_cut)
    float scale;
    uint32_t * queue;         // pull counters of this pass, one per KV head (every call leaves them zero)
    PrefillStat * stats;      // [n_kv][n_qt][2 parts][kCols columns]
    float * partial;          // [n_kv][n_qt - qt_cut][2 parts][kPfPartialFloats]
    uint32_t * counters;      // [n_kv][n_qt - qt_cut][kPfCounterStride]
};

__device__ inline uint64_t pack2(float a, float b) {
    return static_cast<uint64_t>(__float_as_uint(a)) | (static_cast<uint64_t>(__float_as_uint(b)) << 32);
}
__device__ inline float lo_float(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v)); }
__device__ inline float hi_float(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v >> 32)); }

// Global -> register staging of one tile by the 512 threads.  K: thread t loads 16-byte slices idx =
// it * 512 + t (row idx / 16, slice idx % 16).  V: thread t loads dims 8 dg .. 8 dg + 7 (dg = t / 32) of
// the key pair 2 kp, 2 kp + 1 (kp = t % 32), which it writes transposed.  Rows past the end re-read the
// last row (masked keys get p = 0; no branch splits the loads).
struct TileRegs {
    u4 k[2];
    u4 v[2];
};

__device__ inline void load_tile(const _Float16 * kh, const _Float16 * vh, int kt, int kend, bool with_v,
                                 TileRegs & r) {
    const int t = threadIdx.x;
    const int kp = t & 31, dg = t >> 5;
    const int row0 = kt * kBK;
    if (row0 + kBK <= kend) {
        // whole tile: a uniform tile base and fixed per-thread offsets (scalar base + 32-bit vector
        // offset addressing, no per-load address arithmetic)
        const _Float16 * kb = kh + static_cast<int64_t>(row0) * kHeadDim;
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            r.k[it] = *reinterpret_cast<const u4 *>(kb + (it * 32 + (t >> 4)) * kHeadDim + (t & 15) * 8);
        }
        if (!with_v) return;
        const _Float16 * vb = vh + static_cast<int64_t>(row0) * kHeadDim;
#pragma unroll
        for (int e = 0; e < 2; ++e) r.v[e] = *reinterpret_cast<const u4 *>(vb + (kp * 2 + e) * kHeadDim + dg * 8);
        return;
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int idx = it * kPfThreads + t;
        const int row = min(row0 + (idx >> 4), kend - 1);
        r.k[it] = *reinterpret_cast<const u4 *>(kh + static_cast<int64_t>(row) * kHeadDim + (idx & 15) * 8);
    }
    if (!with_v) return;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int row = min(row0 + kp * 2 + e, kend - 1);
        r.v[e] = *reinterpret_cast<const u4 *>(vh + static_cast<int64_t>(row) * kHeadDim + dg * 8);
    }
}

// (a.lo, b.lo) and (a.hi, b.hi) half pairs: one v_perm_b32 each (selector bytes 0-3 pick from the
// second operand, 4-7 from the first)
__device__ inline uint32_t lo_pair(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ inline uint32_t hi_pair(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

__device__ inline void store_tile(const TileRegs & r, _Float16 * sK, _Float16 * sV, bool with_v) {
    const int t = threadIdx.x;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int idx = it * kPfThreads + t;
        *reinterpret_cast<u4 *>(sK + (idx >> 4) * kKS + (idx & 15) * 8) = r.k[it];
    }
    if (!with_v) return;
    const int kp = t & 31, dg = t >> 5;
    // V^T columns are keys in PV order: key j sits at column (j / 32) * 32 + ((j % 16) / 4) * 8 +
    // ((j / 16) % 2) * 4 + j % 4, so the 8 keys one lane multiplies in a 32-key step (4 from each 16-key
    // block) are 8 consecutive halfs: one 16-byte read.  Keys 2 kp and 2 kp + 1 stay adjacent.
    const int j = 2 * kp;
    const int col = (j >> 5) * 32 + ((j & 15) >> 2) * 8 + ((j >> 4) & 1) * 4 + (j & 3);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        // dims 2w and 2w + 1 of the slice, keys 2 kp and 2 kp + 1
        *reinterpret_cast<uint32_t *>(sV + (dg * 8 + 2 * w) * kVS + col) = lo_pair(r.v[0][w], r.v[1][w]);
        *reinterpret_cast<uint32_t *>(sV + (dg * 8 + 2 * w + 1) * kVS + col) = hi_pair(r.v[0][w], r.v[1][w]);
    }
}

// S^T tiles of this wave: S[qb][kb] = 16 keys (kb) x the 16 queries of block qb; each K fragment is
// read once for both blocks.
__device__ inline void scores_tile(const _Float16 * sK, const h8 (&qf)[kQB][4], int c16, int g4, f4 (&S)[kQB][4]) {
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) S[qb][kb] = f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const h8 a = *reinterpret_cast<const h8 *>(sK + (kb * 16 + c16) * kKS + ks * 32 + g4 * 8);
#pragma unroll
            for (int qb = 0; qb < kQB; ++qb) {
                S[qb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[qb][ks], S[qb][kb], 0, 0, 0);
            }
        }
    }
}

// Masks the keys of a diagonal tile: key j of this lane's query column is attended iff j <= lim.
__device__ inline void mask_tile(f4 (&S)[4], int lim, int kt, int g4) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = kt * kBK + kb * 16 + g4 * 4 + i;
            if (j > lim) S[kb][i] = -INFINITY;
        }
    }
}

// Pass-1 update of one lane's running max m (raw score units) and double sum of exp(s - m).
__device__ inline void stats_update(const f4 (&S)[4], float c, float & m, double & sum) {
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, S[kb][i]);
    }
    const float mn = fmaxf(m, tmax);
    if (mn == -INFINITY) return;                 // every key so far masked for this lane
    const float mc = mn * c;
    float part = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) part += __builtin_amdgcn_exp2f(fmaf(S[kb][i], c, -mc));
    }
    // exp2(-inf) = 0 when the lane had nothing before this tile
    const float f = __builtin_amdgcn_exp2f(fmaf(m, c, -mc));
    sum = sum * static_cast<double>(f) + static_cast<double>(part);
    m = mn;
}

// O^T += V^T P^T for the P^T fragments pf[qb][ksv] (element e <-> key (2 ksv + e / 4) * 16 + g4 * 4 + e % 4 of
// the tile).  Each V^T fragment is read once for both blocks.
__device__ inline void pv_frags(const h8 (&pf)[kQB][2], const _Float16 * sV, int c16, int g4, f4 (&O)[kQB][8]) {
#pragma unroll
    for (int ksv = 0; ksv < 2; ++ksv) {
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const h8 a = *reinterpret_cast<const h8 *>(sV + (db * 16 + c16) * kVS + ksv * 32 + g4 * 8);
#pragma unroll
            for (int qb = 0; qb < kQB; ++qb) {
                O[qb][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pf[qb][ksv], O[qb][db], 0, 0, 0);
            }
        }
    }
}

// mc[qb] = (M scale - log2 S) log2 e for this lane's query column of block qb: p = exp2(s c - mc) =
// exp(s scale - M) / S.
__device__ inline void pv_tile(const f4 (&S)[kQB][4], const _Float16 * sV, const float (&mc)[kQB], float c, int c16,
                               int g4, f4 (&O)[kQB][8]) {
    h8 pf[kQB][2];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pf[qb][kb >> 1][(kb & 1) * 4 + i] =
                    static_cast<_Float16>(__builtin_amdgcn_exp2f(fmaf(S[qb][kb][i], c, -mc[qb])));
            }
        }
    }
    pv_frags(pf, sV, c16, g4, O);
}

// Rescale threshold of the single pass, in log2 units of the exponentials: a column's reference max is moved
// up only when the tile's max exceeds it by more than this, so the exponentials stay below 2^8 (f16 holds
// them with room) and the O accumulators are rescaled only when some column's max grows that much.
constexpr float kLazyLog2 = 8.0f;

// Single-pass (online softmax) update of one key tile: m[qb] is the reference max of this lane's query column
// (raw score units, -inf while no key is attended), l[qb] the sum of exp(s - m) over the keys this lane
// holds; e = exp(s - m) is rounded to f16 for the PV MFMA.
__device__ inline void online_tile(const f4 (&S)[kQB][4], const _Float16 * sV, float c, int c16, int g4,
                                   float (&m)[kQB], double (&l)[kQB], f4 (&O)[kQB][8]) {
    float mn[kQB];
    bool up[kQB];
    bool any = false;
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        float t = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) t = fmaxf(t, S[qb][kb][i]);
        }
        // the column's 64 keys are held by lanes c16 + 16 g4, g4 = 0..3
        t = fmaxf(t, __shfl_xor(t, 16, kWave));
        t = fmaxf(t, __shfl_xor(t, 32, kWave));
        mn[qb] = fmaxf(m[qb], t);
        // -inf -> finite compares as +inf > threshold; -inf -> -inf gives NaN, which is no move
        up[qb] = (mn[qb] - m[qb]) * c > kLazyLog2;
        any = any || up[qb];
    }
    if (__any(any)) {
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
            // lanes whose column keeps its max multiply by 1
            const float f = up[qb] ? __builtin_amdgcn_exp2f((m[qb] - mn[qb]) * c) : 1.0f;
#pragma unroll
            for (int db = 0; db < 8; ++db) O[qb][db] *= f;
            l[qb] *= static_cast<double>(f);
            if (up[qb]) m[qb] = mn[qb];
        }
    }
    h8 pf[kQB][2];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        const float mc = m[qb] == -INFINITY ? INFINITY : m[qb] * c;   // nothing attended yet: every e is 0
        float part = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = __builtin_amdgcn_exp2f(fmaf(S[qb][kb][i], c, -mc));
                part += e;
                pf[qb][kb >> 1][(kb & 1) * 4 + i] = static_cast<_Float16>(e);
            }
        }
        l[qb] += static_cast<double>(part);
    }
    pv_frags(pf, sV, c16, g4, O);
}

// One work item: KV head g, part j of query tile qt, key tiles [kt0, kt1); cut says whether qt has
// two parts.  Item order per head (k = 0, 1, ...): first the first parts of the cut tiles (cap key
// tiles each, longest query tile first), then the uncut tiles and the second parts alternately, both
// in descending order of size: about the order a longest-first scheduler would pick.
struct Item {
    int g, qt, j, kt0, kt1, n_kt;
    bool cut;
};

__device__ inline Item item_of(const MfmaParams & p, int g, int k) {
    Item it;
    it.g = g;
    const int n_cut = p.n_qt - p.qt_cut;          // cut tiles = second parts
    const int n_whole = p.qt_cut;                  // uncut tiles
    if (k < n_cut) {
        it.qt = p.n_qt - 1 - k;
        it.j = 0;
    } else {
        const int m = k - n_cut;
        const int both = 2 * min(n_cut, n_whole);
        int i;
        bool second;
        if (m < both) {
            i = m >> 1;
            second = (m & 1) != 0;
        } else {
            i = m - both + min(n_cut, n_whole);
            second = n_cut > n_whole;
        }
        it.qt = second ? p.n_qt - 1 - i : p.qt_cut - 1 - i;
        it.j = second ? 1 : 0;
    }
    const int t0 = it.qt * kBQ;
    it.n_kt = (min(p.n_past + p.n_tokens, p.n_past + min(t0 + kBQ, p.n_tokens)) + kBK - 1) / kBK;
    it.cut = it.qt >= p.qt_cut;
    it.kt0 = it.j == 0 ? 0 : p.cap;
    it.kt1 = it.cut && it.j == 0 ? p.cap : it.n_kt;
    return it;
}

// One work item.  PASS 1: the part's row statistics (max and sum of exp) of its kCols query columns.
// PASS 2: p over the part's keys with the statistics of both parts of its query tile, and
// O^T += V^T P^T; the two parts of a cut tile are added by whichever finishes second.
// PASS 3 (single pass): online softmax over the part's keys (online_tile); the part's O, max and sum are
// combined with the other part's by whichever finishes second, then O / sum is stored.
template <int PASS>
__device__ inline void run_item(const MfmaParams & p, const Item & it, _Float16 (*sK)[kBK * kKS],
                                _Float16 (*sV)[kHeadDim * kVS]) {
    constexpr bool kWithV = PASS != 1;
    const int g = it.g;
    const int t0 = it.qt * kBQ;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int hh = wave >> 2;
    const int h = g * 2 + hh;
    const int c16 = lane & 15;
    const int g4 = lane >> 4;
    const int L_total = p.n_past + p.n_tokens;
    const int kend = min(L_total, p.n_past + min(t0 + kBQ, p.n_tokens));
    // tiles below kt_full hold only keys <= n_past + t0, attended by every query of the workgroup
    const int kt_full = min((p.n_past + t0 + 1) / kBK, it.n_kt);
    const _Float16 * kh = p.k + g * p.head_stride;
    const _Float16 * vh = p.v + g * p.head_stride;
    const float c = p.scale * kLog2e;

    // this lane's query column of block qb and its causal key limit (keys j <= lim are attended)
    int tq[kQB], lim[kQB], col[kQB];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        tq[qb] = t0 + (wave & 3) * 32 + qb * 16 + c16;
        lim[qb] = tq[qb] < p.n_tokens ? p.n_past + tq[qb] : -1;
        col[qb] = hh * kBQ + (wave & 3) * 32 + qb * 16 + c16;   // statistics column
    }
    // statistics of part j of this query tile: [g][qt][j][column]
    PrefillStat * st = p.stats + (static_cast<int64_t>(g) * p.n_qt + it.qt) * 2 * kCols;

    // Q fragments, the B operand of S^T: lane holds query column c16 of each block and 8 dims of each
    // 32-dim step, rounded to f16 (GGML's conversion of src1 for an f16 src0); absent tokens are zero
    h8 qf[kQB][4];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        const int tqc = min(tq[qb], p.n_tokens - 1);
        const bool ok = tq[qb] < p.n_tokens;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const float * qp = p.q + static_cast<int64_t>(tqc) * p.q_stride + h * kHeadDim + ks * 32 + g4 * 8;
            const float4 a = *reinterpret_cast<const float4 *>(qp);
            const float4 b = *reinterpret_cast<const float4 *>(qp + 4);
            qf[qb][ks] = h8{static_cast<_Float16>(ok ? a.x : 0.f), static_cast<_Float16>(ok ? a.y : 0.f),
                            static_cast<_Float16>(ok ? a.z : 0.f), static_cast<_Float16>(ok ? a.w : 0.f),
                            static_cast<_Float16>(ok ? b.x : 0.f), static_cast<_Float16>(ok ? b.y : 0.f),
                            static_cast<_Float16>(ok ? b.z : 0.f), static_cast<_Float16>(ok ? b.w : 0.f)};
        }
    }

    float mc[kQB];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) mc[qb] = 0.f;
    if constexpr (PASS == 2) {
        // row max M and sum S over the parts: S = s_0 exp(m_0 - M) + s_1 exp(m_1 - M), in double; the
        // normalisation 1 / S folded into the exponent: exp2(s c - M c - log2 S); a column without keys
        // (padding) gets an exponent of -inf, so p = 0
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
            const PrefillStat a = st[col[qb]];
            PrefillStat b{-INFINITY, 0.f, 0.0};
            if (it.cut) b = st[kCols + col[qb]];
            const float M = fmaxf(a.m, b.m);
            double S = 0.0;
            if (M != -INFINITY) {
                S = a.s * static_cast<double>(__builtin_amdgcn_exp2f((a.m - M) * c));
                if (it.cut) S += b.s * static_cast<double>(__builtin_amdgcn_exp2f((b.m - M) * c));
            }
            mc[qb] = M == -INFINITY || !(S > 0.0) ? INFINITY
                                                  : static_cast<float>(static_cast<double>(M * c) + std::log2(S));
        }
    }

    float m[kQB];
    double sum[kQB];
    f4 O[kQB][8];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        m[qb] = -INFINITY;
        sum[qb] = 0.0;
#pragma unroll
        for (int db = 0; db < 8; ++db) O[qb][db] = f4{0.f, 0.f, 0.f, 0.f};
    }
    TileRegs regs;
    const int kt0 = it.kt0, kt1 = it.kt1;
    load_tile(kh, vh, kt0, kend, kWithV, regs);
    store_tile(regs, sK[0], sV[0], kWithV);
    if (kt0 + 1 < kt1) load_tile(kh, vh, kt0 + 1, kend, kWithV, regs);
    __syncthreads();
    auto step = [&](int kt, auto mask) {
        const int b = (kt - kt0) & 1;
        f4 S[kQB][4];
        scores_tile(sK[b], qf, c16, g4, S);
        if constexpr (decltype(mask)::value) {
#pragma unroll
            for (int qb = 0; qb < kQB; ++qb) mask_tile(S[qb], lim[qb], kt, g4);
        }
        if constexpr (PASS == 1) {
#pragma unroll
            for (int qb = 0; qb < kQB; ++qb) stats_update(S[qb], c, m[qb], sum[qb]);
        } else if constexpr (PASS == 2) {
            pv_tile(S, sV[b], mc, c, c16, g4, O);
        } else {
            online_tile(S, sV[b], c, c16, g4, m, sum, O);
        }
        if (kt + 1 < kt1) {
            store_tile(regs, sK[b ^ 1], sV[PASS != 1 ? (b ^ 1) : 0], kWithV);
            if (kt + 2 < kt1) load_tile(kh, vh, kt + 2, kend, kWithV, regs);
        }
        __syncthreads();
    };
    auto run = [&](int kt, auto mask) { step(kt, mask); };
    int kt = kt0;
    for (; kt < min(kt1, kt_full); ++kt) run(kt, std::false_type{});
    for (; kt < kt1; ++kt) run(kt, std::true_type{});

    if constexpr (PASS == 1) {
        // combine the 4 lanes of each query column (lane bits 4, 5) and store the part's statistics
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
            float M = fmaxf(m[qb], __shfl_xor(m[qb], 16, kWave));
            M = fmaxf(M, __shfl_xor(M, 32, kWave));
            double sm = M == -INFINITY ? 0.0 : sum[qb] * static_cast<double>(__builtin_amdgcn_exp2f((m[qb] - M) * c));
            sm += __shfl_xor(sm, 16, kWave);
            sm += __shfl_xor(sm, 32, kWave);
            if (g4 == 0) st[it.j * kCols + col[qb]] = PrefillStat{M, 0.0f, sm};
        }
        return;
    }

    // PASS 3: the column's sum over the 4 lanes that hold its keys (fixed order; every lane gets the same value)
    double lt[kQB];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        lt[qb] = sum[qb];
        if constexpr (PASS == 3) {
            lt[qb] += __shfl_xor(lt[qb], 16, kWave);
            lt[qb] += __shfl_xor(lt[qb], 32, kWave);
        }
    }
    if (it.cut) {
        // Publish this part's O (thread-major: element e of every thread is 512 consecutive float4; with a single
        // pass also the max and sum of the thread's columns), then count; the second part to arrive combines
        // both, in part order, so the result is the same whichever part arrives second.  That needs every
        // product rounded before the sum: a contracted (fused) product would be the merging part's own, and
        // the result would depend on which part arrived second (measured: runs differed in the last query tiles).
#pragma clang fp contract(off)
        const int64_t unit = static_cast<int64_t>(g) * (p.n_qt - p.qt_cut) + (it.qt - p.qt_cut);
        uint64_t * mine = reinterpret_cast<uint64_t *>(p.partial + (unit * 2 + it.j) * kPfPartialFloats);
        const uint64_t * other = reinterpret_cast<const uint64_t *>(p.partial + (unit * 2 + (it.j ^ 1)) * kPfPartialFloats);
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                const int e = ((qb * 8 + db) * kPfThreads + static_cast<int>(threadIdx.x)) * 2;
                __hip_atomic_store(mine + e, pack2(O[qb][db][0], O[qb][db][1]), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(mine + e + 1, pack2(O[qb][db][2], O[qb][db][3]), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        constexpr int kStatOff = static_cast<int>(kPfOFloats / 2);    // uint64 offset of the (m, sum) entries
        if constexpr (PASS == 3) {
#pragma unroll
            for (int qb = 0; qb < kQB; ++qb) {
                const int e = kStatOff + static_cast<int>(threadIdx.x) * 4 + 2 * qb;
                __hip_atomic_store(mine + e, pack2(m[qb], 0.0f), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(mine + e + 1, static_cast<uint64_t>(__double_as_longlong(lt[qb])), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        __shared__ int s_last;
        if (threadIdx.x == 0) {
            uint32_t * ctr = p.counters + unit * kPfCounterStride;
            const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = prev == 1u;
            if (s_last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!s_last) return;
        // factors of this part (fm) and the other (fo) in the combined state (PASS 3; 1 for PASS 2)
        float fm[kQB], fo[kQB];
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
            fm[qb] = 1.0f;
            fo[qb] = 1.0f;
            if constexpr (PASS == 3) {
                const int e = kStatOff + static_cast<int>(threadIdx.x) * 4 + 2 * qb;
                const float mo = lo_float(__hip_atomic_load(other + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                const double lo = __longlong_as_double(static_cast<long long>(
                    __hip_atomic_load(other + e + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)));
                const float M = fmaxf(m[qb], mo);
                fm[qb] = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m[qb] - M) * c);
                fo[qb] = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((mo - M) * c);
                const double a = lt[qb] * static_cast<double>(fm[qb]), b = lo * static_cast<double>(fo[qb]);
                lt[qb] = it.j == 0 ? a + b : b + a;
            }
        }
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                const int e = ((qb * 8 + db) * kPfThreads + static_cast<int>(threadIdx.x)) * 2;
                const uint64_t lo = __hip_atomic_load(other + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint64_t hi = __hip_atomic_load(other + e + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const f4 ov = f4{lo_float(lo), hi_float(lo), lo_float(hi), hi_float(hi)} * fo[qb];
                const f4 mv = O[qb][db] * fm[qb];
                O[qb][db] = it.j == 0 ? mv + ov : ov + mv;
            }
        }
    }
    if constexpr (PASS == 3) {
        // O / sum, with the sum's reciprocal in f32 (the reference's soft_max multiplies by 1 / sum)
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
            const float r = lt[qb] > 0.0 ? static_cast<float>(1.0 / lt[qb]) : 0.0f;
#pragma unroll
            for (int db = 0; db < 8; ++db) O[qb][db] *= r;
        }
    }

    // O^T: lane holds dims db * 16 + g4 * 4 + i of its query column of each block
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        if (tq[qb] < p.n_tokens) {
            float * op = p.out + static_cast<int64_t>(tq[qb]) * p.q_stride + h * kHeadDim + g4 * 4;
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                *reinterpret_cast<float4 *>(op + db * 16) =
                    make_float4(O[qb][db][0], O[qb][db][1], O[qb][db][2], O[qb][db][3]);
            }
        }
    }
}

// A grid of at most the workgroups that fit on the GPU pulls items until the queues are empty.
// Workgroup b serves KV head b % n_kv and pulls that head's items from the head's own queue: the
// workgroups are dispatched round-robin over the 8 XCDs, so with 8 KV heads every XCD works on one
// head, whose K/V (2 MB at 4k positions) then stays in that XCD's L2.  Each workgroup makes exactly one
// pull past the end of its queue; the last of those resets the counter to zero for the next call.
// Pass 1 holds no V tile and no O: 128 registers give two workgroups per CU.
template <int PASS>
__global__ __launch_bounds__(kPfThreads, 2) void prefill_mfma_kernel(MfmaParams p) {
    __shared__ __attribute__((aligned(16))) _Float16 sK[2][kBK * kKS];
    __shared__ __attribute__((aligned(16))) _Float16 sV[PASS != 1 ? 2 : 1][PASS != 1 ? kHeadDim * kVS : 8];
    __shared__ int s_pull;
    const int g = static_cast<int>(blockIdx.x) % p.n_kv;
    // workgroups serving head g, hence pulls past the end of its queue
    const int n_wg = (static_cast<int>(gridDim.x) - g + p.n_kv - 1) / p.n_kv;
    uint32_t * queue = p.queue + g * kPfCounterStride;
    for (;;) {
        if (threadIdx.x == 0) s_pull = static_cast<int>(__hip_atomic_fetch_add(queue, 1u, __ATOMIC_RELAXED,
                                                                                 __HIP_MEMORY_SCOPE_AGENT));
        __syncthreads();
        const int k = s_pull;
        __syncthreads();
        if (k >= p.n_items) {
            if (threadIdx.x == 0 && k == p.n_items + n_wg - 1) {
                __hip_atomic_store(queue, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return;
        }
        run_item<PASS>(p, item_of(p, g, k), sK, reinterpret_cast<_Float16 (*)[kHeadDim * kVS]>(sV));
    }
}

}  // namespace

// QA_PREFILL_EXACT=1: the two-pass kernels, which round the normalised probabilities to f16 before PV as
// the reference's GGML graph does (soft_max_ext, then mul_mat converting p to the f16 dot type of V).  The
// default single pass rounds exp(s - m) to f16 instead and divides by the sum at the end: same f32
// accumulation, another rounding point of p, attention outputs within 1.2e-4 of the oracle at T = 3913.
bool prefill_exact() {
    static const bool v = [] {
        const char * e = std::getenv("QA_PREFILL_EXACT");
        return e && std::strcmp(e, "1") == 0;
    }();
    return v;
}

// Workgroups of one pass that fit on the device at once (the size of the pulling grid).
template <int PASS>
int resident_grid() {
    static const int n = [] {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, prefill_mfma_kernel<PASS>, kPfThreads, 0) != hipSuccess) {
            return 512;
        }
        return std::max(1, cus * std::max(1, per_cu));
    }();
    return n;
}

// Workspace: the fixed region (queue and merge counters), then the statistics of two parts per
// (KV head, query tile), then (grids of at most kPfCutUnits units) two partial outputs per unit.
size_t prefill_mfma_workspace_bytes(int32_t n_tokens, int32_t n_kv) {
    if (n_tokens <= 0 || n_kv <= 0) return 256;
    const int64_t units = (static_cast<int64_t>(n_tokens) + kBQ - 1) / kBQ * n_kv;
    return kPfFixedBytes + static_cast<size_t>(units) * 2 * kCols * sizeof(PrefillStat) +
           (units <= kPfCutUnits ? static_cast<size_t>(units) * 2 * kPfPartialFloats * sizeof(float) : 0);
}

int prefill_mfma_launch(const float * q, int32_t q_stride, const void * k, const void * v, int64_t head_stride,
                        int32_t n_past, int32_t n_tokens, int32_t n_kv, float scale, float * out, void * workspace,
                        size_t workspace_bytes, hipStream_t stream) {
    MfmaParams p{};
    p.q = q;
    p.k = static_cast<const _Float16 *>(k);
    p.v = static_cast<const _Float16 *>(v);
    p.out = out;
    p.head_stride = head_stride;
    p.q_stride = q_stride;
    p.n_past = n_past;
    p.n_tokens = n_tokens;
    p.n_kv = n_kv;
    p.n_qt = (n_tokens + kBQ - 1) / kBQ;
    p.scale = scale;
    if (static_cast<int64_t>(p.n_qt) * n_kv <= 0) return QA_OK;
    if (n_kv > kPfMaxHeads) return fail(QA_ERR_INVALID, "prefill attention: more than 8 KV heads");
    // Cut the tiles with more than ceil(n_kt_last / 2) key tiles in two when the grid is small enough for
    // the longest tiles to set the duration (larger grids balance themselves through the queue) and the
    // workspace holds the partial outputs; otherwise every tile is one item.
    const int n_kt_last = (n_past + n_tokens + kBK - 1) / kBK;
    const int64_t units = static_cast<int64_t>(p.n_qt) * n_kv;
    const size_t stats_bytes = static_cast<size_t>(units) * 2 * kCols * sizeof(PrefillStat);
    if (!workspace || workspace_bytes < kPfFixedBytes + stats_bytes) {
        return fail(QA_ERR_INVALID, "prefill attention: workspace too small (qa_prefill_attn_workspace_bytes)");
    }
    const bool can_cut = units <= kPfCutUnits && n_kt_last >= 2 &&
                         workspace_bytes >= prefill_mfma_workspace_bytes(n_tokens, n_kv);
    p.cap = can_cut ? (n_kt_last + 1) / 2 : n_kt_last;
    int qt = 0;
    while (qt < p.n_qt && (n_past + std::min((qt + 1) * kBQ, n_tokens) + kBK - 1) / kBK <= p.cap) ++qt;
    p.qt_cut = qt;
    p.n_items = p.n_qt + (p.n_qt - p.qt_cut);
    char * base = static_cast<char *>(workspace);
    p.counters = reinterpret_cast<uint32_t *>(base + kPfQueueBytes);
    p.stats = reinterpret_cast<PrefillStat *>(base + kPfFixedBytes);
    p.partial = reinterpret_cast<float *>(base + kPfFixedBytes + stats_bytes);
    // grids: whole multiples of n_kv (every head gets as many workgroups), at most one per item
    const int64_t total = static_cast<int64_t>(p.n_items) * n_kv;
    auto grid_of = [&](int resident) {
        const int64_t gsz = std::max<int64_t>(n_kv, resident / n_kv * n_kv);
        return dim3(static_cast<unsigned>(std::min(total, gsz)));
    };
    p.queue = reinterpret_cast<uint32_t *>(base);
    if (!prefill_exact()) {
        hipLaunchKernelGGL(prefill_mfma_kernel<3>, grid_of(resident_grid<3>()), dim3(kPfThreads), 0, stream, p);
        QA_LAUNCH_CHECK("prefill_mfma_kernel<3>");
        return QA_OK;
    }
    hipLaunchKernelGGL(prefill_mfma_kernel<1>, grid_of(resident_grid<1>()), dim3(kPfThreads), 0, stream, p);
    QA_LAUNCH_CHECK("prefill_mfma_kernel<1>");
    p.queue = reinterpret_cast<uint32_t *>(base) + kPfMaxHeads * kPfCounterStride;
    hipLaunchKernelGGL(prefill_mfma_kernel<2>, grid_of(resident_grid<2>()), dim3(kPfThreads), 0, stream, p);
    QA_LAUNCH_CHECK("prefill_mfma_kernel<2>");
    return QA_OK;
}

}  // namespace qa
