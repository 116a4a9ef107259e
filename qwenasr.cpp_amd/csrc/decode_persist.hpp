// Persistent decode step at batch 1: every layer of one token in a single launch.  The kernel, its barrier and
// the per-unit instantiation machinery; the units are decode_persist_h*.hip, the host side decode_persist.hip.
//
// The reference rebuilds and re-schedules its GGML graph for every token (text-decoder.cpp:1658-1739).
// The eager step of this library already replaces that with a fixed sequence of launches driven by
// device-side lengths (six per layer).  This kernel replaces the sequence itself: one launch of G resident
// workgroups walks the 28 layers, each layer in six phases separated by grid barriers:
//   q|k|v GEMV (RMSNorm input) -> scores (append + q/k prep) -> values (+ merge) -> o GEMV (+ residual)
//   -> gate|up GEMV (RMSNorm input, SwiGLU) -> down GEMV (+ residual).
// Each phase runs the eager kernel's device function (gemv_body.hpp, decode_attn_body.hpp) over the same
// virtual grid, so the results are bit-identical to the eager step; the LM head and the pick stay
// separate launches.  The attended length comes from the device length array, as in the eager step.
//
// Coherence.  Phases hand activations (x, q|k|v, scores, statistics, attention output, SwiGLU output)
// to workgroups on other XCDs whose L2s are not coherent with the writer's.  Producers store them with
// write-through agent-scope stores and wait for the acknowledgements before the barrier (coherent.hpp),
// and every address is written at most once per launch and read only after that write (each layer has
// its own buffers; the residual GEMVs read the old x from one buffer and write the new x to the next), so
// no cache holds a stale copy when a consumer reads it with plain loads.  The launch's input row, d->x,
// is read by layer 0 only and written by the last layer only, for the LM head's launch.  The new K/V row
// (written once, by the owner of its position) follows the same rule; weights are read-only.
//
// Barrier.  Two levels of arrival counters, each on its own 256-byte line (device-scope atomics on one
// line are serialised): groups of kGroup workgroups, then the group leaders.  Counters only grow; with a
// fixed grid per sync buffer the k-th barrier since the buffer was cleared completes at group count
// k * members and top count k * n_groups (mod 2^32).  The last arrival stores k into the release word,
// which the other workgroups poll (one lane, with a pause between polls).  Every wait is bounded: after
// wait_ticks of the 100 MHz wall clock (200 ms unless the caller sets another bound) without release the
// workgroup sets the error word and leaves, and a workgroup that sees the error word leaves at its next
// barrier, so the grid always drains.  The host reads the error word after the call, and then clears the
// sync buffer and the attention merge counters, whose state an abandoned launch leaves undefined.
//
// Grid and occupancy.  One workgroup of 4 waves per CU (one wave per SIMD, up to 512 registers): each
// GEMV phase then covers its rows in one pass, every wave issuing all its weight loads at once.  Measured
// at config 3 (MI355X): 1.740 ms per token against 1.505 ms for the eager step with f32 weights, 1.275
// against 1.065 ms with bf16 copies (ids identical); two workgroups per CU at a 256-register cap spilled
// and took 2.06 ms, and 256 workgroups with the eager rows per wave 1.78 ms.  The barrier and its
// write-through handoff cost about 1.3 us more than the kernel boundary each replaces.
#pragma once

#include "decode_attn_body.hpp"
#include "gemv_body.hpp"
#include "ops.hpp"

#include <cstddef>
#include <type_traits>

namespace qa {
namespace {


constexpr int kGroup = 16;                    // workgroups per first-level counter
constexpr int kLine = 64;                     // uint32 words per 256-byte line

// sync buffer: [n_groups lines of group counters][top][release][error]
struct SyncLayout {
    int n_groups;
    __host__ __device__ int top() const { return n_groups * kLine; }
    __host__ __device__ int release() const { return (n_groups + 1) * kLine; }
    __host__ __device__ int error() const { return (n_groups + 2) * kLine; }
    __host__ __device__ int words() const { return (n_groups + 3) * kLine; }
};

struct PersistParams {
    const PersistLayer * layers;   // device array [n_layers]
    int32_t n_layers;
    float * x;                     // [hidden]: the input row of layer 0 and the output row of the last layer
    float * xbuf;                  // [2 n_layers - 1][hidden]: x after each o and each down projection but the last
    float * qkv;                   // [n_layers][q_dim + 2 kv_dim]
    float * attn;                  // [n_layers][q_dim]
    float * act;                   // [n_layers][inter]
    size_t ws_stride;              // bytes between the layers' attention workspaces
    int32_t hidden, inter, q_dim, kv_dim;
    float eps;
    DecodeParams dp;               // attention of stream 0, layer 0's workspace (set per layer)
    int32_t n_scores_blocks, n_values_blocks;
    uint32_t * sync;
    int32_t n_groups;
    uint64_t wait_ticks;           // bound of every barrier wait, in s_memrealtime ticks (100 MHz)
};

__device__ inline uint64_t wall_ticks() { return __builtin_amdgcn_s_memrealtime(); }

// Grid barrier number `k` (absolute, counted since the sync buffer was cleared); false if the launch is
// abandoned (this workgroup timed out, or another one did).
__device__ inline bool grid_barrier(const PersistParams & P, uint32_t k) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this thread's agent-scope stores acknowledged
    __syncthreads();                                   // ... and every thread's
    __shared__ int s_ok;
    if (threadIdx.x == 0) {
        const SyncLayout sl{P.n_groups};
        const int grp = static_cast<int>(blockIdx.x) / kGroup;
        const uint32_t members = static_cast<uint32_t>(min(kGroup, static_cast<int>(gridDim.x) - grp * kGroup));
        uint32_t * sync = P.sync;
        const uint32_t prev = __hip_atomic_fetch_add(sync + grp * kLine, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == k * members - 1u) {
            const uint32_t pt = __hip_atomic_fetch_add(sync + sl.top(), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (pt == k * static_cast<uint32_t>(P.n_groups) - 1u) {
                __hip_atomic_store(sync + sl.release(), k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        int ok = 1;
        const uint64_t t0 = wall_ticks();
        for (;;) {
            const uint32_t r = __hip_atomic_load(sync + sl.release(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (static_cast<int32_t>(r - k) >= 0) break;
            if (__hip_atomic_load(sync + sl.error(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
                ok = 0;
                break;
            }
            if (wall_ticks() - t0 > P.wait_ticks) {
                __hip_atomic_store(sync + sl.error(), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        s_ok = ok;
    }
    __syncthreads();
    return s_ok != 0;
}

// HID4 = hidden / 256, QD4 = q_dim / 256 (the o projection's input), INT4 = intermediate / 256; SCH / VCH /
// SR / MB: the attention tiling the eager step picks for the cache capacity; NR*: weight rows per wave of
// each GEMV (any value gives the same sums).
template <int HID4, int QD4, int INT4, bool B16, typename CT, bool R16, int SCH, int VCH, int SR, int MB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
void decode_layers_kernel(PersistParams P, RopeTable rope) {
    // rows per wave so that one pass of 1024 waves (256 workgroups) covers each projection and every wave
    // issues all its weight loads at once: q|k|v 4096 rows, o and down `hidden` rows, gate|up `inter` row
    // pairs (two passes for f32 rows at inter 6144, for the register budget)
    constexpr int NRQ = 4, NRO = HID4 / 4 > 1 ? HID4 / 4 : 1, NRD = NRO;
    constexpr int NRGU = B16 || INT4 <= 12 ? INT4 / 4 : INT4 / 8;
    const int G = static_cast<int>(gridDim.x);
    // barriers completed since the sync buffer was cleared: every workgroup reads it before its first
    // arrival, and the first barrier of this launch cannot complete before every workgroup has arrived
    __shared__ uint32_t s_base;
    if (threadIdx.x == 0) {
        s_base = __hip_atomic_load(P.sync + SyncLayout{P.n_groups}.release(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    uint32_t k = s_base;
    const int W3 = P.q_dim + 2 * P.kv_dim;
    for (int l = 0; l < P.n_layers; ++l) {
        const PersistLayer L = P.layers[l];
        const float * x_in = l == 0 ? P.x : P.xbuf + static_cast<int64_t>(2 * l - 1) * P.hidden;
        float * x_mid = P.xbuf + static_cast<int64_t>(2 * l) * P.hidden;
        float * x_out = l + 1 == P.n_layers ? P.x : P.xbuf + static_cast<int64_t>(2 * l + 1) * P.hidden;
        float * qkv = P.qkv + static_cast<int64_t>(l) * W3;
        float * attn = P.attn + static_cast<int64_t>(l) * P.q_dim;
        float * act = P.act + static_cast<int64_t>(l) * P.inter;
        {
            const GemvParams g{L.qkv, x_in, qkv, L.attn_norm, W3, P.hidden, P.eps, nullptr};
            gemv_body<HID4, NRQ, kEpiStore, true, B16, true>(g, blockIdx.x, G);
        }
        if (!grid_barrier(P, ++k)) return;
        DecodeParams dp = P.dp;
        const size_t wo = static_cast<size_t>(l) * P.ws_stride;
        dp.layer = l;
        dp.q = qkv;
        dp.out = attn;
        dp.q_norm_w = L.q_norm;
        dp.k_norm_w = L.k_norm;
        dp.scores = reinterpret_cast<float *>(reinterpret_cast<char *>(dp.scores) + wo);
        dp.stats = reinterpret_cast<SplitStat *>(reinterpret_cast<char *>(dp.stats) + wo);
        dp.partial = reinterpret_cast<float *>(reinterpret_cast<char *>(dp.partial) + wo);
        dp.counters = reinterpret_cast<uint32_t *>(reinterpret_cast<char *>(dp.counters) + wo);
        for (int b = blockIdx.x; b < P.n_scores_blocks; b += G) {
            decode_scores_body<CT, R16, SCH, true, true>(dp, rope, b, 0);
            __syncthreads();   // the next block reuses the LDS
        }
        if (!grid_barrier(P, ++k)) return;
        for (int b = blockIdx.x; b < P.n_values_blocks; b += G) {
            decode_values_body<CT, R16, VCH, SR, MB, true>(dp, b, 0);
            __syncthreads();
        }
        if (!grid_barrier(P, ++k)) return;
        {
            const GemvParams g{L.o, attn, x_mid, nullptr, P.hidden, P.q_dim, 0.0f, x_in};
            gemv_body<QD4, NRO, kEpiAccum, false, B16, true>(g, blockIdx.x, G);
        }
        if (!grid_barrier(P, ++k)) return;
        {
            const GemvParams g{L.gu, x_mid, act, L.ffn_norm, P.inter, P.hidden, P.eps, nullptr};
            gemv_body<HID4, NRGU, kEpiSwiglu, true, B16, true>(g, blockIdx.x, G);
        }
        if (!grid_barrier(P, ++k)) return;
        {
            const GemvParams g{L.down, act, x_out, nullptr, P.hidden, P.inter, 0.0f, x_mid};
            gemv_body<INT4, NRD, kEpiAccum, false, B16, true>(g, blockIdx.x, G);
        }
        // the last phase ends with the launch; the next launch's first phase reads x after the boundary
        if (l + 1 < P.n_layers && !grid_barrier(P, ++k)) return;
    }
}

typedef void (*LayersKernel)(PersistParams, RopeTable);

struct Variant {
    int hid4, qd4, int4;
    bool b16, f16;
    int sch, vch, sr, mb;
    LayersKernel fn;
};

#define QA_PERSIST_VARIANT(H4, I4, B, F, S, V, SRV, MBV)                                                    \
    Variant{H4, 8, I4, B, F, S, V, SRV, MBV,                                                                \
            decode_layers_kernel<H4, 8, I4, B, std::conditional_t<F, _Float16, float>, F, S, V, SRV, MBV>}

// Every batch-1 tiling pick_chunks can choose (capacities 1 to 65536) for one cache dtype and weight type:
// (scores chunk, values chunk, statistics register slots, merge loads).
#define QA_PERSIST_TILINGS_F16(H4, I4, B)                                                                   \
    QA_PERSIST_VARIANT(H4, I4, B, true, 32, 32, 1, 8), QA_PERSIST_VARIANT(H4, I4, B, true, 32, 64, 1, 8),     \
        QA_PERSIST_VARIANT(H4, I4, B, true, 64, 128, 1, 8), QA_PERSIST_VARIANT(H4, I4, B, true, 128, 128, 1, 16), \
        QA_PERSIST_VARIANT(H4, I4, B, true, 144, 256, 1, 16), QA_PERSIST_VARIANT(H4, I4, B, true, 160, 256, 1, 16), \
        QA_PERSIST_VARIANT(H4, I4, B, true, 192, 256, 1, 16), QA_PERSIST_VARIANT(H4, I4, B, true, 128, 256, 1, 16), \
        QA_PERSIST_VARIANT(H4, I4, B, true, 128, 256, 2, 40), QA_PERSIST_VARIANT(H4, I4, B, true, 128, 256, 4, 40), \
        QA_PERSIST_VARIANT(H4, I4, B, true, 128, 256, 8, 40)
#define QA_PERSIST_TILINGS_F32(H4, I4, B)                                                                   \
    QA_PERSIST_VARIANT(H4, I4, B, false, 32, 32, 1, 8), QA_PERSIST_VARIANT(H4, I4, B, false, 32, 32, 1, 16),  \
        QA_PERSIST_VARIANT(H4, I4, B, false, 32, 64, 1, 16), QA_PERSIST_VARIANT(H4, I4, B, false, 64, 64, 1, 16), \
        QA_PERSIST_VARIANT(H4, I4, B, false, 64, 128, 1, 16), QA_PERSIST_VARIANT(H4, I4, B, false, 128, 128, 1, 16), \
        QA_PERSIST_VARIANT(H4, I4, B, false, 144, 256, 1, 16), QA_PERSIST_VARIANT(H4, I4, B, false, 160, 256, 1, 16), \
        QA_PERSIST_VARIANT(H4, I4, B, false, 192, 256, 1, 16), QA_PERSIST_VARIANT(H4, I4, B, false, 128, 256, 1, 16), \
        QA_PERSIST_VARIANT(H4, I4, B, false, 128, 256, 2, 40), QA_PERSIST_VARIANT(H4, I4, B, false, 128, 256, 4, 40), \
        QA_PERSIST_VARIANT(H4, I4, B, false, 128, 256, 8, 40)

// The variant of `table` for a decoder, or null.
inline const Variant * find_in(const Variant * table, size_t n, const PersistPlanIn & in) {
    if (in.hidden % 256 || in.q_dim % 256 || in.inter % 256) return nullptr;
    const Chunks ch = pick_chunks(in.layout);
    const int sr = values_stat_regs(in.layout.max_seq, ch.scores);
    const int mb = values_merge_loads(in.layout.max_seq, ch.values);
    const bool f16 = in.layout.cache_type == QA_CACHE_F16;
    for (size_t i = 0; i < n; ++i) {
        const Variant & v = table[i];
        if (v.hid4 == in.hidden / 256 && v.qd4 == in.q_dim / 256 && v.int4 == in.inter / 256 && v.b16 == in.b16 &&
            v.f16 == f16 && v.sch == ch.scores && v.vch == ch.values && v.sr == sr && v.mb == mb) {
            return &v;
        }
    }
    return nullptr;
}

inline int occupancy_of(const Variant * v, int * per_cu) {
    QA_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, reinterpret_cast<const void *>(v->fn), 256, 0));
    return QA_OK;
}

inline int launch_variant(const Variant * v, const PersistLaunch & a, hipStream_t stream) {
    if (a.grid <= 0 || a.max_len <= 0 || a.max_len > a.plan.layout.max_seq) {
        return fail(QA_ERR_INVALID, "persistent decode step: invalid grid or length");
    }
    PersistParams P{};
    P.layers = static_cast<const PersistLayer *>(a.layers);
    P.n_layers = a.n_layers;
    P.x = a.x;
    P.xbuf = a.xbuf;
    P.qkv = a.qkv;
    P.attn = a.attn;
    P.act = a.act;
    P.ws_stride = align256(workspace_layout(a.plan.layout.n_streams, a.plan.layout.n_kv_heads,
                                            a.plan.layout.max_seq).total);
    P.hidden = a.plan.hidden;
    P.inter = a.plan.inter;
    P.q_dim = a.plan.q_dim;
    P.kv_dim = a.plan.layout.n_kv_heads * kHeadDim;
    P.eps = a.eps;
    DecodeParams & p = P.dp;
    p.q = a.qkv;
    p.cache = a.cache;
    p.out = a.attn;
    p.lens = a.lens;
    p.lens_add = 1;
    p.eps = a.eps;
    p.q_stride = P.q_dim + 2 * P.kv_dim;
    p.out_stride = P.q_dim;
    p.n_heads = a.n_heads;
    p.max_len = a.max_len;
    p.scale = a.scale;
    if (a.n_heads * kHeadDim != a.plan.q_dim || a.attn_ws_bytes < P.ws_stride * static_cast<size_t>(a.n_layers) ||
        !set_workspace(p, a.plan.layout, a.attn_ws, P.ws_stride)) {
        return fail(QA_ERR_INVALID, "persistent decode step: inconsistent heads or attention workspaces too small");
    }
    p.stat_chunk = v->sch;
    P.n_scores_blocks = (a.max_len + v->sch - 1) / v->sch * p.n_kv_heads;
    P.n_values_blocks = (a.max_len + v->vch - 1) / v->vch * p.n_kv_heads;
    P.sync = a.sync;
    P.n_groups = (a.grid + kGroup - 1) / kGroup;
    P.wait_ticks = a.wait_ticks;
    RopeTable rope = make_rope_table(a.rope_theta);
    // A plain launch: the grid is one workgroup per CU and the occupancy check at enable time showed that one
    // fits, so on a device this stream has to itself every workgroup is resident from the start (a workgroup
    // kept out by other work would end the launch through the bounded waits, not hang it).  A cooperative
    // launch would guarantee residency, but after one process had made cooperative launches, another
    // process's cooperative launch failed (hipErrorIllegalState), as if the device-wide wave-sync resource
    // that cooperative launches take stayed with the first process.
    void * args[] = {&P, &rope};
    QA_HIP(hipLaunchKernel(reinterpret_cast<const void *>(v->fn), dim3(static_cast<unsigned>(a.grid)), dim3(256),
                           args, 0, stream));
    return QA_OK;
}

}  // namespace

// One translation unit per (model shape, cache dtype: F16 or F32) instantiates its kernels (11 tilings of an
// f16 cache or 13 of an f32 cache, x f32 weights and bf16 copies) and defines persist_find_NAME (QA_OK and the resident workgroups per CU if it
// holds the decoder's kernel, QA_ERR_INVALID otherwise) and persist_launch_NAME.
#define QA_PERSIST_UNIT(NAME, H4, I4, CACHE)                                                                \
    namespace {                                                                                             \
    const Variant kUnit[] = {QA_PERSIST_TILINGS_##CACHE(H4, I4, false), QA_PERSIST_TILINGS_##CACHE(H4, I4, true)}; \
    }                                                                                                       \
    int persist_find_##NAME(const PersistPlanIn & in, int * per_cu) {                                       \
        const Variant * v = find_in(kUnit, sizeof(kUnit) / sizeof(kUnit[0]), in);                           \
        if (!v) return QA_ERR_INVALID;                                                                      \
        return occupancy_of(v, per_cu);                                                                     \
    }                                                                                                       \
    int persist_launch_##NAME(const PersistLaunch & a, hipStream_t stream) {                                \
        const Variant * v = find_in(kUnit, sizeof(kUnit) / sizeof(kUnit[0]), a.plan);                       \
        if (!v) return QA_ERR_INVALID;                                                                      \
        return launch_variant(v, a, stream);                                                                \
    }

#define QA_PERSIST_UNITS(X) X(h2048_f16) X(h2048_f32) X(h1024_f16) X(h1024_f32)
#define QA_PERSIST_DECLARE(NAME)                                                                            \
    int persist_find_##NAME(const PersistPlanIn & in, int * per_cu);                                        \
    int persist_launch_##NAME(const PersistLaunch & a, hipStream_t stream);
QA_PERSIST_UNITS(QA_PERSIST_DECLARE)

}  // namespace qa
