// The rest of a Qwen3 decoder step on gfx950: f32 GEMV with fused pre-RMSNorm / residual / SwiGLU
// epilogues, row RMSNorm, SwiGLU, residual add, greedy argmax, embedding gather, length bookkeeping.
//
// These replace the GGML ops around the KV-cache path in text-decoder.cpp:365-373 and 465-493
// (linear_ggml with PREC_F32, rms_norm * w, silu * up, add, logits view) and the host argmax of
// 2266-2274.  Weights are f32 (the reference requires f32 tensors, require_f32_tensor 29-42), so a
// decode step streams every weight byte once: the GEMV is HBM-bound and is written for that --
// each wave keeps its input row in registers and walks whole weight rows with 16-byte loads.
//
// A checkpoint converted from the released bf16 weights (convert.py:386-387 widens bf16 tensors
// with tensor.float()) holds f32 values whose low 16 bits are zero.  For such weights the GEMV can
// read a bf16 copy (the high halves) and widen each value back to the same f32 in registers: the
// products and sums are the f32 kernel's, operation for operation, at half the bytes.
#include "gemv_body.hpp"
#include "ops.hpp"
#include "split3.hpp"
#include "wave.hpp"

#include <algorithm>
#include <cstdlib>
#include <cmath>

namespace qa {
namespace {

// One GEMV per launch (the body is in gemv_body.hpp, shared with the persistent decode step).
template <int IN4, int NR, int EPI, bool PRENORM, bool B16>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
    gemv_body<IN4, NR, EPI, PRENORM, B16, false>(p, blockIdx.x, gridDim.x);
}

template <int IN4, int NR, int EPI, bool PRENORM, bool B16>
int launch_gemv_t(const GemvParams & p, hipStream_t stream) {
    const int64_t waves = (static_cast<int64_t>(p.out_dim) + NR - 1) / NR;
    int64_t blocks = (waves + 3) / 4;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL((gemv_kernel<IN4, NR, EPI, PRENORM, B16>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       stream, p);
    QA_LAUNCH_CHECK("gemv_kernel");
    return QA_OK;
}

// Rows per wave: the default keeps 16-32 KB of weights in flight per wave (measured on the 1.7B decode
// step: 2 f32 rows at in_dim 2048 beat 4 by 1.6%); QA_GEMV_NR = 1, 2 or 4 overrides it (tuning).
int gemv_rows_override() {
    static const int v = [] {
        const char * e = std::getenv("QA_GEMV_NR");
        const int n = e ? std::atoi(e) : 0;
        return n == 1 || n == 2 || n == 4 ? n : 0;
    }();
    return v;
}

template <int IN4, int EPI, bool PRENORM, bool B16>
int launch_gemv_nr(int nr, const GemvParams & p, hipStream_t stream) {
    switch (nr) {
        case 1: return launch_gemv_t<IN4, 1, EPI, PRENORM, B16>(p, stream);
        case 2: return launch_gemv_t<IN4, 2, EPI, PRENORM, B16>(p, stream);
        default: return launch_gemv_t<IN4, 4, EPI, PRENORM, B16>(p, stream);
    }
}

// default rows per wave: 8-32 KB of f32 weights per wave; bf16 rows at least 2 per wave (the 1.7B
// decode step's bf16 GEMVs, traced at 1, 2 and 4 rows: 2 is fastest for every shape, by up to 20%
// over 4 for o-proj, 10% over 1 for q|k|v).  f32 rows at in_dim 2048 (the 1.7B q|k|v, o, gate|up and
// LM head): one row per wave, i.e. twice the workgroups in flight (config-3 token with f32 weights:
// 1.515-1.518 ms against 1.574-1.576 ms with 2 rows and 1.668 ms with 4).  A row's sum is the same
// whatever the rows per wave, so the results do not change.
template <int EPI, bool PRENORM, bool B16>
int launch_gemv_in(const GemvParams & p, hipStream_t stream) {
    const int forced = gemv_rows_override();
    const bool sw = EPI == kEpiSwiglu;
    auto nr = [&](int f32_rows) { return forced ? forced : B16 ? std::max(2, f32_rows) : f32_rows; };
    switch (p.in_dim) {
        case 1024: return launch_gemv_nr<4, EPI, PRENORM, B16>(nr(sw ? 2 : 4), p, stream);
        case 2048: return launch_gemv_nr<8, EPI, PRENORM, B16>(nr(B16 ? 2 : 1), p, stream);
        case 3072: return launch_gemv_nr<12, EPI, PRENORM, B16>(nr(sw ? 1 : 2), p, stream);
        case 4096: return launch_gemv_nr<16, EPI, PRENORM, B16>(nr(sw ? 1 : 2), p, stream);
        case 6144: return launch_gemv_nr<24, EPI, PRENORM, B16>(nr(1), p, stream);
        default: return fail(QA_ERR_INVALID, "gemv: in_dim must be one of 1024, 2048, 3072, 4096, 6144");
    }
}

template <int EPI, bool PRENORM>
int launch_gemv_w(const GemvParams & p, bool b16, hipStream_t stream) {
    return b16 ? launch_gemv_in<EPI, PRENORM, true>(p, stream) : launch_gemv_in<EPI, PRENORM, false>(p, stream);
}

// dst[i] = high half of src[i]; *inexact |= 1 where a low half is non-zero (src not bf16-exact)
__global__ __launch_bounds__(256) void pack_bf16_kernel(const float * src, int64_t n, uint16_t * dst,
                                                        uint32_t * inexact) {
    uint32_t bad = 0;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
        const uint32_t b = __float_as_uint(src[i]);
        bad |= b & 0xffffu;
        dst[i] = static_cast<uint16_t>(b >> 16);
    }
    if (__any(bad != 0) && (threadIdx.x & (kWave - 1)) == 0) atomicOr(inexact, 1u);
}

// ---------------------------------------------------------------- skinny GEMM (2..64 token rows)
// Y[rows][N] (+)= X[rows][K] W[N][K]^T for the multi-stream decode step (one token per stream), on
// f32 MFMA (v_mfma_f32_16x16x4_f32: exact f32 products, f32 sums, as the reference's PREC_F32 GEMM).
// The weights dominate the bytes (each W element meets every token row once), so the kernel is built
// to stream W at HBM rate:
// - a workgroup owns 64 output rows (16 per wave) over one K slice; the tile's slices are consecutive
//   workgroups, and the number of slices is chosen so that ~512 workgroups cover the matrix;
// - the X slice of every token (<= 64 KB) is staged once in LDS and read as the B operand;
// - W streams straight from HBM into the A operand: lane l reads row l % 16 of its wave's block,
//   k 4 (l / 16) + 0..3 and 16 + 4 (l / 16) + 0..3 of each 32-k step, i.e. 64 contiguous bytes per
//   row per wave instruction; the k order inside an MFMA step is a permutation shared by A and B,
//   which the sum does not see.  The B operand reads X from LDS with the same two 16-byte offsets,
//   whose 16 rows x 4 lane groups at +16 bytes are bank-conflict-free at a row stride of 8 mod 16
//   dwords (8 consecutive k per lane, +32 bytes per lane group, conflicts at every stride);
// - slices are merged by the last workgroup of each tile (agent-scope publish + counter on its own
//   cache line), in slice order, so the result does not depend on scheduling.
constexpr int kGrTile = 64;          // output rows per workgroup
constexpr int kGrMaxRows = 64;       // token rows supported
constexpr int kGrLdsBytes = 52 * 1024;  // X slice budget: 3 workgroups per CU
// X staging: every token row of the slice, 16-byte vectors over 256 threads, at most 13 per thread
static_assert(kGrLdsBytes / 16 <= 13 * 256, "X staging registers per thread");
constexpr int kGrCounterStride = 64; // uint32 per tile counter (256 bytes)
// The workspace starts with a fixed counter region for kGrMaxTiles tiles, followed by the partials:
// one layout for every shape, so calls of different shapes can share a workspace without one call's
// partials landing on another call's counters.
constexpr int kGrMaxTiles = 4096;    // N <= 262144
constexpr size_t kGrCounterBytes = static_cast<size_t>(kGrMaxTiles) * kGrCounterStride * sizeof(uint32_t);

struct GemmRowsParams {
    const float * W;          // [N][K]
    const float * X;          // [rows][K]
    float * Y;                // [rows][N]
    float * partial;          // [ks][rows][N] (ks > 1)
    uint32_t * counters;      // [tiles][kGrCounterStride]
    int32_t N, K, rows, ks, slice, accumulate;
    uint32_t x_magic;         // ceil(2^32 / (slice / 4)): X staging index / vectors per token row
    uint32_t x_magic_last;    // the same for the last slice (K - (ks - 1) slice)
    const uint16_t * W16;     // gemm_rows32_kernel: the weights as bf16 bits, read instead of W when set
    // fusions of gemm_rows32_kernel (null / 0: none)
    const float * norm_w;     // X is RMSNorm(X) * norm_w, with the row sums of squares in stats_in
    const double * stats_in;  // [n_stats_in][32]: partial sums of squares of each X row (summed in order)
    double * stats_out;       // [tiles][32]: sums of squares of each stored Y row over the tile's 32 columns
    int32_t n_stats_in, swiglu;
    float eps;
};

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

template <int TB>
__global__ __launch_bounds__(256) void gemm_rows_kernel(GemmRowsParams p) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float sX[];      // [16 TB][slice + 8]
    const int tile = static_cast<int>(blockIdx.x) / p.ks;
    const int sl = static_cast<int>(blockIdx.x) - tile * p.ks;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int k_begin = sl * p.slice;
    const int k_len = min(p.slice, p.K - k_begin);                 // multiple of 32
    const uint32_t x_magic = k_len == p.slice ? p.x_magic : p.x_magic_last;
    // LDS row stride (floats): 16-byte reads of 16 consecutive rows are conflict-free on gfx950 when the
    // stride in dwords is 8 mod 16 (slices are multiples of 32)
    const int xs = p.slice + 8;

    // W rows of this lane: row n0 + lane % 16 (clamped; rows past N are not stored)
    const int n0 = tile * kGrTile + wave * 16;
    const int nrow = min(n0 + (lane & 15), p.N - 1);
    const int g = lane >> 4;
    const float * wr = p.W + static_cast<int64_t>(nrow) * p.K + k_begin + 4 * g;

    // X slice first (at most 16 16-byte loads per thread; token rows past `rows` are zero), then the
    // first batch of W: vector loads complete in issue order, so staging X into LDS waits for X only
    // while W streams in
    // 16 TB rows x slice / 4 vectors <= 13 per thread within the LDS budget (static_assert below)
    constexpr int kXPer = 13;
    const int x_vecs = 16 * TB * (k_len / 4);
    v4f xv[kXPer];
#pragma unroll
    for (int u = 0; u < kXPer; ++u) {
        const int i = min(static_cast<int>(threadIdx.x) + 256 * u, x_vecs - 1);
        // i / cols by multiplication with ceil(2^32 / cols) (exact for i < 2^19 / cols)
        const int cols = k_len / 4;
        const int q = static_cast<int>(__umulhi(static_cast<uint32_t>(i), x_magic));
        const int t = min(q, p.rows - 1), c = i - q * cols;
        xv[u] = *reinterpret_cast<const v4f *>(p.X + static_cast<int64_t>(t) * p.K + k_begin + 4 * c);
    }
    asm volatile("" ::: "memory");
    constexpr int kB = 6;                                            // 32-k steps per batch
    const int n_steps = k_len / 32;
    v4f wa[kB][2];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
        const int st = min(u, n_steps - 1);
        wa[u][0] = *reinterpret_cast<const v4f *>(wr + 32 * st);
        wa[u][1] = *reinterpret_cast<const v4f *>(wr + 32 * st + 16);
    }
#pragma unroll
    for (int u = 0; u < kXPer; ++u) {
        const int i = static_cast<int>(threadIdx.x) + 256 * u;
        if (i < x_vecs) {
            const int t = static_cast<int>(__umulhi(static_cast<uint32_t>(i), x_magic)), c = i - t * (k_len / 4);
            *reinterpret_cast<v4f *>(sX + t * xs + 4 * c) = t < p.rows ? xv[u] : v4f{0.f, 0.f, 0.f, 0.f};
        }
    }
    __syncthreads();

    // two accumulator chains per token block (even and odd 4-k substeps), added at the end in a fixed
    // order: twice the independent MFMAs in flight
    v4f acc[TB], acc2[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) { acc[tb] = v4f{0.f, 0.f, 0.f, 0.f}; acc2[tb] = acc[tb]; }
    const float * xr = sX + (lane & 15) * xs + 4 * g;
    for (int s0 = 0; s0 < n_steps; s0 += kB) {
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            if (s0 + u < n_steps) {
                const int kk = 32 * (s0 + u);
#pragma unroll
                for (int tb = 0; tb < TB; ++tb) {
                    const v4f x0 = *reinterpret_cast<const v4f *>(xr + tb * 16 * xs + kk);
                    const v4f x1 = *reinterpret_cast<const v4f *>(xr + tb * 16 * xs + kk + 16);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        acc[tb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[u][0][j], x0[j], acc[tb], 0, 0, 0);
                        acc2[tb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[u][1][j], x1[j], acc2[tb], 0, 0, 0);
                    }
                }
            }
        }
        // slices longer than one batch (one token block only): the next batch
        if (s0 + kB < n_steps) {
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                const int st = min(s0 + kB + u, n_steps - 1);
                wa[u][0] = *reinterpret_cast<const v4f *>(wr + 32 * st);
                wa[u][1] = *reinterpret_cast<const v4f *>(wr + 32 * st + 16);
            }
        }
    }

#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[tb] += acc2[tb];
    // acc[tb][i] = sum for W row n0 + 4 g + i and token 16 tb + lane % 16
    const int nr = n0 + 4 * g;
    // the old values of this lane's outputs (accumulate): loads issued together, addresses clamped to the
    // matrix and no branch, so that they cost one round trip
    auto old_values = [&](int tb) {
        v4f o = v4f{};
        if (p.accumulate) {
            const float * y = p.Y + static_cast<int64_t>(min(16 * tb + (lane & 15), p.rows - 1)) * p.N;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = y[min(nr + i, p.N - 1)];
        }
        return o;
    };
    if (p.ks == 1) {
        v4f old[TB];
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) old[tb] = old_values(tb);
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
            const int t = 16 * tb + (lane & 15);
            if (t >= p.rows) continue;
            float * y = p.Y + static_cast<int64_t>(t) * p.N + nr;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (nr + i < p.N) y[i] = p.accumulate ? old[tb][i] + acc[tb][i] : acc[tb][i];
            }
        }
        return;
    }
    // publish this slice's partial (rows nr .. nr + 3 of a token: two 8-byte agent-scope stores; the
    // partial buffer is padded to whole 4-row groups), then the last slice of the tile merges in slice
    // order
    const int np = (p.N + 3) / 4 * 4;                                // partial row pitch
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
        const int t = 16 * tb + (lane & 15);
        if (t >= p.rows || nr >= p.N) continue;
        uint64_t * q = reinterpret_cast<uint64_t *>(p.partial + (static_cast<int64_t>(sl) * p.rows + t) * np + nr);
        const uint64_t lo = static_cast<uint64_t>(__float_as_uint(acc[tb][0])) |
                            (static_cast<uint64_t>(__float_as_uint(acc[tb][1])) << 32);
        const uint64_t hi = static_cast<uint64_t>(__float_as_uint(acc[tb][2])) |
                            (static_cast<uint64_t>(__float_as_uint(acc[tb][3])) << 32);
        __hip_atomic_store(q, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(q + 1, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ int s_last;
    if (threadIdx.x == 0) {
        uint32_t * ctr = p.counters + static_cast<int64_t>(tile) * kGrCounterStride;
        const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == static_cast<uint32_t>(p.ks - 1);
        if (s_last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
    // all loads of a group of 8 slices in flight before the sums (slice order kept)
    float sum[TB][4];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sum[tb][i] = 0.0f;
    }
    const bool live = nr < p.N;
    for (int k0 = 0; k0 < p.ks; k0 += 8) {
        uint64_t v[8][TB][2];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                const int t = min(16 * tb + (lane & 15), p.rows - 1);
                const int k = min(k0 + u, p.ks - 1);
                const uint64_t * q =
                    reinterpret_cast<const uint64_t *>(p.partial + (static_cast<int64_t>(k) * p.rows + t) * np + min(nr, np - 4));
                v[u][tb][0] = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                v[u][tb][1] = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (k0 + u >= p.ks) break;
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                sum[tb][0] += __uint_as_float(static_cast<uint32_t>(v[u][tb][0]));
                sum[tb][1] += __uint_as_float(static_cast<uint32_t>(v[u][tb][0] >> 32));
                sum[tb][2] += __uint_as_float(static_cast<uint32_t>(v[u][tb][1]));
                sum[tb][3] += __uint_as_float(static_cast<uint32_t>(v[u][tb][1] >> 32));
            }
        }
    }
    v4f old[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) old[tb] = old_values(tb);
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
        const int t = 16 * tb + (lane & 15);
        if (t >= p.rows || !live) continue;
        float * y = p.Y + static_cast<int64_t>(t) * p.N + nr;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (nr + i < p.N) y[i] = p.accumulate ? old[tb][i] + sum[tb][i] : sum[tb][i];
        }
    }
}

// ---------------------------------------------------------------- skinny GEMM, up to 32 token rows
// The multi-stream decode step (one token per stream, 32 streams) on v_mfma_f32_32x32x2_f32: a
// workgroup owns 32 weight rows over one K slice; its 4 waves take the slice's 64-k blocks in turn
// (wave w: blocks w, w + 4, ...) and are summed through LDS in wave order at the end.
// Memory access is what sets the speed here.  The MFMA operand layout puts 32 different rows on the
// lanes of one load, i.e. 32 B per weight row per instruction, and the memory system moves such
// loads at ~3 TB/s even with no arithmetic at all; 4 rows x 256 contiguous bytes per instruction
// reach ~5.4 TB/s.  So both W and X blocks (32 x 64 f32 = 8 KB each) are loaded 4 rows x 256 B per
// instruction into registers, written to a per-wave LDS block and read back in operand layout (row
// stride 68 floats: the 16-byte reads of 16 consecutive rows fall on distinct banks).  P blocks of
// loads are in flight per wave while one block is computed.
// B16: W16 holds the weights as bf16 bits (bf16-exact weights).  W is loaded 8 rows x 128 B per
// instruction and kept in LDS as bf16; the products run on v_mfma_f32_32x32x16_bf16 with each x split
// into three bf16 parts by truncation, x = hi + mid + lo exactly (hi takes the top 8 significant bits,
// mid the next 8, lo the last 8), so every weight x part product is exact in f32 and the MFMA sums them
// in f32: f32 products and f32 sums, as the f32 path, in another order (5x fewer MFMA cycles: 3 bf16
// MFMAs per 16 k against 8 f32 ones of 4x the cycles).  hi products go to one accumulator, mid and lo
// products to the other.
constexpr int kG32Rows = 32;         // weight rows per workgroup (one MFMA block)
constexpr int kG32Blk = 64;          // k per block
constexpr int kG32Ls = kG32Blk + 4;  // LDS row stride (floats)
constexpr int kG32LsB = kG32Blk + 8; // LDS row stride of bf16 weight rows (elements: 144 B, 16 B aligned)
constexpr int kG32MaxSlices = 8;     // K slices merged per tile group at most (gemm_rows_plan)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u4v __attribute__((ext_vector_type(4)));

// The high halves of two dwords packed into one (lo's high half in bits 0-15, hi's in 16-31): one
// v_perm_b32 (selector bytes 2, 3 of the second source, then 2, 3 of the first).
__device__ inline uint32_t pack_high_halves(uint32_t lo, uint32_t hi) {
    return __builtin_amdgcn_perm(hi, lo, 0x07060302u);
}

// the hi, mid, lo bf16 parts (x = hi + mid + lo exactly) of 8 floats, packed two per dword.  hi and mid
// are truncations to the top 8 significant bits; the last remainder has at most 8 significant bits, so
// its own high half is already the part (the packing keeps high halves only).
__device__ inline void split_bf16x3(const v4f a, const v4f b, u4v & hi, u4v & mid, u4v & lo) {
    float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    uint32_t h[8], m[8], l[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t u = __float_as_uint(x[e]);
        h[e] = u;
        const float r1 = x[e] - __uint_as_float(u & 0xffff0000u);
        const uint32_t v = __float_as_uint(r1);
        m[e] = v;
        l[e] = __float_as_uint(r1 - __uint_as_float(v & 0xffff0000u));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        hi[j] = pack_high_halves(h[2 * j], h[2 * j + 1]);
        mid[j] = pack_high_halves(m[2 * j], m[2 * j + 1]);
        lo[j] = pack_high_halves(l[2 * j], l[2 * j + 1]);
    }
}

// T tiles of 32 weight rows per workgroup (T = 2 with bf16 weights and more than 1024 tiles, i.e. the LM
// head): every X block is loaded, normalised and split into its three bf16 parts once for all T tiles,
// whose MFMAs then share it.
template <int P, bool B16, int T>
__global__ __launch_bounds__(256) void gemm_rows32_kernel(GemmRowsParams p) {
#pragma clang fp contract(off)
    static_assert(T == 1 || (T == 2 && B16), "two tiles per workgroup with bf16 weights only");
    // per wave: a block of f32 weight rows, or T blocks of bf16 weight rows; then reused for the cross-wave
    // sums of T accumulator sets (4 waves x 16 entries x 64 lanes x T)
    constexpr int kLw = kG32Rows * kG32Ls > T * kG32Rows * kG32LsB / 2 ? kG32Rows * kG32Ls : T * kG32Rows * kG32LsB / 2;
    static_assert(4 * kLw >= 4 * 16 * kWave * T, "LDS for the cross-wave sums");
    __shared__ __attribute__((aligned(16))) float lw[4][kLw];
    __shared__ __attribute__((aligned(16))) float lx[4][kG32Rows * kG32Ls];
    __shared__ double s_part[8][32];
    __shared__ float s_scale[32];
    __shared__ int s_last;
    const int grp = static_cast<int>(blockIdx.x) / p.ks;            // tiles T grp .. T grp + T - 1
    const int sl = static_cast<int>(blockIdx.x) - grp * p.ks;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int k_begin = sl * p.slice;
    const int k_len = min(p.slice, p.K - k_begin);                  // multiple of 64
    const int n_blk = k_len / kG32Blk;
    const int my = (n_blk - wave + 3) / 4;                          // this wave's blocks
    const int last = max(my - 1, 0);
    const bool prenorm = p.norm_w != nullptr;
    // RMSNorm input: thread (token tid % 32, part tid / 32) loads the partial sums of squares k = part,
    // part + 8, ... (at most 16: K <= 4096 with 32-column partials) before any weight load
    double sq[16];
    if (prenorm) {
        const int tk = threadIdx.x & 31, part = threadIdx.x >> 5;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int k = min(part + 8 * j, p.n_stats_in - 1);
            sq[j] = p.stats_in[32 * k + tk];
        }
    }
    // load lanes: row 4 i + lane / 16 of a block (i = 0..7), k 4 (lane % 16) .. + 3; rows past N re-read
    // the last row and tokens past `rows` the last token (neither is stored).  SwiGLU tiles hold 16
    // gate rows and the 16 matching up rows (W = [gate rows; up rows], N = 2 I).
    const int lr = lane >> 4, lc = 4 * (lane & 15);
    const float * wbase = p.W + k_begin + kG32Blk * wave + lc;
    // bf16 rows: lane loads 8 elements, row 8 i + lane / 8 (i = 0..3) of each tile, k 8 (lane % 8) .. + 7
    const int lr16 = lane >> 3, lc16 = 8 * (lane & 7);
    const uint16_t * wbase16 = p.W16 + k_begin + kG32Blk * wave + lc16;
    const float * xbase = p.X + k_begin + kG32Blk * wave + lc;
    const float * nbase = prenorm ? p.norm_w + k_begin + kG32Blk * wave + lc : nullptr;
    auto weight_row = [&](int tile, int line) {
        const int wr_row = p.swiglu ? (line < 16 ? 16 * tile + line : (p.N >> 1) + 16 * tile + line - 16)
                                    : tile * kG32Rows + line;
        return static_cast<int64_t>(min(wr_row, p.N - 1)) * p.K;
    };
    int64_t wrow[8];
    int xrow[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int line = 4 * i + lr;
        // B16: entry 4 t + j is row 8 j + lane / 8 of tile T grp + t
        wrow[i] = B16 ? weight_row(T * grp + (i >> 2), 8 * (i & 3) + lr16) : weight_row(grp, line);
        xrow[i] = min(line, p.rows - 1) * p.K;
    }
    v4f wr[P][8], xr[P][8], nw[P];
    u4v wb[P][4 * T];
    auto load = [&](int u, int b) {
        const int o = min(b, last) * 4 * kG32Blk;
#pragma unroll
        for (int i = 0; i < 8; ++i) xr[u][i] = *reinterpret_cast<const v4f *>(xbase + xrow[i] + o);
        if (prenorm) nw[u] = *reinterpret_cast<const v4f *>(nbase + o);
        if constexpr (B16) {
#pragma unroll
            for (int i = 0; i < 4 * T; ++i) wb[u][i] = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(wbase16 + wrow[i] + o));
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) wr[u][i] = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(wbase + wrow[i] + o));
        }
    };
    if (my > 0) {
        // (a wave with fewer than P blocks re-reads its last one: no branch around a load here, which would
        // leave the wait counts of the loop below unknown)
#pragma unroll
        for (int u = 0; u < P; ++u) load(u, u);
    }
    float sc[8];
    if (prenorm) {
        // rms_norm_row (text-decoder.cpp:542-557): sum of squares in double, float scale, (x * scale) * w;
        // partial sums are added in a fixed order (k = part + 8 j by j, then the 8 parts in order)
        const int tk = threadIdx.x & 31, part = threadIdx.x >> 5;
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (part + 8 * j < p.n_stats_in) ss += sq[j];
        }
        s_part[part][tk] = ss;
        __syncthreads();
        if (threadIdx.x < 32) {
            double tot = 0.0;
#pragma unroll
            for (int q = 0; q < 8; ++q) tot += s_part[q][threadIdx.x];
            s_scale[threadIdx.x] = 1.0f / sqrtf(static_cast<float>(tot / static_cast<double>(p.K)) + p.eps);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; ++i) sc[i] = s_scale[min(4 * i + lr, p.rows - 1)];
    }
    float * myw = lw[wave];
    float * myx = lx[wave];
    const int r = lane & 31, h = lane >> 5;
    v16f acc0[T], acc1[T];
#pragma unroll
    for (int t = 0; t < T; ++t) { acc0[t] = v16f{}; acc1[t] = v16f{}; }
    uint16_t * myw16 = reinterpret_cast<uint16_t *>(myw);
    auto compute = [&](int u) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v4f xv = xr[u][i];
            if (prenorm) {
#pragma unroll
                for (int e = 0; e < 4; ++e) xv[e] = xv[e] * sc[i] * nw[u][e];
            }
            if constexpr (!B16) *reinterpret_cast<v4f *>(myw + (4 * i + lr) * kG32Ls + lc) = wr[u][i];
            *reinterpret_cast<v4f *>(myx + (4 * i + lr) * kG32Ls + lc) = xv;
        }
        if constexpr (B16) {
#pragma unroll
            for (int i = 0; i < 4 * T; ++i) {
                *reinterpret_cast<u4v *>(myw16 + ((i >> 2) * kG32Rows + 8 * (i & 3) + lr16) * kG32LsB + lc16) = wb[u][i];
            }
        }
        // the block is read back by other lanes of this wave: LDS operations of a wave complete in order
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if constexpr (B16) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                // MFMA step s: k 16 s + 8 h + 0..7 for lane half h (A: weight row r, B: token r); the split
                // of X serves the T tiles
                const v4f x0 = *reinterpret_cast<const v4f *>(myx + r * kG32Ls + 16 * s + 8 * h);
                const v4f x1 = *reinterpret_cast<const v4f *>(myx + r * kG32Ls + 16 * s + 8 * h + 4);
                u4v bh, bm, bl;
                split_bf16x3(x0, x1, bh, bm, bl);
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const u4v a = *reinterpret_cast<const u4v *>(myw16 + (t * kG32Rows + r) * kG32LsB + 16 * s + 8 * h);
                    const bf16x8 av = __builtin_bit_cast(bf16x8, a);
                    acc0[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, __builtin_bit_cast(bf16x8, bh), acc0[t], 0, 0, 0);
                    acc1[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, __builtin_bit_cast(bf16x8, bm), acc1[t], 0, 0, 0);
                    acc1[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, __builtin_bit_cast(bf16x8, bl), acc1[t], 0, 0, 0);
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            return;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            // MFMA step s: k 16 s + 4 h + j (acc0) and 16 s + 8 + 4 h + j (acc1), j = 0..3 -- the same
            // permutation of k for the W (A) and X (B) operands
            const v4f a0 = *reinterpret_cast<const v4f *>(myw + r * kG32Ls + 16 * s + 4 * h);
            const v4f a1 = *reinterpret_cast<const v4f *>(myw + r * kG32Ls + 16 * s + 8 + 4 * h);
            const v4f b0 = *reinterpret_cast<const v4f *>(myx + r * kG32Ls + 16 * s + 4 * h);
            const v4f b1 = *reinterpret_cast<const v4f *>(myx + r * kG32Ls + 16 * s + 8 + 4 * h);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc0[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[j], b0[j], acc0[0], 0, 0, 0);
                acc1[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[j], b1[j], acc1[0], 0, 0, 0);
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };
    // block b is computed from register set b % P; the loads of block b + P follow its arithmetic.  Only
    // blocks of this wave are loaded, so nothing is in flight when the accumulators are summed.
    const int full = my / P * P;
    for (int b0 = 0; b0 + P < full; b0 += P) {
#pragma unroll
        for (int u = 0; u < P; ++u) {
            compute(u);
            load(u, b0 + P + u);
            // keep the loads of block b + P right behind the arithmetic of block b
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (full > 0) {
        // the last whole group of P blocks loads only the remaining my - full blocks
#pragma unroll
        for (int u = 0; u < P; ++u) {
            compute(u);
            if (u < my - full) load(u, full + u);
        }
    }
#pragma unroll
    for (int u = 0; u < P - 1; ++u) {
        if (u < my - full) compute(u);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // sum the 4 waves (wave order) through LDS: accumulator entry i of lane (r, h) is row
    // 8 (i / 4) + 4 h + i % 4 of token r (32x32 MFMA output layout); tile t's sums at t 4096
    __syncthreads();
    float * red = &lw[0][0];
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int i = 0; i < 16; ++i) red[((t * 4 + wave) * 16 + i) * kWave + lane] = acc0[t][i] + acc1[t][i];
    }
    __syncthreads();
    auto entry = [&](int t, int i) {
        float a = red[(t * 64 + i) * kWave + lane];
#pragma unroll
        for (int v = 1; v < 4; ++v) a += red[((t * 4 + v) * 16 + i) * kWave + lane];
        return a;
    };
    const int tk = r;   // token of this lane's outputs
    if (p.swiglu) {
        // one slice (ks = 1): waves 0 and 1 own gate rows 8 w + 4 h + 0..3 (entries 4 w + j) and their up
        // rows 16 + 8 w + 4 h + 0..3 (entries 4 w + 8 + j) of each tile; silu(gate) * up as
        // text-decoder.cpp:602
        if (wave < 2 && tk < p.rows) {
            const int I = p.N >> 1;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int c = 16 * (T * grp + t) + 8 * wave + 4 * h;
                float * y = p.Y + static_cast<int64_t>(tk) * I + c;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float g = entry(t, 4 * wave + j), u = entry(t, 4 * wave + 8 + j);
                    if (c + j < I) y[j] = (g / (1.0f + expf(-g))) * u;
                }
            }
        }
        return;
    }
    // wave w owns entries 4 w .. 4 w + 3 of each tile: rows 8 w + 4 h + 0..3 of token r
    v4f sv[T];
    int nr[T];
    bool live[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int j = 0; j < 4; ++j) sv[t][j] = entry(t, 4 * wave + j);
        nr[t] = (T * grp + t) * kG32Rows + 8 * wave + 4 * h;
        live[t] = tk < p.rows && nr[t] < p.N;
    }
    // store (or accumulate) the final values of tile t; with stats_out also the tile's per-token sum of
    // squares of the stored values (a workgroup-uniform step: every thread of the workgroup calls it)
    // the old values of tile t's 4 outputs of this lane (accumulate), read by 4 loads issued together
    // (addresses clamped to the matrix, no branch), so that they cost one round trip
    auto old_values = [&](int t) {
        v4f o = v4f{};
        if (p.accumulate) {
            const float * y = p.Y + static_cast<int64_t>(min(tk, p.rows - 1)) * p.N;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = y[min(nr[t] + i, p.N - 1)];
        }
        return o;
    };
    auto finish = [&](int t, v4f v, v4f old) {
        double ss = 0.0;
        if (live[t]) {
            float * y = p.Y + static_cast<int64_t>(tk) * p.N + nr[t];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (nr[t] + i < p.N) {
                    const float o = p.accumulate ? old[i] + v[i] : v[i];
                    y[i] = o;
                    ss += static_cast<double>(o) * o;
                }
            }
        }
        if (p.stats_out) {
            double * sst = &s_part[0][0];                           // [4 waves][2 halves][32 tokens]
            sst[(2 * wave + h) * 32 + tk] = ss;
            __syncthreads();
            if (threadIdx.x < 32) {
                double tot = 0.0;
#pragma unroll
                for (int q = 0; q < 8; ++q) tot += sst[q * 32 + threadIdx.x];
                p.stats_out[32 * (T * grp + t) + threadIdx.x] = tot;
            }
            __syncthreads();   // sst is written again by the next tile's step
        }
    };
    if (p.ks == 1) {
        v4f old[T];
#pragma unroll
        for (int t = 0; t < T; ++t) old[t] = old_values(t);
#pragma unroll
        for (int t = 0; t < T; ++t) finish(t, sv[t], old[t]);
        return;
    }
    // publish (partial rows padded to whole 4-row groups), then the last slice of the tile group merges in
    // slice order -- the same protocol as gemm_rows_kernel
    const int np = (p.N + 3) / 4 * 4;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        if (live[t]) {
            uint64_t * q = reinterpret_cast<uint64_t *>(p.partial + (static_cast<int64_t>(sl) * p.rows + tk) * np + nr[t]);
            const uint64_t lo = static_cast<uint64_t>(__float_as_uint(sv[t][0])) | (static_cast<uint64_t>(__float_as_uint(sv[t][1])) << 32);
            const uint64_t hi = static_cast<uint64_t>(__float_as_uint(sv[t][2])) | (static_cast<uint64_t>(__float_as_uint(sv[t][3])) << 32);
            __hip_atomic_store(q, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(q + 1, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t * ctr = p.counters + static_cast<int64_t>(grp) * kGrCounterStride;
        const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == static_cast<uint32_t>(p.ks - 1);
        if (s_last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
    const int tt = min(tk, p.rows - 1);
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int nn = min(nr[t], np - 4);
        // one round of loads: the plan merges at most kG32MaxSlices slices; no loop, whose back edge would
        // make the compiler wait for earlier loads before reusing their registers
        uint64_t v[kG32MaxSlices][2];
#pragma unroll
        for (int u = 0; u < kG32MaxSlices; ++u) {
            const int k = min(u, p.ks - 1);
            const uint64_t * q = reinterpret_cast<const uint64_t *>(p.partial + (static_cast<int64_t>(k) * p.rows + tt) * np + nn);
            v[u][0] = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v[u][1] = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const v4f old = old_values(t);   // issued behind the partials' loads, waited for with them
        float sum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < kG32MaxSlices; ++u) {
            if (u >= p.ks) break;
            sum[0] += __uint_as_float(static_cast<uint32_t>(v[u][0]));
            sum[1] += __uint_as_float(static_cast<uint32_t>(v[u][0] >> 32));
            sum[2] += __uint_as_float(static_cast<uint32_t>(v[u][1]));
            sum[3] += __uint_as_float(static_cast<uint32_t>(v[u][1] >> 32));
        }
        finish(t, v4f{sum[0], sum[1], sum[2], sum[3]}, old);
    }
}

struct GemmRowsPlan {
    int ks, slice, tiles;
    bool rows32;     // gemm_rows32_kernel (else gemm_rows_kernel)
    int depth;       // blocks in flight per wave (gemm_rows32_kernel)
    int tpw;         // tiles per workgroup (gemm_rows32_kernel: 2 with bf16 weights, an even tile count and > 1024 tiles)
};

// tuning overrides of the <= 32-row plan: QA_GR32_WGS (workgroup target, default 256) and QA_GR32_DEPTH
// (blocks in flight per wave, 1 or 2)
int env_int(const char * name, int fallback) {
    const char * e = std::getenv(name);
    return e ? std::atoi(e) : fallback;
}

GemmRowsPlan gemm_rows_plan(int32_t N, int32_t K, int32_t rows, bool one_slice = false, bool b16 = false) {
    GemmRowsPlan pl{};
    static const int target_wgs = std::max(64, env_int("QA_GR32_WGS", 256));
    static const int forced_depth = env_int("QA_GR32_DEPTH", 0);
    static const int forced_tpw = env_int("QA_GR32_TPW", 0);
    if (rows <= kG32Rows && K % kG32Blk == 0) {
        // ~256 workgroups at least (one per CU); a K slice keeps >= 4 blocks (one per wave) and at most
        // 8 slices are merged.  Two blocks in flight per wave when the grid is one workgroup per CU (the
        // register file then holds 2 waves per SIMD either way), one when there are more workgroups.
        // With bf16 weights and more than 1024 tiles (the LM head) a workgroup takes two tiles, which
        // share each X block and its split (config-4 step: LM head 0.198 -> 0.171 ms); with fewer tiles
        // the grid would drop below two workgroups per CU (layer projections 1.95 -> 2.40 ms per step).
        pl.rows32 = true;
        pl.tiles = (N + kG32Rows - 1) / kG32Rows;
        pl.tpw = b16 && pl.tiles % 2 == 0 && (pl.tiles > 1024 || forced_tpw == 2) && forced_tpw != 1 ? 2 : 1;
        const int groups = pl.tiles / pl.tpw;
        int ks = std::max(1, std::min({(target_wgs + groups / 2) / groups, kG32MaxSlices, K / (4 * kG32Blk)}));
        if (groups > kGrMaxTiles || one_slice) ks = 1;             // counters exist for kGrMaxTiles groups
        pl.slice = ((K + ks - 1) / ks + kG32Blk - 1) / kG32Blk * kG32Blk;
        pl.ks = (K + pl.slice - 1) / pl.slice;
        pl.depth = forced_depth == 1 || forced_depth == 2 ? forced_depth : groups * pl.ks <= 256 ? 2 : 1;
        return pl;
    }
    pl.tiles = (N + kGrTile - 1) / kGrTile;
    const int rows_pad = (rows + 15) / 16 * 16;
    // ~512 workgroups but at most 8 slices (the merge then takes one round of loads), and the X slice of
    // every token (padded row stride) within the LDS budget
    int ks = std::max(1, std::min(std::min((512 + pl.tiles - 1) / pl.tiles, 8), K / 32));
    for (;; ++ks) {
        pl.slice = ((K + ks - 1) / ks + 31) / 32 * 32;
        if (static_cast<size_t>(rows_pad) * (pl.slice + 8) * sizeof(float) <= kGrLdsBytes || pl.slice == 32) break;
    }
    pl.ks = (K + pl.slice - 1) / pl.slice;
    return pl;
}

// ---------------------------------------------------------------- row RMSNorm (T > 1 paths)
// y = RMSNorm(x) w per row, as f32 rows of y or (split != null) as the three-part split rows of the
// prefill GEMM's input ([rows][3 dim] bf16 bits)
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float * x, const float * w, int dim, float eps,
                                                           float * y, uint16_t * split) {
#pragma clang fp contract(off)
    const int r = blockIdx.x;
    const float * xr = x + static_cast<int64_t>(r) * dim;
    double ss = 0.0;
    for (int i = threadIdx.x; i < dim; i += 256) ss += static_cast<double>(xr[i]) * xr[i];
    ss = wave_sum_d_all(ss);
    __shared__ double part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float scale = 1.0f / sqrtf(static_cast<float>(tot / static_cast<double>(dim)) + eps);
    if (split) {
        uint16_t * sr = split + static_cast<int64_t>(r) * 3 * dim;
        for (int i = threadIdx.x; i < dim; i += 256) store_split3(sr + i, dim, xr[i] * scale * w[i]);
        return;
    }
    float * yr = y + static_cast<int64_t>(r) * dim;
    for (int i = threadIdx.x; i < dim; i += 256) yr[i] = xr[i] * scale * w[i];
}

// a = silu(gate) up per row (gu rows = [gate | up], dim each), text-decoder.cpp:602; as f32 rows of a or
// (split != null) as the three-part split rows of the prefill GEMM's input.  blockIdx.y = row.
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const float * gu, int dim, float * a, uint16_t * split) {
#pragma clang fp contract(off)
    const int c = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    if (c >= dim) return;
    const int64_t r = blockIdx.y;
    const float g = gu[r * 2 * dim + c];
    const float u = gu[r * 2 * dim + dim + c];
    const float v = (g / (1.0f + expf(-g))) * u;
    if (split) store_split3(split + r * 3 * dim + c, dim, v);
    else a[r * dim + c] = v;
}

__global__ void add_inplace_kernel(float * y, const float * x, size_t n) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        y[i] += x[i];
    }
}

// Row `row` of the next step's input: the embedding row t (zeros unless valid) copied to o, and, with
// stats, the row's sums of squares per 32-column group (in double, the columns in increasing order),
// stored at stats[32 * group + row] for the fused RMSNorm input of the multi-stream GEMM.  256 threads;
// each pass issues all its loads (8 per thread, 2048 columns) before the first use and stages the
// values in LDS for the sums, so a row costs one memory round trip per 2048 columns.
constexpr int kGatherCols = 2048;

__device__ void gather_row(const float * t, bool valid, int dim, float * o, double * stats, int row) {
#pragma clang fp contract(off)
    __shared__ float s_row[kGatherCols];
    for (int base = 0; base < dim; base += kGatherCols) {
        const int n = min(kGatherCols, dim - base);
        float v[kGatherCols / 256];
#pragma unroll
        for (int u = 0; u < kGatherCols / 256; ++u) v[u] = t[base + min(static_cast<int>(threadIdx.x) + 256 * u, n - 1)];
#pragma unroll
        for (int u = 0; u < kGatherCols / 256; ++u) {
            const int i = static_cast<int>(threadIdx.x) + 256 * u;
            const float x = valid ? v[u] : 0.0f;
            if (i < n) {
                o[base + i] = x;
                s_row[i] = x;
            }
        }
        if (!stats) continue;
        __syncthreads();
        for (int k = threadIdx.x; 32 * k < n; k += 256) {
            double ss = 0.0;
            for (int i = 32 * k; i < min(32 * k + 32, n); ++i) {
                const double x = s_row[i];
                ss = fma(x, x, ss);
            }
            stats[32 * (base / 32 + k) + row] = ss;
        }
        __syncthreads();   // s_row is refilled by the next pass
    }
}

// out[r] = table[ids[r]] (zeros for ids out of range); stats (optional): stats[k][r] = sum of squares of columns
// 32 k .. 32 k + 31 of row r (the partial layout gemm_rows32_kernel takes for its RMSNorm input; r < 32)
__global__ __launch_bounds__(256) void embed_rows_kernel(const float * table, int n_rows, int dim, const int32_t * ids,
                                                         float * out, double * stats) {
    const int r = blockIdx.x;
    const int id = ids[r];
    const bool valid = id >= 0 && id < n_rows;
    gather_row(table + static_cast<int64_t>(valid ? id : 0) * dim, valid, dim, out + static_cast<int64_t>(r) * dim,
               stats, r);
}

__global__ void advance_lens_kernel(int32_t * lens, int n, int delta) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) lens[i] += delta;
}

// ---------------------------------------------------------------- argmax
// Reference rule (text-decoder.cpp:2266-2274): best = -inf, take i when logits[i] > best, so the
// lowest index among equal maxima wins, NaN and -inf never win, and -1 means nothing was taken.
struct Cand {
    float v;
    int32_t i;
};

__device__ inline Cand better(Cand a, Cand b) {
    if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}

constexpr int kArgmaxBlocks = 64;
// uint32 words between the rows' block counters: one 256-byte line each.  Device-scope atomics on one
// line are serialised, so with the counters of 32 rows packed into one line the 2048 increments of a
// 32-row pick queued behind each other (32 us per config-4 step, against 8 us for one row).
constexpr int kArgmaxCounterStride = 64;
constexpr int kArgmaxBatch = 10;   // loads per thread in flight: a 1.7B vocabulary chunk (2374) in one round
constexpr int32_t kNoIndex = 0x7fffffff;

// Block candidates are published as one 8-byte agent-scope atomic store each and read back by the
// last block with agent-scope atomic loads (coherent across XCDs without an L2 write-back/invalidate
// fence); a vmcnt wait orders the store before the counter increment.
__device__ inline uint64_t pack_cand(Cand c) {
    return static_cast<uint64_t>(__float_as_uint(c.v)) | (static_cast<uint64_t>(static_cast<uint32_t>(c.i)) << 32);
}

__device__ inline Cand unpack_cand(uint64_t u) {
    Cand c;
    c.v = __uint_as_float(static_cast<uint32_t>(u));
    c.i = static_cast<int32_t>(static_cast<uint32_t>(u >> 32));
    return c;
}

__device__ inline Cand wave_best(Cand c) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        Cand o;
        o.v = __shfl_xor(c.v, off, kWave);
        o.i = __shfl_xor(c.i, off, kWave);
        c = better(c, o);
    }
    return c;
}

__global__ __launch_bounds__(256) void argmax_kernel(const float * logits, int vocab, uint64_t * partial,
                                                     uint32_t * counters, int32_t * ids, StepTail tail) {
    const int row = blockIdx.y;
    const int chunk = (vocab + kArgmaxBlocks - 1) / kArgmaxBlocks;
    const int lo = blockIdx.x * chunk;
    const int hi = min(vocab, lo + chunk);
    const float * lr = logits + static_cast<int64_t>(row) * vocab;
    Cand c{-INFINITY, kNoIndex};
    // kArgmaxBatch loads per thread in flight at once (indices past the chunk re-read its last element
    // and are skipped), then scanned in increasing index order: the first maximum of the thread wins and
    // NaN never does, as in a plain loop.  A loop with one load per iteration waited a full memory round
    // trip per element (10 us for the 1.7B vocabulary at batch 1).
    for (int i0 = lo + static_cast<int>(threadIdx.x); i0 < hi; i0 += 256 * kArgmaxBatch) {
        float v[kArgmaxBatch];
#pragma unroll
        for (int u = 0; u < kArgmaxBatch; ++u) v[u] = lr[min(i0 + 256 * u, hi - 1)];
#pragma unroll
        for (int u = 0; u < kArgmaxBatch; ++u) {
            const int i = i0 + 256 * u;
            if (i < hi && v[u] > c.v) { c.v = v[u]; c.i = i; }
        }
    }
    c = wave_best(c);
    __shared__ Cand wc[4];
    if ((threadIdx.x & 63) == 0) wc[threadIdx.x >> 6] = c;
    __syncthreads();
    __shared__ int is_last;
    if (threadIdx.x == 0) {
        const Cand b = better(better(wc[0], wc[1]), better(wc[2], wc[3]));
        __hip_atomic_store(partial + row * kArgmaxBlocks + blockIdx.x, pack_cand(b), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        uint32_t * ctr = counters + static_cast<int64_t>(row) * kArgmaxCounterStride;
        const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = old == kArgmaxBlocks - 1;
        if (is_last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!is_last) return;
    __shared__ int s_id;
    if (threadIdx.x < kArgmaxBlocks) {
        Cand b = unpack_cand(__hip_atomic_load(partial + row * kArgmaxBlocks + threadIdx.x, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT));
        b = wave_best(b);
        if (threadIdx.x == 0) {
            const int id = b.i == kNoIndex ? -1 : b.i;
            ids[row] = id;
            s_id = id;
            if (tail.host_ids) tail.host_ids[row] = id;
            if (tail.lens) tail.lens[row] += 1;
        }
    }
    if (!tail.embd) return;
    // the next step's input: embed_rows_kernel's gather and row statistics, for the picked id
    __syncthreads();
    const int id = s_id;
    const bool valid = id >= 0 && id < vocab;
    gather_row(tail.embd + static_cast<int64_t>(valid ? id : 0) * tail.dim, valid, tail.dim,
               tail.x + static_cast<int64_t>(row) * tail.dim, tail.stats, row);
}

}  // namespace

int gemv_launch(int epi, bool prenorm, const float * W, int32_t out_dim, int32_t in_dim, const float * x,
                float * y, const float * norm_w, float eps, hipStream_t stream, const uint16_t * W16) {
    GemvParams p{W16 ? static_cast<const void *>(W16) : static_cast<const void *>(W), x, y, norm_w, out_dim, in_dim,
                 eps, y};
    const bool b16 = W16 != nullptr;
    if (!p.W || !x || !y || out_dim <= 0 || (prenorm && !norm_w)) return fail(QA_ERR_INVALID, "gemv: invalid arguments");
    if (epi == kEpiStore) return prenorm ? launch_gemv_w<kEpiStore, true>(p, b16, stream) : launch_gemv_w<kEpiStore, false>(p, b16, stream);
    if (epi == kEpiAccum) return prenorm ? launch_gemv_w<kEpiAccum, true>(p, b16, stream) : launch_gemv_w<kEpiAccum, false>(p, b16, stream);
    return prenorm ? launch_gemv_w<kEpiSwiglu, true>(p, b16, stream) : launch_gemv_w<kEpiSwiglu, false>(p, b16, stream);
}

// Row t of out = [hi | mid | lo] of row t of x (rows x K floats): the exact three-part bf16 split,
// x = hi + mid + lo (truncations to 8 significant bits, then the same of the remainder; the last
// remainder has at most 8 significant bits).  blockIdx.y = row, 4 consecutive elements per thread.
__device__ inline uint32_t split3_pair(float a, float b, uint32_t & mid, uint32_t & lo) {
    const uint32_t ha = __float_as_uint(a) & 0xffff0000u, hb = __float_as_uint(b) & 0xffff0000u;
    const float ra = a - __uint_as_float(ha), rb = b - __uint_as_float(hb);
    const uint32_t ma = __float_as_uint(ra) & 0xffff0000u, mb = __float_as_uint(rb) & 0xffff0000u;
    const float qa = ra - __uint_as_float(ma), qb = rb - __uint_as_float(mb);
    mid = (ma >> 16) | mb;
    lo = (__float_as_uint(qa) >> 16) | (__float_as_uint(qb) & 0xffff0000u);
    return (ha >> 16) | hb;
}

__global__ __launch_bounds__(256) void split_bf16x3_rows_kernel(const float * x, int32_t K, uint16_t * out) {
    const int k = (static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x)) * 4;
    if (k >= K) return;
    const int64_t t = blockIdx.y;
    const float4 v = *reinterpret_cast<const float4 *>(x + t * K + k);
    uint32_t m0, m1, l0, l1;
    const uint32_t h0 = split3_pair(v.x, v.y, m0, l0), h1 = split3_pair(v.z, v.w, m1, l1);
    uint16_t * o = out + t * 3 * K + k;
    *reinterpret_cast<uint2 *>(o) = make_uint2(h0, h1);
    *reinterpret_cast<uint2 *>(o + K) = make_uint2(m0, m1);
    *reinterpret_cast<uint2 *>(o + 2 * K) = make_uint2(l0, l1);
}

int split_bf16x3_rows_launch(const float * x, int64_t rows, int32_t K, uint16_t * out, hipStream_t stream) {
    if (!x || !out || rows < 0 || K <= 0 || K % 4 != 0) return fail(QA_ERR_INVALID, "split_bf16x3_rows: invalid arguments");
    for (int64_t r0 = 0; r0 < rows; r0 += 65535) {     // grid.y <= 65535 rows per launch
        const dim3 grid(static_cast<unsigned>((K / 4 + 255) / 256), static_cast<unsigned>(std::min<int64_t>(rows - r0, 65535)));
        hipLaunchKernelGGL(split_bf16x3_rows_kernel, grid, dim3(256), 0, stream, x + r0 * K, K, out + r0 * 3 * K);
        QA_LAUNCH_CHECK("split_bf16x3_rows_kernel");
    }
    return QA_OK;
}

int pack_bf16_launch(const float * src, int64_t n, uint16_t * dst, uint32_t * inexact, hipStream_t stream) {
    if (!src || !dst || !inexact || n < 0) return fail(QA_ERR_INVALID, "pack_bf16: invalid arguments");
    if (n == 0) return QA_OK;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(pack_bf16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, src, n, dst, inexact);
    QA_LAUNCH_CHECK("pack_bf16_kernel");
    return QA_OK;
}

size_t gemm_rows_workspace_bytes(int32_t N, int32_t K, int32_t rows) {
    if (N <= 0 || N > kGrMaxTiles * kGrTile || K <= 0 || rows <= 0 || rows > kGrMaxRows || K % 32 != 0) return 0;
    // the larger of the f32-weight and bf16-weight plans (their slice counts differ)
    const int ks = std::max(gemm_rows_plan(N, K, rows).ks, gemm_rows_plan(N, K, rows, false, true).ks);
    const size_t partial = ks > 1 ? static_cast<size_t>(ks) * rows * ((N + 3) / 4 * 4) * sizeof(float) : 0;
    return kGrCounterBytes + partial;
}

bool gemm_rows_fusable(int32_t N, int32_t K, int32_t rows) {
    return N > 0 && N <= kGrMaxTiles * kGrTile && rows >= 1 && rows <= kG32Rows && K > 0 && K % kG32Blk == 0;
}

int gemm_rows_launch(const float * W, int32_t N, int32_t K, const float * X, int32_t rows, float * Y, bool accumulate,
                     void * workspace, size_t workspace_bytes, hipStream_t stream, const GemmRowsFusion * fusion,
                     const uint16_t * W16) {
    if ((!W && !W16) || !X || !Y || N <= 0 || N > kGrMaxTiles * kGrTile || K <= 0 || K % 32 != 0 || rows < 1 ||
        rows > kGrMaxRows) {
        return fail(QA_ERR_INVALID, "gemm_rows: invalid shape");
    }
    const bool fused = fusion && (fusion->norm_w || fusion->stats_out || fusion->swiglu);
    if (fused) {
        if (!gemm_rows_fusable(N, K, rows)) return fail(QA_ERR_INVALID, "gemm_rows: fusions need <= 32 rows, K % 64 == 0");
        if (fusion->norm_w && (!fusion->stats_in || fusion->n_stats_in < 1 || fusion->n_stats_in > 128)) {
            return fail(QA_ERR_INVALID, "gemm_rows: RMSNorm input needs 1..128 partial sums per row");
        }
        if (fusion->swiglu && (N % 32 != 0 || accumulate || fusion->stats_out)) {
            return fail(QA_ERR_INVALID, "gemm_rows: SwiGLU needs N = 2 I with I % 16 == 0 and a plain store");
        }
    }
    const GemmRowsPlan pl = gemm_rows_plan(N, K, rows, fused && fusion->swiglu, W16 != nullptr);
    if (!W && !pl.rows32) return fail(QA_ERR_INVALID, "gemm_rows: bf16 weights need rows <= 32 and K % 64 == 0");
    const size_t need = gemm_rows_workspace_bytes(N, K, rows);
    if (!workspace || workspace_bytes < need) return fail(QA_ERR_INVALID, "gemm_rows: workspace too small");
    GemmRowsParams p{};
    p.W = W;
    p.X = X;
    p.Y = Y;
    p.counters = static_cast<uint32_t *>(workspace);
    p.partial = reinterpret_cast<float *>(static_cast<char *>(workspace) + kGrCounterBytes);
    p.N = N;
    p.K = K;
    p.rows = rows;
    p.ks = pl.ks;
    p.slice = pl.slice;
    p.accumulate = accumulate ? 1 : 0;
    auto magic = [](int k_len) {
        const uint64_t cols = static_cast<uint64_t>(k_len / 4);
        return static_cast<uint32_t>(((uint64_t{1} << 32) + cols - 1) / cols);
    };
    if (fused) {
        p.norm_w = fusion->norm_w;
        p.stats_in = fusion->stats_in;
        p.n_stats_in = fusion->n_stats_in;
        p.eps = fusion->eps;
        p.stats_out = fusion->stats_out;
        p.swiglu = fusion->swiglu ? 1 : 0;
    }
    if (pl.rows32) {
        const dim3 grid(static_cast<unsigned>(pl.tiles / pl.tpw * pl.ks));
        p.W16 = W16;
        if (W16 && pl.tpw == 2) {
            if (pl.depth == 2) hipLaunchKernelGGL((gemm_rows32_kernel<2, true, 2>), grid, dim3(256), 0, stream, p);
            else hipLaunchKernelGGL((gemm_rows32_kernel<1, true, 2>), grid, dim3(256), 0, stream, p);
        } else if (W16) {
            if (pl.depth == 2) hipLaunchKernelGGL((gemm_rows32_kernel<2, true, 1>), grid, dim3(256), 0, stream, p);
            else hipLaunchKernelGGL((gemm_rows32_kernel<1, true, 1>), grid, dim3(256), 0, stream, p);
        } else {
            if (pl.depth == 2) hipLaunchKernelGGL((gemm_rows32_kernel<2, false, 1>), grid, dim3(256), 0, stream, p);
            else hipLaunchKernelGGL((gemm_rows32_kernel<1, false, 1>), grid, dim3(256), 0, stream, p);
        }
        QA_LAUNCH_CHECK("gemm_rows32_kernel");
        return QA_OK;
    }
    p.x_magic = magic(pl.slice);
    p.x_magic_last = magic(K - (pl.ks - 1) * pl.slice);
    const int tb = (rows + 15) / 16;
    const size_t lds = static_cast<size_t>(16 * tb) * (pl.slice + 8) * sizeof(float);
    const dim3 grid(static_cast<unsigned>(pl.tiles * pl.ks));
    switch (tb) {
        case 1: hipLaunchKernelGGL((gemm_rows_kernel<1>), grid, dim3(256), lds, stream, p); break;
        case 2: hipLaunchKernelGGL((gemm_rows_kernel<2>), grid, dim3(256), lds, stream, p); break;
        case 3: hipLaunchKernelGGL((gemm_rows_kernel<3>), grid, dim3(256), lds, stream, p); break;
        default: hipLaunchKernelGGL((gemm_rows_kernel<4>), grid, dim3(256), lds, stream, p); break;
    }
    QA_LAUNCH_CHECK("gemm_rows_kernel");
    return QA_OK;
}

size_t argmax_workspace_bytes(int32_t rows) {
    return (sizeof(Cand) * kArgmaxBlocks + sizeof(uint32_t) * kArgmaxCounterStride) * static_cast<size_t>(rows) + 256;
}

int argmax_launch(const float * logits, int32_t rows, int32_t vocab, int32_t * ids, void * workspace,
                  hipStream_t stream, const StepTail & tail) {
    static_assert(sizeof(Cand) == sizeof(uint64_t), "a candidate is published as one 8-byte store");
    if (tail.embd && (!tail.x || tail.dim <= 0 || (tail.stats && rows > 32))) {
        return fail(QA_ERR_INVALID, "argmax: invalid embedding gather of the step tail");
    }
    uint64_t * partial = static_cast<uint64_t *>(workspace);
    uint32_t * counters = reinterpret_cast<uint32_t *>(partial + static_cast<size_t>(rows) * kArgmaxBlocks);
    hipLaunchKernelGGL(argmax_kernel, dim3(kArgmaxBlocks, static_cast<unsigned>(rows)), dim3(256), 0, stream,
                       logits, vocab, partial, counters, ids, tail);
    QA_LAUNCH_CHECK("argmax_kernel");
    return QA_OK;
}

int rmsnorm_rows_launch(const float * x, const float * w, int32_t rows, int32_t dim, float eps, float * y,
                        hipStream_t stream, uint16_t * split) {
    if (rows <= 0) return QA_OK;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, x, w, dim,
                       eps, y, split);
    QA_LAUNCH_CHECK("rmsnorm_rows_kernel");
    return QA_OK;
}

int swiglu_rows_launch(const float * gu, int32_t rows, int32_t dim, float * a, hipStream_t stream, uint16_t * split) {
    if (rows <= 0 || dim <= 0) return QA_OK;
    for (int32_t r0 = 0; r0 < rows; r0 += 65535) {     // grid.y <= 65535 rows per launch
        const dim3 grid(static_cast<unsigned>((dim + 255) / 256), static_cast<unsigned>(std::min(rows - r0, 65535)));
        const int64_t off = static_cast<int64_t>(r0) * dim;
        hipLaunchKernelGGL(swiglu_rows_kernel, grid, dim3(256), 0, stream, gu + 2 * off, dim, split ? nullptr : a + off,
                           split ? split + 3 * off : nullptr);
        QA_LAUNCH_CHECK("swiglu_rows_kernel");
    }
    return QA_OK;
}

int embed_rows_launch(const float * table, int32_t n_rows, int32_t dim, const int32_t * ids, int32_t rows,
                      float * out, hipStream_t stream, double * stats) {
    if (rows <= 0) return QA_OK;
    if (stats && rows > 32) return fail(QA_ERR_INVALID, "embed_rows: row statistics cover at most 32 rows");
    hipLaunchKernelGGL(embed_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, table, n_rows,
                       dim, ids, out, stats);
    QA_LAUNCH_CHECK("embed_rows_kernel");
    return QA_OK;
}

int advance_lens_launch(int32_t * lens, int32_t n, int32_t delta, hipStream_t stream) {
    if (n <= 0) return QA_OK;
    hipLaunchKernelGGL(advance_lens_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream,
                       lens, n, delta);
    QA_LAUNCH_CHECK("advance_lens_kernel");
    return QA_OK;
}

}  // namespace qa

extern "C" int qa_gemv(const float * W, int32_t out_dim, int32_t in_dim, const float * x, int32_t rows, float * y,
                       int32_t accumulate, void * stream) {
    using namespace qa;
    for (int32_t r = 0; r < rows; ++r) {
        const int rc = gemv_launch(accumulate ? kEpiAccum : kEpiStore, false, W, out_dim, in_dim,
                                   x + static_cast<int64_t>(r) * in_dim, y + static_cast<int64_t>(r) * out_dim,
                                   nullptr, 0.0f, as_stream(stream));
        if (rc != QA_OK) return rc;
    }
    return QA_OK;
}

extern "C" int qa_gemv_fused(const float * W, const uint16_t * W_bf16, int32_t out_dim, int32_t in_dim,
                             const float * x, float * y, int32_t epilogue, const float * norm_w, float eps,
                             void * stream) {
    using namespace qa;
    if ((W == nullptr) == (W_bf16 == nullptr)) return fail(QA_ERR_INVALID, "qa_gemv_fused: pass exactly one of W, W_bf16");
    if (epilogue < kEpiStore || epilogue > kEpiSwiglu) return fail(QA_ERR_INVALID, "qa_gemv_fused: unknown epilogue");
    return gemv_launch(epilogue, norm_w != nullptr, W, out_dim, in_dim, x, y, norm_w, eps, as_stream(stream), W_bf16);
}

extern "C" int qa_pack_bf16(const float * src, int64_t n, uint16_t * dst, uint32_t * inexact, void * stream) {
    return qa::pack_bf16_launch(src, n, dst, inexact, qa::as_stream(stream));
}

extern "C" size_t qa_argmax_workspace_bytes(int32_t rows) {
    return rows > 0 ? qa::argmax_workspace_bytes(rows) : 0;
}

extern "C" int qa_argmax_rows(const float * logits, int32_t rows, int32_t vocab, int32_t * ids, void * workspace,
                              size_t workspace_bytes, void * stream) {
    if (!logits || !ids || !workspace || rows <= 0 || vocab <= 0 ||
        workspace_bytes < qa::argmax_workspace_bytes(rows)) {
        return qa::fail(QA_ERR_INVALID, "qa_argmax_rows: invalid arguments");
    }
    return qa::argmax_launch(logits, rows, vocab, ids, workspace, qa::as_stream(stream));
}

extern "C" int qa_rmsnorm_rows(const float * x, const float * w, int32_t rows, int32_t dim, float eps, float * y,
                               void * stream) {
    if (!x || !w || !y || rows < 0 || dim <= 0) return qa::fail(QA_ERR_INVALID, "qa_rmsnorm_rows: invalid arguments");
    return qa::rmsnorm_rows_launch(x, w, rows, dim, eps, y, qa::as_stream(stream));
}

extern "C" int qa_swiglu_rows(const float * gu, int32_t rows, int32_t dim, float * a, void * stream) {
    if (!gu || !a || rows < 0 || dim <= 0) return qa::fail(QA_ERR_INVALID, "qa_swiglu_rows: invalid arguments");
    return qa::swiglu_rows_launch(gu, rows, dim, a, qa::as_stream(stream));
}

extern "C" int qa_add_inplace(float * y, const float * x, size_t n, void * stream) {
    if (!y || !x) return qa::fail(QA_ERR_INVALID, "qa_add_inplace: null pointer");
    if (n == 0) return QA_OK;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(qa::add_inplace_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       qa::as_stream(stream), y, x, n);
    QA_LAUNCH_CHECK("add_inplace_kernel");
    return QA_OK;
}

extern "C" int qa_embed_rows(const float * table, int32_t n_rows, int32_t dim, const int32_t * ids, int32_t rows,
                             float * out, void * stream) {
    if (!table || !ids || !out || dim <= 0) return qa::fail(QA_ERR_INVALID, "qa_embed_rows: invalid arguments");
    return qa::embed_rows_launch(table, n_rows, dim, ids, rows, out, qa::as_stream(stream));
}

extern "C" int qa_advance_lens(int32_t * lens, int32_t n, int32_t delta, void * stream) {
    if (!lens) return qa::fail(QA_ERR_INVALID, "qa_advance_lens: null pointer");
    return qa::advance_lens_launch(lens, n, delta, qa::as_stream(stream));
}

namespace qa {
namespace {

__global__ void set_values_kernel(int32_t * dst, int n, int32_t value) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = value;
}

// f32 rows -> cache dtype (f16 rounds to nearest even, like ggml_cpy).
__global__ void cast_rows_kernel(const float * src, void * dst, int f16, int64_t n) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        if (f16) static_cast<_Float16 *>(dst)[i] = static_cast<_Float16>(src[i]);
        else static_cast<float *>(dst)[i] = src[i];
    }
}

}  // namespace

int set_values_launch(int32_t * dst, int32_t n, int32_t value, hipStream_t stream) {
    if (n <= 0) return QA_OK;
    hipLaunchKernelGGL(set_values_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, dst,
                       n, value);
    QA_LAUNCH_CHECK("set_values_kernel");
    return QA_OK;
}

int cast_rows_launch(const float * src, void * dst, int32_t cache_type, int64_t n, hipStream_t stream) {
    if (n <= 0) return QA_OK;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 16384);
    hipLaunchKernelGGL(cast_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, src, dst,
                       cache_type == QA_CACHE_F16 ? 1 : 0, n);
    QA_LAUNCH_CHECK("cast_rows_kernel");
    return QA_OK;
}

}  // namespace qa

extern "C" size_t qa_gemm_rows_workspace_bytes(int32_t out_dim, int32_t in_dim, int32_t rows) {
    return qa::gemm_rows_workspace_bytes(out_dim, in_dim, rows);
}

extern "C" int qa_gemm_rows(const float * W, int32_t out_dim, int32_t in_dim, const float * x, int32_t rows, float * y,
                            int32_t accumulate, void * workspace, size_t workspace_bytes, void * stream) {
    return qa::gemm_rows_launch(W, out_dim, in_dim, x, rows, y, accumulate != 0, workspace, workspace_bytes,
                                qa::as_stream(stream));
}

extern "C" int qa_gemm_rows_fused(const float * W, int32_t out_dim, int32_t in_dim, const float * x, int32_t rows,
                                  float * y, int32_t accumulate, const float * norm_w, const double * stats_in,
                                  int32_t n_stats_in, float eps, double * stats_out, int32_t swiglu,
                                  void * workspace, size_t workspace_bytes, void * stream) {
    qa::GemmRowsFusion f;
    f.norm_w = norm_w;
    f.stats_in = stats_in;
    f.n_stats_in = n_stats_in;
    f.eps = eps;
    f.stats_out = stats_out;
    f.swiglu = swiglu != 0;
    return qa::gemm_rows_launch(W, out_dim, in_dim, x, rows, y, accumulate != 0, workspace, workspace_bytes,
                                qa::as_stream(stream), &f);
}

extern "C" int qa_gemm_rows_fused_bf16(const uint16_t * W_bf16, int32_t out_dim, int32_t in_dim, const float * x,
                                       int32_t rows, float * y, int32_t accumulate, const float * norm_w,
                                       const double * stats_in, int32_t n_stats_in, float eps, double * stats_out,
                                       int32_t swiglu, void * workspace, size_t workspace_bytes, void * stream) {
    if (!W_bf16) return qa::fail(QA_ERR_INVALID, "qa_gemm_rows_fused_bf16: null weights");
    qa::GemmRowsFusion f;
    f.norm_w = norm_w;
    f.stats_in = stats_in;
    f.n_stats_in = n_stats_in;
    f.eps = eps;
    f.stats_out = stats_out;
    f.swiglu = swiglu != 0;
    return qa::gemm_rows_launch(nullptr, out_dim, in_dim, x, rows, y, accumulate != 0, workspace, workspace_bytes,
                                qa::as_stream(stream), &f, W_bf16);
}
