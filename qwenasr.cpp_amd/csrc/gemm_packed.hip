// Multi-stream decode projections on f32 weights (2..32 token rows), from weights packed at decoder creation in
// the A-operand order of v_mfma_f32_16x16x4_f32.
//
// The f32 path of gemm_rows32_kernel stages 4 weight rows x 256 bytes per load through LDS and merges K slices
// across workgroups (publish, counter, reload); at 32 rows its q|k|v and o projections take ~19.7 us for 33.6 and
// 16.8 MB.  Here the weights are reordered once, so each load instruction reads 1 KB that lands in the MFMA
// A operand as loaded:
//   packed chunk (16-row tile t, step s of 32 k, half j): lane l = (r = l % 16, g = l / 16) holds
//   W[16 t + r][32 s + 16 j + 4 g + e], e = 0..3, at float index ((t S + s) 2 + j) 256 + 4 l + e (S = K / 32).
// The MFMA's k order inside a step is a permutation shared by the A (weights) and B (X) operands, which the
// sum does not see: lane (r, g) of token half h reads X[16 h + r][32 s + 16 j + 4 g + e].
//
// gemm_packed_kernel: one workgroup per 16-row tile over the whole K (8 waves, each a contiguous eighth of the
// steps, 4 steps in flight), X read from L2 per wave, the 8 partial tiles summed in LDS in wave order: no
// cross-workgroup merge.  Fusions as in gemm_rows32_kernel: RMSNorm of X from partial row sums of squares
// (x * scale) * w (text-decoder.cpp:92-98), and accumulation into Y with the 16-column sums of squares of the
// stored rows (the next RMSNorm's statistics).
// gemm_packed_lm_kernel (the LM head, 151936 rows): 128 rows per workgroup (8 waves x 16-row tiles) over the
// whole K; the normalised X is staged in LDS, 256 k at a time in fragment order, and read by all 8 waves, which
// keeps the L2 reads of X at a quarter of the weight bytes (per-wave X reads cost more than the weight stream).
#include "ops.hpp"

namespace qa {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kPkWaves = 8;
constexpr int kPkThreads = kPkWaves * kWave;
constexpr int kPkDepth = 4;      // steps in flight per wave

struct PackedParams {
    const float * Wp;            // packed weights
    const float * X;             // [rows][K]
    float * Y;                   // [rows][N]
    const float * norm_w;        // RMSNorm weight (prenorm) or null
    const double * stats_in;     // [n_stats_in][32]
    double * stats_out;          // [N / 16][32] or null
    int32_t N, K, rows, n_stats_in, accumulate;
    float eps;
};

__global__ __launch_bounds__(256) void pack_f32_kernel(const float * W, int64_t N, int32_t K, float * Wp) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= N * K) return;
    const int64_t S = K / 32;
    const int e = static_cast<int>(i & 3), lane = static_cast<int>((i >> 2) & 63), j = static_cast<int>((i >> 8) & 1);
    const int64_t ts = i >> 9;
    const int64_t s = ts % S, t = ts / S;
    Wp[i] = W[(16 * t + (lane & 15)) * K + 32 * s + 16 * j + 4 * (lane >> 4) + e];
}

// Per-token RMSNorm scale from the partial sums of squares, summed in the order of gemm_rows32_kernel
// (thread (token tid % 32, part tid / 32) adds partials part + 8 j, then the 8 parts in order), so both kernels
// give the same scale: 1 / sqrt(float(sum / K) + eps) (rms_norm_row, text-decoder.cpp:542-557).  The partials
// are loaded first (stats_load, before any weight load: loads complete in issue order) and summed afterwards.
__device__ inline void stats_load(const PackedParams & p, double (&sq)[16]) {
    const int tk = threadIdx.x & 31, part = (threadIdx.x >> 5) & 7;
#pragma unroll
    for (int j = 0; j < 16; ++j) sq[j] = p.stats_in[32 * min(part + 8 * j, p.n_stats_in - 1) + tk];
}

__device__ inline void prenorm_scales(const PackedParams & p, const double (&sq)[16], float * s_scale) {
    __shared__ double s_part[8][32];
    if (threadIdx.x < 256) {
        const int tk = threadIdx.x & 31, part = threadIdx.x >> 5;
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (part + 8 * j < p.n_stats_in) ss += sq[j];
        }
        s_part[part][tk] = ss;
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        double tot = 0.0;
#pragma unroll
        for (int q = 0; q < 8; ++q) tot += s_part[q][threadIdx.x];
        s_scale[threadIdx.x] = 1.0f / sqrtf(static_cast<float>(tot / static_cast<double>(p.K)) + p.eps);
    }
    __syncthreads();
}

// SPW steps of 32 k per wave (K = 32 SPW kPkWaves).
template <int SPW, bool PRENORM>
__global__ __launch_bounds__(kPkThreads) void gemm_packed_kernel(PackedParams p) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int t = blockIdx.x;
    constexpr int S_WAVE = SPW;
    const int S = p.K / 32;
    const int sb = wave * S_WAVE;
    const f4 * wb = reinterpret_cast<const f4 *>(p.Wp) + (static_cast<int64_t>(t) * S + sb) * 128 + lane;
    const int tok0 = min(r16, p.rows - 1), tok1 = min(16 + r16, p.rows - 1);
    const float * x0 = p.X + static_cast<int64_t>(tok0) * p.K + 32 * sb + 4 * g;
    const float * x1 = p.X + static_cast<int64_t>(tok1) * p.K + 32 * sb + 4 * g;
    const float * nb = PRENORM ? p.norm_w + 32 * sb + 4 * g : nullptr;
    constexpr int D = SPW < kPkDepth ? SPW : kPkDepth;
    f4 wv[D][2], xa[D][2], xc[D][2], nv[D][2];
    auto load = [&](int u, int s) {
        wv[u][0] = __builtin_nontemporal_load(wb + s * 128);
        wv[u][1] = __builtin_nontemporal_load(wb + s * 128 + 64);
        xa[u][0] = *reinterpret_cast<const f4 *>(x0 + 32 * s);
        xa[u][1] = *reinterpret_cast<const f4 *>(x0 + 32 * s + 16);
        xc[u][0] = *reinterpret_cast<const f4 *>(x1 + 32 * s);
        xc[u][1] = *reinterpret_cast<const f4 *>(x1 + 32 * s + 16);
        if constexpr (PRENORM) {
            nv[u][0] = *reinterpret_cast<const f4 *>(nb + 32 * s);
            nv[u][1] = *reinterpret_cast<const f4 *>(nb + 32 * s + 16);
        }
    };
    double sq[16];
    if constexpr (PRENORM) stats_load(p, sq);
#pragma unroll
    for (int u = 0; u < D; ++u) load(u, u);
    __builtin_amdgcn_sched_barrier(0);
    __shared__ float s_scale[32];
    float sc0 = 1.0f, sc1 = 1.0f;
    if constexpr (PRENORM) {
        prenorm_scales(p, sq, s_scale);
        sc0 = s_scale[tok0];
        sc1 = s_scale[tok1];
    }
    f4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < S_WAVE; ++s) {
        const int u = s % D;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            f4 b0 = xa[u][j], b1 = xc[u][j];
            if constexpr (PRENORM) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    b0[e] = b0[e] * sc0 * nv[u][j][e];
                    b1[e] = b1[e] * sc1 * nv[u][j][e];
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[u][j][e], b0[e], a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[u][j][e], b1[e], a1, 0, 0, 0);
            }
        }
        if (s + D < S_WAVE) load(u, s + D);
        __builtin_amdgcn_sched_barrier(0);
    }
    // the 8 waves' partial tiles summed in wave order; waves 0 and 1 finish token halves 0 and 1
    __shared__ f4 red[kPkWaves][2][kWave];
    red[wave][0][lane] = a0;
    red[wave][1][lane] = a1;
    __syncthreads();
    if (wave >= 2) return;
    f4 v = red[0][wave][lane];
#pragma unroll
    for (int w = 1; w < kPkWaves; ++w) v += red[w][wave][lane];
    // lane (r16, g) of half h: token 16 h + r16, rows 16 t + 4 g + i (16x16 MFMA output layout)
    const int tok = 16 * wave + r16;
    const bool live = tok < p.rows;
    float * y = p.Y + static_cast<int64_t>(min(tok, p.rows - 1)) * p.N + 16 * t + 4 * g;
    // the 4 old values in one 16-byte load (N is a multiple of 16)
    const f4 old = p.accumulate ? *reinterpret_cast<const f4 *>(y) : f4{};
    double ss = 0.0;
    if (live) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float o = p.accumulate ? old[i] + v[i] : v[i];
            y[i] = o;
            ss += static_cast<double>(o) * o;
        }
    }
    if (p.stats_out) {
        // the token's 16 rows are held by lanes r16 + 16 g: sums in a fixed order
        ss += __shfl_xor(ss, 16, kWave);
        ss += __shfl_xor(ss, 32, kWave);
        if (g == 0 && live) p.stats_out[32 * t + tok] = ss;
    }
}

constexpr int kLmChunk = 256;             // k per staged X chunk
constexpr int kLmSteps = kLmChunk / 32;   // 8 steps per chunk

// LM head: workgroup = 8 waves x 16-row tiles (128 rows) over the whole K, X (normalised) staged in LDS.
__global__ __launch_bounds__(kPkThreads) void gemm_packed_lm_kernel(PackedParams p) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int tile = blockIdx.x * kPkWaves + wave;
    const int S = p.K / 32;
    const int n_chunks = p.K / kLmChunk;
    const f4 * wb = reinterpret_cast<const f4 *>(p.Wp) + static_cast<int64_t>(tile) * S * 128 + lane;
    __shared__ f4 xs[2][kLmSteps * 4 * kWave];   // [buffer][step][half * 2 + j][lane]: 2 x 32 KB
    __shared__ float s_scale[32];
    // staging: slot q of thread tt is tt + 512 q (2048 slots per chunk, 4 per thread)
    auto stage_load = [&](int c, f4 (&v)[4], f4 (&w)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int slot = static_cast<int>(threadIdx.x) + kPkThreads * q;
            const int l = slot & 63, hj = (slot >> 6) & 3, s = slot >> 8;
            const int tok = min(16 * (hj >> 1) + (l & 15), p.rows - 1);
            const int k = c * kLmChunk + 32 * s + 16 * (hj & 1) + 4 * (l >> 4);
            v[q] = *reinterpret_cast<const f4 *>(p.X + static_cast<int64_t>(tok) * p.K + k);
            w[q] = *reinterpret_cast<const f4 *>(p.norm_w + k);
        }
    };
    auto stage_store = [&](int b, const f4 (&v)[4], const f4 (&w)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int slot = static_cast<int>(threadIdx.x) + kPkThreads * q;
            const int l = slot & 63, hj = (slot >> 6) & 3;
            const float sc = s_scale[min(16 * (hj >> 1) + (l & 15), p.rows - 1)];
            f4 x = v[q];
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = x[e] * sc * w[q][e];
            xs[b][slot] = x;
        }
    };
    f4 wv[kPkDepth][2];
    auto wload = [&](int u, int s) {
        wv[u][0] = __builtin_nontemporal_load(wb + s * 128);
        wv[u][1] = __builtin_nontemporal_load(wb + s * 128 + 64);
    };
    double sq[16];
    stats_load(p, sq);
    f4 xv[4], nw[4];
    stage_load(0, xv, nw);
#pragma unroll
    for (int u = 0; u < kPkDepth; ++u) wload(u, u);
    __builtin_amdgcn_sched_barrier(0);
    prenorm_scales(p, sq, s_scale);
    stage_store(0, xv, nw);
    __syncthreads();
    f4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < n_chunks; ++c) {
        const int b = c & 1;
        const bool more = c + 1 < n_chunks;
        if (more) stage_load(c + 1, xv, nw);
#pragma unroll
        for (int s = 0; s < kLmSteps; ++s) {
            const int gs = c * kLmSteps + s;
            const int u = s % kPkDepth;             // kLmSteps is a multiple of kPkDepth
            const f4 * xb = &xs[b][s * 256 + lane];
            const f4 x00 = xb[0], x01 = xb[64], x10 = xb[128], x11 = xb[192];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[u][0][e], x00[e], a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[u][0][e], x10[e], a1, 0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[u][1][e], x01[e], a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[u][1][e], x11[e], a1, 0, 0, 0);
            }
            // unconditional (past the end: the last step again, an L2 hit) so the waits stay exact
            wload(u, min(gs + kPkDepth, S - 1));
            __builtin_amdgcn_sched_barrier(0);
        }
        if (more) stage_store(b ^ 1, xv, nw);
        __syncthreads();
    }
    const int row = 16 * tile + 4 * g;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int tok = 16 * h + r16;
        const f4 v = h ? a1 : a0;
        if (tok < p.rows) {
            float * y = p.Y + static_cast<int64_t>(tok) * p.N + row;
#pragma unroll
            for (int i = 0; i < 4; ++i) y[i] = v[i];
        }
    }
}

}  // namespace

bool packed_gemm_shape_ok(int32_t N, int32_t K, bool lm_head) {
    if (N <= 0 || K <= 0) return false;
    if (lm_head) return N % 128 == 0 && K % kLmChunk == 0 && K / 32 >= kPkDepth;
    return N % 16 == 0 && (K == 1024 || K == 2048);
}

int pack_f32_launch(const float * W, int32_t N, int32_t K, float * Wp, hipStream_t stream) {
    if (!W || !Wp || N <= 0 || N % 16 != 0 || K <= 0 || K % 32 != 0) return fail(QA_ERR_INVALID, "pack_f32: invalid shape");
    const int64_t n = static_cast<int64_t>(N) * K;
    hipLaunchKernelGGL(pack_f32_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, W,
                       static_cast<int64_t>(N), K, Wp);
    QA_LAUNCH_CHECK("pack_f32_kernel");
    return QA_OK;
}

int gemm_packed_launch(const float * Wp, int32_t N, int32_t K, const float * X, int32_t rows, float * Y, bool accumulate,
                       const GemmRowsFusion * fusion, bool lm_head, hipStream_t stream) {
    if (!Wp || !X || !Y || rows < 1 || rows > 32 || !packed_gemm_shape_ok(N, K, lm_head)) {
        return fail(QA_ERR_INVALID, "gemm_packed: invalid shape");
    }
    PackedParams p{};
    p.Wp = Wp;
    p.X = X;
    p.Y = Y;
    p.N = N;
    p.K = K;
    p.rows = rows;
    p.accumulate = accumulate ? 1 : 0;
    const bool prenorm = fusion && fusion->norm_w;
    if (prenorm) {
        if (!fusion->stats_in || fusion->n_stats_in < 1 || fusion->n_stats_in > 128) {
            return fail(QA_ERR_INVALID, "gemm_packed: RMSNorm input needs 1..128 partial sums per row");
        }
        p.norm_w = fusion->norm_w;
        p.stats_in = fusion->stats_in;
        p.n_stats_in = fusion->n_stats_in;
        p.eps = fusion->eps;
    }
    if (fusion) p.stats_out = fusion->stats_out;
    if (lm_head) {
        if (!prenorm || accumulate || p.stats_out) return fail(QA_ERR_INVALID, "gemm_packed: the LM head form is RMSNorm -> store");
        hipLaunchKernelGGL(gemm_packed_lm_kernel, dim3(static_cast<unsigned>(N / 128)), dim3(kPkThreads), 0, stream, p);
        QA_LAUNCH_CHECK("gemm_packed_lm_kernel");
        return QA_OK;
    }
    const dim3 grid(static_cast<unsigned>(N / 16));
    if (K == 2048) {
        if (prenorm) hipLaunchKernelGGL((gemm_packed_kernel<8, true>), grid, dim3(kPkThreads), 0, stream, p);
        else hipLaunchKernelGGL((gemm_packed_kernel<8, false>), grid, dim3(kPkThreads), 0, stream, p);
    } else {
        if (prenorm) hipLaunchKernelGGL((gemm_packed_kernel<4, true>), grid, dim3(kPkThreads), 0, stream, p);
        else hipLaunchKernelGGL((gemm_packed_kernel<4, false>), grid, dim3(kPkThreads), 0, stream, p);
    }
    QA_LAUNCH_CHECK("gemm_packed_kernel");
    return QA_OK;
}

}  // namespace qa
