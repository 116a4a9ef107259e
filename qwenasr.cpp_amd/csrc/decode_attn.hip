// Split-K GQA decode attention over the KV cache, gfx950.
//
// Replaces the decode half of backend_text_layer_forward_cached_ggml (text-decoder.cpp:435-463):
//   scores = mul_mat(K[0,L), q); soft_max_ext(scores, mask, 1/sqrt(d)); out = mul_mat(cont(V^T), p)
// including the transposed copy of V that the reference materialises on every call (459): V is read
// row-wise here, so each K and V byte of the prefix is read from HBM exactly once.
//
// The reference's arithmetic with an f16 cache rounds q to f16 before QK^T and the *normalised*
// probabilities to f16 before PV (GGML mul_mat converts src1 to src0's dot type).  Normalised p needs
// the global max and sum before any PV, so the work is split in two launches:
//   K pass  grid (split, kv_head, stream): scores of both query heads of the group for 64 positions,
//           written to the workspace with that split's max and sum(exp(x - max)) (sum in double).
//   V pass  same grid: global max/sum from the split stats, p = f16(expf(x - max) * (1/sum)),
//           partial o for the split, then the last workgroup of each (stream, kv_head) adds the
//           partials in split order and writes o.  Its counter is reset by that same workgroup, so no
//           memset is ever needed between calls (the launch sequence is graph-capturable).
// Memory layout inside a split: 16 lanes cover one 128-wide row (8 elements = 16 B of f16 per lane),
// so one wave load fetches 4 consecutive rows = 1 KB; both query heads of the GQA group use every
// loaded K/V element from registers, which is where the reference's broadcast of KV head h/2 lives.
#include "ops.hpp"

#include <cmath>

namespace qa {
namespace {

constexpr int kSplit = 64;          // positions per workgroup
constexpr int kThreads = 256;       // 4 waves, 16 positions each
constexpr int kRep = 2;             // query heads per KV head (Qwen3-ASR: 16 / 8)

struct SplitStat {
    float m;
    float pad;
    double s;
};

struct DecodeParams {
    const float * q;          // [S][q_stride]
    const void * cache;
    float * out;              // [S][q_stride]
    const int32_t * lens;     // attended length = lens[s] + lens_add
    float * scores;           // [S][H][score_stride]
    SplitStat * stats;        // [S][H][max_splits]
    float * partial;          // [S][max_splits][H][128]
    uint32_t * counters;      // [S][n_kv]
    int32_t lens_add;
    int32_t q_stride;
    int32_t n_heads, n_kv_heads, n_streams, max_seq, layer;
    int32_t max_len, max_splits, score_stride;
    float scale;
};

struct Workspace {
    size_t scores, stats, partial, counters, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

Workspace workspace_layout(int32_t n_streams, int32_t n_heads, int32_t max_len) {
    const size_t splits = (static_cast<size_t>(max_len) + kSplit - 1) / kSplit;
    const size_t stride = splits * kSplit;
    Workspace w{};
    w.scores = 0;
    w.stats = align256(w.scores + sizeof(float) * n_streams * n_heads * stride);
    w.partial = align256(w.stats + sizeof(SplitStat) * n_streams * n_heads * splits);
    w.counters = align256(w.partial + sizeof(float) * n_streams * splits * n_heads * kHeadDim);
    w.total = align256(w.counters + sizeof(uint32_t) * n_streams * (n_heads / kRep));
    return w;
}

template <typename CT>
struct RowSlice;

// 8 consecutive elements of a row as floats (16 B load for f16, 2 x 16 B for f32).
template <>
struct RowSlice<_Float16> {
    static __device__ inline void load(const _Float16 * p, float (&v)[8]) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        const h8 x = *reinterpret_cast<const h8 *>(p);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(x[i]);
    }
};

template <>
struct RowSlice<float> {
    static __device__ inline void load(const float * p, float (&v)[8]) {
        const float4 a = *reinterpret_cast<const float4 *>(p);
        const float4 b = *reinterpret_cast<const float4 *>(p + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
};

__device__ inline float round_f16(float x) { return static_cast<float>(static_cast<_Float16>(x)); }

__device__ inline float group16_sum(float v) {
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

template <typename CT, bool R16>
__global__ __launch_bounds__(kThreads) void decode_scores_kernel(DecodeParams p) {
    const int c = blockIdx.x, g = blockIdx.y, s = blockIdx.z;
    const int L = min(p.lens[s] + p.lens_add, p.max_len);   // never past the rows the launch was sized for
    const int row0 = c * kSplit;
    if (row0 >= L) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int sub = lane >> 4;
    const int part = lane & 15;
    const int h0 = g * kRep;

    float q0[8], q1[8];
    {
        const float * qp = p.q + static_cast<int64_t>(s) * p.q_stride + h0 * kHeadDim + part * 8;
        RowSlice<float>::load(qp, q0);
        RowSlice<float>::load(qp + kHeadDim, q1);
        if (R16) {
#pragma unroll
            for (int i = 0; i < 8; ++i) { q0[i] = round_f16(q0[i]); q1[i] = round_f16(q1[i]); }
        }
    }
    const CT * kbase = static_cast<const CT *>(p.cache) +
        cache_row_offset(p.layer, 0, s, g, 0, p.n_streams, p.n_kv_heads, p.max_seq) + part * 8;

    float kv[4][8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int j = row0 + wave * 16 + k * 4 + sub;
        if (j < L) {
            RowSlice<CT>::load(kbase + static_cast<int64_t>(j) * kHeadDim, kv[k]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) kv[k][i] = 0.0f;
        }
    }
    float x0[4], x1[4];
    float m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            a = fmaf(q0[i], kv[k][i], a);
            b = fmaf(q1[i], kv[k][i], b);
        }
        a = group16_sum(a) * p.scale;
        b = group16_sum(b) * p.scale;
        const int j = row0 + wave * 16 + k * 4 + sub;
        const bool valid = j < L;
        x0[k] = valid ? a : -INFINITY;
        x1[k] = valid ? b : -INFINITY;
        if (valid && part == 0) {
            float * sp = p.scores + (static_cast<int64_t>(s) * p.n_heads + h0) * p.score_stride + j;
            sp[0] = a;
            sp[p.score_stride] = b;
        }
        m0 = fmaxf(m0, x0[k]);
        m1 = fmaxf(m1, x1[k]);
    }
    // max over the 4 row groups of the wave, then over the 4 waves
    m0 = fmaxf(m0, __shfl_xor(m0, 16, kWave)); m0 = fmaxf(m0, __shfl_xor(m0, 32, kWave));
    m1 = fmaxf(m1, __shfl_xor(m1, 16, kWave)); m1 = fmaxf(m1, __shfl_xor(m1, 32, kWave));
    __shared__ float smax[2][4];
    __shared__ double ssum[2][4];
    if (lane == 0) { smax[0][wave] = m0; smax[1][wave] = m1; }
    __syncthreads();
    m0 = fmaxf(fmaxf(smax[0][0], smax[0][1]), fmaxf(smax[0][2], smax[0][3]));
    m1 = fmaxf(fmaxf(smax[1][0], smax[1][1]), fmaxf(smax[1][2], smax[1][3]));

    double e0 = 0.0, e1 = 0.0;
    if (part == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (x0[k] != -INFINITY) e0 += static_cast<double>(expf(x0[k] - m0));
            if (x1[k] != -INFINITY) e1 += static_cast<double>(expf(x1[k] - m1));
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        e0 += __shfl_xor(e0, off, kWave);
        e1 += __shfl_xor(e1, off, kWave);
    }
    if (lane == 0) { ssum[0][wave] = e0; ssum[1][wave] = e1; }
    __syncthreads();
    if (threadIdx.x < 2) {
        const int h = threadIdx.x;
        SplitStat st;
        st.m = h == 0 ? m0 : m1;
        st.pad = 0.0f;
        st.s = (ssum[h][0] + ssum[h][1]) + (ssum[h][2] + ssum[h][3]);
        p.stats[(static_cast<int64_t>(s) * p.n_heads + h0 + h) * p.max_splits + c] = st;
    }
}

template <typename CT, bool R16>
__global__ __launch_bounds__(kThreads) void decode_values_kernel(DecodeParams p) {
    const int c = blockIdx.x, g = blockIdx.y, s = blockIdx.z;
    const int L = min(p.lens[s] + p.lens_add, p.max_len);   // never past the rows the launch was sized for
    const int n_splits = (L + kSplit - 1) / kSplit;
    if (c >= n_splits) return;
    const int row0 = c * kSplit;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int sub = lane >> 4;
    const int part = lane & 15;
    const int h0 = g * kRep;

    // global max and sum of the two heads from the split statistics (every wave, redundantly)
    const SplitStat * st0 = p.stats + (static_cast<int64_t>(s) * p.n_heads + h0) * p.max_splits;
    const SplitStat * st1 = st0 + p.max_splits;
    float M0 = -INFINITY, M1 = -INFINITY;
    for (int i = lane; i < n_splits; i += kWave) {
        M0 = fmaxf(M0, st0[i].m);
        M1 = fmaxf(M1, st1[i].m);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        M0 = fmaxf(M0, __shfl_xor(M0, off, kWave));
        M1 = fmaxf(M1, __shfl_xor(M1, off, kWave));
    }
    double S0 = 0.0, S1 = 0.0;
    for (int i = lane; i < n_splits; i += kWave) {
        S0 += st0[i].s * exp(static_cast<double>(st0[i].m) - static_cast<double>(M0));
        S1 += st1[i].s * exp(static_cast<double>(st1[i].m) - static_cast<double>(M1));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        S0 += __shfl_xor(S0, off, kWave);
        S1 += __shfl_xor(S1, off, kWave);
    }
    const float r0 = static_cast<float>(1.0 / S0);
    const float r1 = static_cast<float>(1.0 / S1);

    const CT * vbase = static_cast<const CT *>(p.cache) +
        cache_row_offset(p.layer, 1, s, g, 0, p.n_streams, p.n_kv_heads, p.max_seq) + part * 8;
    const float * sc0 = p.scores + (static_cast<int64_t>(s) * p.n_heads + h0) * p.score_stride;
    const float * sc1 = sc0 + p.score_stride;

    float vv[4][8];
    float p0[4], p1[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int j = row0 + wave * 16 + k * 4 + sub;
        if (j < L) {
            RowSlice<CT>::load(vbase + static_cast<int64_t>(j) * kHeadDim, vv[k]);
            float a = expf(sc0[j] - M0) * r0;
            float b = expf(sc1[j] - M1) * r1;
            if (R16) { a = round_f16(a); b = round_f16(b); }
            p0[k] = a;
            p1[k] = b;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) vv[k][i] = 0.0f;
            p0[k] = 0.0f;
            p1[k] = 0.0f;
        }
    }
    float a0[8], a1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { a0[i] = 0.0f; a1[i] = 0.0f; }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            a0[i] = fmaf(p0[k], vv[k][i], a0[i]);
            a1[i] = fmaf(p1[k], vv[k][i], a1[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a0[i] += __shfl_xor(a0[i], 16, kWave); a0[i] += __shfl_xor(a0[i], 32, kWave);
        a1[i] += __shfl_xor(a1[i], 16, kWave); a1[i] += __shfl_xor(a1[i], 32, kWave);
    }
    __shared__ float red[4][kRep][kHeadDim];
    if (sub == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            red[wave][0][part * 8 + i] = a0[i];
            red[wave][1][part * 8 + i] = a1[i];
        }
    }
    __syncthreads();
    const int hh = threadIdx.x >> 7;          // 0..1
    const int d = threadIdx.x & (kHeadDim - 1);
    const float sum = (red[0][hh][d] + red[1][hh][d]) + (red[2][hh][d] + red[3][hh][d]);
    float * part_out = p.partial +
        ((static_cast<int64_t>(s) * p.max_splits + c) * p.n_heads + h0 + hh) * kHeadDim;
    part_out[d] = sum;

    __threadfence();
    __syncthreads();
    __shared__ int is_last;
    if (threadIdx.x == 0) {
        uint32_t * ctr = p.counters + static_cast<int64_t>(s) * p.n_kv_heads + g;
        const uint32_t old = atomicAdd(ctr, 1u);
        is_last = old == static_cast<uint32_t>(n_splits - 1);
        if (is_last) atomicExch(ctr, 0u);
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    const float * pp = p.partial +
        (static_cast<int64_t>(s) * p.max_splits * p.n_heads + h0 + hh) * kHeadDim + d;
    const int64_t step = static_cast<int64_t>(p.n_heads) * kHeadDim;
    float acc = 0.0f;
    for (int i = 0; i < n_splits; ++i) acc += __builtin_nontemporal_load(pp + i * step);
    p.out[static_cast<int64_t>(s) * p.q_stride + (h0 + hh) * kHeadDim + d] = acc;
}

}  // namespace

int decode_attn_launch(const float * q, int32_t q_stride, const void * cache, const qa_kv_layout & layout,
                       int32_t layer, const int32_t * lens, int32_t lens_add, int32_t n_streams,
                       int32_t max_len, int32_t n_heads, float scale, float * out, void * workspace,
                       size_t workspace_bytes, hipStream_t stream) {
    if (layout.head_dim != kHeadDim || n_heads != kRep * layout.n_kv_heads) {
        return fail(QA_ERR_INVALID, "decode attention: only head_dim 128 with 2 query heads per KV head");
    }
    if (n_streams <= 0 || n_streams > layout.n_streams || max_len <= 0 || max_len > layout.max_seq ||
        layer < 0 || layer >= layout.n_layers) {
        return fail(QA_ERR_INVALID, "decode attention: invalid streams, length or layer");
    }
    const Workspace w = workspace_layout(n_streams, n_heads, max_len);
    if (!workspace || workspace_bytes < w.total) {
        return fail(QA_ERR_INVALID, "decode attention: workspace too small");
    }
    char * base = static_cast<char *>(workspace);
    DecodeParams p{};
    p.q = q;
    p.cache = cache;
    p.out = out;
    p.lens = lens;
    p.lens_add = lens_add;
    p.scores = reinterpret_cast<float *>(base + w.scores);
    p.stats = reinterpret_cast<SplitStat *>(base + w.stats);
    p.partial = reinterpret_cast<float *>(base + w.partial);
    p.counters = reinterpret_cast<uint32_t *>(base + w.counters);
    p.q_stride = q_stride;
    p.n_heads = n_heads;
    p.n_kv_heads = layout.n_kv_heads;
    p.n_streams = layout.n_streams;
    p.max_seq = layout.max_seq;
    p.layer = layer;
    p.max_len = max_len;
    p.max_splits = (max_len + kSplit - 1) / kSplit;
    p.score_stride = p.max_splits * kSplit;
    p.scale = scale;
    const dim3 grid(static_cast<unsigned>(p.max_splits), static_cast<unsigned>(layout.n_kv_heads),
                    static_cast<unsigned>(n_streams));
    if (layout.cache_type == QA_CACHE_F16) {
        hipLaunchKernelGGL((decode_scores_kernel<_Float16, true>), grid, dim3(kThreads), 0, stream, p);
        QA_LAUNCH_CHECK("decode_scores_kernel");
        hipLaunchKernelGGL((decode_values_kernel<_Float16, true>), grid, dim3(kThreads), 0, stream, p);
        QA_LAUNCH_CHECK("decode_values_kernel");
    } else {
        hipLaunchKernelGGL((decode_scores_kernel<float, false>), grid, dim3(kThreads), 0, stream, p);
        QA_LAUNCH_CHECK("decode_scores_kernel");
        hipLaunchKernelGGL((decode_values_kernel<float, false>), grid, dim3(kThreads), 0, stream, p);
        QA_LAUNCH_CHECK("decode_values_kernel");
    }
    return QA_OK;
}

size_t decode_attn_workspace(int32_t n_streams, int32_t n_heads, int32_t max_len) {
    if (n_streams <= 0 || n_heads <= 0 || max_len <= 0) return 0;
    return workspace_layout(n_streams, n_heads, max_len).total;
}

}  // namespace qa

extern "C" size_t qa_decode_attn_workspace_bytes(int32_t n_streams, int32_t n_heads, int32_t max_len) {
    return qa::decode_attn_workspace(n_streams, n_heads, max_len);
}

extern "C" int qa_decode_attn(const float * q, const void * cache, const qa_kv_layout * layout, int32_t layer,
                              const int32_t * lens, int32_t n_streams, int32_t max_len, int32_t n_heads,
                              float scale, float * out, void * workspace, size_t workspace_bytes, void * stream) {
    using namespace qa;
    if (qa_kv_layout_check(layout) != QA_OK) return QA_ERR_INVALID;
    if (!q || !cache || !lens || !out) return fail(QA_ERR_INVALID, "qa_decode_attn: null pointer");
    return decode_attn_launch(q, n_heads * kHeadDim, cache, *layout, layer, lens, 0, n_streams, max_len,
                              n_heads, scale, out, workspace, workspace_bytes, as_stream(stream));
}
