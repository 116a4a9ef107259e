// Causal prefill attention, gfx950.
//
// Replaces the prefill half of the cached layer graph (text-decoder.cpp:435-463 with T > 1 and the
// dense mask of 1729-1735) and the non-cached causal graph (320-334, ggml_diag_mask_inf).  The
// reference materialises the f32 score tensor [L, T, 16] (980 MB per layer at T = 3913) and a
// transposed copy of V; nothing of that size exists here.
//
// Arithmetic = the reference's GGML graph for the K/V dtype: with f16 K/V, q is rounded to f16
// before QK^T and the normalised probabilities are rounded to f16 before PV; scores are scaled,
// the max is exact, expf(x - max) is summed in double and multiplied by (float)(1/sum).
//
// f16 caches run on CDNA4 f16 MFMA (prefill_mfma.hip).  prefill_rows_kernel serves f32 K/V (the
// non-cached layer of text-decoder.cpp:265-345 and f32 caches), where the reference's arithmetic is
// f32 throughout: one workgroup per (query, KV head), both query heads of the GQA group share every
// loaded K/V element, the scores of the query stay in LDS (keys <= 8192).
#include "ops.hpp"

#include <cmath>

namespace qa {
namespace {

constexpr int kRep = 2;
constexpr int kMaxRowsKeys = 8192;

struct RowsParams {
    const float * q;          // [T][q_stride]
    const void * k;           // key row (head 0, position 0)
    const void * v;
    float * out;              // [T][q_stride]
    int64_t head_stride;      // elements between KV heads
    int64_t row_stride;       // elements between positions
    int32_t q_stride;         // elements between the q rows of two tokens
    int32_t out_stride;       // elements between the output rows of two tokens
    int32_t n_past, n_tokens;
    float scale;
};

template <typename CT>
__device__ inline void load8(const CT * p, float (&v)[8]);

template <>
__device__ inline void load8<float>(const float * p, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4 *>(p);
    const float4 b = *reinterpret_cast<const float4 *>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ inline float round_f16(float x) { return static_cast<float>(static_cast<_Float16>(x)); }

template <typename CT, bool R16>
__global__ __launch_bounds__(256) void prefill_rows_kernel(RowsParams p) {
    extern __shared__ float sc[];               // [2][nk_pad]
    const int t = blockIdx.x;
    const int g = blockIdx.y;
    const int nk = p.n_past + t + 1;
    const int nk_pad = (p.n_past + p.n_tokens + 63) & ~63;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int sub = lane >> 4;
    const int part = lane & 15;
    const int h0 = g * kRep;

    float q0[8], q1[8];
    {
        const float * qp = p.q + static_cast<int64_t>(t) * p.q_stride + h0 * kHeadDim + part * 8;
        load8<float>(qp, q0);
        load8<float>(qp + kHeadDim, q1);
        if (R16) {
#pragma unroll
            for (int i = 0; i < 8; ++i) { q0[i] = round_f16(q0[i]); q1[i] = round_f16(q1[i]); }
        }
    }
    const CT * kb = static_cast<const CT *>(p.k) + g * p.head_stride + part * 8;
    const CT * vb = static_cast<const CT *>(p.v) + g * p.head_stride + part * 8;

    // pass 1: scores into LDS, running max
    float m0 = -INFINITY, m1 = -INFINITY;
    for (int j0 = 0; j0 < nk; j0 += 64) {
        float kv[4][8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int j = j0 + k * 16 + wave * 4 + sub;
            if (j < nk) {
                load8<CT>(kb + j * p.row_stride, kv[k]);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) kv[k][i] = 0.0f;
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float a = 0.0f, b = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                a = fmaf(q0[i], kv[k][i], a);
                b = fmaf(q1[i], kv[k][i], b);
            }
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) {
                a += __shfl_xor(a, off, kWave);
                b += __shfl_xor(b, off, kWave);
            }
            const int j = j0 + k * 16 + wave * 4 + sub;
            if (j < nk) {
                a *= p.scale;
                b *= p.scale;
                if (part == 0) { sc[j] = a; sc[nk_pad + j] = b; }
                m0 = fmaxf(m0, a);
                m1 = fmaxf(m1, b);
            }
        }
    }
    __shared__ float smax[2][4];
    __shared__ double ssum[2][4];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        m0 = fmaxf(m0, __shfl_xor(m0, off, kWave));
        m1 = fmaxf(m1, __shfl_xor(m1, off, kWave));
    }
    if (lane == 0) { smax[0][wave] = m0; smax[1][wave] = m1; }
    __syncthreads();
    m0 = fmaxf(fmaxf(smax[0][0], smax[0][1]), fmaxf(smax[0][2], smax[0][3]));
    m1 = fmaxf(fmaxf(smax[1][0], smax[1][1]), fmaxf(smax[1][2], smax[1][3]));

    // pass 2: sum of expf(x - max) in double
    double e0 = 0.0, e1 = 0.0;
    for (int j = threadIdx.x; j < nk; j += 256) {
        e0 += static_cast<double>(expf(sc[j] - m0));
        e1 += static_cast<double>(expf(sc[nk_pad + j] - m1));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        e0 += __shfl_xor(e0, off, kWave);
        e1 += __shfl_xor(e1, off, kWave);
    }
    if (lane == 0) { ssum[0][wave] = e0; ssum[1][wave] = e1; }
    __syncthreads();
    const float r0 = static_cast<float>(1.0 / ((ssum[0][0] + ssum[0][1]) + (ssum[0][2] + ssum[0][3])));
    const float r1 = static_cast<float>(1.0 / ((ssum[1][0] + ssum[1][1]) + (ssum[1][2] + ssum[1][3])));

    // pass 3: o = sum_j p_j V_j
    float a0[8], a1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { a0[i] = 0.0f; a1[i] = 0.0f; }
    for (int j0 = 0; j0 < nk; j0 += 64) {
        float vv[4][8];
        float pa[4], pb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int j = j0 + k * 16 + wave * 4 + sub;
            if (j < nk) {
                load8<CT>(vb + j * p.row_stride, vv[k]);
                float x = expf(sc[j] - m0) * r0;
                float y = expf(sc[nk_pad + j] - m1) * r1;
                if (R16) { x = round_f16(x); y = round_f16(y); }
                pa[k] = x;
                pb[k] = y;
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) vv[k][i] = 0.0f;
                pa[k] = 0.0f;
                pb[k] = 0.0f;
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                a0[i] = fmaf(pa[k], vv[k][i], a0[i]);
                a1[i] = fmaf(pb[k], vv[k][i], a1[i]);
            }
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
    const int hh = threadIdx.x >> 7;
    const int d = threadIdx.x & (kHeadDim - 1);
    p.out[static_cast<int64_t>(t) * p.out_stride + (h0 + hh) * kHeadDim + d] =
        (red[0][hh][d] + red[1][hh][d]) + (red[2][hh][d] + red[3][hh][d]);
}

template <typename CT, bool R16>
int launch_rows(const RowsParams & p, int n_kv_heads, hipStream_t stream) {
    const int nk_pad = (p.n_past + p.n_tokens + 63) & ~63;
    const size_t lds = sizeof(float) * 2 * static_cast<size_t>(nk_pad);
    hipLaunchKernelGGL((prefill_rows_kernel<CT, R16>), dim3(static_cast<unsigned>(p.n_tokens),
                       static_cast<unsigned>(n_kv_heads)), dim3(256), lds, stream, p);
    QA_LAUNCH_CHECK("prefill_rows_kernel");
    return QA_OK;
}

}  // namespace

int prefill_attn_launch(const float * q, int32_t q_stride, const void * cache, const qa_kv_layout & layout,
                        int32_t layer, int32_t stream_idx, int32_t n_past, int32_t n_tokens, int32_t n_heads,
                        float scale, float * out, void * workspace, size_t workspace_bytes, hipStream_t stream) {
    if (layout.head_dim != kHeadDim || n_heads != kRep * layout.n_kv_heads) {
        return fail(QA_ERR_INVALID, "prefill attention: only head_dim 128 with 2 query heads per KV head");
    }
    if (layer < 0 || layer >= layout.n_layers || stream_idx < 0 || stream_idx >= layout.n_streams ||
        n_past < 0 || n_tokens <= 0 || n_past + n_tokens > layout.max_seq) {
        return fail(QA_ERR_INVALID, "prefill attention: invalid layer, stream or range");
    }
    const size_t esz = qa_kv_elem_bytes(layout.cache_type);
    const char * base = static_cast<const char *>(cache);
    const void * k0 = base + esz * cache_row_offset(layer, 0, stream_idx, 0, 0, layout.n_streams, layout.n_kv_heads,
                                                    layout.max_seq);
    const void * v0 = base + esz * cache_row_offset(layer, 1, stream_idx, 0, 0, layout.n_streams, layout.n_kv_heads,
                                                    layout.max_seq);
    if (layout.cache_type == QA_CACHE_F16) {
        return prefill_mfma_launch(q, q_stride, k0, v0, static_cast<int64_t>(layout.max_seq) * kHeadDim, n_past,
                                   n_tokens, layout.n_kv_heads, scale, out, workspace, workspace_bytes, stream);
    }
    if (n_past + n_tokens > kMaxRowsKeys) {
        return fail(QA_ERR_INVALID, "prefill attention: more than 8192 keys with an f32 cache");
    }
    RowsParams p{};
    p.q = q;
    p.out = out;
    p.q_stride = q_stride;
    p.out_stride = q_stride;
    p.n_past = n_past;
    p.n_tokens = n_tokens;
    p.scale = scale;
    p.head_stride = static_cast<int64_t>(layout.max_seq) * kHeadDim;
    p.row_stride = kHeadDim;
    p.k = k0;
    p.v = v0;
    return launch_rows<float, false>(p, layout.n_kv_heads, stream);
}

}  // namespace qa

extern "C" size_t qa_prefill_attn_workspace_bytes(int32_t n_tokens, int32_t n_heads) {
    return qa::prefill_mfma_workspace_bytes(n_tokens, n_heads / qa::kRep);
}

extern "C" int qa_prefill_attn(const float * q, const void * cache, const qa_kv_layout * layout, int32_t layer,
                               int32_t stream_idx, int32_t n_past, int32_t n_tokens, int32_t n_heads, float scale,
                               float * out, void * workspace, size_t workspace_bytes, void * stream) {
    using namespace qa;
    if (qa_kv_layout_check(layout) != QA_OK) return QA_ERR_INVALID;
    if (!q || !cache || !out) return fail(QA_ERR_INVALID, "qa_prefill_attn: null pointer");
    return prefill_attn_launch(q, n_heads * kHeadDim, cache, *layout, layer, stream_idx, n_past, n_tokens, n_heads,
                               scale, out, workspace, workspace_bytes, as_stream(stream));
}

namespace qa {

int causal_f32_launch(const float * q, int32_t q_stride, const float * k, const float * v, int64_t row_stride,
                      int32_t n_tokens, int32_t n_heads, int32_t n_kv_heads, float scale, float * out,
                      int32_t out_stride, hipStream_t stream) {
    if (!q || !k || !v || !out || n_tokens <= 0 || n_kv_heads <= 0 || n_heads != kRep * n_kv_heads) {
        return fail(QA_ERR_INVALID, "causal f32 attention: invalid arguments");
    }
    // every row of q and of the output holds all n_heads heads: the kernel reads and writes
    // [t * stride, t * stride + n_heads * head_dim) of each
    if (q_stride < n_heads * kHeadDim || out_stride < n_heads * kHeadDim || row_stride < kHeadDim * n_kv_heads) {
        return fail(QA_ERR_INVALID, "causal f32 attention: a row stride is shorter than its row");
    }
    if (n_tokens > kMaxRowsKeys) return fail(QA_ERR_INVALID, "causal f32 attention: more than 8192 tokens");
    RowsParams p{};
    p.q = q;
    p.k = k;
    p.v = v;
    p.out = out;
    p.q_stride = q_stride;
    p.out_stride = out_stride;
    p.n_past = 0;
    p.n_tokens = n_tokens;
    p.scale = scale;
    p.head_stride = kHeadDim;
    p.row_stride = row_stride;
    return launch_rows<float, false>(p, n_kv_heads, stream);
}

}  // namespace qa

extern "C" int qa_causal_attn_f32(const float * q, const float * k, const float * v, int32_t n_tokens,
                                  int32_t n_heads, int32_t n_kv_heads, float scale, float * out, void * stream) {
    return qa::causal_f32_launch(q, n_heads * qa::kHeadDim, k, v, static_cast<int64_t>(n_kv_heads) * qa::kHeadDim,
                                 n_tokens, n_heads, n_kv_heads, scale, out, n_heads * qa::kHeadDim,
                                 qa::as_stream(stream));
}
