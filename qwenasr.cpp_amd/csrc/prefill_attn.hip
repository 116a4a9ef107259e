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
#include <cstdlib>

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

// f32 K/V on f32 MFMA (v_mfma_f32_16x16x4_f32: exact f32 products, f32 sums).  A workgroup owns 64
// queries x both query heads of one KV head (8 waves: wave w takes head w % 2 and queries 16 (w / 2) ..
// + 15) and walks the keys in tiles of 32, staged in LDS (double-buffered, the next tile in registers
// while the current one is computed).  Each wave computes S^T = K Q^T (keys x queries): the operand
// layout of the product then holds, in each lane, 4 keys of one query, which is exactly the B operand
// of O^T = V^T P^T, so P never moves.  Softmax is online, in f32, with the running sum in double:
// p_j = exp(s_j - m) rescaled as m grows, and o / l at the end -- the same f32 arithmetic as
// prefill_rows_kernel in another association (about 1e-6 relative).
// Lane layouts of v_mfma_f32_16x16x4_f32 (lane l, g = l / 16): A[m = l % 16][k = g], B[k = g][n = l % 16],
// C[m = 4 g + i][n = l % 16], i = 0..3.
constexpr int kF32Tile = 32;                  // keys per tile
constexpr int kF32KLs = kHeadDim + 8;         // K row stride in LDS (floats): 16-byte reads of 16 rows
constexpr int kF32VLs = kHeadDim + 16;        // V row stride: the 4 lane groups read 4 rows of one column
constexpr int kF32Queries = 64;

typedef float f4v __attribute__((ext_vector_type(4)));

// One query block of 64 (8 waves) against its causal key range.
__device__ inline void f32mfma_block(const RowsParams & p, float (*ks)[kF32Tile * kF32KLs],
                                     float (*vs)[kF32Tile * kF32VLs], int qb) {
    const int kvh = blockIdx.y;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int hh = wave & 1, qi = wave >> 1;
    const int q0 = qb * kF32Queries;
    const int qrow = q0 + 16 * qi + c;                              // this lane's query (token index)
    const int qpos = p.n_past + min(qrow, p.n_tokens - 1);          // its position (rows past T: the last)
    const int n_keys = p.n_past + min(q0 + kF32Queries, p.n_tokens);   // keys of the workgroup's last query
    const int n_tiles = (n_keys + kF32Tile - 1) / kF32Tile;

    // q of this lane's query, d = 16 u + 4 g + 0..3 (the B operand order)
    f4v qreg[8];
    {
        const float * qp = p.q + static_cast<int64_t>(min(qrow, p.n_tokens - 1)) * p.q_stride +
                           (kRep * kvh + hh) * kHeadDim + 4 * g;
#pragma unroll
        for (int u = 0; u < 8; ++u) qreg[u] = *reinterpret_cast<const f4v *>(qp + 16 * u);
    }
    const float * kbase = static_cast<const float *>(p.k) + kvh * p.head_stride;
    const float * vbase = static_cast<const float *>(p.v) + kvh * p.head_stride;
    // tile staging: thread t loads 16 bytes at key t / 32 (+ 16), d 4 (t % 32), for K and for V
    const int lk = threadIdx.x >> 5, ld = 4 * (threadIdx.x & 31);
    f4v kr[2], vr[2];
    auto load_tile = [&](int tile) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int key = min(tile * kF32Tile + lk + 16 * h, n_keys - 1);
            kr[h] = *reinterpret_cast<const f4v *>(kbase + static_cast<int64_t>(key) * p.row_stride + ld);
            vr[h] = *reinterpret_cast<const f4v *>(vbase + static_cast<int64_t>(key) * p.row_stride + ld);
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            *reinterpret_cast<f4v *>(&ks[buf][(lk + 16 * h) * kF32KLs + ld]) = kr[h];
            *reinterpret_cast<f4v *>(&vs[buf][(lk + 16 * h) * kF32VLs + ld]) = vr[h];
        }
    };
    load_tile(0);
    store_tile(0);
    if (n_tiles > 1) load_tile(1);
    __syncthreads();

    f4v oacc[8];
#pragma unroll
    for (int db = 0; db < 8; ++db) oacc[db] = f4v{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    double l_run = 0.0;
    for (int t = 0; t < n_tiles; ++t) {
        const int buf = t & 1;
        const float * kt = ks[buf];
        const float * vt = vs[buf];
        // S^T for keys 16 b + 0..15 of the tile
        f4v sacc[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            sacc[b] = f4v{0.f, 0.f, 0.f, 0.f};
            const float * kr_l = kt + (16 * b + c) * kF32KLs + 4 * g;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const f4v a = *reinterpret_cast<const f4v *>(kr_l + 16 * u);
#pragma unroll
                for (int j = 0; j < 4; ++j) sacc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], qreg[u][j], sacc[b], 0, 0, 0);
            }
        }
        // scale, causal mask, online softmax of this lane's query over the tile's 32 keys
        float sv[2][4];
        float mx = -INFINITY;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kp = t * kF32Tile + 16 * b + 4 * g + i;
                const float x = kp <= qpos ? sacc[b][i] * p.scale : -INFINITY;
                sv[b][i] = x;
                mx = fmaxf(mx, x);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float m_new = fmaxf(m_run, mx);
        const float corr = m_run == -INFINITY ? 0.0f : expf(m_run - m_new);
        float psum = 0.0f;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = sv[b][i] == -INFINITY ? 0.0f : expf(sv[b][i] - m_new);
                sv[b][i] = e;
                psum += e;
            }
        }
        psum += __shfl_xor(psum, 16, kWave);
        psum += __shfl_xor(psum, 32, kWave);
        l_run = l_run * static_cast<double>(corr) + static_cast<double>(psum);
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < 8; ++db) oacc[db] *= corr;
        // O^T[d][q] += V^T[d][key] P^T[key][q]: keys 16 b + 4 g + i of the tile in k-slot g of step (b, i)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float * vrow = vt + (16 * b + 4 * g + i) * kF32VLs + c;
#pragma unroll
                for (int db = 0; db < 8; ++db) {
                    oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[16 * db], sv[b][i], oacc[db], 0, 0, 0);
                }
            }
        }
        // stage the next tile (its loads were issued a tile ago) and issue the loads of the one after.
        // Buffer buf ^ 1 last held tile t - 1, which every wave finished before the previous barrier.
        if (t + 1 < n_tiles) {
            store_tile(buf ^ 1);
            if (t + 2 < n_tiles) load_tile(t + 2);
            __syncthreads();
        }
    }
    // oacc[db][i] = O^T[d = 16 db + 4 g + i][q = c]; normalise and store
    if (qrow < p.n_tokens) {
        const float r = static_cast<float>(1.0 / l_run);
        float * out = p.out + static_cast<int64_t>(qrow) * p.out_stride + (kRep * kvh + hh) * kHeadDim + 4 * g;
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            f4v o = oacc[db] * r;
            *reinterpret_cast<f4v *>(out + 16 * db) = o;
        }
    }
}

__global__ __launch_bounds__(512) void prefill_f32mfma_kernel(RowsParams p) {
    __shared__ __attribute__((aligned(16))) float ks[2][kF32Tile * kF32KLs];
    __shared__ __attribute__((aligned(16))) float vs[2][kF32Tile * kF32VLs];
    const int n_qb = (p.n_tokens + kF32Queries - 1) / kF32Queries;
    // causal balance: workgroup i takes query block n_qb - 1 - i, then block i, so every workgroup
    // walks about the same number of key tiles
    const int first = n_qb - 1 - static_cast<int>(blockIdx.x);
    f32mfma_block(p, ks, vs, first);
    const int second = static_cast<int>(blockIdx.x);
    if (second < first) {
        __syncthreads();                 // every wave is done with the first block's LDS tiles
        f32mfma_block(p, ks, vs, second);
    }
}

int launch_f32mfma(const RowsParams & p, int n_kv_heads, hipStream_t stream) {
    const int n_qb = (p.n_tokens + kF32Queries - 1) / kF32Queries;
    hipLaunchKernelGGL(prefill_f32mfma_kernel, dim3(static_cast<unsigned>((n_qb + 1) / 2), static_cast<unsigned>(n_kv_heads)),
                       dim3(512), 0, stream, p);
    QA_LAUNCH_CHECK("prefill_f32mfma_kernel");
    return QA_OK;
}

// QA_PREFILL_F32_ROWS=1 keeps the f32 row kernel (comparison)
bool f32_rows_forced() {
    const char * e = std::getenv("QA_PREFILL_F32_ROWS");
    return e && std::atoi(e) != 0;
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
    if (!f32_rows_forced()) return launch_f32mfma(p, layout.n_kv_heads, stream);
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
    if (!f32_rows_forced()) return launch_f32mfma(p, n_kv_heads, stream);
    return launch_rows<float, false>(p, n_kv_heads, stream);
}

}  // namespace qa

extern "C" int qa_causal_attn_f32(const float * q, const float * k, const float * v, int32_t n_tokens,
                                  int32_t n_heads, int32_t n_kv_heads, float scale, float * out, void * stream) {
    return qa::causal_f32_launch(q, n_heads * qa::kHeadDim, k, v, static_cast<int64_t>(n_kv_heads) * qa::kHeadDim,
                                 n_tokens, n_heads, n_kv_heads, scale, out, n_heads * qa::kHeadDim,
                                 qa::as_stream(stream));
}
