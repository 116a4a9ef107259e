// Fused q/k/v preparation and KV-cache append for gfx950.
//
// Replaces, per cached layer call, the GGML chain of text-decoder.cpp:377-433:
//   rms_norm(q,k) * {q,k}_norm_w -> rope_ext(NEOX) -> cont(permute) -> cpy into the cache view.
// One wavefront owns one 128-wide head row; lane i holds elements i and i + 64, which is exactly a
// NEOX rotation pair, so RMSNorm needs one wave reduction and RoPE needs no data exchange at all.
// The arithmetic follows the reference's scalar statement bit for bit where it can
// (rms_norm_row 542-557, apply_rope_position 604-625): squares summed in double, float scale,
// (x * scale) * w, angles in double from a host-computed inv_freq table, no FMA contraction.
#include "ops.hpp"
#include "prep.hpp"

#include <cmath>

namespace qa {

RopeTable make_rope_table(float theta) {
    RopeTable t;
    const double log_theta = std::log(static_cast<double>(theta));
    for (int i = 0; i < kHeadDim / 2; ++i) {
        t.inv_freq[i] = std::exp(-log_theta * static_cast<double>(2 * i) / static_cast<double>(kHeadDim));
    }
    return t;
}

namespace {

enum PrepMode { kPrepCacheF32 = 0, kPrepCacheF16 = 1, kPrepInPlace = 2 };

struct PrepParams {
    float * qkv;              // [rows][q_dim + 2 kv_dim]; written in place only in kPrepInPlace
    const float * q_norm_w;
    const float * k_norm_w;
    float * q_out;            // [rows][q_dim]            (cache modes)
    void * cache;             // K+V allocation          (cache modes)
    const int32_t * n_past;   // [n_streams]             (cache modes)
    int32_t pos0;             //                          (in-place mode)
    int32_t n_rows, n_tokens, n_heads, n_kv_heads, n_streams, max_seq, layer;
    float eps;
};

// One workgroup per token row; wave w prepares the head slots w, w + 4, w + 8, ... of the row (q heads,
// then k heads, then v heads).  The RoPE angles depend only on the position, so each wave evaluates
// its lane's cos/sin once for all of its q and k heads.  Every load of a group of 8 slots is issued
// before the first arithmetic; slots past the end re-read the last slot and are not stored.
template <int MODE>
__global__ __launch_bounds__(256) void qkv_prep_kernel(PrepParams p, RopeTable rope) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int row = blockIdx.x;
    const int slots = MODE == kPrepInPlace ? p.n_heads + p.n_kv_heads : p.n_heads + 2 * p.n_kv_heads;
    if (row >= p.n_rows) return;

    const int stream = row / p.n_tokens;
    const int t = row - stream * p.n_tokens;
    const int pos = MODE == kPrepInPlace ? p.pos0 + t : p.n_past[stream] + t;
    if (MODE != kPrepInPlace && (pos < 0 || pos >= p.max_seq)) return;   // uniform for the workgroup

    const int q_dim = p.n_heads * kHeadDim;
    const int row_width = (p.n_heads + 2 * p.n_kv_heads) * kHeadDim;
    float * src_row = p.qkv + static_cast<int64_t>(row) * row_width;
    const double inv_freq = rope.inv_freq[lane];
    const float wqa = p.q_norm_w[lane], wqb = p.q_norm_w[lane + 64];
    const float wka = p.k_norm_w[lane], wkb = p.k_norm_w[lane + 64];
    constexpr int kPer = 8;
    float a[kPer], b[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int slot = min(wave + 4 * u, slots - 1);
        a[u] = src_row[slot * kHeadDim + lane];
        b[u] = src_row[slot * kHeadDim + lane + 64];
    }
    float c, s;
    rope_cos_sin(pos, inv_freq, c, s);
    for (int s0 = wave;; s0 += 4 * kPer) {
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int slot = s0 + 4 * u;
            if (slot >= slots) break;                   // uniform for the wave
            float ra = a[u], rb = b[u];
            if (slot < p.n_heads + p.n_kv_heads) {
                const bool is_q = slot < p.n_heads;
                norm_rope_pair_cs(ra, rb, is_q ? wqa : wka, is_q ? wqb : wkb, p.eps, c, s);
                if (MODE == kPrepInPlace) {
                    src_row[slot * kHeadDim + lane] = ra;
                    src_row[slot * kHeadDim + lane + 64] = rb;
                    continue;
                }
                if (is_q) {
                    float * dst = p.q_out + static_cast<int64_t>(row) * q_dim + slot * kHeadDim;
                    dst[lane] = ra;
                    dst[lane + 64] = rb;
                    continue;
                }
            }
            // k (normed and rotated above) or v (stored raw, text-decoder.cpp:411, 433), cast to the
            // cache dtype
            const bool is_v = slot >= p.n_heads + p.n_kv_heads;
            const int head = slot - p.n_heads - (is_v ? p.n_kv_heads : 0);
            const int64_t off = cache_row_offset(p.layer, is_v ? 1 : 0, stream, head, pos, p.n_streams, p.n_kv_heads,
                                                 p.max_seq);
            if (MODE == kPrepCacheF16) {
                _Float16 * dst = static_cast<_Float16 *>(p.cache) + off;
                dst[lane] = static_cast<_Float16>(ra);
                dst[lane + 64] = static_cast<_Float16>(rb);
            } else {
                float * dst = static_cast<float *>(p.cache) + off;
                dst[lane] = ra;
                dst[lane + 64] = rb;
            }
        }
        if (s0 + 4 * kPer >= slots) break;
        // next group of slots (more than 32 head slots per row)
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int slot = min(s0 + 4 * kPer + 4 * u, slots - 1);
            a[u] = src_row[slot * kHeadDim + lane];
            b[u] = src_row[slot * kHeadDim + lane + 64];
        }
    }
}

int launch_prep(int mode, const PrepParams & p, float rope_theta, hipStream_t stream) {
    const int64_t blocks = p.n_rows;
    if (blocks <= 0) return QA_OK;
    const RopeTable rope = make_rope_table(rope_theta);
    const dim3 grid(static_cast<unsigned>(blocks));
    switch (mode) {
        case kPrepCacheF32: hipLaunchKernelGGL(qkv_prep_kernel<kPrepCacheF32>, grid, dim3(256), 0, stream, p, rope); break;
        case kPrepCacheF16: hipLaunchKernelGGL(qkv_prep_kernel<kPrepCacheF16>, grid, dim3(256), 0, stream, p, rope); break;
        default: hipLaunchKernelGGL(qkv_prep_kernel<kPrepInPlace>, grid, dim3(256), 0, stream, p, rope); break;
    }
    QA_LAUNCH_CHECK("qkv_prep_kernel");
    return QA_OK;
}

}  // namespace
}  // namespace qa

extern "C" int qa_kv_append(const float * qkv, const float * q_norm_w, const float * k_norm_w,
                            float * q_out, void * cache, const qa_kv_layout * layout, int32_t layer,
                            const int32_t * n_past, int32_t n_streams, int32_t n_tokens, int32_t n_heads,
                            float rope_theta, float eps, void * stream) {
    using namespace qa;
    if (qa_kv_layout_check(layout) != QA_OK) return QA_ERR_INVALID;
    if (!qkv || !q_norm_w || !k_norm_w || !q_out || !cache || !n_past) {
        return fail(QA_ERR_INVALID, "qa_kv_append: null pointer");
    }
    if (layout->head_dim != kHeadDim || layer < 0 || layer >= layout->n_layers || n_streams <= 0 ||
        n_streams > layout->n_streams || n_tokens <= 0 || n_heads <= 0 || n_heads % layout->n_kv_heads != 0) {
        return fail(QA_ERR_INVALID, "qa_kv_append: invalid shape");
    }
    PrepParams p{};
    p.qkv = const_cast<float *>(qkv);
    p.q_norm_w = q_norm_w;
    p.k_norm_w = k_norm_w;
    p.q_out = q_out;
    p.cache = cache;
    p.n_past = n_past;
    p.n_rows = n_streams * n_tokens;
    p.n_tokens = n_tokens;
    p.n_heads = n_heads;
    p.n_kv_heads = layout->n_kv_heads;
    p.n_streams = layout->n_streams;
    p.max_seq = layout->max_seq;
    p.layer = layer;
    p.eps = eps;
    return launch_prep(layout->cache_type == QA_CACHE_F16 ? kPrepCacheF16 : kPrepCacheF32, p, rope_theta,
                       as_stream(stream));
}

extern "C" int qa_qk_prep(float * qkv, int32_t n_tokens, int32_t n_heads, int32_t n_kv_heads,
                          const float * q_norm_w, const float * k_norm_w, int32_t pos0, float rope_theta,
                          float eps, void * stream) {
    using namespace qa;
    if (!qkv || !q_norm_w || !k_norm_w || n_tokens <= 0 || n_heads <= 0 || n_kv_heads <= 0) {
        return fail(QA_ERR_INVALID, "qa_qk_prep: invalid arguments");
    }
    PrepParams p{};
    p.qkv = qkv;
    p.q_norm_w = q_norm_w;
    p.k_norm_w = k_norm_w;
    p.pos0 = pos0;
    p.n_rows = n_tokens;
    p.n_tokens = n_tokens;
    p.n_heads = n_heads;
    p.n_kv_heads = n_kv_heads;
    p.n_streams = 1;
    p.eps = eps;
    return launch_prep(kPrepInPlace, p, rope_theta, as_stream(stream));
}
