// qa_decoder: device weights, KV cache, workspaces and the step drivers of the C ABI runtime layer.
//
// Follows the control flow of the reference's cached backend (src/text-decoder.cpp):
//   init            1476-1592 (validate, upload f32 weights) + alloc_kv_cache 1420-1474 (zeroed cache)
//   cached forward  1641-1755 (capacity check, positions n_past + i, 28 layers, last-row logits,
//                   cur_len = n_past + T)
//   greedy generate 2209-2311 (prefill, then argmax / stop check / break before the last forward)
// with the data path replaced by the kernels of this library.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "ops.hpp"

namespace {

using namespace qa;

struct DevLayer {
    float * attn_norm = nullptr;
    float * ffn_norm = nullptr;
    float * qkv = nullptr;     // [q_dim + 2 kv_dim][hidden]  (q rows, k rows, v rows)
    float * o = nullptr;       // [hidden][q_dim]
    float * q_norm = nullptr;
    float * k_norm = nullptr;
    float * gu = nullptr;      // [2 intermediate][hidden]     (gate rows, up rows)
    float * down = nullptr;    // [hidden][intermediate]
    // bf16 copies of the projection weights (their high halves), present only when every weight of
    // the model is bf16-exact; the batch-1 GEMVs read these
    uint16_t * qkv16 = nullptr;
    uint16_t * o16 = nullptr;
    uint16_t * gu16 = nullptr;
    uint16_t * down16 = nullptr;
    // q|k|v and o f32 rows packed for the multi-stream step's MFMA GEMM (gemm_packed.hip): multi-stream
    // decoders on f32 weights only
    float * qkv_p = nullptr;
    float * o_p = nullptr;
};

enum Kind { kDecode = 0, kPrefill = 1, kNoCache = 2 };

constexpr int32_t kSkinnyRows = 64;   // token rows up to which projections use the skinny MFMA GEMM

enum Family { kFamAppend = 0, kFamDecodeAttn, kFamPrefillAttn, kFamProj, kFamLogits, kFamLayers, kFamCount };
// decode_layers: the persistent step's single launch (every layer's projections and attention)
const char * kFamNames[kFamCount] = {"kv_append", "decode_attn", "prefill_attn", "projections", "logits",
                                     "decode_layers"};

}  // namespace

struct qa_decoder {
    qa_text_config cfg{};
    int32_t n_streams = 0, max_seq = 0, cache_type = 0;
    hipStream_t stream = nullptr;
    rocblas_handle blas = nullptr;
    std::vector<DevLayer> layers;
    float * embd = nullptr;
    float * out_norm = nullptr;
    float * out_w = nullptr;
    uint16_t * out_w16 = nullptr;
    float * out_p = nullptr;            // the LM head packed like DevLayer::qkv_p
    std::vector<void *> weight_allocs;
    std::vector<void *> b16_allocs;     // the bf16 weight copies (freed again if the model is not exact)
    void * cache = nullptr;
    qa_kv_layout layout{};
    int32_t * d_lens = nullptr;
    std::vector<int32_t> cur_len;
    // activations, sized for cap_rows rows
    int32_t cap_rows = 0;
    std::vector<void *> act_allocs;
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *qrot = nullptr, *attn = nullptr, *gu = nullptr, *act = nullptr;
    uint16_t * xsplit = nullptr;   // [rows][3 in_dim] bf16: three-part split of a GEMM input (bf16 copies)
    size_t xsplit_elems = 0;       // a third of its size: rows x max in_dim
    uint16_t * actsplit = nullptr; // [rows][3 intermediate] bf16: split of silu(gate) * up (fused SwiGLU)
    float * logits = nullptr;    // [n_streams][vocab]
    void * attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    void * am_ws = nullptr;
    size_t am_ws_bytes = 0;
    void * gr_ws = nullptr;      // skinny-GEMM partials and tile counters (activation allocation)
    size_t gr_ws_bytes = 0;
    void * pf_ws = nullptr;      // prefill attention: row statistics, split partials, merge counters
    size_t pf_ws_bytes = 0;
    double * xstats = nullptr;   // [hidden / 16][32] partial sums of squares of the rows of x (fused steps)
    int32_t * d_ids = nullptr;
    int32_t * h_ids = nullptr;   // pinned
    int32_t * h_ids_dev = nullptr;   // the same memory as the device addresses it
    // qa_decoder_generate's pipeline: completion events of the two decode steps in flight, and (margins
    // only) two pinned logits rows, allocated at first use
    hipEvent_t gen_ev[2] = {nullptr, nullptr};
    float * h_logits = nullptr;
    float * staging = nullptr;
    size_t staging_bytes = 0;
    float scale = 0.0f;
    // persistent decode step (qa_decoder_set_persistent): resident grid, barrier state, device layer table
    bool persist = false;
    bool persist_ran = false;          // a persistent launch since the last check of the error word
    int32_t persist_grid = 0;
    uint64_t persist_wait_ticks = 20000000;   // 200 ms; QA_PERSIST_WAIT_TICKS at enable time overrides it
    uint32_t * persist_sync = nullptr;
    size_t persist_sync_bytes = 0;
    PersistLayer * persist_layers = nullptr;
    // its per-layer activations and attention workspaces (every address written once per launch)
    float * persist_xbuf = nullptr;
    float * persist_qkv = nullptr;
    float * persist_attn = nullptr;
    float * persist_act = nullptr;
    void * persist_ws = nullptr;
    size_t persist_ws_bytes = 0;
    // profiling
    bool prof = false;
    struct Rec { int fam; hipEvent_t a, b; };
    std::vector<Rec> recs;
    size_t n_recs = 0;
};

namespace {

int dmalloc(std::vector<void *> & list, size_t bytes, void ** out) {
    void * p = nullptr;
    if (bytes == 0) bytes = 256;
    if (hipMalloc(&p, bytes) != hipSuccess) return fail(QA_ERR_ALLOC, "device allocation failed");
    list.push_back(p);
    *out = p;
    return QA_OK;
}

template <typename T>
int dmalloc_t(std::vector<void *> & list, size_t count, T ** out) {
    void * p = nullptr;
    const int rc = dmalloc(list, sizeof(T) * count, &p);
    *out = static_cast<T *>(p);
    return rc;
}

int upload(float * dst, const float * src, size_t n) {
    if (!src) return fail(QA_ERR_INVALID, "missing weight tensor");
    QA_HIP(hipMemcpy(dst, src, sizeof(float) * n, hipMemcpyHostToDevice));
    return QA_OK;
}

struct Prof {
    qa_decoder * d;
    int fam;
    int idx = -1;
    Prof(qa_decoder * dec, int family) : d(dec), fam(family) {
        if (!d->prof) return;
        if (d->n_recs == d->recs.size()) {
            qa_decoder::Rec r{family, nullptr, nullptr};
            if (hipEventCreate(&r.a) != hipSuccess || hipEventCreate(&r.b) != hipSuccess) return;
            d->recs.push_back(r);
        }
        idx = static_cast<int>(d->n_recs++);
        d->recs[idx].fam = family;
        (void)hipEventRecord(d->recs[idx].a, d->stream);
    }
    ~Prof() {
        if (idx >= 0) (void)hipEventRecord(d->recs[idx].b, d->stream);
    }
};

void free_acts(qa_decoder * d) {
    for (void * p : d->act_allocs) (void)hipFree(p);
    d->act_allocs.clear();
    d->cap_rows = 0;
    d->gr_ws = nullptr;
    d->gr_ws_bytes = 0;
    d->pf_ws = nullptr;
    d->pf_ws_bytes = 0;
    d->xstats = nullptr;
    d->xsplit = nullptr;
    d->xsplit_elems = 0;
    d->actsplit = nullptr;
}

// Workspace of the skinny GEMM for the layer projections at up to `rows` token rows and the LM head at
// up to `logit_rows` (its size grows with the row count, so the largest count covers all smaller ones).
size_t gemm_rows_bytes_for(const qa_text_config & c, int32_t rows, int32_t logit_rows) {
    const int32_t H = c.hidden, QD = c.n_heads * kHeadDim, KD = c.n_kv_heads * kHeadDim, I = c.intermediate;
    const int32_t shapes[4][2] = {{QD + 2 * KD, H}, {H, QD}, {2 * I, H}, {H, I}};
    size_t m = 0;
    for (const auto & sh : shapes) m = std::max(m, gemm_rows_workspace_bytes(sh[0], sh[1], rows));
    if (logit_rows >= 2) m = std::max(m, gemm_rows_workspace_bytes(c.vocab, H, logit_rows));
    return m;
}

int ensure_rows(qa_decoder * d, int32_t rows) {
    if (rows <= d->cap_rows) return QA_OK;
    (void)hipStreamSynchronize(d->stream);
    free_acts(d);
    const size_t H = d->cfg.hidden, QD = static_cast<size_t>(d->cfg.n_heads) * kHeadDim,
                 KD = static_cast<size_t>(d->cfg.n_kv_heads) * kHeadDim, I = d->cfg.intermediate;
    const size_t R = static_cast<size_t>(rows);
    int rc = QA_OK;
    rc = rc ? rc : dmalloc_t(d->act_allocs, R * H, &d->x);
    rc = rc ? rc : dmalloc_t(d->act_allocs, R * H, &d->xn);
    rc = rc ? rc : dmalloc_t(d->act_allocs, R * (QD + 2 * KD), &d->qkv);
    rc = rc ? rc : dmalloc_t(d->act_allocs, R * QD, &d->qrot);
    rc = rc ? rc : dmalloc_t(d->act_allocs, R * QD, &d->attn);
    rc = rc ? rc : dmalloc_t(d->act_allocs, R * 2 * I, &d->gu);
    rc = rc ? rc : dmalloc_t(d->act_allocs, R * I, &d->act);
    // the LM head runs on one row per stream (decode) or the last row (prefill)
    const size_t gr = rows >= 2 ? gemm_rows_bytes_for(d->cfg, std::min<int32_t>(rows, kSkinnyRows),
                                                      std::min<int32_t>(d->n_streams, kSkinnyRows))
                                : 0;
    if (rc == QA_OK && gr > 0) {
        rc = dmalloc(d->act_allocs, gr, &d->gr_ws);
        // cleared on the decoder's stream (non-blocking: a null-stream memset would not be ordered before
        // the kernels that use the counters)
        if (rc == QA_OK && hipMemsetAsync(d->gr_ws, 0, gr, d->stream) != hipSuccess) {
            rc = fail(QA_ERR_DEVICE, "workspace clear failed");
        }
        if (rc == QA_OK) d->gr_ws_bytes = gr;
    }
    if (rc == QA_OK && rows >= 2) {
        // room for 16-column partials (the packed o projection) as well as 32-column ones
        const size_t n = static_cast<size_t>((H + 15) / 16) * 32;
        rc = dmalloc(d->act_allocs, n * sizeof(double), reinterpret_cast<void **>(&d->xstats));
    }
    // bf16 copies: longer GEMM inputs are split into three bf16 parts ([rows][3 in_dim]) for the bf16 GEMM,
    // and the fused SwiGLU writes its split output beside the gate|up input
    if (rc == QA_OK && rows > kSkinnyRows && !d->layers.empty() && d->layers[0].qkv16) {
        d->xsplit_elems = R * std::max({H, QD, I});
        rc = dmalloc_t(d->act_allocs, 3 * d->xsplit_elems, &d->xsplit);
        rc = rc ? rc : dmalloc_t(d->act_allocs, 3 * R * I, &d->actsplit);
    }
    // prefill attention over up to `rows` tokens (counters cleared once; every call leaves them zero)
    const size_t pf = rows >= 2 ? qa_prefill_attn_workspace_bytes(rows, d->cfg.n_heads) : 0;
    if (rc == QA_OK && pf > 0) {
        rc = dmalloc(d->act_allocs, pf, &d->pf_ws);
        if (rc == QA_OK && hipMemsetAsync(d->pf_ws, 0, pf, d->stream) != hipSuccess) {
            rc = fail(QA_ERR_DEVICE, "workspace clear failed");
        }
        if (rc == QA_OK) d->pf_ws_bytes = pf;
    }
    if (rc != QA_OK) {
        free_acts(d);
        return rc;
    }
    d->cap_rows = rows;
    return QA_OK;
}

bool skinny_path(const qa_decoder * d, int32_t rows, int32_t in_dim) {
    return rows <= kSkinnyRows && in_dim % 32 == 0 && d->gr_ws;
}

// Whether sgemm runs the bf16 GEMM over the three-part split of its input (then the producer of the
// input may write d->xsplit itself, see sgemm's x_split).  W16: the bf16 rows; swiglu: the fused SwiGLU
// GEMM (out_dim = intermediate, W16 = [gate rows; up rows]).
bool split_path(const qa_decoder * d, int32_t rows, int32_t out_dim, int32_t in_dim, const uint16_t * W16,
                bool swiglu = false) {
    return !skinny_path(d, rows, in_dim) && W16 && d->xsplit && static_cast<size_t>(rows) * in_dim <= d->xsplit_elems &&
           gemm_split3_shape_ok(out_dim, in_dim, swiglu);
}

int sgemm(qa_decoder * d, const float * W, int32_t out_dim, int32_t in_dim, const float * X, int32_t rows, float * Y,
          float beta, const uint16_t * W16 = nullptr, const uint16_t * x_split = nullptr) {
    // Y[rows][out] (+)= X[rows][in] * W[out][in]^T.  Up to kSkinnyRows rows (multi-stream decode, short
    // prefills) the weights are streamed once by the skinny MFMA GEMM; longer prefills run gemm_split3 on
    // the bf16 copies, or rocBLAS sgemm on f32 weights.  x_split: the producer of X already wrote its
    // three-part split there (only where split_path holds).
    if (x_split && !split_path(d, rows, out_dim, in_dim, W16)) {
        return fail(QA_ERR_INVALID, "sgemm: split input without split path");
    }
    if (skinny_path(d, rows, in_dim)) {
        return gemm_rows_launch(W, out_dim, in_dim, X, rows, Y, beta != 0.0f, d->gr_ws, d->gr_ws_bytes, d->stream);
    }
    if (split_path(d, rows, out_dim, in_dim, W16)) {
        // bf16-exact weights: each row of X split into three bf16 parts, X = hi + mid + lo exactly, and one
        // bf16 MFMA GEMM over the one bf16 copy uses every W tile for the three parts: every product exact,
        // the sums in f32 (gemm_split3.hip)
        const int rc = x_split ? QA_OK : split_bf16x3_rows_launch(X, rows, in_dim, d->xsplit, d->stream);
        if (rc != QA_OK) return rc;
        return gemm_split3_launch(W16, out_dim, in_dim, x_split ? x_split : d->xsplit, rows, Y, beta != 0.0f, nullptr,
                                  d->stream);
    }
    // column-major C(out x rows) = W^T(out x in) * X(in x rows)
    const float alpha = 1.0f;
    const rocblas_status st = rocblas_sgemm(d->blas, rocblas_operation_transpose, rocblas_operation_none, out_dim,
                                            rows, in_dim, &alpha, W, in_dim, X, in_dim, &beta, Y, out_dim);
    if (st != rocblas_status_success) {
        return fail(QA_ERR_DEVICE, std::string("rocblas_sgemm failed: ") + rocblas_status_to_string(st));
    }
    return QA_OK;
}

// The multi-stream decode step (2..32 streams) runs its projections on the 32-row skinny GEMM with the
// RMSNorms and the SwiGLU fused in: the residual GEMMs (o, down) and the embedding gather leave the
// per-row sums of squares of x in d->xstats, the normalised GEMMs (q|k|v, gate|up, LM head) read them.
bool fused_rows(const qa_decoder * d, int32_t rows) {
    const qa_text_config & c = d->cfg;
    const int32_t H = c.hidden, QD = c.n_heads * kHeadDim, KD = c.n_kv_heads * kHeadDim, I = c.intermediate;
    return rows >= 2 && d->xstats && (H + 31) / 32 <= 128 && (2 * I) % 32 == 0 &&
           gemm_rows_fusable(QD + 2 * KD, H, rows) && gemm_rows_fusable(H, QD, rows) &&
           gemm_rows_fusable(2 * I, H, rows) && gemm_rows_fusable(H, I, rows) && gemm_rows_fusable(c.vocab, H, rows);
}

int fused_gemm(qa_decoder * d, const float * W, int32_t N, int32_t K, const float * X, int32_t rows, float * Y,
               bool accumulate, const GemmRowsFusion & f, const uint16_t * W16) {
    return gemm_rows_launch(W, N, K, X, rows, Y, accumulate, d->gr_ws, d->gr_ws_bytes, d->stream, &f, W16);
}

// cols: columns per partial sum of squares in d->xstats, as the producer of x wrote them (32: embedding gather,
// pick tail, gemm_rows32_kernel; 16: the packed o projection)
GemmRowsFusion norm_in(const qa_decoder * d, const float * norm_w, int32_t cols = 32) {
    GemmRowsFusion f;
    f.norm_w = norm_w;
    f.stats_in = d->xstats;
    f.n_stats_in = (d->cfg.hidden + cols - 1) / cols;
    f.eps = d->cfg.rms_norm_eps;
    return f;
}

GemmRowsFusion stats_out(const qa_decoder * d) {
    GemmRowsFusion f;
    f.stats_out = d->xstats;
    return f;
}

int32_t host_max_len(const qa_decoder * d, int32_t n, int32_t add) {
    int32_t m = 0;
    for (int32_t s = 0; s < n; ++s) m = std::max(m, d->cur_len[s] + add);
    return m;
}

// One layer over `rows` token rows held in d->x.
//   kDecode : rows = number of streams (one token each), positions d_lens[s], keys [0, d_lens[s] + 1)
//   kPrefill: rows = T tokens of stream 0 at positions n_past.., keys [0, n_past + t]
//   kNoCache: rows = T tokens, positions 0..T-1, f32 K/V never stored
int run_layer(qa_decoder * d, int32_t l, int32_t rows, int kind, int32_t n_past, int32_t max_len = 0,
              bool fused = false) {
    const qa_text_config & c = d->cfg;
    const DevLayer & L = d->layers[l];
    const int32_t H = c.hidden, QD = c.n_heads * kHeadDim, KD = c.n_kv_heads * kHeadDim, I = c.intermediate;
    const int32_t W3 = QD + 2 * KD;
    hipStream_t s = d->stream;
    int rc;
    {
        Prof pr(d, kFamProj);
        if (rows == 1) {
            rc = gemv_launch(kEpiStoreOp, true, L.qkv, W3, H, d->x, d->qkv, L.attn_norm, c.rms_norm_eps, s,
                             L.qkv16);
        } else if (fused) {
            const GemmRowsFusion f = norm_in(d, L.attn_norm);
            rc = L.qkv_p ? gemm_packed_launch(L.qkv_p, W3, H, d->x, rows, d->qkv, false, &f, false, s)
                         : fused_gemm(d, L.qkv, W3, H, d->x, rows, d->qkv, false, f, L.qkv16);
        } else {
            // the RMSNorm writes the GEMM's split input directly where the GEMM takes one
            const bool sp = split_path(d, rows, W3, H, L.qkv16);
            rc = rmsnorm_rows_launch(d->x, L.attn_norm, rows, H, c.rms_norm_eps, d->xn, s, sp ? d->xsplit : nullptr);
            if (rc == QA_OK) rc = sgemm(d, L.qkv, W3, H, d->xn, rows, d->qkv, 0.0f, L.qkv16, sp ? d->xsplit : nullptr);
        }
        if (rc != QA_OK) return rc;
    }
    if (kind == kNoCache) {
        {
            Prof pr(d, kFamAppend);
            rc = qa_qk_prep(d->qkv, rows, c.n_heads, c.n_kv_heads, L.q_norm, L.k_norm, 0, c.rope_theta,
                            c.rms_norm_eps, s);
            if (rc != QA_OK) return rc;
        }
        Prof pr(d, kFamPrefillAttn);
        rc = causal_f32_launch(d->qkv, W3, d->qkv + QD, d->qkv + QD + KD, W3, rows, c.n_heads, c.n_kv_heads,
                               d->scale, d->attn, QD, s);
        if (rc != QA_OK) return rc;
    } else if (kind == kDecode) {
        // append + attend in one launch: one token per stream at position d_lens[s]
        Prof pr(d, kFamDecodeAttn);
        rc = decode_step_attn_launch(d->qkv, L.q_norm, L.k_norm, d->cache, d->layout, l, d->d_lens, rows,
                                     max_len > 0 ? max_len : host_max_len(d, rows, 1), c.n_heads, c.rope_theta,
                                     c.rms_norm_eps, d->scale, d->attn, d->attn_ws, d->attn_ws_bytes, s);
        if (rc != QA_OK) return rc;
    } else {
        {
            Prof pr(d, kFamAppend);
            rc = qa_kv_append(d->qkv, L.q_norm, L.k_norm, d->qrot, d->cache, &d->layout, l, d->d_lens, 1, rows,
                              c.n_heads, c.rope_theta, c.rms_norm_eps, s);
            if (rc != QA_OK) return rc;
        }
        Prof pr(d, kFamPrefillAttn);
        rc = prefill_attn_launch(d->qrot, QD, d->cache, d->layout, l, 0, n_past, rows, c.n_heads, d->scale,
                                 d->attn, d->pf_ws, d->pf_ws_bytes, s);
        if (rc != QA_OK) return rc;
    }
    Prof pr(d, kFamProj);
    if (rows == 1) {
        rc = gemv_launch(kEpiAccumOp, false, L.o, H, QD, d->attn, d->x, nullptr, 0.0f, s, L.o16);
        if (rc == QA_OK) {
            rc = gemv_launch(kEpiSwigluOp, true, L.gu, I, H, d->x, d->act, L.ffn_norm, c.rms_norm_eps, s, L.gu16);
        }
        if (rc == QA_OK) rc = gemv_launch(kEpiAccumOp, false, L.down, H, I, d->act, d->x, nullptr, 0.0f, s, L.down16);
    } else if (fused) {
        // the packed o projection leaves 16-column partial sums of squares of x for the gate|up RMSNorm
        GemmRowsFusion gu = norm_in(d, L.ffn_norm, L.o_p ? 16 : 32);
        gu.swiglu = true;
        if (L.o_p) {
            const GemmRowsFusion so = stats_out(d);
            rc = gemm_packed_launch(L.o_p, H, QD, d->attn, rows, d->x, true, &so, false, s);
        } else {
            rc = fused_gemm(d, L.o, H, QD, d->attn, rows, d->x, true, stats_out(d), L.o16);
        }
        if (rc == QA_OK) rc = fused_gemm(d, L.gu, 2 * I, H, d->x, rows, d->act, false, gu, L.gu16);
        if (rc == QA_OK) rc = fused_gemm(d, L.down, H, I, d->act, rows, d->x, true, stats_out(d), L.down16);
    } else {
        rc = sgemm(d, L.o, H, QD, d->attn, rows, d->x, 1.0f, L.o16);
        const bool sd = split_path(d, rows, H, I, L.down16) && d->actsplit;
        // bf16 copies: gate|up with the SwiGLU in its epilogue, writing the split input of down directly
        const bool fuse = sd && split_path(d, rows, I, H, L.gu16, true);
        const bool sg = fuse || split_path(d, rows, 2 * I, H, L.gu16);
        if (rc == QA_OK) rc = rmsnorm_rows_launch(d->x, L.ffn_norm, rows, H, c.rms_norm_eps, d->xn, s, sg ? d->xsplit : nullptr);
        if (fuse) {
            if (rc == QA_OK) rc = gemm_split3_launch(L.gu16, I, H, d->xsplit, rows, nullptr, false, d->actsplit, s);
        } else {
            if (rc == QA_OK) rc = sgemm(d, L.gu, 2 * I, H, d->xn, rows, d->gu, 0.0f, L.gu16, sg ? d->xsplit : nullptr);
            if (rc == QA_OK) rc = swiglu_rows_launch(d->gu, rows, I, d->act, s, sd ? d->actsplit : nullptr);
        }
        if (rc == QA_OK) rc = sgemm(d, L.down, H, I, d->act, rows, d->x, 1.0f, L.down16, sd ? d->actsplit : nullptr);
    }
    return rc;
}

// Logits of `rows` rows starting at row `first` of d->x into d->logits[0..rows), then greedy ids.
int logits_and_pick(qa_decoder * d, int32_t first, int32_t rows, bool pick, bool fused = false,
                    const StepTail & tail = StepTail{}) {
    const qa_text_config & c = d->cfg;
    if (!d->out_w || !d->out_norm) return fail(QA_ERR_INVALID, "decoder has no output weights");
    int rc;
    {
        Prof pr(d, kFamLogits);
        const float * xr = d->x + static_cast<int64_t>(first) * c.hidden;
        if (rows == 1) {
            rc = gemv_launch(kEpiStoreOp, true, d->out_w, c.vocab, c.hidden, xr, d->logits, d->out_norm,
                             c.rms_norm_eps, d->stream, d->out_w16);
        } else if (fused && first == 0) {
            const GemmRowsFusion f = norm_in(d, d->out_norm);
            rc = d->out_p ? gemm_packed_launch(d->out_p, c.vocab, c.hidden, xr, rows, d->logits, false, &f, true, d->stream)
                          : fused_gemm(d, d->out_w, c.vocab, c.hidden, xr, rows, d->logits, false, f, d->out_w16);
        } else {
            rc = rmsnorm_rows_launch(xr, d->out_norm, rows, c.hidden, c.rms_norm_eps, d->xn, d->stream);
            if (rc == QA_OK) rc = sgemm(d, d->out_w, c.vocab, c.hidden, d->xn, rows, d->logits, 0.0f);
        }
        if (rc != QA_OK) return rc;
    }
    if (!pick) return QA_OK;
    return argmax_launch(d->logits, rows, c.vocab, d->d_ids, d->am_ws, d->stream, tail);
}

PersistPlanIn persist_plan_in(const qa_decoder * d) {
    PersistPlanIn in;
    in.layout = d->layout;
    in.hidden = d->cfg.hidden;
    in.q_dim = d->cfg.n_heads * kHeadDim;
    in.inter = d->cfg.intermediate;
    in.b16 = !d->layers.empty() && d->layers[0].qkv16;
    return in;
}

// Every layer of one batch-1 token (stream 0, position d_lens[0]) as one persistent launch; x holds the
// token's input row and ends with the last layer's output, as after the eager layers.
int persist_layers(qa_decoder * d, int32_t max_len) {
    const qa_text_config & c = d->cfg;
    PersistLaunch a;
    a.plan = persist_plan_in(d);
    a.grid = d->persist_grid;
    a.layers = d->persist_layers;
    a.n_layers = c.n_layers;
    a.x = d->x;
    a.xbuf = d->persist_xbuf;
    a.qkv = d->persist_qkv;
    a.attn = d->persist_attn;
    a.act = d->persist_act;
    a.cache = d->cache;
    a.lens = d->d_lens;
    a.max_len = max_len;
    a.n_heads = c.n_heads;
    a.eps = c.rms_norm_eps;
    a.scale = d->scale;
    a.rope_theta = c.rope_theta;
    a.attn_ws = d->persist_ws;
    a.attn_ws_bytes = d->persist_ws_bytes;
    a.sync = d->persist_sync;
    a.wait_ticks = d->persist_wait_ticks;
    Prof pr(d, kFamLayers);
    const int rc = persist_layers_launch(a, d->stream);
    if (rc == QA_OK) d->persist_ran = true;
    return rc;
}

// After a call that ran persistent launches: QA_ERR_DEVICE if one of them abandoned a barrier wait (its
// results are invalid), after clearing the barrier state and the attention merge counters it left behind.
int persist_check(qa_decoder * d) {
    if (!d->persist_ran) return QA_OK;
    d->persist_ran = false;
    uint32_t err = 0;
    QA_HIP(hipMemcpyAsync(&err, d->persist_sync + persist_error_word_offset(d->persist_grid), sizeof(err),
                          hipMemcpyDeviceToHost, d->stream));
    QA_HIP(hipStreamSynchronize(d->stream));
    if (err == 0) return QA_OK;
    QA_HIP(hipMemsetAsync(d->persist_sync, 0, d->persist_sync_bytes, d->stream));
    QA_HIP(hipMemsetAsync(d->persist_ws, 0, d->persist_ws_bytes, d->stream));
    QA_HIP(hipStreamSynchronize(d->stream));
    return fail(QA_ERR_DEVICE, "persistent decode step: a grid barrier wait ran out, the call's results are invalid");
}

int check_forward(const qa_decoder * d, int32_t n_tokens, int32_t n_past) {
    if (n_tokens <= 0 || n_past < 0 || n_past + n_tokens > d->max_seq) {
        return fail(n_past + n_tokens > d->max_seq ? QA_ERR_CAPACITY : QA_ERR_INVALID,
                    "invalid text decoder cached forward configuration");
    }
    return QA_OK;
}

// Cached call of stream 0 with x already on the device.
int forward_device(qa_decoder * d, int32_t n_tokens, int32_t n_past, bool pick) {
    int rc = set_values_launch(d->d_lens, 1, n_past, d->stream);
    if (rc != QA_OK) return rc;
    d->cur_len[0] = n_past;
    const int kind = n_tokens == 1 ? kDecode : kPrefill;
    if (d->persist && n_tokens == 1) {
        rc = persist_layers(d, n_past + 1);
        if (rc != QA_OK) return rc;
    } else {
        for (int32_t l = 0; l < d->cfg.n_layers; ++l) {
            rc = run_layer(d, l, n_tokens, kind, n_past);
            if (rc != QA_OK) return rc;
        }
    }
    rc = logits_and_pick(d, n_tokens - 1, 1, pick);
    if (rc != QA_OK) return rc;
    rc = set_values_launch(d->d_lens, 1, n_past + n_tokens, d->stream);
    d->cur_len[0] = n_past + n_tokens;
    return rc;
}

// One decode step of `rows` streams with the token ids already in d_ids: embedding gather (unless the
// previous step's pick already left the rows in d->x: embed = false), every layer (fused append +
// attention at position d_lens[s]), LM head, and the pick, whose kernel also advances d_lens[s], writes
// the ids to host_ids (device-visible pinned memory, optional) and gathers the next step's embedding
// rows into d->x.  Only device memory is read for lengths and ids, so the sequence is capturable.
int decode_step_ops(qa_decoder * d, int32_t rows, int32_t max_len, bool embed, int32_t * host_ids) {
    const bool fused = fused_rows(d, rows);
    int rc = QA_OK;
    if (embed) {
        rc = embed_rows_launch(d->embd, d->cfg.vocab, d->cfg.hidden, d->d_ids, rows, d->x, d->stream,
                               fused ? d->xstats : nullptr);
    }
    if (d->persist && rows == 1) {
        if (rc == QA_OK) rc = persist_layers(d, max_len);
    } else {
        for (int32_t l = 0; l < d->cfg.n_layers && rc == QA_OK; ++l) {
            rc = run_layer(d, l, rows, kDecode, 0, max_len, fused);
        }
    }
    StepTail tail;
    tail.lens = d->d_lens;
    tail.host_ids = host_ids;
    tail.embd = d->embd;
    tail.x = d->x;
    tail.stats = fused ? d->xstats : nullptr;
    tail.dim = d->cfg.hidden;
    if (rc == QA_OK) rc = logits_and_pick(d, 0, rows, true, fused, tail);
    return rc;
}

// One decode step launched eagerly.  The step reads lengths and ids from device memory only, so the
// host does no per-token bookkeeping beyond the launches (the reference rebuilds its graph and uploads
// a dense mask every token, text-decoder.cpp:1658-1739).  embed: d->x does not hold the embedding rows
// of d_ids yet (the first step after a prefill or after ids came from the host).
int decode_step(qa_decoder * d, int32_t rows, bool embed, int32_t * host_ids = nullptr) {
    const int rc = decode_step_ops(d, rows, host_max_len(d, rows, 1), embed, host_ids);
    if (rc != QA_OK) return rc;
    for (int32_t s = 0; s < rows; ++s) d->cur_len[s] += 1;
    return QA_OK;
}

float top2_margin(const float * v, int32_t n, int32_t best) {
    float second = -INFINITY;
    for (int32_t i = 0; i < n; ++i) {
        if (i != best && v[i] > second) second = v[i];
    }
    return v[best] - second;
}

// bf16 copies of the projection and LM-head weights for the batch-1 GEMVs, kept only when every one
// of them is bf16-exact (a checkpoint converted from bf16 weights); then the GEMVs read half the bytes
// and compute the same f32 results.  QA_WEIGHTS_F32=1 keeps the f32 weights only.
int pack_weights_bf16(qa_decoder * d) {
    const char * e = std::getenv("QA_WEIGHTS_F32");
    if (e && std::strcmp(e, "1") == 0) return QA_OK;
    const qa_text_config & c = d->cfg;
    const size_t H = c.hidden, QD = static_cast<size_t>(c.n_heads) * kHeadDim,
                 KD = static_cast<size_t>(c.n_kv_heads) * kHeadDim, I = c.intermediate;
    uint32_t * flag = nullptr;
    int rc = dmalloc_t(d->b16_allocs, 64, &flag);
    if (rc == QA_OK && hipMemsetAsync(flag, 0, 4, d->stream) != hipSuccess) rc = fail(QA_ERR_DEVICE, "clear failed");
    auto pack = [&](const float * src, size_t n, uint16_t ** dst) {
        if (rc != QA_OK) return;
        rc = dmalloc_t(d->b16_allocs, n, dst);
        if (rc == QA_OK) rc = pack_bf16_launch(src, static_cast<int64_t>(n), *dst, flag, d->stream);
    };
    for (DevLayer & L : d->layers) {
        pack(L.qkv, (QD + 2 * KD) * H, &L.qkv16);
        pack(L.o, H * QD, &L.o16);
        pack(L.gu, 2 * I * H, &L.gu16);
        pack(L.down, H * I, &L.down16);
    }
    if (d->out_w) pack(d->out_w, static_cast<size_t>(c.vocab) * H, &d->out_w16);
    uint32_t inexact = 1;
    if (rc == QA_OK && (hipMemcpyAsync(&inexact, flag, 4, hipMemcpyDeviceToHost, d->stream) != hipSuccess ||
                        hipStreamSynchronize(d->stream) != hipSuccess)) {
        rc = fail(QA_ERR_DEVICE, "bf16 weight check failed");
    }
    if (rc != QA_OK || inexact != 0) {
        for (void * p : d->b16_allocs) (void)hipFree(p);
        d->b16_allocs.clear();
        for (DevLayer & L : d->layers) L.qkv16 = L.o16 = L.gu16 = L.down16 = nullptr;
        d->out_w16 = nullptr;
    }
    return rc;
}

// Multi-stream decoders on f32 weights: the LM head packed for gemm_packed.hip's 128-row MFMA kernel (1.24 GB
// beside the 6.88 GB of f32 weights for the 1.7B model; config-4 step 4.04 -> 3.99 ms, all 2048 oracle ids kept).
// QA_GR_PACKED=1 also packs the q|k|v and o rows of every layer (1.41 GB more; 3.83 ms).  That part is opt-in:
// its sums run in another order than gemm_rows32_kernel's, and on config 4 it takes the oracle's runner-up at one
// near-tie (stream 11, step 36, oracle top-2 margin 4.3e-4), where the default kernels agree.
int pack_weights_mfma(qa_decoder * d) {
    if (d->n_streams < 2 || d->layers.empty() || d->layers[0].qkv16) return QA_OK;
    const char * e = std::getenv("QA_GR_PACKED");
    const bool layers = e && std::strcmp(e, "1") == 0;
    const qa_text_config & c = d->cfg;
    const int32_t H = c.hidden, QD = c.n_heads * kHeadDim, KD = c.n_kv_heads * kHeadDim;
    int rc = QA_OK;
    auto pack = [&](const float * src, int32_t N, int32_t K, float ** dst) {
        if (rc != QA_OK) return;
        rc = dmalloc_t(d->weight_allocs, static_cast<size_t>(N) * K, dst);
        if (rc == QA_OK) rc = pack_f32_launch(src, N, K, *dst, d->stream);
    };
    if (layers && packed_gemm_shape_ok(QD + 2 * KD, H, false) && packed_gemm_shape_ok(H, QD, false)) {
        for (DevLayer & L : d->layers) {
            pack(L.qkv, QD + 2 * KD, H, &L.qkv_p);
            pack(L.o, H, QD, &L.o_p);
        }
    }
    if (d->out_w && packed_gemm_shape_ok(c.vocab, H, true)) pack(d->out_w, c.vocab, H, &d->out_p);
    return rc;
}

}  // namespace

extern "C" int qa_decoder_weights_bf16(const qa_decoder * d) {
    return d && !d->layers.empty() && d->layers[0].qkv16 ? 1 : 0;
}

extern "C" int qa_decoder_create(const qa_text_config * cfg, const qa_model_weights * w, int32_t n_streams,
                                 int32_t max_seq, int32_t cache_type, qa_decoder ** out) {
    if (!out) return fail(QA_ERR_INVALID, "qa_decoder_create: null output");
    *out = nullptr;
    if (!cfg || !w || !w->layers || cfg->n_layers <= 0 || cfg->hidden <= 0 || cfg->n_heads <= 0 ||
        cfg->n_kv_heads <= 0 || cfg->intermediate <= 0 || cfg->vocab <= 0 || cfg->n_heads % cfg->n_kv_heads != 0) {
        return fail(QA_ERR_INVALID, "invalid text decoder backend configuration");
    }
    if (cfg->head_dim != kHeadDim || cfg->n_heads != 2 * cfg->n_kv_heads) {
        return fail(QA_ERR_INVALID, "this build implements head_dim 128 with 2 query heads per KV head");
    }
    if (n_streams <= 0 || max_seq <= 0 || (cache_type != QA_CACHE_F32 && cache_type != QA_CACHE_F16)) {
        return fail(QA_ERR_INVALID, "invalid text decoder KV-cache configuration");
    }
    if (qa_device_count() <= 0) return fail(QA_ERR_NO_DEVICE, "no HIP device visible");
    QA_HIP(hipSetDevice(0));
    // the allocation-free attention entry point's scratch address, resolved here, outside any capture
    if (qa_decode_noalloc_prepare() != QA_OK) return QA_ERR_DEVICE;

    qa_decoder * d = new qa_decoder();
    d->cfg = *cfg;
    d->n_streams = n_streams;
    d->max_seq = max_seq;
    d->cache_type = cache_type;
    d->scale = 1.0f / std::sqrt(static_cast<float>(cfg->head_dim));
    d->cur_len.assign(static_cast<size_t>(n_streams), 0);
    auto bail = [&](int rc) {
        qa_decoder_destroy(d);
        return rc;
    };
    if (hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking) != hipSuccess) {
        return bail(fail(QA_ERR_DEVICE, "hipStreamCreate failed"));
    }
    // no atomics-based GEMM algorithms: their sums land in a different order from run to run, and the
    // prefill's results (and everything decoded after it) are then not repeatable
    if (rocblas_create_handle(&d->blas) != rocblas_status_success ||
        rocblas_set_stream(d->blas, d->stream) != rocblas_status_success ||
        rocblas_set_atomics_mode(d->blas, rocblas_atomics_not_allowed) != rocblas_status_success) {
        return bail(fail(QA_ERR_DEVICE, "rocblas handle creation failed"));
    }

    const size_t H = cfg->hidden, QD = static_cast<size_t>(cfg->n_heads) * kHeadDim,
                 KD = static_cast<size_t>(cfg->n_kv_heads) * kHeadDim, I = cfg->intermediate;
    int rc = QA_OK;
    d->layers.resize(static_cast<size_t>(cfg->n_layers));
    for (int32_t l = 0; l < cfg->n_layers && rc == QA_OK; ++l) {
        const qa_layer_weights & lw = w->layers[l];
        DevLayer & L = d->layers[static_cast<size_t>(l)];
        rc = rc ? rc : dmalloc_t(d->weight_allocs, H, &L.attn_norm);
        rc = rc ? rc : dmalloc_t(d->weight_allocs, H, &L.ffn_norm);
        rc = rc ? rc : dmalloc_t(d->weight_allocs, (QD + 2 * KD) * H, &L.qkv);
        rc = rc ? rc : dmalloc_t(d->weight_allocs, H * QD, &L.o);
        rc = rc ? rc : dmalloc_t(d->weight_allocs, kHeadDim, &L.q_norm);
        rc = rc ? rc : dmalloc_t(d->weight_allocs, kHeadDim, &L.k_norm);
        rc = rc ? rc : dmalloc_t(d->weight_allocs, 2 * I * H, &L.gu);
        rc = rc ? rc : dmalloc_t(d->weight_allocs, H * I, &L.down);
        rc = rc ? rc : upload(L.attn_norm, lw.attn_norm, H);
        rc = rc ? rc : upload(L.ffn_norm, lw.ffn_norm, H);
        rc = rc ? rc : upload(L.qkv, lw.q, QD * H);
        rc = rc ? rc : upload(L.qkv + QD * H, lw.k, KD * H);
        rc = rc ? rc : upload(L.qkv + (QD + KD) * H, lw.v, KD * H);
        rc = rc ? rc : upload(L.o, lw.o, H * QD);
        rc = rc ? rc : upload(L.q_norm, lw.q_norm, kHeadDim);
        rc = rc ? rc : upload(L.k_norm, lw.k_norm, kHeadDim);
        rc = rc ? rc : upload(L.gu, lw.gate, I * H);
        rc = rc ? rc : upload(L.gu + I * H, lw.up, I * H);
        rc = rc ? rc : upload(L.down, lw.down, H * I);
    }
    if (rc != QA_OK) return bail(rc);
    const size_t VH = static_cast<size_t>(cfg->vocab) * H;
    if (w->output && w->output_norm) {
        rc = rc ? rc : dmalloc_t(d->weight_allocs, VH, &d->out_w);
        rc = rc ? rc : upload(d->out_w, w->output, VH);
        rc = rc ? rc : dmalloc_t(d->weight_allocs, H, &d->out_norm);
        rc = rc ? rc : upload(d->out_norm, w->output_norm, H);
    }
    if (rc == QA_OK && w->token_embd) {
        if (w->token_embd == w->output && d->out_w) {
            d->embd = d->out_w;     // tied embeddings: one device copy
        } else {
            rc = dmalloc_t(d->weight_allocs, VH, &d->embd);
            rc = rc ? rc : upload(d->embd, w->token_embd, VH);
        }
    }
    if (rc != QA_OK) return bail(rc);
    rc = pack_weights_bf16(d);
    if (rc == QA_OK) rc = pack_weights_mfma(d);
    if (rc != QA_OK) return bail(rc);

    d->layout.n_layers = cfg->n_layers;
    d->layout.n_streams = n_streams;
    d->layout.n_kv_heads = cfg->n_kv_heads;
    d->layout.head_dim = kHeadDim;
    d->layout.max_seq = max_seq;
    d->layout.cache_type = cache_type;
    rc = qa_kv_cache_alloc(&d->layout, &d->cache);
    if (rc != QA_OK) return bail(rc);

    rc = rc ? rc : dmalloc_t(d->weight_allocs, static_cast<size_t>(n_streams), &d->d_lens);
    rc = rc ? rc : dmalloc_t(d->weight_allocs, static_cast<size_t>(n_streams), &d->d_ids);
    rc = rc ? rc : dmalloc_t(d->weight_allocs, static_cast<size_t>(n_streams) * cfg->vocab, &d->logits);
    d->attn_ws_bytes = decode_attn_workspace(n_streams, cfg->n_kv_heads, max_seq);
    rc = rc ? rc : dmalloc(d->weight_allocs, d->attn_ws_bytes, &d->attn_ws);
    d->am_ws_bytes = argmax_workspace_bytes(n_streams);
    rc = rc ? rc : dmalloc(d->weight_allocs, d->am_ws_bytes, &d->am_ws);
    if (rc != QA_OK) return bail(rc);
    if (hipHostMalloc(reinterpret_cast<void **>(&d->h_ids), sizeof(int32_t) * 4096 * static_cast<size_t>(n_streams)) !=
        hipSuccess) {
        d->h_ids = nullptr;
        return bail(fail(QA_ERR_ALLOC, "pinned host allocation failed"));
    }
    if (hipHostGetDevicePointer(reinterpret_cast<void **>(&d->h_ids_dev), d->h_ids, 0) != hipSuccess || !d->h_ids_dev) {
        return bail(fail(QA_ERR_DEVICE, "pinned id buffer has no device address"));
    }
    // cleared on the decoder's own stream, ahead of every kernel that reads them
    if (hipMemsetAsync(d->d_lens, 0, sizeof(int32_t) * n_streams, d->stream) != hipSuccess ||
        hipMemsetAsync(d->attn_ws, 0, d->attn_ws_bytes, d->stream) != hipSuccess ||
        hipMemsetAsync(d->am_ws, 0, d->am_ws_bytes, d->stream) != hipSuccess) {
        return bail(fail(QA_ERR_DEVICE, "workspace clear failed"));
    }
    rc = ensure_rows(d, n_streams);
    if (rc != QA_OK) return bail(rc);
    // QA_DECODE_PERSISTENT=1: the persistent decode step for callers that cannot call qa_decoder_set_persistent
    // (the drop-in API and its tools); a decoder it does not cover stays eager
    if (const char * e = std::getenv("QA_DECODE_PERSISTENT"); e && std::strcmp(e, "1") == 0) {
        (void)qa_decoder_set_persistent(d, 1);
    }
    *out = d;
    return QA_OK;
}

extern "C" void qa_decoder_destroy(qa_decoder * d) {
    if (!d) return;
    if (d->stream) (void)hipStreamSynchronize(d->stream);
    for (auto & r : d->recs) {
        if (r.a) (void)hipEventDestroy(r.a);
        if (r.b) (void)hipEventDestroy(r.b);
    }
    free_acts(d);
    for (void * p : d->weight_allocs) (void)hipFree(p);
    for (void * p : d->b16_allocs) (void)hipFree(p);
    if (d->staging) (void)hipFree(d->staging);
    if (d->cache) (void)hipFree(d->cache);
    if (d->h_ids) (void)hipHostFree(d->h_ids);
    if (d->h_logits) (void)hipHostFree(d->h_logits);
    for (hipEvent_t e : d->gen_ev) {
        if (e) (void)hipEventDestroy(e);
    }
    if (d->blas) rocblas_destroy_handle(d->blas);
    if (d->stream) (void)hipStreamDestroy(d->stream);
    delete d;
}

extern "C" int qa_decoder_cur_len(const qa_decoder * d, int32_t stream, int32_t * cur_len) {
    if (!d || !cur_len || stream < 0 || stream >= d->n_streams) return fail(QA_ERR_INVALID, "qa_decoder_cur_len");
    *cur_len = d->cur_len[static_cast<size_t>(stream)];
    return QA_OK;
}

extern "C" int qa_decoder_set_cur_len(qa_decoder * d, int32_t stream, int32_t cur_len) {
    if (!d || stream < 0 || stream >= d->n_streams || cur_len < 0 || cur_len > d->max_seq) {
        return fail(QA_ERR_INVALID, "qa_decoder_set_cur_len");
    }
    d->cur_len[static_cast<size_t>(stream)] = cur_len;
    return set_values_launch(d->d_lens + stream, 1, cur_len, d->stream);
}

extern "C" int qa_decoder_device_lens(qa_decoder * d, int32_t * lens) {
    if (!d || !lens) return fail(QA_ERR_INVALID, "qa_decoder_device_lens");
    QA_HIP(hipMemcpyAsync(lens, d->d_lens, sizeof(int32_t) * d->n_streams, hipMemcpyDeviceToHost, d->stream));
    QA_HIP(hipStreamSynchronize(d->stream));
    return QA_OK;
}

extern "C" void * qa_decoder_cache(qa_decoder * d, qa_kv_layout * layout) {
    if (!d) return nullptr;
    if (layout) *layout = d->layout;
    return d->cache;
}

extern "C" void * qa_decoder_stream(qa_decoder * d) { return d ? d->stream : nullptr; }

extern "C" int qa_decoder_forward(qa_decoder * d, const float * x, int32_t n_tokens, int32_t n_past, float * logits) {
    if (!d || !x) return fail(QA_ERR_INVALID, "text_decoder_backend_cached_logits: invalid arguments");
    int rc = check_forward(d, n_tokens, n_past);
    if (rc != QA_OK) return rc;
    rc = ensure_rows(d, n_tokens);
    if (rc != QA_OK) return rc;
    QA_HIP(hipMemcpyAsync(d->x, x, sizeof(float) * n_tokens * d->cfg.hidden, hipMemcpyHostToDevice, d->stream));
    rc = forward_device(d, n_tokens, n_past, false);
    if (rc != QA_OK) return rc;
    if (logits) {
        QA_HIP(hipMemcpyAsync(logits, d->logits, sizeof(float) * d->cfg.vocab, hipMemcpyDeviceToHost, d->stream));
    }
    QA_HIP(hipStreamSynchronize(d->stream));
    return persist_check(d);
}

extern "C" int qa_decoder_generate(qa_decoder * d, const float * x, int32_t n_tokens, int32_t max_new,
                                   const int32_t * stop_ids, int32_t n_stop, int32_t * out_ids, int32_t * n_out,
                                   int32_t * stopped, int32_t * total_tokens, float * margins) {
    if (!d || !x || !n_out || !stopped || !total_tokens || (max_new > 0 && !out_ids)) {
        return fail(QA_ERR_INVALID, "qwenasr_text_generate_cached_backend: backend or out is null");
    }
    *n_out = 0;
    *stopped = 0;
    *total_tokens = n_tokens;
    if (max_new < 0) return fail(QA_ERR_INVALID, "max_new_tokens must be non-negative");
    if (n_tokens <= 0) return fail(QA_ERR_INVALID, "invalid backend cached text generation input");
    if (n_tokens + max_new > d->max_seq) return fail(QA_ERR_CAPACITY, "backend text generation exceeds KV-cache capacity");
    if (max_new == 0) return QA_OK;
    if (!d->embd) return fail(QA_ERR_INVALID, "decoder has no token embedding");
    int rc = ensure_rows(d, n_tokens);
    if (rc != QA_OK) return rc;
    const int32_t V = d->cfg.vocab;
    for (hipEvent_t & e : d->gen_ev) {
        if (!e) QA_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    if (margins && !d->h_logits) {
        QA_HIP(hipHostMalloc(reinterpret_cast<void **>(&d->h_logits), sizeof(float) * 2 * static_cast<size_t>(V)));
    }
    // Pipelined loop: decode step e + 1 (which feeds id e, already on the device) is queued before the host
    // reads id e, so the device never waits for the host's stop check.  Step k writes its id into pinned slot
    // k % 2 and (margins) its logits into pinned row k % 2, then records gen_ev[k % 2]; the host reads slot
    // e % 2 after gen_ev[e % 2], and step e + 2 reuses that slot only after.  When id e ends the loop (stop id,
    // out of range), the one step queued beyond it is rolled back: the length returns to the fed tokens, as if
    // it had never run (its K/V row lies past the length, where no call reads before writing it again).
    QA_HIP(hipMemcpyAsync(d->x, x, sizeof(float) * n_tokens * d->cfg.hidden, hipMemcpyHostToDevice, d->stream));
    rc = forward_device(d, n_tokens, 0, true);
    if (rc != QA_OK) return rc;
    QA_HIP(hipMemcpyAsync(d->h_ids, d->d_ids, sizeof(int32_t), hipMemcpyDeviceToHost, d->stream));
    if (margins) QA_HIP(hipMemcpyAsync(d->h_logits, d->logits, sizeof(float) * V, hipMemcpyDeviceToHost, d->stream));
    QA_HIP(hipEventRecord(d->gen_ev[0], d->stream));
    int32_t queued = 0;   // decode steps queued; step k (1-based) produces id k
    int32_t fed = 0;      // ids appended to the cache by the steps the loop keeps
    for (int32_t e = 0; e < max_new; ++e) {
        if (queued == e && e + 1 < max_new) {
            const int32_t k = e + 1;
            rc = decode_step(d, 1, k == 1, d->h_ids_dev + (k % 2));
            if (rc != QA_OK) return rc;
            if (margins) {
                QA_HIP(hipMemcpyAsync(d->h_logits + static_cast<size_t>(k % 2) * V, d->logits, sizeof(float) * V,
                                      hipMemcpyDeviceToHost, d->stream));
            }
            QA_HIP(hipEventRecord(d->gen_ev[k % 2], d->stream));
            queued = k;
        }
        QA_HIP(hipEventSynchronize(d->gen_ev[e % 2]));
        const int32_t id = d->h_ids[e % 2];
        bool stop = id < 0 || id >= V;
        if (!stop) {
            if (margins) margins[e] = top2_margin(d->h_logits + static_cast<size_t>(e % 2) * V, V, id);
            out_ids[(*n_out)++] = id;
            *total_tokens = n_tokens + *n_out;
            for (int32_t k = 0; k < n_stop; ++k) stop = stop || stop_ids[k] == id;
            if (stop) *stopped = 1;
        }
        if (stop) break;
        fed = e + 1;
    }
    QA_HIP(hipStreamSynchronize(d->stream));
    if (queued > fed) {
        // the step queued beyond the last kept id: length back to n_tokens + fed (device and host)
        rc = set_values_launch(d->d_lens, 1, n_tokens + fed, d->stream);
        if (rc != QA_OK) return rc;
        d->cur_len[0] = n_tokens + fed;
        QA_HIP(hipStreamSynchronize(d->stream));
    }
    rc = persist_check(d);
    if (rc != QA_OK) return rc;
    if (*n_out < max_new && !*stopped) return fail(QA_ERR_RANGE, "generated token id is out of range");
    return QA_OK;
}

extern "C" int qa_decoder_decode_streams(qa_decoder * d, const int32_t * first_ids, int32_t n_steps, int32_t * out_ids) {
    if (!d || !first_ids || (n_steps > 0 && !out_ids) || n_steps < 0) {
        return fail(QA_ERR_INVALID, "qa_decoder_decode_streams: invalid arguments");
    }
    const int32_t S = d->n_streams;
    for (int32_t s = 0; s < S; ++s) {
        if (d->cur_len[s] + n_steps > d->max_seq) {
            return fail(QA_ERR_CAPACITY, "decode steps exceed the KV-cache capacity of a stream");
        }
        if (first_ids[s] < 0 || first_ids[s] >= d->cfg.vocab) return fail(QA_ERR_RANGE, "first id out of range");
    }
    if (n_steps == 0) return QA_OK;
    if (static_cast<int64_t>(n_steps) * S > 4096LL * S) return fail(QA_ERR_INVALID, "too many steps");
    int rc = ensure_rows(d, S);
    if (rc != QA_OK) return rc;
    QA_HIP(hipMemcpyAsync(d->d_ids, first_ids, sizeof(int32_t) * S, hipMemcpyHostToDevice, d->stream));
    for (int32_t k = 0; k < n_steps; ++k) {
        rc = decode_step(d, S, k == 0, d->h_ids_dev + static_cast<size_t>(k) * S);
        if (rc != QA_OK) return rc;
    }
    QA_HIP(hipStreamSynchronize(d->stream));
    rc = persist_check(d);
    if (rc != QA_OK) return rc;
    std::memcpy(out_ids, d->h_ids, sizeof(int32_t) * static_cast<size_t>(n_steps) * S);
    return QA_OK;
}

extern "C" int qa_decoder_set_persistent(qa_decoder * d, int32_t enable) {
    if (!d) return fail(QA_ERR_INVALID, "qa_decoder_set_persistent: null decoder");
    if (!enable) {
        d->persist = false;
        return QA_OK;
    }
    int32_t grid = 0;
    int rc = persist_plan(persist_plan_in(d), &grid);
    if (rc != QA_OK) return rc;
    // the barrier wait bound in 100 MHz ticks (tests set a tiny bound to force the give-up path)
    d->persist_wait_ticks = 20000000;
    if (const char * e = std::getenv("QA_PERSIST_WAIT_TICKS")) d->persist_wait_ticks = std::strtoull(e, nullptr, 10);
    if (!d->persist_layers) {
        const qa_text_config & c = d->cfg;
        const size_t nl = static_cast<size_t>(c.n_layers), H = static_cast<size_t>(c.hidden);
        const size_t QD = static_cast<size_t>(c.n_heads) * kHeadDim, KD = static_cast<size_t>(c.n_kv_heads) * kHeadDim;
        if (!d->persist_ws) {
            rc = dmalloc_t(d->weight_allocs, (2 * nl - 1) * H, &d->persist_xbuf);
            rc = rc ? rc : dmalloc_t(d->weight_allocs, nl * (QD + 2 * KD), &d->persist_qkv);
            rc = rc ? rc : dmalloc_t(d->weight_allocs, nl * QD, &d->persist_attn);
            rc = rc ? rc : dmalloc_t(d->weight_allocs, nl * static_cast<size_t>(c.intermediate), &d->persist_act);
            const size_t ws_bytes = nl * persist_ws_stride(d->layout);
            rc = rc ? rc : dmalloc(d->weight_allocs, ws_bytes, &d->persist_ws);
            if (rc != QA_OK) return rc;
            d->persist_ws_bytes = ws_bytes;
            QA_HIP(hipMemsetAsync(d->persist_ws, 0, d->persist_ws_bytes, d->stream));
        }
        std::vector<PersistLayer> table(d->layers.size());
        for (size_t l = 0; l < d->layers.size(); ++l) {
            const DevLayer & L = d->layers[l];
            PersistLayer & t = table[l];
            t.qkv = L.qkv16 ? static_cast<const void *>(L.qkv16) : L.qkv;
            t.o = L.o16 ? static_cast<const void *>(L.o16) : L.o;
            t.gu = L.gu16 ? static_cast<const void *>(L.gu16) : L.gu;
            t.down = L.down16 ? static_cast<const void *>(L.down16) : L.down;
            t.attn_norm = L.attn_norm;
            t.ffn_norm = L.ffn_norm;
            t.q_norm = L.q_norm;
            t.k_norm = L.k_norm;
        }
        void * p = nullptr;
        rc = dmalloc(d->weight_allocs, sizeof(PersistLayer) * table.size(), &p);
        if (rc != QA_OK) return rc;
        QA_HIP(hipMemcpyAsync(p, table.data(), sizeof(PersistLayer) * table.size(), hipMemcpyHostToDevice, d->stream));
        QA_HIP(hipStreamSynchronize(d->stream));
        d->persist_layers = static_cast<PersistLayer *>(p);
    }
    // the barrier counters assume one grid per sync buffer: a new buffer (cleared) for a new grid
    if (!d->persist_sync || grid != d->persist_grid) {
        void * p = nullptr;
        rc = dmalloc(d->weight_allocs, persist_sync_bytes(grid), &p);
        if (rc != QA_OK) return rc;
        d->persist_sync = static_cast<uint32_t *>(p);
        d->persist_sync_bytes = persist_sync_bytes(grid);
        QA_HIP(hipMemsetAsync(p, 0, d->persist_sync_bytes, d->stream));
        d->persist_grid = grid;
    }
    QA_HIP(hipStreamSynchronize(d->stream));
    d->persist = true;
    return QA_OK;
}

extern "C" int qa_decoder_fill_cache(qa_decoder * d, int32_t stream, const float * k, const float * v, int32_t len) {
    if (!d || !k || !v || stream < 0 || stream >= d->n_streams || len < 0 || len > d->max_seq) {
        return fail(QA_ERR_INVALID, "qa_decoder_fill_cache: invalid arguments");
    }
    const size_t per_head = static_cast<size_t>(len) * kHeadDim;
    const size_t per_layer = per_head * d->cfg.n_kv_heads;
    if (per_layer * sizeof(float) > d->staging_bytes) {
        if (d->staging) (void)hipFree(d->staging);
        d->staging = nullptr;
        d->staging_bytes = 0;
        if (hipMalloc(reinterpret_cast<void **>(&d->staging), per_layer * sizeof(float)) != hipSuccess) {
            return fail(QA_ERR_ALLOC, "staging allocation failed");
        }
        d->staging_bytes = per_layer * sizeof(float);
    }
    const size_t esz = qa_kv_elem_bytes(d->cache_type);
    for (int32_t l = 0; l < d->cfg.n_layers; ++l) {
        for (int kv = 0; kv < 2; ++kv) {
            const float * src = (kv == 0 ? k : v) + per_layer * l;
            QA_HIP(hipMemcpyAsync(d->staging, src, per_layer * sizeof(float), hipMemcpyHostToDevice, d->stream));
            for (int32_t h = 0; h < d->cfg.n_kv_heads; ++h) {
                char * dst = static_cast<char *>(d->cache) +
                    esz * cache_row_offset(l, kv, stream, h, 0, d->n_streams, d->cfg.n_kv_heads, d->max_seq);
                const int rc = cast_rows_launch(d->staging + per_head * h, dst, d->cache_type,
                                                static_cast<int64_t>(per_head), d->stream);
                if (rc != QA_OK) return rc;
            }
            QA_HIP(hipStreamSynchronize(d->stream));
        }
    }
    return qa_decoder_set_cur_len(d, stream, len);
}

extern "C" int qa_decoder_layer_forward(qa_decoder * d, int32_t layer, const float * x, int32_t n_tokens, int32_t n_past,
                                        float * y) {
    if (!d || !x || !y || layer < 0 || layer >= d->cfg.n_layers) return fail(QA_ERR_INVALID, "qa_decoder_layer_forward");
    int rc = check_forward(d, n_tokens, n_past);
    if (rc != QA_OK) return rc;
    rc = ensure_rows(d, n_tokens);
    if (rc != QA_OK) return rc;
    QA_HIP(hipMemcpyAsync(d->x, x, sizeof(float) * n_tokens * d->cfg.hidden, hipMemcpyHostToDevice, d->stream));
    rc = set_values_launch(d->d_lens, 1, n_past, d->stream);
    d->cur_len[0] = n_past;
    if (rc == QA_OK) rc = run_layer(d, layer, n_tokens, n_tokens == 1 ? kDecode : kPrefill, n_past);
    if (rc == QA_OK) rc = set_values_launch(d->d_lens, 1, n_past + n_tokens, d->stream);
    if (rc != QA_OK) return rc;
    d->cur_len[0] = n_past + n_tokens;
    QA_HIP(hipMemcpyAsync(y, d->x, sizeof(float) * n_tokens * d->cfg.hidden, hipMemcpyDeviceToHost, d->stream));
    QA_HIP(hipStreamSynchronize(d->stream));
    return QA_OK;
}

extern "C" int qa_decoder_layer_forward_nocache(qa_decoder * d, int32_t layer, const float * x, int32_t n_tokens,
                                                float * y) {
    if (!d || !x || !y || layer < 0 || layer >= d->cfg.n_layers || n_tokens <= 0) {
        return fail(QA_ERR_INVALID, "invalid decoder input for text layer backend");
    }
    int rc = ensure_rows(d, n_tokens);
    if (rc != QA_OK) return rc;
    QA_HIP(hipMemcpyAsync(d->x, x, sizeof(float) * n_tokens * d->cfg.hidden, hipMemcpyHostToDevice, d->stream));
    rc = run_layer(d, layer, n_tokens, kNoCache, 0);
    if (rc != QA_OK) return rc;
    QA_HIP(hipMemcpyAsync(y, d->x, sizeof(float) * n_tokens * d->cfg.hidden, hipMemcpyDeviceToHost, d->stream));
    QA_HIP(hipStreamSynchronize(d->stream));
    return QA_OK;
}

extern "C" int qa_decoder_prefill_nocache(qa_decoder * d, const float * x, int32_t n_tokens, float * logits) {
    if (!d || !x || !logits || n_tokens <= 0) return fail(QA_ERR_INVALID, "invalid decoder input for text prefill backend");
    int rc = ensure_rows(d, n_tokens);
    if (rc != QA_OK) return rc;
    QA_HIP(hipMemcpyAsync(d->x, x, sizeof(float) * n_tokens * d->cfg.hidden, hipMemcpyHostToDevice, d->stream));
    for (int32_t l = 0; l < d->cfg.n_layers && rc == QA_OK; ++l) rc = run_layer(d, l, n_tokens, kNoCache, 0);
    if (rc == QA_OK) rc = logits_and_pick(d, n_tokens - 1, 1, false);
    if (rc != QA_OK) return rc;
    QA_HIP(hipMemcpyAsync(logits, d->logits, sizeof(float) * d->cfg.vocab, hipMemcpyDeviceToHost, d->stream));
    QA_HIP(hipStreamSynchronize(d->stream));
    return QA_OK;
}

extern "C" int qa_decoder_profile_enable(qa_decoder * d, int32_t enable) {
    if (!d) return fail(QA_ERR_INVALID, "qa_decoder_profile_enable");
    d->prof = enable != 0;
    return QA_OK;
}

extern "C" int qa_decoder_profile_reset(qa_decoder * d) {
    if (!d) return fail(QA_ERR_INVALID, "qa_decoder_profile_reset");
    QA_HIP(hipStreamSynchronize(d->stream));
    d->n_recs = 0;
    return QA_OK;
}

extern "C" int qa_decoder_profile_read(qa_decoder * d, const char * family, double * total_ms, int64_t * launches) {
    if (!d || !family || !total_ms || !launches) return fail(QA_ERR_INVALID, "qa_decoder_profile_read");
    int fam = -1;
    for (int i = 0; i < kFamCount; ++i) {
        if (std::strcmp(kFamNames[i], family) == 0) fam = i;
    }
    if (fam < 0) return fail(QA_ERR_INVALID, std::string("unknown kernel family: ") + family);
    QA_HIP(hipStreamSynchronize(d->stream));
    double total = 0.0;
    int64_t n = 0;
    for (size_t i = 0; i < d->n_recs; ++i) {
        if (d->recs[i].fam != fam) continue;
        float ms = 0.0f;
        QA_HIP(hipEventElapsedTime(&ms, d->recs[i].a, d->recs[i].b));
        total += ms;
        ++n;
    }
    *total_ms = total;
    *launches = n;
    return QA_OK;
}
