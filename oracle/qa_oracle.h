/*
 * qa_oracle.h -- CPU restatement of the Qwen3-ASR text-decoder KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The product library
 * never links or calls it.
 *
 * What it restates (citations into the reference, andimarafioti/qwenasr.cpp):
 *   - RMSNorm: src/text-decoder.cpp:542-557 (rms_norm_row; mean square in double)
 *   - NEOX RoPE: src/text-decoder.cpp:604-625 (apply_rope_position; angle in double)
 *   - linear: src/text-decoder.cpp:561-600 (f32 dot products; summation order differs, see below)
 *   - cached layer graph: src/text-decoder.cpp:347-474 (append into cache view, then attend)
 *   - logits: src/text-decoder.cpp:476-493; greedy loop: src/text-decoder.cpp:2209-2311
 *   - cache layout: src/text-decoder.cpp:1420-1474; bookkeeping: 1641-1755
 *   - non-cached causal layer: src/text-decoder.cpp:265-345
 * GGML op semantics that the reference relies on but does not contain (GGML is an absent
 * submodule) are restated from upstream GGML's public CPU code and marked [ggml-sem]:
 *   - ggml_cpy f32 -> f16 rounds to nearest even;
 *   - mul_mat with an f16 src0 converts src1 to f16 first (q before QK^T, probabilities before PV);
 *   - soft_max_ext: x * scale (+ mask), max, expf(x - max), sum in double, multiply by (float)(1/sum).
 * Parity of those three against real GGML is unpinned at bit level (GGML cannot be built here).
 *
 * Summation order: every dot product here sums in a fixed order that differs from the reference's
 * sequential loops and from GGML's SIMD order; results agree to f32 rounding, not bitwise.
 */
#ifndef QA_ORACLE_H
#define QA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_config {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab;
    float rope_theta, rms_norm_eps;
} orc_config;

typedef struct orc_layer {
    const float *attn_norm, *ffn_norm, *q, *k, *v, *o, *q_norm, *k_norm, *gate, *up, *down;
} orc_layer;

typedef struct orc_model {
    orc_config cfg;
    const orc_layer * layers;
    const float *token_embd, *output_norm, *output;
} orc_model;

/* Cache of one stream: K and V each [n_layers][n_kv_heads][max_seq][head_dim] in `dtype`
 * (0 = f32, 1 = f16 bits).  Same per-layer layout as the reference (text-decoder.cpp:1451-1462). */
typedef struct orc_cache {
    int32_t dtype, n_layers, n_kv_heads, head_dim, max_seq, cur_len;
    void *k, *v;
} orc_cache;

/* scalar helpers */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_array(const float * x, uint16_t * h, size_t n);
void orc_f16_to_f32_array(const uint16_t * h, float * x, size_t n);
void orc_rms_norm_row(const float * x, int32_t n, const float * w, float eps, float * y);
void orc_rope_rows(float * rows, int32_t position, int32_t n_heads, int32_t head_dim, float theta);
int64_t orc_slot_index(int32_t head, int32_t pos, int32_t dim, int32_t max_seq, int32_t head_dim);
void orc_positions(int32_t n_past, int32_t n_tokens, int32_t * out);
void orc_causal_mask(int32_t n_past, int32_t n_tokens, float * mask);
void orc_linear(const float * x, int32_t rows, int32_t in_dim, const float * w, int32_t out_dim, float * y);
int32_t orc_argmax(const float * logits, int32_t n);
int orc_set_threads(int32_t n);

/* Pieces of the path, each on explicit buffers. */
void orc_qk_prep(float * q, float * k, int32_t n_tokens, int32_t n_heads, int32_t n_kv_heads,
                 int32_t head_dim, const float * q_norm_w, const float * k_norm_w, int32_t pos0,
                 float theta, float eps);
/* Writes T rows (already prepared k and raw v, [T][kv_dim] f32) at positions n_past.. of `layer`. */
void orc_cache_write(orc_cache * cache, int32_t layer, const float * k, const float * v,
                     int32_t n_past, int32_t n_tokens);
/* Attention of T queries q [T][q_dim] at positions n_past.. over cache rows [0, n_past + t]. */
void orc_cache_attention(const orc_cache * cache, int32_t layer, const float * q, int32_t n_past,
                         int32_t n_tokens, int32_t n_heads, float scale, float * out);
/* Causal f32 attention, K/V never cached (text-decoder.cpp:320-334). */
void orc_causal_attention_f32(const float * q, const float * k, const float * v, int32_t n_tokens,
                              int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, float scale,
                              float * out);

/* Whole layers and the model. */
int orc_layer_forward_cached(const orc_model * m, int32_t layer, const float * x, int32_t n_tokens,
                             int32_t n_past, orc_cache * cache, float * y);
int orc_layer_forward_nocache(const orc_model * m, int32_t layer, const float * x, int32_t n_tokens,
                              float * y);
int orc_logits(const orc_model * m, const float * state, float * logits);
int orc_forward_cached(const orc_model * m, const float * x, int32_t n_tokens, int32_t n_past,
                       orc_cache * cache, float * logits);
/* margins[k] / runner_up[k] (either may be NULL): gap between the greedy pick of step k and the
 * runner-up, and the runner-up's id (first index of the largest other logit).                 */
int orc_generate_cached(const orc_model * m, const float * x, int32_t n_tokens, int32_t max_new,
                        const int32_t * stop_ids, int32_t n_stop, orc_cache * cache,
                        int32_t * out_ids, int32_t * n_out, int32_t * stopped, int32_t * total_tokens,
                        float * margins, int32_t * runner_up);
/* n_steps single-token steps starting from token first_id at cache->cur_len; out_ids[k] is the
 * greedy pick after step k (config 4 per-stream statement). */
int orc_decode_steps(const orc_model * m, orc_cache * cache, int32_t first_id, int32_t n_steps,
                     int32_t * out_ids, float * margins, int32_t * runner_up);

#ifdef __cplusplus
}
#endif

#endif
