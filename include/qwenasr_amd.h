/*
 * qwenasr_amd.h -- C ABI of the MI355X (gfx950) Qwen3-ASR text-decoder KV-cache path.
 *
 * Three layers, all plain C: raw device pointers, sizes, an opaque hipStream_t passed as void*,
 * and an int status (QA_OK == 0).  No torch or C++ types cross this boundary.
 *
 *  1. Kernel layer  (qa_kv_*, qa_decode_attn*, qa_prefill_attn*, qa_*gemv*, ...): one call = one
 *     or two kernel launches on the given stream.  These replace the GGML op chains that
 *     src/text-decoder.cpp builds for the cached layer (lines 347-474).
 *  2. Runtime layer (qa_decoder_*): device weights, KV cache, workspaces and the decode-step
 *     driver.  It replaces QwenAsrTextDecoderBackend (src/text-decoder.cpp:165-189) and the
 *     per-call bookkeeping of text_decoder_backend_cached_logits (1641-1755).
 *  3. Model layer   (qa_synth_*, qa_model_*): seeded synthetic weights and inputs on the host.
 *
 * The C++ drop-in of the reference's src/text-decoder.h and src/ggml-backends.h is implemented on
 * top of layers 2 and 3 (include/text-decoder.h, include/ggml-backends.h).
 */
#ifndef QWENASR_AMD_H
#define QWENASR_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status codes */
enum {
    QA_OK = 0,
    QA_ERR_INVALID = 1,      /* bad argument or shape (reference: "invalid ... configuration") */
    QA_ERR_CAPACITY = 2,     /* n_past + T > max_seq_len (text-decoder.cpp:1652-1656, 2230-2233) */
    QA_ERR_DEVICE = 3,       /* a HIP call failed */
    QA_ERR_NO_DEVICE = 4,    /* no gfx950 device visible */
    QA_ERR_ALLOC = 5,        /* device or host allocation failed */
    QA_ERR_RANGE = 6         /* generated token id out of range (text-decoder.cpp:2275-2278) */
};

/* Last error message of the calling thread (never NULL). */
const char * qa_last_error(void);

/* ---------------------------------------------------------------- device */
/* Number of visible HIP devices; 0 when none (never an error). */
int qa_device_count(void);
/* Fills name (e.g. "gfx950") of device 0; returns QA_ERR_NO_DEVICE when there is none. */
int qa_device_arch(char * name, size_t name_len);

/* Synchronous device -> host copy (test and inspection helper). */
int qa_copy_to_host(void * host_dst, const void * dev_src, size_t bytes);
/* Waits for all work on device 0 (hipDeviceSynchronize). */
int qa_device_synchronize(void);

/* Device memory, copies and timing on device 0, so hosts (tests, benchmarks, FFI callers) need no
 * second HIP runtime of their own.  stream NULL is the default stream. */
int qa_device_malloc(void ** out, size_t bytes);
int qa_device_free(void * dev_ptr);
int qa_copy_to_device(void * dev_dst, const void * host_src, size_t bytes);
/* Device-to-device copy on `stream` (also the known-size reference for HBM traffic counters). */
int qa_copy_device(void * dev_dst, const void * dev_src, size_t bytes, void * stream);
int qa_memset_device(void * dev_dst, int value, size_t bytes);
int qa_event_create(void ** event);
int qa_event_destroy(void * event);
int qa_event_record(void * event, void * stream);
/* Waits for `stop`, then ms = time between the two recorded events. */
int qa_event_elapsed_ms(void * start, void * stop, float * ms);
int qa_stream_synchronize(void * stream);

/* ---------------------------------------------------------------- KV cache layout (rows a1, a2)
 * One allocation holds K and V for every layer and stream.  Element (layer, kv, stream, head, pos, i)
 * with kv = 0 for K and 1 for V lives at element index
 *
 *     ((((layer * 2 + kv) * n_streams + stream) * n_kv_heads + head) * max_seq + pos) * head_dim + i
 *
 * so for one (layer, kv, stream) the block is exactly the reference's per-layer tensor
 * ne = [head_dim, max_seq_len, n_kv_heads] (text-decoder.cpp:1451-1462): head-major, then
 * position, then dim, i.e. slot (h, p, i) at (h * max_seq_len + p) * head_dim + i.            */
typedef enum { QA_CACHE_F32 = 0, QA_CACHE_F16 = 1 } qa_cache_type;

typedef struct qa_kv_layout {
    int32_t n_layers;
    int32_t n_streams;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t max_seq;
    int32_t cache_type;      /* qa_cache_type */
} qa_kv_layout;

int qa_kv_layout_check(const qa_kv_layout * layout);
size_t qa_kv_elem_bytes(int32_t cache_type);
/* Total bytes of the K+V allocation; 0 for an invalid layout. */
size_t qa_kv_cache_bytes(const qa_kv_layout * layout);
/* Element index of one slot (see the formula above); -1 when out of range. */
int64_t qa_kv_slot_index(const qa_kv_layout * layout, int32_t layer, int32_t kv, int32_t stream,
                         int32_t head, int32_t pos, int32_t dim);
/* hipMalloc + zero fill (the reference clears its KV buffer, text-decoder.cpp:1472). */
int qa_kv_cache_alloc(const qa_kv_layout * layout, void ** dev_cache);
int qa_kv_cache_free(void * dev_cache);

/* Host bookkeeping of one cached call (text-decoder.cpp:1724-1735): positions[i] = n_past + i and
 * the dense causal mask mask[q][k] = 0 if k <= n_past + q else -inf, row length n_past + T.
 * The GPU kernels never read the mask; these exist so the bookkeeping can be checked bit-exactly. */
int qa_positions(int32_t n_past, int32_t n_tokens, int32_t * positions);
int qa_causal_mask(int32_t n_past, int32_t n_tokens, float * mask);

/* ---------------------------------------------------------------- kernel layer
 * Shapes use row-major C order.  q_dim = n_heads * head_dim, kv_dim = n_kv_heads * head_dim.
 * Only head_dim == 128 and n_heads == 2 * n_kv_heads are implemented (Qwen3-ASR 0.6B and 1.7B);
 * other shapes are rejected with QA_ERR_INVALID before any launch.                              */

/* Fused q/k/v preparation and cache write (rows a5, a10).
 * qkv      : [n_streams * n_tokens][q_dim + 2 * kv_dim] f32, projection outputs (q | k | v) of each
 *            token; row r belongs to stream r / n_tokens, token r % n_tokens.
 * n_past   : device int32[n_streams]; token t of stream s is at position n_past[s] + t.
 * q_out    : [n_streams * n_tokens][q_dim] f32 <- RoPE(RMSNorm(q_h) * q_norm_w).
 * cache    : K row  <- cast(RoPE(RMSNorm(k_h) * k_norm_w)),  V row <- cast(v_h), at that position.
 * RMSNorm and RoPE follow the reference's scalar statement (text-decoder.cpp:542-557, 604-625):
 * mean square in double, scale = 1/sqrtf(float(ms) + eps), NEOX pairs (i, i + head_dim/2) with
 * angle = pos * exp(-ln(theta) * 2i / head_dim) in double; the cast to f16 rounds to nearest even. */
int qa_kv_append(const float * qkv, const float * q_norm_w, const float * k_norm_w,
                 float * q_out, void * cache, const qa_kv_layout * layout, int32_t layer,
                 const int32_t * n_past, int32_t n_streams, int32_t n_tokens, int32_t n_heads,
                 float rope_theta, float eps, void * stream);

/* Split-K GQA decode attention over the cache (row a6), one query token per stream (two launches:
 * scores + chunk statistics, then normalised PV + merge).
 * q       : [n_streams][q_dim] f32 (post norm + RoPE), out: [n_streams][q_dim] f32.
 * lens    : device int32[n_streams]; stream s attends positions [0, lens[s]).  Every lens[s] must be
 *           in [1, max_len] and max_len <= layout->max_seq.
 * Q head h reads KV head h / (n_heads / n_kv_heads) (text-decoder.cpp:725, 1035).
 * Arithmetic is that of the reference's GGML graph (text-decoder.cpp:454-461) for the cache dtype:
 *   f16 cache: s_j = f32dot(f16(q), K_j) * scale; p = expf(s - max) * (float)(1 / sum), the sum in
 *              double; p -> f16; o = f32dot(p, V).   f32 cache: no f16 rounding of q or p.
 * workspace: device scratch of qa_decode_attn_workspace_bytes(layout->n_streams, n_heads,
 * layout->max_seq) bytes, i.e. sized by the cache CAPACITY so its internal offsets never move.  Its
 * counters must be zero before the first call (qa_workspace_clear); every call leaves them zero
 * again, so one workspace serves any sequence of calls on that cache.  Calls that share a
 * workspace must be stream-ordered.                                                             */
size_t qa_decode_attn_workspace_bytes(int32_t n_streams, int32_t n_heads, int32_t max_seq);
int qa_workspace_clear(void * workspace, size_t bytes, void * stream);
int qa_decode_attn(const float * q, const void * cache, const qa_kv_layout * layout, int32_t layer,
                   const int32_t * lens, int32_t n_streams, int32_t max_len, int32_t n_heads,
                   float scale, float * out, void * workspace, size_t workspace_bytes, void * stream);

/* One decode step of a layer's KV-cache path with the append fused in (rows a5 + a6): for each stream s,
 * the token at position n_past[s] is appended and attended.  qkv: [n_streams][q_dim + 2 * kv_dim]
 * raw projection rows (q | k | v).  The kernel applies q_norm/k_norm RMSNorm and NEOX RoPE exactly
 * as qa_kv_append does (same bits), writes the new K and V rows into the cache at n_past[s], and
 * computes what qa_decode_attn computes over positions [0, n_past[s] + 1).  n_past[s] + 1 must be
 * in [1, max_len], max_len <= layout->max_seq.  n_past itself is not advanced (qa_advance_lens).
 * out: [n_streams][q_dim].  Workspace as for qa_decode_attn.  Equals qa_kv_append followed by
 * qa_decode_attn on lens = n_past + 1 (text-decoder.cpp:410-463 at T = 1).                      */
int qa_decode_step_attn(const float * qkv, const float * q_norm_w, const float * k_norm_w, void * cache,
                        const qa_kv_layout * layout, int32_t layer, const int32_t * n_past, int32_t n_streams,
                        int32_t max_len, int32_t n_heads, float rope_theta, float eps, float scale, float * out,
                        void * workspace, size_t workspace_bytes, void * stream);

/* Allocation-free qa_decode_step_attn.  No counterpart in the reference: it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * kernels, arguments and results as qa_decode_step_attn, without the workspace: it lives in a
 * file-scope device array of QA_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until
 * the process ends.  The call allocates nothing (no hipMalloc, hipFree or allocating library routine);
 * it zeroes its merge counters with a small kernel each time, so any sequence of calls with different
 * layouts is correct.  A layout whose workspace (qa_decode_attn_workspace_bytes(layout->n_streams,
 * n_heads, layout->max_seq)) exceeds the maximum is rejected with QA_ERR_INVALID before any launch;
 * 48 MiB covers 32 streams of 4.5k positions or one stream of 150k.  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (different streams, threads or processes' graphs replayed
 * concurrently) race and must be serialised by the caller.                                        */
#define QA_NOALLOC_SCRATCH_BYTES ((size_t)48 << 20)
int qa_decode_step_attn_noalloc(const float * qkv, const float * q_norm_w, const float * k_norm_w, void * cache,
                                const qa_kv_layout * layout, int32_t layer, const int32_t * n_past, int32_t n_streams,
                                int32_t max_len, int32_t n_heads, float rope_theta, float eps, float scale, float * out,
                                void * stream);
/* Set-up of qa_decode_step_attn_noalloc on the current device: resolves the device address of its
 * scratch array (hipGetSymbolAddress), once per device.  No counterpart in the reference.  The entry
 * point does this itself on a device's first call, but refuses a first call made while its stream is
 * being captured (QA_ERR_INVALID), so callers that capture call this (or the entry point once) before
 * capturing.  qa_decoder_create calls it for the device it runs on.                              */
int qa_decode_noalloc_prepare(void);

/* Causal prefill attention over the cache (row a7): the n_tokens queries of stream `stream_idx` at
 * positions n_past .. n_past + n_tokens - 1, query t attending keys [0, n_past + t].  Same
 * arithmetic as qa_decode_attn.  f16 caches run on CDNA4 f16 MFMA as two kernels (row statistics,
 * then p and PV) over work items pulled from per-KV-head queues.
 * workspace (f16 caches): qa_prefill_attn_workspace_bytes(n_tokens, n_heads) bytes, cleared once
 * with qa_workspace_clear before the first call; it holds the queue and merge counters (every call
 * leaves them zero, so one workspace serves any sequence of calls with at most n_tokens tokens),
 * the statistics and the partial outputs of the longest query tiles.  A smaller workspace that
 * still holds the counters and statistics runs without cutting tiles; a missing one is an error.
 * Calls that share a workspace must be stream-ordered.  f32 caches use no workspace.            */
size_t qa_prefill_attn_workspace_bytes(int32_t n_tokens, int32_t n_heads);
int qa_prefill_attn(const float * q, const void * cache, const qa_kv_layout * layout, int32_t layer,
                    int32_t stream_idx, int32_t n_past, int32_t n_tokens, int32_t n_heads, float scale,
                    float * out, void * workspace, size_t workspace_bytes, void * stream);

/* Causal attention with f32 K/V that are never cached (row a8: text-decoder.cpp:265-345, used by
 * qwenasr_text_prefill_backend_forward and the layer backend).  q: [T][q_dim], k, v: [T][kv_dim]
 * (k post norm + RoPE), out: [T][q_dim]; positions are 0..T-1.                                 */
int qa_causal_attn_f32(const float * q, const float * k, const float * v, int32_t n_tokens,
                       int32_t n_heads, int32_t n_kv_heads, float scale, float * out, void * stream);

/* Non-cached q/k preparation: q, k (in place, rows of q_dim / kv_dim) <- RoPE(RMSNorm(.) * w)
 * at positions pos0 + t.  v is left untouched.                                                  */
int qa_qk_prep(float * qkv, int32_t n_tokens, int32_t n_heads, int32_t n_kv_heads,
               const float * q_norm_w, const float * k_norm_w, int32_t pos0, float rope_theta,
               float eps, void * stream);

/* ---------------------------------------------------------------- adjacent decoder ops (row f1)
 * f32 weights stored row-major [out][in] (GGML ne = [in, out], text-decoder.cpp:219-227).       */
/* Skinny GEMM for the multi-stream decode step (one token per stream): y[rows][out] (+)= x[rows][in] *
 * W[out][in]^T for 1 <= rows <= 64 and in_dim a multiple of 32, on f32 MFMA (exact f32 products,  *
 * f32 sums).  Replaces the decode-time linear_ggml calls (text-decoder.cpp:83-90) at batch > 1.     *
 * The workspace (qa_gemm_rows_workspace_bytes, zeroed once) holds tile counters that every call  *
 * leaves at zero, in a fixed region, then per-slice partials: a workspace sized for the largest   *
 * shape serves every smaller one; calls sharing it must be stream-ordered.  out_dim <= 262144.    */
size_t qa_gemm_rows_workspace_bytes(int32_t out_dim, int32_t in_dim, int32_t rows);
int qa_gemm_rows(const float * W, int32_t out_dim, int32_t in_dim, const float * x, int32_t rows, float * y,
                 int32_t accumulate, void * workspace, size_t workspace_bytes, void * stream);
/* qa_gemm_rows with the decode step's neighbouring ops fused (rows <= 32, in_dim % 64 == 0), replacing  *
 * the rms_norm * w before q/k/v and gate/up and the silu * up after gate/up (text-decoder.cpp:92-98,   *
 * 365-373, 602) and the separate RMSNorm/SwiGLU passes:                                               *
 *  - norm_w != NULL: x is replaced by RMSNorm(x) * norm_w (eps).  stats_in = [n_stats_in][32] doubles, *
 *    partial sums of squares of each x row (row r at [k][r]), added in order k = 0, 8, 16, .. then     *
 *    1, 9, .. (8 interleaved parts), 1 <= n_stats_in <= 128;                                           *
 *  - stats_out != NULL: [ceil(out_dim / 32)][32] partial sums of squares of each stored y row (after   *
 *    accumulation), the stats_in of a following normalised GEMM;                                      *
 *  - swiglu != 0: W = [gate rows; up rows] (out_dim = 2 I, I % 16 == 0), y[rows][I] = silu(g) * u;     *
 *    needs accumulate == 0 and stats_out == NULL.                                                     */
int qa_gemm_rows_fused(const float * W, int32_t out_dim, int32_t in_dim, const float * x, int32_t rows,
                       float * y, int32_t accumulate, const float * norm_w, const double * stats_in,
                       int32_t n_stats_in, float eps, double * stats_out, int32_t swiglu,
                       void * workspace, size_t workspace_bytes, void * stream);
/* qa_gemm_rows_fused with the weights given as bf16 bits (the high halves of bf16-exact f32 weights,  *
 * see qa_pack_bf16), reading half the bytes.  The products run on bf16 MFMAs with each x split into    *
 * three bf16 parts (x = hi + mid + lo exactly): every product is exact and the sums are f32, as in     *
 * qa_gemm_rows_fused, in another order.  rows <= 32 and in_dim % 64 == 0.                             */
int qa_gemm_rows_fused_bf16(const uint16_t * W_bf16, int32_t out_dim, int32_t in_dim, const float * x, int32_t rows,
                            float * y, int32_t accumulate, const float * norm_w, const double * stats_in,
                            int32_t n_stats_in, float eps, double * stats_out, int32_t swiglu,
                            void * workspace, size_t workspace_bytes, void * stream);
/* The prefill GEMM on bf16-exact weights (T > 32 rows), replacing linear_ggml (text-decoder.cpp:83-90)  *
 * there: x_split = [rows][3 in_dim] bf16 bits, each row the three-part split [hi | mid | lo] of an f32  *
 * input row (x = hi + mid + lo exactly), and y[rows][out_dim] (+)= sum of the three parts times W^T:    *
 * exact f32 products, f32 sums (bf16 MFMA).  in_dim % 64 == 0, out_dim % 256 == 0.  With act_split    *
 * != NULL (y NULL, accumulate 0) W_bf16 = [gate rows; up rows] (2 out_dim rows, out_dim % 128 == 0)    *
 * and act_split[rows][3 out_dim] receives the split of silu(gate) * up (text-decoder.cpp:602).         */
int qa_gemm_split3_bf16(const uint16_t * W_bf16, int32_t out_dim, int32_t in_dim, const uint16_t * x_split,
                        int32_t rows, float * y, int32_t accumulate, uint16_t * act_split, void * stream);

/* y[r][o] = sum_i W[o][i] * x[r][i]  (+ y[r][o] when accumulate != 0); rows small (decode).     */
int qa_gemv(const float * W, int32_t out_dim, int32_t in_dim, const float * x, int32_t rows,
            float * y, int32_t accumulate, void * stream);
/* One decode-step GEMV with its fused neighbours (text-decoder.cpp:365-373, 465-493, 602), the     *
 * kernel the decoder runs at batch 1: y = W x (epilogue 0), y += W x (1), or y[o] = silu(g) * u     *
 * with W = [gate rows; up rows] of 2 out_dim rows (2); norm_w != NULL first replaces x by           *
 * RMSNorm(x) * norm_w (eps).  Pass the weights as f32 (W) or, for bf16-exact weights, as their     *
 * bf16 bits (W_bf16, see qa_pack_bf16): both give the same result bit for bit.                     *
 * in_dim one of 1024, 2048, 3072, 4096, 6144.                                                       */
int qa_gemv_fused(const float * W, const uint16_t * W_bf16, int32_t out_dim, int32_t in_dim, const float * x,
                  float * y, int32_t epilogue, const float * norm_w, float eps, void * stream);
/* dst[i] = the high 16 bits of src[i] (device buffers); *inexact (device, cleared by the caller)     *
 * gets bit 0 set when any low half is non-zero, i.e. when src is not bf16-exact.  A checkpoint      *
 * converted from bf16 weights (convert.py:386-387 widens them with tensor.float()) is bf16-exact.  */
int qa_pack_bf16(const float * src, int64_t n, uint16_t * dst, uint32_t * inexact, void * stream);
/* RMSNorm of each row (text-decoder.cpp:92-98): y = x * (1/sqrtf(mean(x^2) + eps)) * w.          */
int qa_rmsnorm_rows(const float * x, const float * w, int32_t rows, int32_t dim, float eps, float * y,
                    void * stream);
/* a[r][i] = silu(g[r][i]) * u[r][i] over rows of width dim, reading gu = [rows][2*dim] (g | u).   */
int qa_swiglu_rows(const float * gu, int32_t rows, int32_t dim, float * a, void * stream);
/* y += x elementwise. */
int qa_add_inplace(float * y, const float * x, size_t n, void * stream);
/* Greedy pick per row: first index of the maximum, NaN never wins (text-decoder.cpp:2266-2274).
 * ids[r] = -1 when no value beats -inf.  The workspace (qa_argmax_workspace_bytes) must be cleared
 * once with qa_workspace_clear; each call leaves its counters zero again.                        */
size_t qa_argmax_workspace_bytes(int32_t rows);
int qa_argmax_rows(const float * logits, int32_t rows, int32_t vocab, int32_t * ids, void * workspace,
                   size_t workspace_bytes, void * stream);
/* out[r] = table[ids[r]] (rows of width dim); ids out of [0, n_rows) give a zero row.            */
int qa_embed_rows(const float * table, int32_t n_rows, int32_t dim, const int32_t * ids, int32_t rows,
                  float * out, void * stream);
/* lens[s] += delta for s < n (device bookkeeping of a decode step). */
int qa_advance_lens(int32_t * lens, int32_t n, int32_t delta, void * stream);

/* ---------------------------------------------------------------- model layer (host) */
typedef struct qa_text_config {
    int32_t n_layers;
    int32_t hidden;
    int32_t n_heads;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t intermediate;
    int32_t vocab;
    float rope_theta;
    float rms_norm_eps;
} qa_text_config;

/* Host pointers to f32 weights, GGML/GGUF layout (linear weights row-major [out][in]). */
typedef struct qa_layer_weights {
    const float * attn_norm;   /* [hidden] */
    const float * ffn_norm;    /* [hidden] */
    const float * q;           /* [q_dim][hidden] */
    const float * k;           /* [kv_dim][hidden] */
    const float * v;           /* [kv_dim][hidden] */
    const float * o;           /* [hidden][q_dim] */
    const float * q_norm;      /* [head_dim] */
    const float * k_norm;      /* [head_dim] */
    const float * gate;        /* [intermediate][hidden] */
    const float * up;          /* [intermediate][hidden] */
    const float * down;        /* [hidden][intermediate] */
} qa_layer_weights;

typedef struct qa_model_weights {
    const qa_layer_weights * layers;   /* n_layers entries */
    const float * token_embd;          /* [vocab][hidden] */
    const float * output_norm;         /* [hidden] */
    const float * output;              /* [vocab][hidden] */
} qa_model_weights;

/* Seeded generator (counter-based splitmix64 + Box-Muller); see csrc/synth.cpp. */
uint64_t qa_synth_key(uint64_t base_seed, const char * name);
uint64_t qa_synth_word(uint64_t key, uint64_t index);
void qa_synth_fill_normal(float * out, size_t n, uint64_t base_seed, const char * name, double stddev);
void qa_synth_fill_const(float * out, size_t n, float value);
void qa_synth_fill_ids(int32_t * out, size_t n, uint64_t base_seed, const char * name, int32_t lo, int32_t hi);

/* Synthetic Qwen3-ASR text model: every linear weight and the embedding N(0, 0.02) keyed by its
 * GGUF tensor name, norm weights 1.0, output.weight tied to token_embd (same host buffer).       */
typedef struct qa_model qa_model;
int qa_model_synthetic(const qa_text_config * cfg, uint64_t seed, qa_model ** out);
/* Rounds every tensor of the model to the nearest bf16 value (ties to even), kept as f32: the      *
 * values a checkpoint converted from the released bf16 weights holds (convert.py:386-387).        */
int qa_model_round_bf16(qa_model * model);
void qa_model_free(qa_model * model);
/* Host view of one tensor by GGUF name (e.g. "text.blk.3.attn_q.weight"); NULL if absent. */
const float * qa_model_tensor(const qa_model * model, const char * name, int64_t * n_elems);
int qa_model_config(const qa_model * model, qa_text_config * cfg);

/* Decoder-input assembly (qwenasr_decoder_input_from_audio, decoder-input.cpp:26-101, after the
 * prompt has been tokenized): row t of out [n_tokens][hidden] is the embedding row of ids[t], except
 * that the i-th id equal to audio_token_id takes audio row i of audio [audio_tokens][hidden].  All
 * host memory.  Everything is validated before out is written, with the reference's errors: no ids,
 * a negative audio_token_id, an empty audio block, an id outside [0, vocab), more placeholders than
 * audio rows, or fewer.                                                                          */
int qa_decoder_input_assemble(const float * token_embd, int32_t vocab, int32_t hidden, const int32_t * ids,
                              int32_t n_tokens, int32_t audio_token_id, const float * audio, int32_t audio_tokens,
                              float * out);
int qa_model_weights_view(const qa_model * model, qa_layer_weights * layers, int32_t n_layers,
                          qa_model_weights * weights);

/* Special-token ids of Qwen3-ASR (convert.py:334-354 defaults; native-model.cpp:411-434). */
enum {
    QA_TOKEN_ENDOFTEXT = 151643,
    QA_TOKEN_IM_START = 151644,
    QA_TOKEN_IM_END = 151645,
    QA_TOKEN_AUDIO_START = 151669,
    QA_TOKEN_AUDIO_END = 151670,
    QA_TOKEN_AUDIO_PAD = 151676,
    QA_TOKEN_ASR_TEXT = 151704
};

/* Writes `model` as a GGUF v3 checkpoint that the reference's loader accepts: the metadata keys of
 * qwenasr_load_gguf_metadata (native-model.cpp:188-218), a placeholder tokenizer vocabulary with the
 * special tokens at their ids (the reference's fixture layout, native-model.cpp:407-431; a vocabulary
 * smaller than Qwen3-ASR's holds them at its last seven ids, in the order of the enum above) and every
 * text tensor in f32 with GGML ne order (load_text_layer_tensors, text-decoder.cpp:191-228).  Replaces
 * the checkpoint side of convert.py:357-397 for synthetic models.                                 */
int qa_gguf_write_model(const qa_model * model, const char * path);

/* The ASR prompt of qwenasr_build_asr_prompt (tokenizer.cpp:529-549): system turn with system_text,
 * user turn holding audio_tokens <|audio_pad|> placeholders between <|audio_start|> and <|audio_end|>
 * (a negative count counts as 0), the assistant turn, and "language NAME<asr_text>" when language is
 * non-empty.  Writes at most cap bytes including the terminating NUL; *len (may be NULL) receives the
 * full length without the NUL.  QA_ERR_RANGE when cap is too small (nothing is written then).     */
int qa_build_asr_prompt(int32_t audio_tokens, const char * system_text, const char * language, char * out,
                        size_t cap, size_t * len);

/* Audio-encoder output length for `input_frames` mel frames (qwenasr_audio_output_length,
 * audio-features.cpp:14-19): 13 tokens per 100 frames plus the tail's two stride-2 stages.      */
int32_t qa_audio_output_length(int32_t input_frames);

/* Header of a WAV file as the reference's reader sees it (qwenasr_read_wav_16k_mono,
 * audio-features.cpp:120-200): the sample-frame count of the data chunk and the sample rate.
 * QA_ERR_INVALID with the reference's messages for a missing file, a rate other than 16 kHz, no
 * data, or an encoding other than PCM16, PCM24 or f32.                                           */
int qa_wav_info(const char * path, int64_t * n_samples, int32_t * sample_rate);

/* ---------------------------------------------------------------- runtime layer */
typedef struct qa_decoder qa_decoder;

/* Uploads the weights, allocates the cache (zeroed) and workspaces on device 0. */
int qa_decoder_create(const qa_text_config * cfg, const qa_model_weights * weights, int32_t n_streams,
                      int32_t max_seq, int32_t cache_type, qa_decoder ** out);
void qa_decoder_destroy(qa_decoder * dec);
/* 1 when the decoder holds bf16 copies of its projection and LM-head weights (every one of them was   *
 * bf16-exact at creation, as in a checkpoint converted from bf16 weights, convert.py:386-387, and    *
 * QA_WEIGHTS_F32=1 was not set), which the batch-1 GEMVs then read with unchanged f32 results.     */
int qa_decoder_weights_bf16(const qa_decoder * dec);
/* Host mirror of the per-stream lengths (cur_len of the reference, text-decoder.cpp:186). */
int qa_decoder_cur_len(const qa_decoder * dec, int32_t stream, int32_t * cur_len);
/* Reads the device-side lengths (what the kernels use) into lens[n_streams]. */
int qa_decoder_device_lens(qa_decoder * dec, int32_t * lens);
int qa_decoder_set_cur_len(qa_decoder * dec, int32_t stream, int32_t cur_len);
void * qa_decoder_cache(qa_decoder * dec, qa_kv_layout * layout);
void * qa_decoder_stream(qa_decoder * dec);

/* One cached call of stream 0 (text_decoder_backend_cached_logits, text-decoder.cpp:1641-1755):
 * x: [T][hidden] host f32 at positions n_past.., logits (host, may be NULL): [vocab] of the last
 * token.  Sets cur_len = n_past + T.                                                            */
int qa_decoder_forward(qa_decoder * dec, const float * x, int32_t n_tokens, int32_t n_past, float * logits);

/* Greedy generation of stream 0 (qwenasr_text_generate_cached_backend, text-decoder.cpp:2209-2311).
 * out_ids must hold max_new_tokens entries.  margins (may be NULL) receives the top1 - top2 logit
 * gap of each produced token.                                                                    */
int qa_decoder_generate(qa_decoder * dec, const float * x, int32_t n_tokens, int32_t max_new_tokens,
                        const int32_t * stop_ids, int32_t n_stop, int32_t * out_ids, int32_t * n_out,
                        int32_t * stopped, int32_t * total_tokens, float * margins);

/* Lock-step decode of all streams (config 4): stream s starts at cur_len[s] with token first_ids[s]
 * and runs n_steps steps, each appending one token per stream.  out_ids: [n_steps][n_streams]. */
int qa_decoder_decode_streams(qa_decoder * dec, const int32_t * first_ids, int32_t n_steps,
                              int32_t * out_ids);

/* Decode-step capture without a graph (text-decoder.cpp:1658-1739 rebuilds and schedules a graph per
 * token): with enable = 1, every batch-1 decode step of this decoder (generate, and cached forwards of
 * one token) runs all its layers as ONE persistent launch (one workgroup per CU), whose workgroups walk
 * the layers' six phases behind grid barriers, driven by the device-side length; the LM head and the
 * pick follow as two launches.  Results are bit-identical to the eager step (same device code per
 * phase).  QA_ERR_INVALID if no persistent kernel is instantiated for the decoder's shapes (streams,
 * hidden/intermediate size, weight copies, cache dtype and the capacity's attention tiling); the decoder
 * then stays eager.  Every barrier wait is bounded (200 ms): an abandoned launch makes the call that
 * ran it return QA_ERR_DEVICE, and the decoder clears its barrier and merge state.  enable = 0 returns to
 * the eager step.                                                                                  */
int qa_decoder_set_persistent(qa_decoder * dec, int32_t enable);

/* Copies host K/V rows into stream `stream`'s cache slot for every layer (config 4 prefill of
 * random K/V).  k, v: [n_layers][n_kv_heads][len][head_dim] f32 (cast to the cache dtype).      */
int qa_decoder_fill_cache(qa_decoder * dec, int32_t stream, const float * k, const float * v, int32_t len);

/* Single decoder layer (config 0 / row a5-a6): one cached call of layer `layer` only,
 * x: [T][hidden] host in, y: [T][hidden] host out. The cache and cur_len advance like a forward. */
int qa_decoder_layer_forward(qa_decoder * dec, int32_t layer, const float * x, int32_t n_tokens,
                             int32_t n_past, float * y);

/* Non-cached single layer (row a8; qwenasr_text_layer_backend_forward, text-decoder.cpp:1305-1390):
 * positions 0..T-1, causal f32 attention with K/V never stored; the cache is not touched.       */
int qa_decoder_layer_forward_nocache(qa_decoder * dec, int32_t layer, const float * x, int32_t n_tokens,
                                     float * y);
/* Non-cached prefill of all layers + last-row logits (qwenasr_text_prefill_backend_forward,
 * text-decoder.cpp:1757-1854).  logits: host [vocab].                                          */
int qa_decoder_prefill_nocache(qa_decoder * dec, const float * x, int32_t n_tokens, float * logits);

/* Timing hooks used by bench.py: total device time of the named kernel family recorded with HIP
 * events on the decoder's stream since the last reset ("decode_attn", "kv_append", ...).       */
int qa_decoder_profile_enable(qa_decoder * dec, int32_t enable);
int qa_decoder_profile_read(qa_decoder * dec, const char * family, double * total_ms, int64_t * launches);
int qa_decoder_profile_reset(qa_decoder * dec);

#ifdef __cplusplus
}
#endif

#endif /* QWENASR_AMD_H */
