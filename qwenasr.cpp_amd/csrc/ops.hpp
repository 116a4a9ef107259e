// Internal launch functions shared by the runtime (not part of the C ABI).
#pragma once

#include "common.hpp"

namespace qa {

enum { kEpiStoreOp = 0, kEpiAccumOp = 1, kEpiSwigluOp = 2 };

// W16 (optional): the same weights as bf16 bits, read instead of W when given (bf16-exact weights)
int gemv_launch(int epi, bool prenorm, const float * W, int32_t out_dim, int32_t in_dim, const float * x, float * y,
                const float * norm_w, float eps, hipStream_t stream, const uint16_t * W16 = nullptr);
// out[t] = [hi | mid | lo] of x[t] (rows x K): the exact three-part bf16 split, x = hi + mid + lo (bf16 bits)
int split_bf16x3_rows_launch(const float * x, int64_t rows, int32_t K, uint16_t * out, hipStream_t stream);
// Prefill GEMM on bf16-exact weights over the three-part split input (gemm_split3.hip):
// Y[M][N] (+)= sum_p Xs[M][p K .. p K + K) W16[N][K]^T, f32 products and sums; with act != nullptr (Y null,
// no accumulate) W16 = [gate rows; up rows] (2 N rows) and act[M][3 N] = split of silu(gate) * up.
bool gemm_split3_shape_ok(int32_t N, int32_t K, bool swiglu);
int gemm_split3_launch(const uint16_t * W16, int32_t N, int32_t K, const uint16_t * Xs, int32_t M, float * Y,
                       bool accumulate, uint16_t * act, hipStream_t stream);
// dst = high halves of src; *inexact |= 1 if any low half of src is non-zero
int pack_bf16_launch(const float * src, int64_t n, uint16_t * dst, uint32_t * inexact, hipStream_t stream);
// Y[rows][N] (+)= X[rows][K] W[N][K]^T for 1..64 rows (K a multiple of 32), f32 MFMA.
size_t gemm_rows_workspace_bytes(int32_t N, int32_t K, int32_t rows);
// Fusions of the <= 32-row kernel (gemm_rows_fusable):
//  - norm_w: X is replaced by RMSNorm(X) * norm_w; the per-row sums of squares come as n_stats_in
//    partials [n_stats_in][32] (double), e.g. the stats_out of the GEMM that produced X;
//  - stats_out: [ceil(N / 32)][32] partial sums of squares of the stored rows of Y (after accumulation);
//  - swiglu: W = [gate rows; up rows] (N = 2 I, I % 16 == 0), Y = silu(gate) * up, [rows][I].
struct GemmRowsFusion {
    const float * norm_w = nullptr;
    const double * stats_in = nullptr;
    int32_t n_stats_in = 0;
    float eps = 0.0f;
    double * stats_out = nullptr;
    bool swiglu = false;
};
bool gemm_rows_fusable(int32_t N, int32_t K, int32_t rows);
// W16 (optional): the same weights as bf16 bits (bf16-exact weights), read instead of W by the <= 32-row
// kernel with the same results; the longer-row kernel reads W
int gemm_rows_launch(const float * W, int32_t N, int32_t K, const float * X, int32_t rows, float * Y, bool accumulate,
                     void * workspace, size_t workspace_bytes, hipStream_t stream,
                     const GemmRowsFusion * fusion = nullptr, const uint16_t * W16 = nullptr);
// f32 weights packed for the multi-stream projections (gemm_packed.hip): Wp = W [N][K] reordered into the
// A-operand order of the f32 MFMA (N % 16 == 0, K % 32 == 0; same size as W).
int pack_f32_launch(const float * W, int32_t N, int32_t K, float * Wp, hipStream_t stream);
// Shapes the packed GEMM takes: layer projections N % 16 == 0 with K 1024 or 2048; the LM head N % 128 == 0 and
// K % 256 == 0.
bool packed_gemm_shape_ok(int32_t N, int32_t K, bool lm_head);
// Y[rows][N] (+)= X[rows][K] W[N][K]^T from packed weights, 1..32 rows, with the fusion's RMSNorm input and
// stats_out ([N / 16][32]: 16-column partial sums of squares of the stored rows).  lm_head: the 128-row kernel
// (RMSNorm input, plain store).
int gemm_packed_launch(const float * Wp, int32_t N, int32_t K, const float * X, int32_t rows, float * Y, bool accumulate,
                       const GemmRowsFusion * fusion, bool lm_head, hipStream_t stream);
size_t argmax_workspace_bytes(int32_t rows);
// What the decode step's last kernel does after picking row r's id (each part optional): lens[r] += 1,
// host_ids[r] = id (a device-visible pointer into pinned host memory), and the picked token's
// embedding row gathered into x[r] as the next step's input, exactly as embed_rows_launch gathers it
// (with its 32-column sums of squares in stats when given; rows <= 32 then).
struct StepTail {
    int32_t * lens = nullptr;
    int32_t * host_ids = nullptr;
    const float * embd = nullptr;
    float * x = nullptr;
    double * stats = nullptr;
    int32_t dim = 0;
};
int argmax_launch(const float * logits, int32_t rows, int32_t vocab, int32_t * ids, void * workspace,
                  hipStream_t stream, const StepTail & tail = StepTail{});
// split (optional): write the rows as the three-part bf16 split of the prefill GEMM's input ([rows][3 dim],
// see split_bf16x3_rows_launch) instead of f32 rows of y / a
int rmsnorm_rows_launch(const float * x, const float * w, int32_t rows, int32_t dim, float eps, float * y,
                        hipStream_t stream, uint16_t * split = nullptr);
int swiglu_rows_launch(const float * gu, int32_t rows, int32_t dim, float * a, hipStream_t stream,
                       uint16_t * split = nullptr);
// stats (optional, rows <= 32): [ceil(dim / 32)][32] partial sums of squares of each gathered row
int embed_rows_launch(const float * table, int32_t n_rows, int32_t dim, const int32_t * ids, int32_t rows,
                      float * out, hipStream_t stream, double * stats = nullptr);
int advance_lens_launch(int32_t * lens, int32_t n, int32_t delta, hipStream_t stream);
int set_values_launch(int32_t * dst, int32_t n, int32_t value, hipStream_t stream);
int cast_rows_launch(const float * src, void * dst, int32_t cache_type, int64_t n, hipStream_t stream);

int decode_attn_launch(const float * q, int32_t q_stride, const void * cache, const qa_kv_layout & layout,
                       int32_t layer, const int32_t * lens, int32_t lens_add, int32_t n_streams, int32_t max_len,
                       int32_t n_heads, float scale, float * out, void * workspace, size_t workspace_bytes,
                       hipStream_t stream);
int decode_step_attn_launch(const float * qkv, const float * q_norm_w, const float * k_norm_w, void * cache,
                            const qa_kv_layout & layout, int32_t layer, const int32_t * n_past, int32_t n_streams,
                            int32_t max_len, int32_t n_heads, float rope_theta, float eps, float scale, float * out,
                            void * workspace, size_t workspace_bytes, hipStream_t stream);
size_t decode_attn_workspace(int32_t n_streams, int32_t n_kv_heads, int32_t max_seq);

// Persistent decode step (decode_persist.hip): every layer of one batch-1 token in one launch,
// bit-identical to the eager step.  The layer table lives in device memory.
struct PersistLayer {
    const void * qkv;   // f32 rows, or their bf16 copies when b16
    const void * o;
    const void * gu;
    const void * down;
    const float * attn_norm;
    const float * ffn_norm;
    const float * q_norm;
    const float * k_norm;
};
struct PersistPlanIn {
    qa_kv_layout layout;
    int32_t hidden = 0, q_dim = 0, inter = 0;
    bool b16 = false;
};
// the grid (resident workgroups) for a decoder, or an error if no persistent kernel covers its shapes
int persist_plan(const PersistPlanIn & in, int32_t * grid);
size_t persist_sync_bytes(int32_t grid);
// bytes of one layer's attention workspace in the persistent step (each layer has its own)
size_t persist_ws_stride(const qa_kv_layout & layout);
int persist_error_word_offset(int32_t grid);   // in uint32 words from the start of the sync buffer
struct PersistLaunch {
    PersistPlanIn plan;
    int32_t grid = 0;
    const PersistLayer * layers = nullptr;
    int32_t n_layers = 0;
    // every address is written at most once per launch, so each layer has its own buffers
    float * x = nullptr;      // [hidden]: layer 0's input, the last layer's output
    float * xbuf = nullptr;   // [2 n_layers - 1][hidden]
    float * qkv = nullptr;    // [n_layers][q_dim + 2 kv_dim]
    float * attn = nullptr;   // [n_layers][q_dim]
    float * act = nullptr;    // [n_layers][inter]
    void * cache = nullptr;
    const int32_t * lens = nullptr;
    int32_t max_len = 0;
    int32_t n_heads = 0;
    float eps = 0.0f, scale = 0.0f, rope_theta = 0.0f;
    void * attn_ws = nullptr;    // [n_layers][persist_ws_stride], cleared before the first launch
    size_t attn_ws_bytes = 0;
    uint32_t * sync = nullptr;   // cleared before the first launch and after an abandoned one
    uint64_t wait_ticks = 20000000;   // bound of each barrier wait (100 MHz ticks: 200 ms)
};
int persist_layers_launch(const PersistLaunch & a, hipStream_t stream);

int prefill_attn_launch(const float * q, int32_t q_stride, const void * cache, const qa_kv_layout & layout,
                        int32_t layer, int32_t stream_idx, int32_t n_past, int32_t n_tokens, int32_t n_heads,
                        float scale, float * out, void * workspace, size_t workspace_bytes, hipStream_t stream);
size_t prefill_mfma_workspace_bytes(int32_t n_tokens, int32_t n_kv);
int prefill_mfma_launch(const float * q, int32_t q_stride, const void * k, const void * v, int64_t head_stride,
                        int32_t n_past, int32_t n_tokens, int32_t n_kv, float scale, float * out, void * workspace,
                        size_t workspace_bytes, hipStream_t stream);
int causal_f32_launch(const float * q, int32_t q_stride, const float * k, const float * v, int64_t row_stride,
                      int32_t n_tokens, int32_t n_heads, int32_t n_kv_heads, float scale, float * out,
                      int32_t out_stride, hipStream_t stream);

}  // namespace qa
