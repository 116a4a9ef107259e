// Drop-in for the reference's src/text-decoder.h: the same output structs, opaque backends and 13
// functions with the same parameters, defaults, ownership and error behaviour
// (text-decoder.h:10-179).  The *_backend_* functions run on the MI355X through the C ABI of
// qwenasr_amd.h.  The four *_cpu functions and qwenasr_text_layer_forward_ggml are the reference's
// host statements of the same maths; this build keeps their signatures but returns false with an
// explanatory error, because its CPU statement of the path is test infrastructure, not a product
// path.
#pragma once

#include "decoder-input.h"
#include "ggml-backends.h"
#include "gguf-model.h"

#include <string>
#include <vector>

struct QwenAsrTextLayerOutput {
    int tokens = 0;
    int hidden = 0;
    std::vector<float> values; // [token, hidden]
};

struct QwenAsrTextPrefillOutput {
    int tokens = 0;
    int hidden = 0;
    int vocab = 0;
    std::vector<float> logits; // [vocab], next-token logits from the last prompt position
};

struct QwenAsrTextGenerateOutput {
    int prompt_tokens = 0;
    int total_tokens = 0;
    int hidden = 0;
    int vocab = 0;
    bool stopped = false;
    std::vector<int32_t> generated_ids;
};

struct QwenAsrTextLayerBackend;
struct QwenAsrTextDecoderBackend;

bool qwenasr_text_layer_forward_cpu(
    const QwenAsrGgufModel & model,
    const QwenAsrDecoderInputOutput & input,
    int layer,
    int n_heads,
    int n_kv_heads,
    int head_dim,
    int intermediate,
    float rope_theta,
    float rms_norm_eps,
    QwenAsrTextLayerOutput * out,
    std::string * error);

bool qwenasr_text_layer_forward_ggml(
    const QwenAsrGgufModel & model,
    const QwenAsrDecoderInputOutput & input,
    int layer,
    int n_threads,
    int n_heads,
    int n_kv_heads,
    int head_dim,
    int intermediate,
    float rope_theta,
    float rms_norm_eps,
    QwenAsrTextLayerOutput * out,
    std::string * error);

bool qwenasr_text_layer_backend_init(
    const QwenAsrGgufModel & model,
    int layer,
    int n_threads,
    int hidden,
    int n_heads,
    int n_kv_heads,
    int head_dim,
    int intermediate,
    float rope_theta,
    float rms_norm_eps,
    QwenAsrTextLayerBackend ** out,
    std::string * error,
    QwenAsrGgmlDevice device = qwenasr_ggml_device_auto());

void qwenasr_text_layer_backend_free(QwenAsrTextLayerBackend * backend);

bool qwenasr_text_layer_backend_forward(
    QwenAsrTextLayerBackend * backend,
    const QwenAsrDecoderInputOutput & input,
    QwenAsrTextLayerOutput * out,
    std::string * error);

bool qwenasr_text_decoder_backend_init(
    const QwenAsrGgufModel & model,
    int n_threads,
    int n_layers,
    int hidden,
    int n_heads,
    int n_kv_heads,
    int head_dim,
    int intermediate,
    int vocab,
    float rope_theta,
    float rms_norm_eps,
    QwenAsrTextDecoderBackend ** out,
    std::string * error,
    QwenAsrGgmlDevice device = qwenasr_ggml_device_auto());

bool qwenasr_text_decoder_backend_init_cached(
    const QwenAsrGgufModel & model,
    int n_threads,
    int n_layers,
    int hidden,
    int n_heads,
    int n_kv_heads,
    int head_dim,
    int intermediate,
    int vocab,
    int max_seq_len,
    float rope_theta,
    float rms_norm_eps,
    QwenAsrTextDecoderBackend ** out,
    std::string * error,
    QwenAsrGgmlDevice device = qwenasr_ggml_device_auto());

void qwenasr_text_decoder_backend_free(QwenAsrTextDecoderBackend * backend);

bool qwenasr_text_prefill_backend_forward(
    QwenAsrTextDecoderBackend * backend,
    const QwenAsrDecoderInputOutput & input,
    QwenAsrTextPrefillOutput * out,
    std::string * error);

bool qwenasr_text_prefill_forward_cpu(
    const QwenAsrGgufModel & model,
    const QwenAsrDecoderInputOutput & input,
    int n_layers,
    int n_heads,
    int n_kv_heads,
    int head_dim,
    int intermediate,
    int vocab,
    float rope_theta,
    float rms_norm_eps,
    QwenAsrTextPrefillOutput * out,
    std::string * error);

bool qwenasr_text_generate_greedy_cpu(
    const QwenAsrGgufModel & model,
    const QwenAsrDecoderInputOutput & input,
    int max_new_tokens,
    int n_layers,
    int n_heads,
    int n_kv_heads,
    int head_dim,
    int intermediate,
    int vocab,
    float rope_theta,
    float rms_norm_eps,
    const std::vector<int32_t> & stop_ids,
    QwenAsrTextGenerateOutput * out,
    std::string * error);

bool qwenasr_text_generate_cached_backend(
    QwenAsrTextDecoderBackend * backend,
    const QwenAsrGgufModel & model,
    const QwenAsrDecoderInputOutput & input,
    int max_new_tokens,
    const std::vector<int32_t> & stop_ids,
    QwenAsrTextGenerateOutput * out,
    std::string * error);

bool qwenasr_text_generate_cached_cpu(
    const QwenAsrGgufModel & model,
    const QwenAsrDecoderInputOutput & input,
    int max_new_tokens,
    int n_layers,
    int n_heads,
    int n_kv_heads,
    int head_dim,
    int intermediate,
    int vocab,
    float rope_theta,
    float rms_norm_eps,
    const std::vector<int32_t> & stop_ids,
    QwenAsrTextGenerateOutput * out,
    std::string * error);

// ---- Additions of this build (no counterpart in the reference) ----------------------------------
// KV-cache element type for *_init_cached: "f32" (the reference's only type, default) or "f16".
// The environment variable QWENASR_KV_CACHE_TYPE selects it for unmodified callers.
enum class QwenAsrKvCacheType { F32 = 0, F16 = 1 };

bool qwenasr_text_decoder_backend_init_cached_typed(
    const QwenAsrGgufModel & model,
    int n_threads,
    int n_layers,
    int hidden,
    int n_heads,
    int n_kv_heads,
    int head_dim,
    int intermediate,
    int vocab,
    int max_seq_len,
    float rope_theta,
    float rms_norm_eps,
    QwenAsrKvCacheType cache_type,
    QwenAsrTextDecoderBackend ** out,
    std::string * error,
    QwenAsrGgmlDevice device = qwenasr_ggml_device_auto());

// Underlying C-ABI decoder of a backend (for timing hooks and cache inspection).
struct qa_decoder;
qa_decoder * qwenasr_text_decoder_backend_handle(QwenAsrTextDecoderBackend * backend);
