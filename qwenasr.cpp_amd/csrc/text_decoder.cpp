// text-decoder.h drop-in over the C ABI.
//
// Validation, ownership and error text follow the reference (src/text-decoder.cpp):
//   weights by name, f32 only, exact shapes         load_text_layer_tensors 191-228, require_* 29-65
//   *out = nullptr first, free on every failure     1222, 1495, 1614
//   null-safe *_free                                1184-1202, 1392-1418
//   outputs filled by move only on success
// The data path is the C-ABI decoder (qa_decoder_*): weights are copied to the GPU at init like the
// reference copies them to its primary backend (1586-1588).
#include "text-decoder.h"

#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "qwenasr_amd.h"

struct QwenAsrTextLayerBackend {
    qa_decoder * dec = nullptr;
    int layer = 0;
    int hidden = 0;
};

struct QwenAsrTextDecoderBackend {
    qa_decoder * dec = nullptr;
    bool cached = false;
    int hidden = 0;
    int vocab = 0;
    int max_seq_len = 0;
};

namespace {

void set_error(std::string * error, const std::string & message) {
    if (error) *error = message;
}

bool require_f32(const QwenAsrGgufModel & model, const std::string & name, QwenAsrGgufTensorView * out,
                 std::string * error) {
    if (!qwenasr_gguf_model_tensor_by_name(model, name.c_str(), out, error)) return false;
    if (out->type != GGML_TYPE_F32) {
        set_error(error, "tensor is not f32: " + name);
        return false;
    }
    return true;
}

bool require_shape(const QwenAsrGgufTensorView & t, std::vector<int64_t> ne, std::string * error) {
    if (t.ne != ne) {
        set_error(error, "tensor shape mismatch: " + t.name);
        return false;
    }
    return true;
}

const float * f32(const QwenAsrGgufTensorView & t) { return static_cast<const float *>(t.data); }

bool load_layer(const QwenAsrGgufModel & model, int layer, int hidden, int q_dim, int kv_dim, int head_dim,
                int intermediate, qa_layer_weights * w, std::string * error) {
    const std::string p = "text.blk." + std::to_string(layer) + ".";
    QwenAsrGgufTensorView an, fn, q, k, v, o, qn, kn, g, u, d;
    if (!require_f32(model, p + "attn_norm.weight", &an, error) || !require_f32(model, p + "ffn_norm.weight", &fn, error) ||
        !require_f32(model, p + "attn_q.weight", &q, error) || !require_f32(model, p + "attn_k.weight", &k, error) ||
        !require_f32(model, p + "attn_v.weight", &v, error) || !require_f32(model, p + "attn_output.weight", &o, error) ||
        !require_f32(model, p + "attn_q_norm.weight", &qn, error) ||
        !require_f32(model, p + "attn_k_norm.weight", &kn, error) || !require_f32(model, p + "ffn_gate.weight", &g, error) ||
        !require_f32(model, p + "ffn_up.weight", &u, error) || !require_f32(model, p + "ffn_down.weight", &d, error)) {
        return false;
    }
    if (!require_shape(an, {hidden}, error) || !require_shape(fn, {hidden}, error) ||
        !require_shape(q, {hidden, q_dim}, error) || !require_shape(k, {hidden, kv_dim}, error) ||
        !require_shape(v, {hidden, kv_dim}, error) || !require_shape(o, {q_dim, hidden}, error) ||
        !require_shape(qn, {head_dim}, error) || !require_shape(kn, {head_dim}, error) ||
        !require_shape(g, {hidden, intermediate}, error) || !require_shape(u, {hidden, intermediate}, error) ||
        !require_shape(d, {intermediate, hidden}, error)) {
        return false;
    }
    w->attn_norm = f32(an);
    w->ffn_norm = f32(fn);
    w->q = f32(q);
    w->k = f32(k);
    w->v = f32(v);
    w->o = f32(o);
    w->q_norm = f32(qn);
    w->k_norm = f32(kn);
    w->gate = f32(g);
    w->up = f32(u);
    w->down = f32(d);
    return true;
}

bool check_device(QwenAsrGgmlDevice device, int n_threads, std::string * error) {
    QwenAsrGgmlBackendSet set;
    if (!qwenasr_ggml_backend_set_init(device, n_threads, &set, error)) return false;
    qwenasr_ggml_backend_set_free(&set);
    return true;
}

bool cpu_path_unavailable(const char * fn, std::string * error) {
    set_error(error, std::string(fn) +
                         ": the host statement of the text decoder is not part of the MI355X build; use the "
                         "*_backend_* functions (HIP device 0)");
    return false;
}

QwenAsrKvCacheType env_cache_type() {
    const char * v = std::getenv("QWENASR_KV_CACHE_TYPE");
    if (v && (std::strcmp(v, "f16") == 0 || std::strcmp(v, "F16") == 0)) return QwenAsrKvCacheType::F16;
    return QwenAsrKvCacheType::F32;
}

bool decoder_init(const QwenAsrGgufModel & model, int n_threads, int n_layers, int hidden, int n_heads,
                  int n_kv_heads, int head_dim, int intermediate, int vocab, int max_seq_len, bool cached,
                  QwenAsrKvCacheType cache_type, float rope_theta, float rms_norm_eps,
                  QwenAsrTextDecoderBackend ** out, std::string * error, QwenAsrGgmlDevice device) {
    if (!out) {
        set_error(error, "qwenasr_text_decoder_backend_init: out is null");
        return false;
    }
    *out = nullptr;
    const int q_dim = n_heads * head_dim;
    const int kv_dim = n_kv_heads * head_dim;
    if (n_layers <= 0 || hidden <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || intermediate <= 0 ||
        vocab <= 0 || n_heads % n_kv_heads != 0 || q_dim <= 0 || kv_dim <= 0) {
        set_error(error, "invalid text decoder backend configuration");
        return false;
    }
    if (cached && max_seq_len <= 0) {
        set_error(error, "invalid text decoder KV-cache configuration");
        return false;
    }
    if (!check_device(device, n_threads, error)) return false;
    std::vector<qa_layer_weights> layers(static_cast<size_t>(n_layers));
    for (int l = 0; l < n_layers; ++l) {
        if (!load_layer(model, l, hidden, q_dim, kv_dim, head_dim, intermediate, &layers[static_cast<size_t>(l)],
                        error)) {
            return false;
        }
    }
    QwenAsrGgufTensorView on, ow, emb;
    if (!require_f32(model, "text.output_norm.weight", &on, error) || !require_f32(model, "text.output.weight", &ow, error) ||
        !require_shape(on, {hidden}, error) || !require_shape(ow, {hidden, vocab}, error)) {
        return false;
    }
    qa_model_weights w{};
    w.layers = layers.data();
    w.output_norm = f32(on);
    w.output = f32(ow);
    std::string emb_error;
    if (require_f32(model, "text.token_embd.weight", &emb, &emb_error) && emb.ne == std::vector<int64_t>{hidden, vocab}) {
        w.token_embd = f32(emb);
    }
    qa_text_config cfg{n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab, rope_theta, rms_norm_eps};
    qa_decoder * dec = nullptr;
    const int rc = qa_decoder_create(&cfg, &w, 1, cached ? max_seq_len : 1,
                                     cache_type == QwenAsrKvCacheType::F16 ? QA_CACHE_F16 : QA_CACHE_F32, &dec);
    if (rc != QA_OK) {
        set_error(error, qa_last_error());
        return false;
    }
    QwenAsrTextDecoderBackend * b = new QwenAsrTextDecoderBackend();
    b->dec = dec;
    b->cached = cached;
    b->hidden = hidden;
    b->vocab = vocab;
    b->max_seq_len = cached ? max_seq_len : 0;
    *out = b;
    return true;
}

}  // namespace

bool qwenasr_text_layer_forward_cpu(const QwenAsrGgufModel &, const QwenAsrDecoderInputOutput &, int, int, int, int,
                                    int, float, float, QwenAsrTextLayerOutput *, std::string * error) {
    return cpu_path_unavailable("qwenasr_text_layer_forward_cpu", error);
}

bool qwenasr_text_layer_forward_ggml(const QwenAsrGgufModel &, const QwenAsrDecoderInputOutput &, int, int, int, int,
                                     int, int, float, float, QwenAsrTextLayerOutput *, std::string * error) {
    return cpu_path_unavailable("qwenasr_text_layer_forward_ggml", error);
}

bool qwenasr_text_layer_backend_init(const QwenAsrGgufModel & model, int layer, int n_threads, int hidden, int n_heads,
                                     int n_kv_heads, int head_dim, int intermediate, float rope_theta,
                                     float rms_norm_eps, QwenAsrTextLayerBackend ** out, std::string * error,
                                     QwenAsrGgmlDevice device) {
    if (!out) {
        set_error(error, "qwenasr_text_layer_backend_init: out is null");
        return false;
    }
    *out = nullptr;
    const int q_dim = n_heads * head_dim;
    const int kv_dim = n_kv_heads * head_dim;
    if (layer < 0 || hidden <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || intermediate <= 0 ||
        n_heads % n_kv_heads != 0 || q_dim <= 0 || kv_dim <= 0) {
        set_error(error, "invalid text layer backend configuration");
        return false;
    }
    if (!check_device(device, n_threads, error)) return false;
    qa_layer_weights lw{};
    if (!load_layer(model, layer, hidden, q_dim, kv_dim, head_dim, intermediate, &lw, error)) return false;
    qa_model_weights w{};
    w.layers = &lw;
    qa_text_config cfg{1, hidden, n_heads, n_kv_heads, head_dim, intermediate, 1, rope_theta, rms_norm_eps};
    qa_decoder * dec = nullptr;
    if (qa_decoder_create(&cfg, &w, 1, 1, QA_CACHE_F32, &dec) != QA_OK) {
        set_error(error, qa_last_error());
        return false;
    }
    QwenAsrTextLayerBackend * b = new QwenAsrTextLayerBackend();
    b->dec = dec;
    b->layer = layer;
    b->hidden = hidden;
    *out = b;
    return true;
}

void qwenasr_text_layer_backend_free(QwenAsrTextLayerBackend * backend) {
    if (!backend) return;
    qa_decoder_destroy(backend->dec);
    delete backend;
}

bool qwenasr_text_layer_backend_forward(QwenAsrTextLayerBackend * backend, const QwenAsrDecoderInputOutput & input,
                                        QwenAsrTextLayerOutput * out, std::string * error) {
    if (!backend || !out) {
        set_error(error, "qwenasr_text_layer_backend_forward: backend or out is null");
        return false;
    }
    if (input.tokens <= 0 || input.hidden != backend->hidden ||
        input.values.size() != static_cast<size_t>(input.tokens) * input.hidden) {
        set_error(error, "invalid decoder input for text layer backend");
        return false;
    }
    QwenAsrTextLayerOutput result;
    result.tokens = input.tokens;
    result.hidden = input.hidden;
    result.values.assign(input.values.size(), 0.0f);
    if (qa_decoder_layer_forward_nocache(backend->dec, 0, input.values.data(), input.tokens, result.values.data()) !=
        QA_OK) {
        set_error(error, qa_last_error());
        return false;
    }
    *out = std::move(result);
    return true;
}

bool qwenasr_text_decoder_backend_init(const QwenAsrGgufModel & model, int n_threads, int n_layers, int hidden,
                                       int n_heads, int n_kv_heads, int head_dim, int intermediate, int vocab,
                                       float rope_theta, float rms_norm_eps, QwenAsrTextDecoderBackend ** out,
                                       std::string * error, QwenAsrGgmlDevice device) {
    return decoder_init(model, n_threads, n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab, 0,
                        false, QwenAsrKvCacheType::F32, rope_theta, rms_norm_eps, out, error, device);
}

bool qwenasr_text_decoder_backend_init_cached(const QwenAsrGgufModel & model, int n_threads, int n_layers, int hidden,
                                              int n_heads, int n_kv_heads, int head_dim, int intermediate, int vocab,
                                              int max_seq_len, float rope_theta, float rms_norm_eps,
                                              QwenAsrTextDecoderBackend ** out, std::string * error,
                                              QwenAsrGgmlDevice device) {
    return decoder_init(model, n_threads, n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab,
                        max_seq_len, true, env_cache_type(), rope_theta, rms_norm_eps, out, error, device);
}

bool qwenasr_text_decoder_backend_init_cached_typed(const QwenAsrGgufModel & model, int n_threads, int n_layers,
                                                    int hidden, int n_heads, int n_kv_heads, int head_dim,
                                                    int intermediate, int vocab, int max_seq_len, float rope_theta,
                                                    float rms_norm_eps, QwenAsrKvCacheType cache_type,
                                                    QwenAsrTextDecoderBackend ** out, std::string * error,
                                                    QwenAsrGgmlDevice device) {
    return decoder_init(model, n_threads, n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab,
                        max_seq_len, true, cache_type, rope_theta, rms_norm_eps, out, error, device);
}

void qwenasr_text_decoder_backend_free(QwenAsrTextDecoderBackend * backend) {
    if (!backend) return;
    qa_decoder_destroy(backend->dec);
    delete backend;
}

qa_decoder * qwenasr_text_decoder_backend_handle(QwenAsrTextDecoderBackend * backend) {
    return backend ? backend->dec : nullptr;
}

bool qwenasr_text_prefill_backend_forward(QwenAsrTextDecoderBackend * backend, const QwenAsrDecoderInputOutput & input,
                                          QwenAsrTextPrefillOutput * out, std::string * error) {
    if (!backend || !out) {
        set_error(error, "qwenasr_text_prefill_backend_forward: backend or out is null");
        return false;
    }
    if (input.tokens <= 0 || input.hidden != backend->hidden ||
        input.values.size() != static_cast<size_t>(input.tokens) * input.hidden) {
        set_error(error, "invalid decoder input for text prefill backend");
        return false;
    }
    QwenAsrTextPrefillOutput result;
    result.tokens = input.tokens;
    result.hidden = input.hidden;
    result.vocab = backend->vocab;
    result.logits.assign(static_cast<size_t>(backend->vocab), 0.0f);
    if (qa_decoder_prefill_nocache(backend->dec, input.values.data(), input.tokens, result.logits.data()) != QA_OK) {
        set_error(error, qa_last_error());
        return false;
    }
    *out = std::move(result);
    return true;
}

bool qwenasr_text_prefill_forward_cpu(const QwenAsrGgufModel &, const QwenAsrDecoderInputOutput &, int, int, int, int,
                                      int, int, float, float, QwenAsrTextPrefillOutput *, std::string * error) {
    return cpu_path_unavailable("qwenasr_text_prefill_forward_cpu", error);
}

bool qwenasr_text_generate_greedy_cpu(const QwenAsrGgufModel &, const QwenAsrDecoderInputOutput &, int, int, int, int,
                                      int, int, int, float, float, const std::vector<int32_t> &,
                                      QwenAsrTextGenerateOutput *, std::string * error) {
    return cpu_path_unavailable("qwenasr_text_generate_greedy_cpu", error);
}

bool qwenasr_text_generate_cached_backend(QwenAsrTextDecoderBackend * backend, const QwenAsrGgufModel & model,
                                          const QwenAsrDecoderInputOutput & input, int max_new_tokens,
                                          const std::vector<int32_t> & stop_ids, QwenAsrTextGenerateOutput * out,
                                          std::string * error) {
    if (!backend || !out) {
        set_error(error, "qwenasr_text_generate_cached_backend: backend or out is null");
        return false;
    }
    if (max_new_tokens < 0) {
        set_error(error, "max_new_tokens must be non-negative");
        return false;
    }
    if (input.tokens <= 0 || input.hidden != backend->hidden ||
        input.values.size() != static_cast<size_t>(input.tokens) * input.hidden) {
        set_error(error, "invalid backend cached text generation input");
        return false;
    }
    if (!backend->cached) {
        set_error(error, "invalid text decoder cached forward configuration");
        return false;
    }
    if (input.tokens + max_new_tokens > backend->max_seq_len) {
        set_error(error, "backend text generation exceeds KV-cache capacity");
        return false;
    }
    QwenAsrTextGenerateOutput result;
    result.prompt_tokens = input.tokens;
    result.total_tokens = input.tokens;
    result.hidden = input.hidden;
    result.vocab = backend->vocab;
    if (max_new_tokens == 0) {
        *out = std::move(result);
        return true;
    }
    QwenAsrGgufTensorView embd;
    if (!require_f32(model, "text.token_embd.weight", &embd, error) ||
        !require_shape(embd, {backend->hidden, backend->vocab}, error)) {
        return false;
    }
    std::vector<int32_t> ids(static_cast<size_t>(max_new_tokens), 0);
    int32_t n_out = 0, stopped = 0, total = 0;
    if (qa_decoder_generate(backend->dec, input.values.data(), input.tokens, max_new_tokens, stop_ids.data(),
                            static_cast<int32_t>(stop_ids.size()), ids.data(), &n_out, &stopped, &total,
                            nullptr) != QA_OK) {
        set_error(error, qa_last_error());
        return false;
    }
    ids.resize(static_cast<size_t>(n_out));
    result.generated_ids = std::move(ids);
    result.stopped = stopped != 0;
    result.total_tokens = total;
    *out = std::move(result);
    return true;
}

bool qwenasr_text_generate_cached_cpu(const QwenAsrGgufModel &, const QwenAsrDecoderInputOutput &, int, int, int, int,
                                      int, int, int, float, float, const std::vector<int32_t> &,
                                      QwenAsrTextGenerateOutput *, std::string * error) {
    return cpu_path_unavailable("qwenasr_text_generate_cached_cpu", error);
}
