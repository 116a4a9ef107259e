// Synthetic-input counterpart of the reference's tools/qwen-asr-text-layer.cpp.
//
// The reference tool builds its decoder input from a WAV file through the GGML audio encoder
// (tools/qwen-asr-text-layer.cpp:265-386), which is outside this build.  This driver builds the same
// QwenAsrDecoderInputOutput from seeded synthetic data instead (audio-embedding rows N(0, 1) followed
// by random prompt ids embedded through text.token_embd.weight), then calls the text-decoder.h
// drop-in exactly like the reference tool does (layer / --prefill / --generate dispatch, 430-469) and
// prints the same key=value contract (487-517, 603-625, 715-733) plus timing keys of this build.
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <limits>
#include <string>
#include <thread>
#include <vector>

#include "qwenasr_amd.h"
#include "text-decoder.h"

namespace {

void usage(const char * argv0) {
    std::cerr << "Usage: " << argv0 << " [--model model.gguf | --size 0.6b|1.7b] [--layers N] [--audio-tokens N]\n"
              << "       [--prompt-tokens N] [--seed S] [--device auto|cpu|gpu] [--kv-cache-type f32|f16]\n"
              << "       [--layer N | --prefill | --generate N] [--threads N]\n";
}

bool parse_int(const char * s, long lo, long hi, int * out) {
    char * end = nullptr;
    const long v = std::strtol(s, &end, 10);
    if (!end || *end != '\0' || v < lo || v > hi) return false;
    *out = static_cast<int>(v);
    return true;
}

}  // namespace

int main(int argc, char ** argv) {
    const unsigned hw = std::thread::hardware_concurrency();
    int n_threads = hw == 0 ? 1 : static_cast<int>(hw);
    std::string model_path, size = "0.6b", cache_type = "f32";
    int n_layers = -1, audio_tokens = 143, prompt_tokens = 13, layer = 0, generate = -1;
    bool prefill = false;
    uint64_t seed = 20260101;
    QwenAsrGgmlDevice device = qwenasr_ggml_device_auto();
    std::string error;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&](const char * what) -> const char * {
            if (++i >= argc) {
                std::cerr << a << " requires " << what << "\n";
                std::exit(2);
            }
            return argv[i];
        };
        if (a == "-h" || a == "--help") { usage(argv[0]); return 0; }
        else if (a == "--model") model_path = next("a path");
        else if (a == "--size") size = next("0.6b or 1.7b");
        else if (a == "--layers") { if (!parse_int(next("an integer"), 1, 1000, &n_layers)) { std::cerr << "--layers requires a positive integer\n"; return 2; } }
        else if (a == "--audio-tokens") { if (!parse_int(next("an integer"), 0, 1 << 20, &audio_tokens)) { std::cerr << "bad --audio-tokens\n"; return 2; } }
        else if (a == "--prompt-tokens") { if (!parse_int(next("an integer"), 0, 1 << 20, &prompt_tokens)) { std::cerr << "bad --prompt-tokens\n"; return 2; } }
        else if (a == "--seed") seed = std::strtoull(next("an integer"), nullptr, 10);
        else if (a == "--kv-cache-type") cache_type = next("f32 or f16");
        else if (a == "--layer") { if (!parse_int(next("an integer"), 0, 1000, &layer)) { std::cerr << "--layer requires a non-negative integer\n"; return 2; } }
        else if (a == "--prefill") prefill = true;
        else if (a == "--generate") { if (!parse_int(next("an integer"), 0, 1024, &generate)) { std::cerr << "--generate requires a non-negative integer up to 1024\n"; return 2; } }
        else if (a == "--threads") { if (!parse_int(next("an integer"), 1, 4096, &n_threads)) { std::cerr << "--threads requires a positive integer\n"; return 2; } }
        else if (a == "--device") { if (!qwenasr_ggml_device_from_string(next("auto, cpu, or gpu"), &device, &error)) { std::cerr << error << "\n"; return 2; } }
        else { std::cerr << "unknown argument: " << a << "\n"; usage(argv[0]); return 2; }
    }
    if (prefill && generate >= 0) {
        std::cerr << "--prefill and --generate are mutually exclusive\n";
        return 2;
    }
    if (cache_type != "f32" && cache_type != "f16") {
        std::cerr << "--kv-cache-type requires f32 or f16\n";
        return 2;
    }
    const int tokens = audio_tokens + prompt_tokens;
    if (tokens <= 0) {
        std::cerr << "the prompt needs at least one position\n";
        return 2;
    }

    // ---- model: a GGUF file or a seeded synthetic model of the named size
    QwenAsrGgufModel model{};
    qa_model * synth = nullptr;
    qa_text_config cfg{};
    const auto load_start = std::chrono::steady_clock::now();
    if (!model_path.empty()) {
        if (!qwenasr_gguf_model_open(model_path.c_str(), &model, &error)) {
            std::cerr << error << "\n";
            return 1;
        }
        uint32_t v = 0;
        auto u = [&](const char * k, int32_t * dst) { if (qwenasr_gguf_model_get_u32(model, k, &v)) *dst = static_cast<int32_t>(v); };
        u("qwen3-asr.text.num_hidden_layers", &cfg.n_layers);
        u("qwen3-asr.text.hidden_size", &cfg.hidden);
        u("qwen3-asr.text.num_attention_heads", &cfg.n_heads);
        u("qwen3-asr.text.num_key_value_heads", &cfg.n_kv_heads);
        u("qwen3-asr.text.head_dim", &cfg.head_dim);
        u("qwen3-asr.text.intermediate_size", &cfg.intermediate);
        u("qwen3-asr.text.vocab_size", &cfg.vocab);
        qwenasr_gguf_model_get_f32(model, "qwen3-asr.text.rope_theta", &cfg.rope_theta);
        qwenasr_gguf_model_get_f32(model, "qwen3-asr.text.rms_norm_eps", &cfg.rms_norm_eps);
    } else {
        if (size == "1.7b") cfg = {28, 2048, 16, 8, 128, 6144, 151936, 1000000.0f, 1e-6f};
        else if (size == "0.6b") cfg = {28, 1024, 16, 8, 128, 3072, 151936, 1000000.0f, 1e-6f};
        else { std::cerr << "--size requires 0.6b or 1.7b\n"; return 2; }
        if (n_layers > 0) cfg.n_layers = n_layers;
        if (qa_model_synthetic(&cfg, seed, &synth) != QA_OK ||
            !qwenasr_gguf_model_from_synthetic(synth, &model, &error)) {
            std::cerr << (error.empty() ? qa_last_error() : error) << "\n";
            return 1;
        }
    }
    const double load_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - load_start).count();
    if (!prefill && generate < 0 && (layer < 0 || layer >= cfg.n_layers)) {
        std::cerr << "--layer is out of range for model\n";
        return 2;
    }

    // ---- decoder input: audio rows N(0, 1) then embedded prompt ids U[0, vocab)
    QwenAsrDecoderInputOutput input;
    input.tokens = tokens;
    input.hidden = cfg.hidden;
    input.audio_tokens = audio_tokens;
    input.values.resize(static_cast<size_t>(tokens) * cfg.hidden);
    qa_synth_fill_normal(input.values.data(), static_cast<size_t>(audio_tokens) * cfg.hidden, seed + 1,
                         "audio_embeddings", 1.0);
    input.input_ids.assign(static_cast<size_t>(audio_tokens), 151676);
    std::vector<int32_t> ids(static_cast<size_t>(prompt_tokens));
    qa_synth_fill_ids(ids.data(), ids.size(), seed + 3, "prompt_ids", 0, cfg.vocab - 1);
    QwenAsrGgufTensorView embd;
    if (prompt_tokens > 0 && !qwenasr_gguf_model_tensor_by_name(model, "text.token_embd.weight", &embd, &error)) {
        std::cerr << error << "\n";
        return 1;
    }
    for (int i = 0; i < prompt_tokens; ++i) {
        input.input_ids.push_back(ids[static_cast<size_t>(i)]);
        std::memcpy(input.values.data() + static_cast<size_t>(audio_tokens + i) * cfg.hidden,
                    static_cast<const float *>(embd.data) + static_cast<size_t>(ids[static_cast<size_t>(i)]) * cfg.hidden,
                    sizeof(float) * cfg.hidden);
    }

    std::cout << "backend=sched\n";
    if (generate >= 0) {
        const std::vector<int32_t> stop_ids = {151645, 151643, 151645};
        QwenAsrTextDecoderBackend * backend = nullptr;
        const auto t0 = std::chrono::steady_clock::now();
        const bool init_ok = qwenasr_text_decoder_backend_init_cached_typed(
            model, n_threads, cfg.n_layers, cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.intermediate,
            cfg.vocab, tokens + generate, cfg.rope_theta, cfg.rms_norm_eps,
            cache_type == "f16" ? QwenAsrKvCacheType::F16 : QwenAsrKvCacheType::F32, &backend, &error, device);
        const double init_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        if (!init_ok) {
            std::cerr << error << "\n";
            return 1;
        }
        QwenAsrTextGenerateOutput out;
        const auto g0 = std::chrono::steady_clock::now();
        const bool ok = qwenasr_text_generate_cached_backend(backend, model, input, generate, stop_ids, &out, &error);
        const double gen_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - g0).count();
        qwenasr_text_decoder_backend_free(backend);
        if (!ok) {
            std::cerr << error << "\n";
            return 1;
        }
        std::cout << "mode=generate\n" << "decode_backend=kv-cache\n" << "audio_backend=synthetic\n"
                  << "device=" << qwenasr_ggml_device_name(device) << "\n" << "threads=" << n_threads << "\n"
                  << "model_load_ms=" << load_ms << "\n" << "text_init_ms=" << init_ms << "\n"
                  << "generate_ms=" << gen_ms << "\n" << "kv_cache_type=" << cache_type << "\n"
                  << "layers=" << cfg.n_layers << "\n" << "prompt_tokens=" << out.prompt_tokens << "\n"
                  << "total_tokens=" << out.total_tokens << "\n" << "hidden=" << out.hidden << "\n"
                  << "vocab=" << out.vocab << "\n" << "requested_tokens=" << generate << "\n"
                  << "generated_tokens=" << out.generated_ids.size() << "\n"
                  << "stopped=" << (out.stopped ? "true" : "false") << "\n" << "generated_ids=";
        for (size_t i = 0; i < out.generated_ids.size(); ++i) std::cout << (i ? "," : "") << out.generated_ids[i];
        std::cout << "\n";
    } else if (prefill) {
        QwenAsrTextDecoderBackend * backend = nullptr;
        const auto t0 = std::chrono::steady_clock::now();
        if (!qwenasr_text_decoder_backend_init(model, n_threads, cfg.n_layers, cfg.hidden, cfg.n_heads, cfg.n_kv_heads,
                                               cfg.head_dim, cfg.intermediate, cfg.vocab, cfg.rope_theta,
                                               cfg.rms_norm_eps, &backend, &error, device)) {
            std::cerr << error << "\n";
            return 1;
        }
        const double init_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        QwenAsrTextPrefillOutput out;
        const auto p0 = std::chrono::steady_clock::now();
        const bool ok = qwenasr_text_prefill_backend_forward(backend, input, &out, &error);
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - p0).count();
        qwenasr_text_decoder_backend_free(backend);
        if (!ok) {
            std::cerr << error << "\n";
            return 1;
        }
        double sum = 0.0;
        float mn = std::numeric_limits<float>::infinity(), mx = -std::numeric_limits<float>::infinity(), top = mx;
        int top_id = -1;
        for (size_t i = 0; i < out.logits.size(); ++i) {
            const float v = out.logits[i];
            mn = std::min(mn, v);
            mx = std::max(mx, v);
            if (v > top) { top = v; top_id = static_cast<int>(i); }
            sum += v;
        }
        std::cout << "mode=prefill\n" << "device=" << qwenasr_ggml_device_name(device) << "\n"
                  << "threads=" << n_threads << "\n" << "text_init_ms=" << init_ms << "\n" << "prefill_ms=" << ms << "\n"
                  << "layers=" << cfg.n_layers << "\n" << "tokens=" << out.tokens << "\n" << "hidden=" << out.hidden << "\n"
                  << "vocab=" << out.vocab << "\n" << "values=" << out.logits.size() << "\n" << "top_id=" << top_id << "\n"
                  << "top_logit=" << top << "\n" << "min=" << mn << "\n" << "max=" << mx << "\n"
                  << "mean=" << (sum / static_cast<double>(out.logits.size())) << "\n";
    } else {
        QwenAsrTextLayerBackend * backend = nullptr;
        const auto t0 = std::chrono::steady_clock::now();
        if (!qwenasr_text_layer_backend_init(model, layer, n_threads, cfg.hidden, cfg.n_heads, cfg.n_kv_heads,
                                             cfg.head_dim, cfg.intermediate, cfg.rope_theta, cfg.rms_norm_eps, &backend,
                                             &error, device)) {
            std::cerr << error << "\n";
            return 1;
        }
        const double init_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        QwenAsrTextLayerOutput out;
        const auto p0 = std::chrono::steady_clock::now();
        const bool ok = qwenasr_text_layer_backend_forward(backend, input, &out, &error);
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - p0).count();
        qwenasr_text_layer_backend_free(backend);
        if (!ok) {
            std::cerr << error << "\n";
            return 1;
        }
        double sum = 0.0;
        float mn = std::numeric_limits<float>::infinity(), mx = -std::numeric_limits<float>::infinity();
        for (float v : out.values) {
            mn = std::min(mn, v);
            mx = std::max(mx, v);
            sum += v;
        }
        std::cout << "device=" << qwenasr_ggml_device_name(device) << "\n" << "threads=" << n_threads << "\n"
                  << "text_init_ms=" << init_ms << "\n" << "text_layer_ms=" << ms << "\n" << "layer=" << layer << "\n"
                  << "tokens=" << out.tokens << "\n" << "hidden=" << out.hidden << "\n" << "values=" << out.values.size()
                  << "\n" << "min=" << mn << "\n" << "max=" << mx << "\n"
                  << "mean=" << (sum / static_cast<double>(out.values.size())) << "\n";
    }
    qwenasr_gguf_model_close(&model);
    qa_model_free(synth);
    return 0;
}
