// Counterpart of the reference's tools/qwen-asr-text-layer.cpp, driving the text-decoder.h drop-in.
//
// It accepts the reference tool's command line (tools/qwen-asr-text-layer.cpp:19-28, 95-262), so the
// reference's benchmark and parity harnesses (benchmarks/bench_text_*.py, check_text_*.py) can run it
// unchanged: positional model.gguf and audio.wav, --out, --threads, --language, --system,
// --audio-backend ggml|sched, --backend scalar|ggml|sched, --device, --layer, --prefill, --generate N,
// --kv-cache, with the same validation messages and exit codes.  It prints the same key=value lines
// (487-517 generate, 603-625 prefill, 715-733 layer) and writes the same --out files.
//
// What differs: the audio front end (WAV -> mel -> audio encoder, 265-386) and the BPE tokenizer are
// outside this build.  The WAV is read for its length only; the audio-encoder rows are seeded N(0, 1)
// draws, as many as the reference's encoder would produce for that clip (13 per 100 mel frames,
// audio-features.cpp:14-19); the prompt ids are seeded random ids; the decoder input is assembled from
// them through qwenasr_decoder_input_from_ids (decoder-input.cpp:26-101).  text_json holds the
// generated ids as text (no tokenizer to decode them).  The scalar and ggml backends are the
// reference's CPU paths, which this build does not ship: they report an error, like --device cpu.
//
// Additions: --size 0.6b|1.7b with --layers N builds a seeded synthetic model in memory instead of
// opening a GGUF file; --audio-tokens / --prompt-tokens / --seed set the synthetic input;
// --kv-cache-type f32|f16 selects the cache dtype (the reference's is f32 only).
#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <limits>
#include <string>
#include <thread>
#include <vector>

#include "decoder-input.h"
#include "qwenasr_amd.h"
#include "text-decoder.h"
#include "tokenizer.h"

namespace {

void usage(const char * argv0) {
    std::cerr
        << "Usage: " << argv0 << " model.gguf audio.wav [--out text-layer0.f32] [--threads N]\n"
        << "       " << argv0 << " model.gguf audio.wav [--language NAME] [--system TEXT]\n"
        << "       " << argv0 << " model.gguf audio.wav [--audio-backend ggml|sched] [--backend scalar|ggml|sched] [--device auto|cpu|gpu] [--layer N]\n"
        << "       " << argv0 << " model.gguf audio.wav --prefill [--out next-token-logits.f32]\n"
        << "       " << argv0 << " model.gguf audio.wav --generate N [--kv-cache]\n"
        << "       " << argv0 << " --size 0.6b|1.7b [--layers N] [--audio-tokens N] [--prompt-tokens N] [--seed S] ...\n"
        << "Options of this build: [--kv-cache-type f32|f16] (model.gguf may be replaced by --size, audio.wav by\n"
        << "--audio-tokens).  The audio rows and prompt ids are seeded synthetic data.\n";
}

bool parse_long(const char * s, long lo, long hi, long * out) {
    char * end = nullptr;
    const long v = std::strtol(s, &end, 10);
    if (!end || *end != '\0' || v < lo || v > hi) return false;
    *out = v;
    return true;
}

template <typename T>
bool write_raw(const std::string & path, const std::vector<T> & v, std::string * error) {
    std::ofstream out(path, std::ios::binary);
    if (out) out.write(reinterpret_cast<const char *>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T)));
    if (!out) *error = "failed to write output file: " + path;
    return static_cast<bool>(out);
}

std::string json_string(const std::string & v) {
    std::string out = "\"";
    for (const unsigned char c : v) {
        if (c == '"' || c == '\\') {
            out.push_back('\\');
            out.push_back(static_cast<char>(c));
        } else if (c == '\n') {
            out += "\\n";
        } else if (c < 0x20) {
            static const char hex[] = "0123456789abcdef";
            out += "\\u00";
            out.push_back(hex[c >> 4]);
            out.push_back(hex[c & 15]);
        } else {
            out.push_back(static_cast<char>(c));
        }
    }
    return out + "\"";
}

double ms_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

}  // namespace

int main(int argc, char ** argv) {
    if (argc < 2) {
        usage(argv[0]);
        return 2;
    }
    const unsigned hw = std::thread::hardware_concurrency();
    long n_threads = hw == 0 ? 1 : static_cast<long>(hw);
    long layer = 0, generate = -1, n_layers = -1, audio_tokens_opt = -1, prompt_tokens = 13, seed = 20260101;
    std::string model_path, audio_path, out_path, language, system_text, size, cache_type = "f32";
    std::string audio_backend = "sched", text_backend = "sched", error;
    bool prefill = false, use_kv_cache = false;
    QwenAsrGgmlDevice device = qwenasr_ggml_device_auto();
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto value = [&](const char * message) -> const char * {
            if (++i >= argc) {
                std::cerr << message << "\n";
                std::exit(2);
            }
            return argv[i];
        };
        if (a == "-h" || a == "--help") {
            usage(argv[0]);
            return 0;
        } else if (a == "--prefill") {
            prefill = true;
        } else if (a == "--kv-cache") {
            use_kv_cache = true;
        } else if (a == "--generate") {
            if (!parse_long(value("--generate requires a non-negative integer"), 0, 1024, &generate)) {
                std::cerr << "--generate requires a non-negative integer up to 1024\n";
                return 2;
            }
        } else if (a == "--out") {
            out_path = value("--out requires a path");
        } else if (a == "--language") {
            language = value("--language requires a value");
        } else if (a == "--system") {
            system_text = value("--system requires a value");
        } else if (a == "--audio-backend") {
            audio_backend = value("--audio-backend requires ggml or sched");
            if (audio_backend != "ggml" && audio_backend != "sched") {
                std::cerr << "--audio-backend requires ggml or sched\n";
                return 2;
            }
        } else if (a == "--backend") {
            text_backend = value("--backend requires scalar, ggml, or sched");
            if (text_backend != "scalar" && text_backend != "ggml" && text_backend != "sched") {
                std::cerr << "--backend requires scalar, ggml, or sched\n";
                return 2;
            }
        } else if (a == "--device") {
            if (!qwenasr_ggml_device_from_string(value("--device requires auto, cpu, or gpu"), &device, &error)) {
                std::cerr << error << "\n";
                return 2;
            }
        } else if (a == "--layer") {
            if (!parse_long(value("--layer requires a non-negative integer"), 0, std::numeric_limits<int>::max(),
                            &layer)) {
                std::cerr << "--layer requires a non-negative integer\n";
                return 2;
            }
        } else if (a == "--threads") {
            if (!parse_long(value("--threads requires a positive integer"), 1, std::numeric_limits<int>::max(),
                            &n_threads)) {
                std::cerr << "--threads requires a positive integer\n";
                return 2;
            }
        } else if (a == "--model") {
            model_path = value("--model requires a path");
        } else if (a == "--size") {
            size = value("--size requires 0.6b or 1.7b");
        } else if (a == "--layers") {
            if (!parse_long(value("--layers requires a positive integer"), 1, 1000, &n_layers)) {
                std::cerr << "--layers requires a positive integer\n";
                return 2;
            }
        } else if (a == "--audio-tokens") {
            if (!parse_long(value("--audio-tokens requires an integer"), 0, 1 << 20, &audio_tokens_opt)) {
                std::cerr << "--audio-tokens requires a non-negative integer\n";
                return 2;
            }
        } else if (a == "--prompt-tokens") {
            if (!parse_long(value("--prompt-tokens requires an integer"), 0, 1 << 20, &prompt_tokens)) {
                std::cerr << "--prompt-tokens requires a non-negative integer\n";
                return 2;
            }
        } else if (a == "--seed") {
            if (!parse_long(value("--seed requires an integer"), 0, std::numeric_limits<long>::max(), &seed)) {
                std::cerr << "--seed requires a non-negative integer\n";
                return 2;
            }
        } else if (a == "--kv-cache-type") {
            cache_type = value("--kv-cache-type requires f32 or f16");
        } else if (!a.empty() && a[0] == '-') {
            std::cerr << "unknown option: " << a << "\n";
            usage(argv[0]);
            return 2;
        } else if (model_path.empty() && size.empty()) {
            model_path = a;
        } else if (audio_path.empty()) {
            audio_path = a;
        } else {
            std::cerr << "too many positional arguments\n";
            return 2;
        }
    }

    // ---- validation, in the reference's order (tools/qwen-asr-text-layer.cpp:241-272)
    if (model_path.empty() && size.empty()) {
        std::cerr << "model GGUF and audio WAV are required\n";
        return 2;
    }
    if (audio_path.empty() && audio_tokens_opt < 0) {
        if (model_path.empty()) {
            audio_tokens_opt = 143;   // synthetic model without a clip: the 11 s clip's 143 audio rows
        } else {
            std::cerr << "model GGUF and audio WAV are required\n";
            return 2;
        }
    }
    if (prefill && generate >= 0) {
        std::cerr << "--prefill and --generate are mutually exclusive\n";
        return 2;
    }
    if (generate >= 0 && text_backend == "sched") use_kv_cache = true;
    if (use_kv_cache && generate < 0) {
        std::cerr << "--kv-cache requires --generate\n";
        return 2;
    }
    if ((generate >= 0 || prefill) && text_backend == "ggml") {
        std::cerr << "--backend ggml currently supports layer mode only\n";
        return 2;
    }
    if (cache_type != "f32" && cache_type != "f16") {
        std::cerr << "--kv-cache-type requires f32 or f16\n";
        return 2;
    }

    // ---- model: a GGUF checkpoint or a seeded synthetic model of the named size
    QwenAsrGgufModel model{};
    qa_model * synth = nullptr;
    qa_text_config cfg{};
    int32_t audio_token_id = QA_TOKEN_AUDIO_PAD;
    std::vector<int32_t> stop_ids = {QA_TOKEN_IM_END, QA_TOKEN_ENDOFTEXT, QA_TOKEN_IM_END};
    auto cleanup = [&]() {
        qwenasr_gguf_model_close(&model);
        qa_model_free(synth);
    };
    if (!model_path.empty()) {
        if (!qwenasr_gguf_model_open(model_path.c_str(), &model, &error)) {
            std::cerr << error << "\n";
            return 1;
        }
        uint32_t v = 0;
        bool ok = true;
        auto need_u32 = [&](const char * key, int32_t * dst) {
            if (!ok) return;
            if (!qwenasr_gguf_model_get_u32(model, key, &v)) {
                error = std::string("missing GGUF key: ") + key;
                ok = false;
                return;
            }
            *dst = static_cast<int32_t>(v);
        };
        auto need_f32 = [&](const char * key, float * dst) {
            if (ok && !qwenasr_gguf_model_get_f32(model, key, dst)) {
                error = std::string("missing GGUF key: ") + key;
                ok = false;
            }
        };
        need_u32("qwen3-asr.text.num_hidden_layers", &cfg.n_layers);
        need_u32("qwen3-asr.text.hidden_size", &cfg.hidden);
        need_u32("qwen3-asr.text.num_attention_heads", &cfg.n_heads);
        need_u32("qwen3-asr.text.num_key_value_heads", &cfg.n_kv_heads);
        need_u32("qwen3-asr.text.head_dim", &cfg.head_dim);
        need_u32("qwen3-asr.text.intermediate_size", &cfg.intermediate);
        need_u32("qwen3-asr.text.vocab_size", &cfg.vocab);
        need_f32("qwen3-asr.text.rope_theta", &cfg.rope_theta);
        need_f32("qwen3-asr.text.rms_norm_eps", &cfg.rms_norm_eps);
        // stop ids im_end, endoftext, tokenizer eos (tools/qwen-asr-text-layer.cpp:395-399)
        need_u32("qwen3-asr.token.im_end_token_id", &stop_ids[0]);
        need_u32("qwen3-asr.token.endoftext_token_id", &stop_ids[1]);
        need_u32("tokenizer.ggml.eos_token_id", &stop_ids[2]);
        need_u32("qwen3-asr.token.audio_token_id", &audio_token_id);
        if (!ok) {
            cleanup();
            std::cerr << error << "\n";
            return 1;
        }
    } else {
        if (size == "1.7b") cfg = {28, 2048, 16, 8, 128, 6144, 151936, 1000000.0f, 1e-6f};
        else if (size == "0.6b") cfg = {28, 1024, 16, 8, 128, 3072, 151936, 1000000.0f, 1e-6f};
        else {
            std::cerr << "--size requires 0.6b or 1.7b\n";
            return 2;
        }
        if (n_layers > 0) cfg.n_layers = static_cast<int32_t>(n_layers);
        if (qa_model_synthetic(&cfg, static_cast<uint64_t>(seed), &synth) != QA_OK ||
            !qwenasr_gguf_model_from_synthetic(synth, &model, &error)) {
            std::cerr << (error.empty() ? qa_last_error() : error) << "\n";
            cleanup();
            return 1;
        }
    }
    if (!prefill && generate < 0 && layer >= cfg.n_layers) {
        cleanup();
        std::cerr << "--layer is out of range for model\n";
        return 2;
    }

    // ---- audio: the clip's length sets the number of audio-encoder rows
    int64_t samples = 0;
    int32_t sample_rate = 16000;
    if (!audio_path.empty() && qa_wav_info(audio_path.c_str(), &samples, &sample_rate) != QA_OK) {
        cleanup();
        std::cerr << qa_last_error() << "\n";
        return 1;
    }
    const int32_t feature_frames = static_cast<int32_t>(samples / 160);   // hop 160 (audio-features.cpp:362-367)
    const int32_t audio_tokens =
        audio_tokens_opt >= 0 ? static_cast<int32_t>(audio_tokens_opt) : qa_audio_output_length(feature_frames);

    // ---- decoder input: audio rows N(0, 1) at the placeholders, then the prompt ids
    const auto decoder_start = std::chrono::steady_clock::now();
    const std::string prompt_text = qwenasr_build_asr_prompt(audio_tokens, system_text, language);
    std::vector<int32_t> ids(static_cast<size_t>(audio_tokens), audio_token_id);
    std::vector<int32_t> prompt_ids(static_cast<size_t>(prompt_tokens));
    qa_synth_fill_ids(prompt_ids.data(), prompt_ids.size(), static_cast<uint64_t>(seed) + 3, "prompt_ids", 0,
                      cfg.vocab - 1);
    ids.insert(ids.end(), prompt_ids.begin(), prompt_ids.end());
    std::vector<float> audio_rows(static_cast<size_t>(audio_tokens) * cfg.hidden);
    qa_synth_fill_normal(audio_rows.data(), audio_rows.size(), static_cast<uint64_t>(seed) + 1, "audio_embeddings", 1.0);
    QwenAsrDecoderInputOutput input;
    bool input_ok = false;
    if (audio_tokens > 0) {
        input_ok = qwenasr_decoder_input_from_ids(model, ids, audio_rows, audio_tokens, audio_token_id, &input, &error);
    } else {   // no audio rows: the prompt ids alone
        QwenAsrGgufTensorView embd;
        input_ok = !ids.empty() && qwenasr_gguf_model_tensor_by_name(model, "text.token_embd.weight", &embd, &error);
        if (ids.empty()) error = "decoder prompt produced no tokens";
        if (input_ok) {
            input.tokens = static_cast<int>(ids.size());
            input.hidden = cfg.hidden;
            input.input_ids = ids;
            input.values.resize(ids.size() * static_cast<size_t>(cfg.hidden));
            for (size_t t = 0; t < ids.size(); ++t) {
                std::memcpy(input.values.data() + t * cfg.hidden,
                            static_cast<const float *>(embd.data) + static_cast<size_t>(ids[t]) * cfg.hidden,
                            sizeof(float) * cfg.hidden);
            }
        }
    }
    const double decoder_input_ms = ms_since(decoder_start);
    if (!input_ok) {
        cleanup();
        std::cerr << error << "\n";
        return 1;
    }

    // lines every mode prints first (tools/qwen-asr-text-layer.cpp:487-497, 603-614, 715-727)
    auto common = [&](double text_init_ms) {
        std::cout << "audio_backend=" << audio_backend << "\n"
                  << "device=" << qwenasr_ggml_device_name(device) << "\n"
                  << "audio_path=synthetic\n"
                  << "threads=" << n_threads << "\n"
                  << "init_ms=0\n"
                  << "prompt_chars=" << prompt_text.size() << "\n"
                  << "text_init_ms=" << text_init_ms << "\n"
                  << "decoder_input_ms=" << decoder_input_ms << "\n";
    };
    auto tail = [&]() {
        std::cout << "sample_rate=" << sample_rate << "\n"
                  << "samples=" << samples << "\n"
                  << "feature_frames=" << feature_frames << "\n"
                  << "layers=" << cfg.n_layers << "\n";
    };
    const int threads = static_cast<int>(n_threads);
    const QwenAsrKvCacheType kv_type = cache_type == "f16" ? QwenAsrKvCacheType::F16 : QwenAsrKvCacheType::F32;

    if (generate >= 0) {
        QwenAsrTextGenerateOutput out;
        double text_init_ms = 0.0, generate_ms = 0.0;
        QwenAsrTextDecoderBackend * backend = nullptr;
        bool ok = false;
        if (text_backend == "sched") {
            const auto t0 = std::chrono::steady_clock::now();
            ok = qwenasr_text_decoder_backend_init_cached_typed(
                model, threads, cfg.n_layers, cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.intermediate,
                cfg.vocab, input.tokens + static_cast<int>(generate), cfg.rope_theta, cfg.rms_norm_eps, kv_type,
                &backend, &error, device);
            text_init_ms = ms_since(t0);
            if (ok) {
                const auto g0 = std::chrono::steady_clock::now();
                ok = qwenasr_text_generate_cached_backend(backend, model, input, static_cast<int>(generate), stop_ids,
                                                          &out, &error);
                generate_ms = ms_since(g0);
            }
            qwenasr_text_decoder_backend_free(backend);
        } else {
            const auto g0 = std::chrono::steady_clock::now();
            ok = use_kv_cache ? qwenasr_text_generate_cached_cpu(model, input, static_cast<int>(generate), cfg.n_layers,
                                                                 cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                                                 cfg.intermediate, cfg.vocab, cfg.rope_theta,
                                                                 cfg.rms_norm_eps, stop_ids, &out, &error)
                              : qwenasr_text_generate_greedy_cpu(model, input, static_cast<int>(generate), cfg.n_layers,
                                                                 cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                                                 cfg.intermediate, cfg.vocab, cfg.rope_theta,
                                                                 cfg.rms_norm_eps, stop_ids, &out, &error);
            generate_ms = ms_since(g0);
        }
        cleanup();
        if (!ok) {
            std::cerr << error << "\n";
            return 1;
        }
        std::string ids_text;
        for (size_t i = 0; i < out.generated_ids.size(); ++i) {
            ids_text += (i ? "," : "") + std::to_string(out.generated_ids[i]);
        }
        if (!out_path.empty()) {
            std::ofstream f(out_path);
            f << ids_text;
            if (!f) {
                std::cerr << "failed to write output file: " << out_path << "\n";
                return 1;
            }
        }
        std::cout << "backend=" << text_backend << "\n"
                  << "mode=generate\n"
                  << "decode_backend=" << (use_kv_cache ? "kv-cache" : "recompute") << "\n";
        common(text_init_ms);
        std::cout << "generate_ms=" << generate_ms << "\n";
        tail();
        std::cout << "kv_cache_type=" << cache_type << "\n"
                  << "prompt_tokens=" << out.prompt_tokens << "\n"
                  << "total_tokens=" << out.total_tokens << "\n"
                  << "hidden=" << out.hidden << "\n"
                  << "vocab=" << out.vocab << "\n"
                  << "requested_tokens=" << generate << "\n"
                  << "generated_tokens=" << out.generated_ids.size() << "\n"
                  << "stopped=" << (out.stopped ? "true" : "false") << "\n"
                  << "generated_ids=" << ids_text << "\n"
                  << "text_json=" << json_string(ids_text) << "\n";
        return 0;
    }

    if (prefill) {
        QwenAsrTextPrefillOutput out;
        double text_init_ms = 0.0, prefill_ms = 0.0;
        bool ok = false;
        if (text_backend == "sched") {
            QwenAsrTextDecoderBackend * backend = nullptr;
            const auto t0 = std::chrono::steady_clock::now();
            ok = qwenasr_text_decoder_backend_init(model, threads, cfg.n_layers, cfg.hidden, cfg.n_heads,
                                                   cfg.n_kv_heads, cfg.head_dim, cfg.intermediate, cfg.vocab,
                                                   cfg.rope_theta, cfg.rms_norm_eps, &backend, &error, device);
            text_init_ms = ms_since(t0);
            if (ok) {
                const auto p0 = std::chrono::steady_clock::now();
                ok = qwenasr_text_prefill_backend_forward(backend, input, &out, &error);
                prefill_ms = ms_since(p0);
            }
            qwenasr_text_decoder_backend_free(backend);
        } else {
            const auto p0 = std::chrono::steady_clock::now();
            ok = qwenasr_text_prefill_forward_cpu(model, input, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads,
                                                  cfg.head_dim, cfg.intermediate, cfg.vocab, cfg.rope_theta,
                                                  cfg.rms_norm_eps, &out, &error);
            prefill_ms = ms_since(p0);
        }
        cleanup();
        if (!ok) {
            std::cerr << error << "\n";
            return 1;
        }
        if (!out_path.empty() && !write_raw(out_path, out.logits, &error)) {
            std::cerr << error << "\n";
            return 1;
        }
        double sum = 0.0;
        float mn = std::numeric_limits<float>::infinity(), mx = -mn, top = -mn;
        int top_id = -1;
        for (size_t i = 0; i < out.logits.size(); ++i) {
            const float v = out.logits[i];
            mn = std::min(mn, v);
            mx = std::max(mx, v);
            if (v > top) {
                top = v;
                top_id = static_cast<int>(i);
            }
            sum += v;
        }
        std::cout << "backend=" << text_backend << "\n" << "mode=prefill\n";
        common(text_init_ms);
        std::cout << "prefill_ms=" << prefill_ms << "\n";
        tail();
        std::cout << "tokens=" << out.tokens << "\n"
                  << "hidden=" << out.hidden << "\n"
                  << "vocab=" << out.vocab << "\n"
                  << "values=" << out.logits.size() << "\n"
                  << "top_id=" << top_id << "\n"
                  << "top_logit=" << top << "\n"
                  << "min=" << mn << "\n"
                  << "max=" << mx << "\n"
                  << "mean=" << (sum / static_cast<double>(out.logits.size())) << "\n";
        return 0;
    }

    QwenAsrTextLayerOutput out;
    double text_init_ms = 0.0, text_layer_ms = 0.0;
    bool ok = false;
    if (text_backend == "sched") {
        QwenAsrTextLayerBackend * backend = nullptr;
        const auto t0 = std::chrono::steady_clock::now();
        ok = qwenasr_text_layer_backend_init(model, static_cast<int>(layer), threads, cfg.hidden, cfg.n_heads,
                                             cfg.n_kv_heads, cfg.head_dim, cfg.intermediate, cfg.rope_theta,
                                             cfg.rms_norm_eps, &backend, &error, device);
        text_init_ms = ms_since(t0);
        if (ok) {
            const auto p0 = std::chrono::steady_clock::now();
            ok = qwenasr_text_layer_backend_forward(backend, input, &out, &error);
            text_layer_ms = ms_since(p0);
        }
        qwenasr_text_layer_backend_free(backend);
    } else {
        const auto p0 = std::chrono::steady_clock::now();
        ok = text_backend == "ggml"
                 ? qwenasr_text_layer_forward_ggml(model, input, static_cast<int>(layer), threads, cfg.n_heads,
                                                   cfg.n_kv_heads, cfg.head_dim, cfg.intermediate, cfg.rope_theta,
                                                   cfg.rms_norm_eps, &out, &error)
                 : qwenasr_text_layer_forward_cpu(model, input, static_cast<int>(layer), cfg.n_heads, cfg.n_kv_heads,
                                                  cfg.head_dim, cfg.intermediate, cfg.rope_theta, cfg.rms_norm_eps,
                                                  &out, &error);
        text_layer_ms = ms_since(p0);
    }
    cleanup();
    if (!ok) {
        std::cerr << error << "\n";
        return 1;
    }
    if (!out_path.empty() && !write_raw(out_path, out.values, &error)) {
        std::cerr << error << "\n";
        return 1;
    }
    double sum = 0.0;
    float mn = std::numeric_limits<float>::infinity(), mx = -mn;
    for (float v : out.values) {
        mn = std::min(mn, v);
        mx = std::max(mx, v);
        sum += v;
    }
    std::cout << "backend=" << text_backend << "\n";
    common(text_init_ms);
    std::cout << "text_layer_ms=" << text_layer_ms << "\n";
    tail();
    std::cout << "layer=" << layer << "\n"
              << "tokens=" << out.tokens << "\n"
              << "hidden=" << out.hidden << "\n"
              << "values=" << out.values.size() << "\n"
              << "min=" << mn << "\n"
              << "max=" << mx << "\n"
              << "mean=" << (sum / static_cast<double>(out.values.size())) << "\n";
    return 0;
}
