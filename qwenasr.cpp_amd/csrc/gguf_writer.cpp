// GGUF v3 writer: the on-disk side of row f3.
//
// The reference writes GGUF through GGML's gguf_write_to_file (tools/qwen-asr-weights.cpp:58-96,
// src/native-model.cpp:370-440) and through the gguf Python package in convert.py:357-397.  Neither is
// available here, so the container format is written directly, following the GGUF specification that
// the reader in gguf_model.cpp parses:
//   magic "GGUF", u32 version 3, u64 tensor count, u64 key/value count,
//   key/value pairs (u64-length string key, u32 value type, value),
//   tensor infos (name, u32 n_dims, u64 ne[n_dims] in GGML order, u32 type, u64 offset into the data),
//   zero padding to `general.alignment` (32 unless set), then each tensor's bytes at its aligned offset.
// qa_gguf_write_model writes a model held in host memory as a checkpoint that the reference's loader
// accepts: the metadata keys qwenasr_load_gguf_metadata requires (native-model.cpp:188-218), a
// placeholder tokenizer vocabulary with the special tokens at their Qwen3-ASR ids (the same layout as
// the reference's metadata fixture, native-model.cpp:407-431), and the text tensors in f32 under the
// names and ne order that load_text_layer_tensors reads (text-decoder.cpp:191-228).
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "common.hpp"
#include "gguf-model.h"

namespace {

// GGUF value type ids (the GGUF specification).
enum : uint32_t { kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kStr, kArr, kU64, kI64, kF64 };

void set_error(std::string * error, const std::string & message) {
    if (error) *error = message;
}

struct Out {
    std::vector<uint8_t> bytes;
    template <typename T>
    void put(T v) {
        const size_t at = bytes.size();
        bytes.resize(at + sizeof(T));
        std::memcpy(bytes.data() + at, &v, sizeof(T));
    }
    void str(const std::string & s) {
        put<uint64_t>(s.size());
        bytes.insert(bytes.end(), s.begin(), s.end());
    }
    void pad(size_t alignment) {
        while (bytes.size() % alignment) bytes.push_back(0);
    }
};

size_t elem_bytes(ggml_type t) {
    if (t == GGML_TYPE_F32) return 4;
    if (t == GGML_TYPE_F16 || t == GGML_TYPE_BF16) return 2;
    return 0;
}

}  // namespace

void qwenasr_gguf_writer_set_u32(QwenAsrGgufWriter * w, const std::string & key, uint32_t v) {
    QwenAsrGgufValue e;
    e.key = key;
    e.type = kU32;
    e.u = v;
    w->values.push_back(std::move(e));
}

void qwenasr_gguf_writer_set_f32(QwenAsrGgufWriter * w, const std::string & key, float v) {
    QwenAsrGgufValue e;
    e.key = key;
    e.type = kF32;
    e.f = v;
    w->values.push_back(std::move(e));
}

void qwenasr_gguf_writer_set_str(QwenAsrGgufWriter * w, const std::string & key, const std::string & v) {
    QwenAsrGgufValue e;
    e.key = key;
    e.type = kStr;
    e.s = v;
    w->values.push_back(std::move(e));
}

void qwenasr_gguf_writer_set_arr_str(QwenAsrGgufWriter * w, const std::string & key, std::vector<std::string> v) {
    QwenAsrGgufValue e;
    e.key = key;
    e.type = kArr;
    e.elem_type = kStr;
    e.strs = std::move(v);
    w->values.push_back(std::move(e));
}

void qwenasr_gguf_writer_set_arr_i32(QwenAsrGgufWriter * w, const std::string & key, std::vector<int32_t> v) {
    QwenAsrGgufValue e;
    e.key = key;
    e.type = kArr;
    e.elem_type = kI32;
    e.i32s = std::move(v);
    w->values.push_back(std::move(e));
}

void qwenasr_gguf_writer_add_tensor(QwenAsrGgufWriter * w, const std::string & name, ggml_type type,
                                    std::vector<int64_t> ne, const void * data) {
    QwenAsrGgufWriter::Tensor t;
    t.name = name;
    t.type = type;
    t.ne = std::move(ne);
    t.data = data;
    w->tensors.push_back(std::move(t));
}

bool qwenasr_gguf_writer_write(const QwenAsrGgufWriter & w, const char * path, std::string * error) {
    if (!path) {
        set_error(error, "GGUF output path is null");
        return false;
    }
    const size_t alignment = w.alignment;
    if (alignment == 0 || (alignment & (alignment - 1)) != 0) {
        set_error(error, "GGUF alignment must be a power of two");
        return false;
    }
    Out h;
    h.bytes.insert(h.bytes.end(), {'G', 'G', 'U', 'F'});
    h.put<uint32_t>(3);
    h.put<uint64_t>(w.tensors.size());
    h.put<uint64_t>(w.values.size() + (alignment != 32 ? 1 : 0));
    for (const QwenAsrGgufValue & v : w.values) {
        h.str(v.key);
        h.put<uint32_t>(v.type);
        switch (v.type) {
            case kU32: h.put<uint32_t>(static_cast<uint32_t>(v.u)); break;
            case kF32: h.put<float>(v.f); break;
            case kStr: h.str(v.s); break;
            case kArr:
                h.put<uint32_t>(v.elem_type);
                if (v.elem_type == kStr) {
                    h.put<uint64_t>(v.strs.size());
                    for (const std::string & s : v.strs) h.str(s);
                } else {
                    h.put<uint64_t>(v.i32s.size());
                    for (int32_t x : v.i32s) h.put<int32_t>(x);
                }
                break;
            default:
                set_error(error, "unsupported GGUF value type for key " + v.key);
                return false;
        }
    }
    if (alignment != 32) {
        h.str("general.alignment");
        h.put<uint32_t>(kU32);
        h.put<uint32_t>(static_cast<uint32_t>(alignment));
    }
    uint64_t offset = 0;
    std::vector<size_t> nbytes;
    for (const auto & t : w.tensors) {
        const size_t es = elem_bytes(t.type);
        if (es == 0 || t.ne.empty() || t.ne.size() > 4 || !t.data) {
            set_error(error, "unsupported GGUF tensor: " + t.name);
            return false;
        }
        size_t n = es;
        for (int64_t d : t.ne) {
            if (d <= 0) {
                set_error(error, "GGUF tensor has an empty dimension: " + t.name);
                return false;
            }
            n *= static_cast<size_t>(d);
        }
        h.str(t.name);
        h.put<uint32_t>(static_cast<uint32_t>(t.ne.size()));
        for (int64_t d : t.ne) h.put<uint64_t>(static_cast<uint64_t>(d));
        h.put<uint32_t>(static_cast<uint32_t>(t.type));
        h.put<uint64_t>(offset);
        nbytes.push_back(n);
        offset += (n + alignment - 1) / alignment * alignment;
    }
    h.pad(alignment);

    FILE * f = std::fopen(path, "wb");
    if (!f) {
        set_error(error, std::string("failed to open GGUF output file: ") + path);
        return false;
    }
    bool ok = std::fwrite(h.bytes.data(), 1, h.bytes.size(), f) == h.bytes.size();
    static const uint8_t zeros[256] = {0};
    for (size_t i = 0; ok && i < w.tensors.size(); ++i) {
        ok = std::fwrite(w.tensors[i].data, 1, nbytes[i], f) == nbytes[i];
        size_t pad = (alignment - nbytes[i] % alignment) % alignment;
        while (ok && pad > 0) {
            const size_t k = pad < sizeof(zeros) ? pad : sizeof(zeros);
            ok = std::fwrite(zeros, 1, k, f) == k;
            pad -= k;
        }
    }
    ok = (std::fclose(f) == 0) && ok;
    if (!ok) set_error(error, std::string("failed to write GGUF output file: ") + path);
    return ok;
}

extern "C" int qa_gguf_write_model(const qa_model * model, const char * path) {
    using namespace qa;
    if (!model || !path) return fail(QA_ERR_INVALID, "qa_gguf_write_model: null argument");
    qa_text_config c{};
    qa_model_config(model, &c);
    QwenAsrGgufWriter w;
    qwenasr_gguf_writer_set_str(&w, "general.name", "Qwen3-ASR synthetic text decoder");
    qwenasr_gguf_writer_set_str(&w, "qwen3-asr.arch", "qwen3-asr");
    // audio-encoder metadata of Qwen3-ASR-0.6B (native-model.cpp:383-390); no audio tensors are written
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.audio.sample_rate", 16000);
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.audio.num_mel_bins", 128);
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.audio.d_model", 896);
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.audio.encoder_layers", 18);
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.audio.encoder_attention_heads", 14);
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.audio.encoder_ffn_dim", 3584);
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.audio.downsample_hidden_size", 480);
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.audio.output_dim", static_cast<uint32_t>(c.hidden));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.text.vocab_size", static_cast<uint32_t>(c.vocab));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.text.hidden_size", static_cast<uint32_t>(c.hidden));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.text.intermediate_size", static_cast<uint32_t>(c.intermediate));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.text.num_hidden_layers", static_cast<uint32_t>(c.n_layers));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.text.num_attention_heads", static_cast<uint32_t>(c.n_heads));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.text.num_key_value_heads", static_cast<uint32_t>(c.n_kv_heads));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.text.head_dim", static_cast<uint32_t>(c.head_dim));
    qwenasr_gguf_writer_set_f32(&w, "qwen3-asr.text.rope_theta", c.rope_theta);
    qwenasr_gguf_writer_set_f32(&w, "qwen3-asr.text.rms_norm_eps", c.rms_norm_eps);
    // placeholder vocabulary: the special tokens at their Qwen3-ASR ids, or, in a synthetic vocabulary too
    // small to hold those ids, at its last seven ids in the same order; every other token is unused
    struct Special { int32_t id; const char * text; };
    Special specials[] = {{QA_TOKEN_ENDOFTEXT, "<|endoftext|>"}, {QA_TOKEN_IM_START, "<|im_start|>"},
                          {QA_TOKEN_IM_END, "<|im_end|>"},       {QA_TOKEN_AUDIO_START, "<|audio_start|>"},
                          {QA_TOKEN_AUDIO_END, "<|audio_end|>"}, {QA_TOKEN_AUDIO_PAD, "<|audio_pad|>"},
                          {QA_TOKEN_ASR_TEXT, "<asr_text>"}};
    constexpr int32_t kSpecials = 7;
    if (c.vocab <= QA_TOKEN_ASR_TEXT) {
        if (c.vocab < kSpecials + 1) return fail(QA_ERR_INVALID, "qa_gguf_write_model: vocabulary too small");
        for (int32_t k = 0; k < kSpecials; ++k) specials[k].id = c.vocab - kSpecials + k;
    }
    const int32_t endoftext = specials[0].id, im_start = specials[1].id, im_end = specials[2].id;
    const int32_t audio_start = specials[3].id, audio_end = specials[4].id, audio_pad = specials[5].id;
    const int32_t asr_text = specials[6].id;
    std::vector<std::string> tokens(static_cast<size_t>(c.vocab));
    std::vector<int32_t> types(static_cast<size_t>(c.vocab), 5);
    for (size_t i = 0; i < tokens.size(); ++i) tokens[i] = "<|unused-" + std::to_string(i) + "|>";
    for (const Special & s : specials) {
        tokens[static_cast<size_t>(s.id)] = s.text;
        types[static_cast<size_t>(s.id)] = 4;
    }
    qwenasr_gguf_writer_set_str(&w, "tokenizer.ggml.model", "gpt2");
    qwenasr_gguf_writer_set_arr_str(&w, "tokenizer.ggml.tokens", std::move(tokens));
    qwenasr_gguf_writer_set_arr_i32(&w, "tokenizer.ggml.token_type", std::move(types));
    qwenasr_gguf_writer_set_arr_str(&w, "tokenizer.ggml.merges", {"a b"});
    auto u = [](int32_t v) { return static_cast<uint32_t>(v); };
    qwenasr_gguf_writer_set_u32(&w, "tokenizer.ggml.eos_token_id", u(im_end));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.token.endoftext_token_id", u(endoftext));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.token.im_start_token_id", u(im_start));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.token.im_end_token_id", u(im_end));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.token.audio_token_id", u(audio_pad));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.token.audio_start_token_id", u(audio_start));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.token.audio_end_token_id", u(audio_end));
    qwenasr_gguf_writer_set_u32(&w, "qwen3-asr.token.asr_text_token_id", u(asr_text));

    const int64_t H = c.hidden, QD = static_cast<int64_t>(c.n_heads) * c.head_dim,
                  KD = static_cast<int64_t>(c.n_kv_heads) * c.head_dim, I = c.intermediate;
    bool missing = false;
    auto add = [&](const std::string & name, std::vector<int64_t> ne) {
        int64_t n = 0;
        const float * p = qa_model_tensor(model, name.c_str(), &n);
        int64_t want = 1;
        for (int64_t d : ne) want *= d;
        if (!p || n != want) {
            missing = true;
            return;
        }
        qwenasr_gguf_writer_add_tensor(&w, name, GGML_TYPE_F32, std::move(ne), p);
    };
    add("text.token_embd.weight", {H, c.vocab});
    for (int l = 0; l < c.n_layers; ++l) {
        const std::string p = "text.blk." + std::to_string(l) + ".";
        add(p + "attn_norm.weight", {H});
        add(p + "attn_q.weight", {H, QD});
        add(p + "attn_k.weight", {H, KD});
        add(p + "attn_v.weight", {H, KD});
        add(p + "attn_output.weight", {QD, H});
        add(p + "attn_q_norm.weight", {c.head_dim});
        add(p + "attn_k_norm.weight", {c.head_dim});
        add(p + "ffn_norm.weight", {H});
        add(p + "ffn_gate.weight", {H, I});
        add(p + "ffn_up.weight", {H, I});
        add(p + "ffn_down.weight", {I, H});
    }
    add("text.output_norm.weight", {H});
    add("text.output.weight", {H, c.vocab});
    if (missing) return fail(QA_ERR_INVALID, "qa_gguf_write_model: the model lacks a text tensor");
    std::string error;
    if (!qwenasr_gguf_writer_write(w, path, &error)) return fail(QA_ERR_INVALID, error);
    return QA_OK;
}
