// Decoder-input assembly: the step before the text decoder, after the prompt has been tokenized.
//
// Follows qwenasr_decoder_input_from_audio (decoder-input.cpp:26-101): the prompt
// "<|im_start|>system\n...<|audio_start|>" + N x "<|audio_pad|>" + "<|audio_end|>..." (tokenizer.cpp:
// 529-549) is tokenized by the caller; every token id selects its embedding row
// (text.token_embd.weight), and the i-th audio placeholder id is replaced by the i-th audio-encoder
// row.  The reference validates while it copies into a local result and moves it out only on
// success; here a first pass validates and a second pass copies, so `out` is written only when the
// whole input is valid.  Host code: the rows are the decoder's host input (qa_decoder_forward).
#include "decoder-input.h"
#include "gguf-model.h"
#include "qwenasr_amd.h"

#include "common.hpp"

#include <cstring>

extern "C" int qa_decoder_input_assemble(const float * token_embd, int32_t vocab, int32_t hidden, const int32_t * ids,
                                         int32_t n_tokens, int32_t audio_token_id, const float * audio,
                                         int32_t audio_tokens, float * out) {
    using qa::fail;
    if (!token_embd || !out || vocab <= 0 || hidden <= 0) {
        return fail(QA_ERR_INVALID, "qa_decoder_input_assemble: invalid arguments");
    }
    if (audio_token_id < 0) return fail(QA_ERR_INVALID, "invalid decoder input configuration");
    if (audio_tokens <= 0 || !audio) return fail(QA_ERR_INVALID, "invalid native audio encoder output");
    if (n_tokens <= 0 || !ids) return fail(QA_ERR_INVALID, "decoder prompt produced no tokens");
    int32_t placeholders = 0;
    for (int32_t t = 0; t < n_tokens; ++t) {
        const int32_t id = ids[t];
        if (id < 0 || id >= vocab) return fail(QA_ERR_INVALID, "decoder input token id is out of embedding range");
        if (id == audio_token_id && ++placeholders > audio_tokens) {
            return fail(QA_ERR_INVALID, "prompt has more audio placeholders than audio encoder outputs");
        }
    }
    if (placeholders != audio_tokens) {
        return fail(QA_ERR_INVALID, "audio placeholder count does not match audio encoder output count");
    }
    const size_t row = static_cast<size_t>(hidden) * sizeof(float);
    int32_t a = 0;
    for (int32_t t = 0; t < n_tokens; ++t) {
        const int32_t id = ids[t];
        const float * src = id == audio_token_id ? audio + static_cast<size_t>(a++) * hidden
                                                 : token_embd + static_cast<size_t>(id) * hidden;
        std::memcpy(out + static_cast<size_t>(t) * hidden, src, row);
    }
    return QA_OK;
}

bool qwenasr_decoder_input_from_ids(const QwenAsrGgufModel & model, const std::vector<int32_t> & input_ids,
                                    const std::vector<float> & audio_values, int audio_tokens, int audio_token_id,
                                    QwenAsrDecoderInputOutput * out, std::string * error) {
    auto set_error = [&](const std::string & m) {
        if (error) *error = m;
        return false;
    };
    if (!out) return set_error("qwenasr_decoder_input_from_ids: out is null");
    if (audio_token_id < 0) return set_error("invalid decoder input configuration");
    if (audio_tokens <= 0 || audio_values.size() % static_cast<size_t>(audio_tokens) != 0) {
        return set_error("invalid native audio encoder output");
    }
    QwenAsrGgufTensorView embd;
    if (!qwenasr_gguf_model_tensor_by_name(model, "text.token_embd.weight", &embd, error)) return false;
    if (embd.type != GGML_TYPE_F32) return set_error("tensor is not f32: text.token_embd.weight");
    const int64_t hidden = audio_values.size() / static_cast<size_t>(audio_tokens);
    if (embd.ne.size() != 2 || embd.ne[0] != hidden || embd.ne[1] <= 0) {
        return set_error("text.token_embd.weight tensor shape mismatch");
    }
    QwenAsrDecoderInputOutput result;
    result.tokens = static_cast<int>(input_ids.size());
    result.hidden = static_cast<int>(hidden);
    result.audio_tokens = audio_tokens;
    result.input_ids = input_ids;
    result.values.assign(input_ids.size() * static_cast<size_t>(hidden), 0.0f);
    if (qa_decoder_input_assemble(static_cast<const float *>(embd.data), static_cast<int32_t>(embd.ne[1]),
                                  static_cast<int32_t>(hidden), input_ids.data(), static_cast<int32_t>(input_ids.size()),
                                  audio_token_id, audio_values.data(), audio_tokens, result.values.data()) != QA_OK) {
        return set_error(qa_last_error());
    }
    *out = std::move(result);
    return true;
}
