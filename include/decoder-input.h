// Drop-in of the decoder-input struct of the reference (src/decoder-input.h:11-17), the input type of
// every text-decoder entry point, and of its assembly from prompt ids and audio-encoder rows
// (decoder-input.cpp:26-101).  The audio front end and the BPE tokenizer that produce those inputs are
// outside this build.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

struct QwenAsrGgufModel;

struct QwenAsrDecoderInputOutput {
    int tokens = 0;
    int hidden = 0;
    int audio_tokens = 0;
    std::vector<int32_t> input_ids;
    std::vector<float> values; // [token, hidden]
};

// qwenasr_decoder_input_from_audio (decoder-input.cpp:26-101) after its tokenizer step: input_ids is the
// tokenized ASR prompt (tokenizer.cpp:529-549), audio_values the audio-encoder rows [audio_tokens][hidden].
// Each id takes its row of text.token_embd.weight; the i-th audio_token_id takes audio row i.  Same
// validation and error messages as the reference; *out is written only on success.
bool qwenasr_decoder_input_from_ids(const QwenAsrGgufModel & model, const std::vector<int32_t> & input_ids,
                                    const std::vector<float> & audio_values, int audio_tokens, int audio_token_id,
                                    QwenAsrDecoderInputOutput * out, std::string * error);
