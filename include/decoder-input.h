// Drop-in of the decoder-input struct of the reference (src/decoder-input.h:11-17), the input type of
// every text-decoder entry point.  Building it from audio (decoder-input.cpp) is outside this build;
// callers fill it from their own audio front end or synthetic embeddings.
#pragma once

#include <cstdint>
#include <vector>

struct QwenAsrDecoderInputOutput {
    int tokens = 0;
    int hidden = 0;
    int audio_tokens = 0;
    std::vector<int32_t> input_ids;
    std::vector<float> values; // [token, hidden]
};
