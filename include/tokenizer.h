// Drop-in subset of the reference's src/tokenizer.h: the ASR prompt builder only.
// The BPE tokenizer itself (qwenasr_tokenizer_load_gguf, _encode, _decode) is outside this build's
// scope; the prompt string is what a tokenizer would encode into the decoder's prompt ids.
#pragma once

#include <string>

// qwenasr_build_asr_prompt, tokenizer.cpp:529-549.
std::string qwenasr_build_asr_prompt(int audio_tokens, const std::string & system_text, const std::string & language);
