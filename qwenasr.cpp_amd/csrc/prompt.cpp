// Host-side pieces around the decoder input: the ASR prompt text, the audio-token count of a clip and
// the WAV header (rows f4 and the driver's positional WAV argument).
//
//   qwenasr_build_asr_prompt  tokenizer.cpp:529-549  (chat turns with the audio placeholders)
//   qa_audio_output_length    audio-features.cpp:14-19 (13 tokens per 100 mel frames + the tail)
//   qa_wav_info               audio-features.cpp:120-200 (RIFF chunks, 16 kHz, PCM16/PCM24/f32)
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "common.hpp"
#include "tokenizer.h"

std::string qwenasr_build_asr_prompt(int audio_tokens, const std::string & system_text, const std::string & language) {
    const int n = audio_tokens < 0 ? 0 : audio_tokens;
    static const char kPad[] = "<|audio_pad|>";
    std::string out;
    out.reserve(160 + system_text.size() + language.size() + static_cast<size_t>(n) * (sizeof(kPad) - 1));
    out.append("<|im_start|>system\n").append(system_text);
    out.append("<|im_end|>\n<|im_start|>user\n<|audio_start|>");
    for (int i = 0; i < n; ++i) out.append(kPad);
    out.append("<|audio_end|><|im_end|>\n<|im_start|>assistant\n");
    if (!language.empty()) out.append("language ").append(language).append("<asr_text>");
    return out;
}

extern "C" int qa_build_asr_prompt(int32_t audio_tokens, const char * system_text, const char * language, char * out,
                                   size_t cap, size_t * len) {
    const std::string p = qwenasr_build_asr_prompt(audio_tokens, system_text ? system_text : "", language ? language : "");
    if (len) *len = p.size();
    if (!out || cap < p.size() + 1) return qa::fail(QA_ERR_RANGE, "qa_build_asr_prompt: output buffer too small");
    std::memcpy(out, p.c_str(), p.size() + 1);
    return QA_OK;
}

extern "C" int32_t qa_audio_output_length(int32_t input_frames) {
    if (input_frames <= 0) return 0;
    const int32_t rest = input_frames % 100;
    // the remainder passes three stride-2 convolutions: ceil(rest / 2), then ceil(. / 2) twice
    const int32_t a = rest == 0 ? 0 : (rest - 1) / 2 + 1;
    const int32_t tail = a == 0 ? 0 : ((a - 1) / 2) / 2 + 1;
    return tail + (input_frames / 100) * 13;
}

namespace {

uint32_t le32(const unsigned char * p) {
    return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8) | (static_cast<uint32_t>(p[2]) << 16) |
           (static_cast<uint32_t>(p[3]) << 24);
}

uint16_t le16(const unsigned char * p) { return static_cast<uint16_t>(p[0] | (p[1] << 8)); }

}  // namespace

extern "C" int qa_wav_info(const char * path, int64_t * n_samples, int32_t * sample_rate) {
    using qa::fail;
    if (!path || !n_samples || !sample_rate) return fail(QA_ERR_INVALID, "qa_wav_info: null argument");
    std::ifstream in(path, std::ios::binary);
    if (!in) return fail(QA_ERR_INVALID, std::string("failed to open WAV: ") + path);
    unsigned char riff[12];
    in.read(reinterpret_cast<char *>(riff), 12);
    if (!in || std::memcmp(riff, "RIFF", 4) != 0 || std::memcmp(riff + 8, "WAVE", 4) != 0) {
        return fail(QA_ERR_INVALID, "not a RIFF/WAVE file");
    }
    uint16_t format = 0, channels = 0, bits = 0;
    uint32_t rate = 0;
    uint64_t data_bytes = 0;
    bool have_data = false;
    for (;;) {
        unsigned char hdr[8];
        in.read(reinterpret_cast<char *>(hdr), 8);
        if (!in) break;
        const uint32_t size = le32(hdr + 4);
        const std::streampos start = in.tellg();
        if (std::memcmp(hdr, "fmt ", 4) == 0 && size >= 16) {
            std::vector<unsigned char> f(size);
            in.read(reinterpret_cast<char *>(f.data()), size);
            if (!in) break;
            format = le16(&f[0]);
            channels = le16(&f[2]);
            rate = le32(&f[4]);
            bits = le16(&f[14]);
            if (format == 0xfffe && size >= 40) {   // WAVE_FORMAT_EXTENSIBLE: the sub-format's first word
                const uint16_t sub = le16(&f[24]);
                if (sub == 1 || sub == 3) format = sub;
            }
        } else if (std::memcmp(hdr, "data", 4) == 0) {
            data_bytes = size;
            have_data = true;
        }
        in.clear();
        in.seekg(start + static_cast<std::streamoff>(size + (size & 1u)));
        if (!in) break;
    }
    if (rate != 16000) return fail(QA_ERR_INVALID, "native feature extractor currently requires 16 kHz WAV input");
    if (channels == 0 || !have_data || data_bytes == 0) return fail(QA_ERR_INVALID, "WAV has no decoded audio data");
    const uint32_t bytes_per_sample = bits / 8u;
    if (bytes_per_sample == 0) return fail(QA_ERR_INVALID, "invalid WAV bits_per_sample");
    if (!((format == 1 && (bits == 16 || bits == 24)) || (format == 3 && bits == 32))) {
        return fail(QA_ERR_INVALID, "unsupported WAV encoding; expected PCM16, PCM24, or F32");
    }
    *n_samples = static_cast<int64_t>(data_bytes / (static_cast<uint64_t>(channels) * bytes_per_sample));
    *sample_rate = static_cast<int32_t>(rate);
    return QA_OK;
}
