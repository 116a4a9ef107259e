// Drop-in for the reference's src/gguf-model.h (same types and functions, gguf-model.h:12-54).
// A model is either a GGUF file mapped read-only (qwenasr_gguf_model_open) or a synthetic model built
// in host memory (qwenasr_gguf_model_from_synthetic, this build's addition).  Tensor views point at
// host memory that stays valid until qwenasr_gguf_model_close.
#pragma once

#include "qwenasr-ggml-types.h"

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

struct qa_model;

struct QwenAsrGgufTensorView {
    std::string name;
    ggml_type type = GGML_TYPE_COUNT;
    std::vector<int64_t> ne;
    size_t nbytes = 0;
    size_t offset = 0;
    const void * data = nullptr;
};

struct QwenAsrGgufModel {
    gguf_context * gguf = nullptr;     // tensor directory and metadata (owned)
    ggml_context * meta = nullptr;     // unused by this build; kept for layout compatibility
    const uint8_t * mapping = nullptr;
    size_t file_size = 0;
    size_t data_offset = 0;
    int fd = -1;
};

bool qwenasr_gguf_model_open(const char * path, QwenAsrGgufModel * model, std::string * error);

void qwenasr_gguf_model_close(QwenAsrGgufModel * model);

int64_t qwenasr_gguf_model_tensor_count(const QwenAsrGgufModel & model);

bool qwenasr_gguf_model_tensor_by_index(
    const QwenAsrGgufModel & model,
    int64_t index,
    QwenAsrGgufTensorView * out,
    std::string * error);

bool qwenasr_gguf_model_tensor_by_name(
    const QwenAsrGgufModel & model,
    const char * name,
    QwenAsrGgufTensorView * out,
    std::string * error);

// Additions of this build (no counterpart in the reference).
// Views a synthetic model (qa_model_synthetic) through this API; `synthetic` must outlive `model`.
bool qwenasr_gguf_model_from_synthetic(const qa_model * synthetic, QwenAsrGgufModel * model, std::string * error);
// Scalar metadata of an opened GGUF file ("qwen3-asr.text.hidden_size", ...); false when absent.
bool qwenasr_gguf_model_get_u32(const QwenAsrGgufModel & model, const char * key, uint32_t * out);
bool qwenasr_gguf_model_get_f32(const QwenAsrGgufModel & model, const char * key, float * out);
