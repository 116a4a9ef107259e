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

// GGUF v3 writer (this build's addition; the reference writes through GGML's gguf_write_to_file,
// tools/qwen-asr-weights.cpp:58-96, and the gguf Python package, convert.py:357-397).  Values and
// tensors are written in the order they were added; tensor data must stay valid until write.
struct QwenAsrGgufValue {
    std::string key;
    uint32_t type = 0;        // GGUF value type id: 4 u32, 6 f32, 8 string, 9 array
    uint32_t elem_type = 0;   // array element type: 8 string or 5 i32
    uint64_t u = 0;
    float f = 0.0f;
    std::string s;
    std::vector<std::string> strs;
    std::vector<int32_t> i32s;
};

struct QwenAsrGgufWriter {
    struct Tensor {
        std::string name;
        ggml_type type = GGML_TYPE_F32;
        std::vector<int64_t> ne;   // GGML order: ne[0] is the contiguous dimension
        const void * data = nullptr;
    };
    std::vector<QwenAsrGgufValue> values;
    std::vector<Tensor> tensors;
    size_t alignment = 32;         // written as general.alignment when not 32
};

void qwenasr_gguf_writer_set_u32(QwenAsrGgufWriter * w, const std::string & key, uint32_t v);
void qwenasr_gguf_writer_set_f32(QwenAsrGgufWriter * w, const std::string & key, float v);
void qwenasr_gguf_writer_set_str(QwenAsrGgufWriter * w, const std::string & key, const std::string & v);
void qwenasr_gguf_writer_set_arr_str(QwenAsrGgufWriter * w, const std::string & key, std::vector<std::string> v);
void qwenasr_gguf_writer_set_arr_i32(QwenAsrGgufWriter * w, const std::string & key, std::vector<int32_t> v);
void qwenasr_gguf_writer_add_tensor(QwenAsrGgufWriter * w, const std::string & name, ggml_type type,
                                    std::vector<int64_t> ne, const void * data);
bool qwenasr_gguf_writer_write(const QwenAsrGgufWriter & w, const char * path, std::string * error);

// String metadata and the element count of an array key of an opened GGUF file; false when absent.
bool qwenasr_gguf_model_get_str(const QwenAsrGgufModel & model, const char * key, std::string * out);
bool qwenasr_gguf_model_get_array_len(const QwenAsrGgufModel & model, const char * key, uint64_t * out);
