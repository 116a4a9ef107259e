// Declarations of the GGML/GGUF type names that the reference's public headers expose
// (src/gguf-model.h:3-33, src/ggml-backends.h:7-23).  GGML itself is not part of this build:
// ggml_backend_t and the two contexts are opaque handles owned by this library, and ggml_type keeps
// the GGUF on-disk type ids (F32 = 0, F16 = 1, BF16 = 30) so tensor views read the same numbers.
#pragma once

#include <cstdint>

enum ggml_type : int32_t {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_BF16 = 30,
    GGML_TYPE_COUNT = 40,
};

struct ggml_context;
struct gguf_context;
struct ggml_backend;
typedef struct ggml_backend * ggml_backend_t;
