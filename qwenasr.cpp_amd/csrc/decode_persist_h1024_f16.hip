// Persistent decode step kernels for the 0.6B (hidden 1024, intermediate 3072) shape with an f16 cache: every batch-1 tiling, f32
// weights and bf16 copies (decode_persist.hpp).
#include "decode_persist.hpp"

namespace qa {
QA_PERSIST_UNIT(h1024_f16, 4, 12, F16)
}  // namespace qa
