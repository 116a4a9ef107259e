// Persistent decode step kernels for the 1.7B (hidden 2048, intermediate 6144) shape with an f16 cache: every batch-1 tiling, f32
// weights and bf16 copies (decode_persist.hpp).
#include "decode_persist.hpp"

namespace qa {
QA_PERSIST_UNIT(h2048_f16, 8, 24, F16)
}  // namespace qa
