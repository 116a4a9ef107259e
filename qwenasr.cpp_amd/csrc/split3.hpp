// The exact three-part bf16 split of an f32 value, for device code only.
//
// v = hi + mid + lo exactly: hi is v truncated to its top 8 significant bits (the high half of its bits),
// mid the same truncation of the remainder, lo the last remainder, which has at most 8 significant bits
// and so is its own high half.  Every product of a bf16 weight with one part is exact in f32, which is how
// the prefill GEMMs on bf16-exact weights reproduce f32 products on bf16 MFMA.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qa {

// the three parts of v as bf16 bits at o[0], o[K], o[2 K]: the layout of one row of a split GEMM input
__device__ inline void store_split3(uint16_t * o, int64_t K, float v) {
    const uint32_t h = __float_as_uint(v) & 0xffff0000u;
    const float r1 = v - __uint_as_float(h);
    const uint32_t m = __float_as_uint(r1) & 0xffff0000u;
    const float r2 = r1 - __uint_as_float(m);
    o[0] = static_cast<uint16_t>(h >> 16);
    o[K] = static_cast<uint16_t>(m >> 16);
    o[2 * K] = static_cast<uint16_t>(__float_as_uint(r2) >> 16);
}

}  // namespace qa
