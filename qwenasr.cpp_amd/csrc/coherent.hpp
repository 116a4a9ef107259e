// Stores of data that workgroups of the same launch on other XCDs read.
//
// gfx950 has one L2 per XCD, and the L2s are not coherent with each other.  Between launches the kernel
// boundary writes back and invalidates them, so plain loads and stores suffice there (COH = false).
// Inside one launch that spans several phases (the persistent decode step) two rules make a handoff
// between XCDs safe without a fence (which on gfx950 writes back and invalidates the whole L2 of the XCD):
//  - the producer stores with agent-scope atomic stores (global_store ... sc1), which write through to
//    memory, and waits for their acknowledgements (s_waitcnt vmcnt(0)) before it arrives at the barrier;
//  - every address is written at most once per launch and read only after the barrier that follows its
//    write, so no L1 or L2 can hold a copy of the line from before the write (the launch starts with
//    invalidated caches), and plain loads miss to memory.  The persistent step therefore gives every
//    layer its own activation and attention-workspace buffers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qa {

template <bool COH>
__device__ __forceinline__ void st_f(float * p, float v) {
    if constexpr (COH) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}

template <bool COH>
__device__ __forceinline__ void st_u64(uint64_t * p, uint64_t v) {
    if constexpr (COH) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}

// One cache element (f16 or f32).
template <bool COH>
__device__ __forceinline__ void st_cache(_Float16 * p, _Float16 v) {
    if constexpr (COH) {
        __hip_atomic_store(reinterpret_cast<uint16_t *>(p), __builtin_bit_cast(uint16_t, v), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    } else {
        *p = v;
    }
}

template <bool COH>
__device__ __forceinline__ void st_cache(float * p, float v) {
    st_f<COH>(p, v);
}

}  // namespace qa
