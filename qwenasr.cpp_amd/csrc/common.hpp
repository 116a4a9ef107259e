// Shared plumbing of the HIP library: error reporting, launch checks, small device helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "qwenasr_amd.h"

namespace qa {

// Thread-local last error, surfaced through qa_last_error().
void set_error(const std::string & msg);
const std::string & last_error();

inline int fail(int code, const std::string & msg) {
    set_error(msg);
    return code;
}

inline int hip_fail(hipError_t e, const char * what) {
    return fail(QA_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

#define QA_HIP(call)                                                   \
    do {                                                               \
        hipError_t qa_e_ = (call);                                     \
        if (qa_e_ != hipSuccess) return ::qa::hip_fail(qa_e_, #call);  \
    } while (0)

#define QA_LAUNCH_CHECK(what)                                          \
    do {                                                               \
        hipError_t qa_e_ = hipGetLastError();                          \
        if (qa_e_ != hipSuccess) return ::qa::hip_fail(qa_e_, what);   \
    } while (0)

inline hipStream_t as_stream(void * s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int kHeadDim = 128;
constexpr int kWave = 64;

// Element offset of (layer, kv, stream, head, pos, 0) in the single K+V allocation.
__host__ __device__ inline int64_t cache_row_offset(int layer, int kv, int stream, int head, int pos,
                                                    int n_streams, int n_kv_heads, int max_seq) {
    return ((((static_cast<int64_t>(layer) * 2 + kv) * n_streams + stream) * n_kv_heads + head) *
                max_seq + pos) * kHeadDim;
}

// Inverse RoPE frequencies, computed on the host with the reference's expression
// exp(-ln(theta) * 2i / d) in double (text-decoder.cpp:611-613) and passed by value.
struct RopeTable {
    double inv_freq[kHeadDim / 2];
};
RopeTable make_rope_table(float theta);

}  // namespace qa
