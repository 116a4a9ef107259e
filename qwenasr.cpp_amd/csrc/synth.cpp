// Seeded synthetic inputs for the Qwen3-ASR text-decoder path.
//
// The reference loads real weights from a GGUF file (src/gguf-model.cpp:164-200) and builds its
// decoder input from audio (src/decoder-input.cpp:26-101).  Neither a checkpoint nor audio exists
// on the machines this build runs on, so every tensor is drawn from a counter-based generator:
//
//   key(name)   = splitmix64_mix(base_seed ^ fnv1a64(name))
//   word(i)     = splitmix64_mix(key + (i + 1) * 0x9E3779B97F4A7C15)   (the i-th splitmix64 output
//                                                                     of a generator seeded with key)
//   uniform(i)  = ((word(i) >> 11) + 0.5) * 2^-53                      in (0, 1), never 0
//   normal(j)   = sqrt(-2 ln uniform(2j)) * cos(2 pi uniform(2j+1))   (Box-Muller, double)
//   value(j)    = (float)(normal(j) * stddev)
//
// Each element depends only on (base_seed, name, index), so the fill is split across host threads
// and still gives the same bits as a serial fill.  The same bits feed the GPU (by upload) and the
// CPU checker, so both sides see identical weights, inputs and cache contents.
#include "qwenasr_amd.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t fnv1a64(const char * s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (; s && *s; ++s) {
        h ^= static_cast<unsigned char>(*s);
        h *= 0x100000001b3ull;
    }
    return h;
}

inline double unit_open(uint64_t w) {
    return (static_cast<double>(w >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

inline uint64_t word_at(uint64_t key, uint64_t i) {
    return mix64(key + (i + 1) * kGamma);
}

inline double normal_at(uint64_t key, uint64_t j) {
    const double u1 = unit_open(word_at(key, 2 * j));
    const double u2 = unit_open(word_at(key, 2 * j + 1));
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586476925286766559 * u2);
}

template <typename Fn>
void parallel_range(size_t n, Fn fn) {
    unsigned hw = std::thread::hardware_concurrency();
    size_t threads = hw == 0 ? 1 : hw;
    threads = std::min<size_t>(threads, 32);
    if (n < (1u << 16) || threads <= 1) {
        fn(size_t{0}, n);
        return;
    }
    std::vector<std::thread> pool;
    const size_t chunk = (n + threads - 1) / threads;
    for (size_t t = 0; t < threads; ++t) {
        const size_t lo = t * chunk;
        const size_t hi = std::min(n, lo + chunk);
        if (lo >= hi) break;
        pool.emplace_back([=] { fn(lo, hi); });
    }
    for (auto & th : pool) th.join();
}

}  // namespace

extern "C" {

uint64_t qa_synth_key(uint64_t base_seed, const char * name) {
    return mix64(base_seed ^ fnv1a64(name));
}

uint64_t qa_synth_word(uint64_t key, uint64_t index) {
    return word_at(key, index);
}

void qa_synth_fill_normal(float * out, size_t n, uint64_t base_seed, const char * name, double stddev) {
    if (!out || n == 0) return;
    const uint64_t key = qa_synth_key(base_seed, name);
    parallel_range(n, [&](size_t lo, size_t hi) {
        for (size_t j = lo; j < hi; ++j) {
            out[j] = static_cast<float>(normal_at(key, j) * stddev);
        }
    });
}

void qa_synth_fill_const(float * out, size_t n, float value) {
    if (!out) return;
    std::fill(out, out + n, value);
}

void qa_synth_fill_ids(int32_t * out, size_t n, uint64_t base_seed, const char * name, int32_t lo, int32_t hi) {
    // Uniform integers in [lo, hi] (inclusive) by the multiply-shift map of the top 32 bits.
    if (!out || n == 0 || hi < lo) return;
    const uint64_t key = qa_synth_key(base_seed, name);
    const uint64_t span = static_cast<uint64_t>(static_cast<int64_t>(hi) - lo + 1);
    for (size_t j = 0; j < n; ++j) {
        const uint64_t top = word_at(key, j) >> 32;
        out[j] = static_cast<int32_t>(lo + static_cast<int64_t>((top * span) >> 32));
    }
}

}  // extern "C"
