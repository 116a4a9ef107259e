// Per-head RMSNorm + NEOX RoPE of one 128-wide head row, computed by one wavefront.
//
// Lane i holds elements i and i + 64, which is exactly one NEOX rotation pair, so the norm needs one
// wave reduction and the rotation needs no data exchange.  The arithmetic follows the reference's
// scalar statement (rms_norm_row, text-decoder.cpp:542-557; apply_rope_position, 604-625):
// squares summed in double, scale = 1 / sqrtf(float(ms) + eps), (x * scale) * w, angle = pos * inv_freq
// in double with inv_freq = exp(-ln(theta) * 2i / d) computed on the host in double, no FMA
// contraction.  Every kernel that prepares q or k goes through this one function, so the fused decode
// kernel and the separate append kernel produce identical bits.
#pragma once

#include "common.hpp"
#include "wave.hpp"

namespace qa {

// cos and sin of the RoPE angle pos * inv_freq, evaluated in double and rounded to f32 (the
// reference's apply_rope_position, text-decoder.cpp:604-625).
__device__ inline void rope_cos_sin(int pos, double inv_freq, float & c, float & s) {
    double sn, cs;
    sincos(static_cast<double>(pos) * inv_freq, &sn, &cs);
    c = static_cast<float>(cs);
    s = static_cast<float>(sn);
}

// a = x[lane], b = x[lane + 64] in, rotated pair out; wa = w[lane], wb = w[lane + 64] of the norm
// weight, (c, s) = rope_cos_sin of this lane's frequency (passed as values, so a caller can issue
// every load of its prologue before the first use and share one angle evaluation between heads).
__device__ inline void norm_rope_pair_cs(float & a, float & b, float wa, float wb, float eps, float c, float s) {
#pragma clang fp contract(off)
    const double ss = wave_sum_d_all(static_cast<double>(a) * a + static_cast<double>(b) * b);
    const double ms = ss / static_cast<double>(kHeadDim);
    const float scale = 1.0f / sqrtf(static_cast<float>(ms) + eps);
    const float na = a * scale * wa;
    const float nb = b * scale * wb;
    a = na * c - nb * s;
    b = nb * c + na * s;
}

__device__ inline void norm_rope_pair(float & a, float & b, float wa, float wb, float eps, int pos,
                                      double inv_freq) {
    float c, s;
    rope_cos_sin(pos, inv_freq, c, s);
    norm_rope_pair_cs(a, b, wa, wb, eps, c, s);
}

__device__ inline void norm_rope_pair(float & a, float & b, const float * w, float eps, int pos,
                                      const RopeTable & rope, int lane) {
    norm_rope_pair(a, b, w[lane], w[lane + 64], eps, pos, rope.inv_freq[lane]);
}

}  // namespace qa
